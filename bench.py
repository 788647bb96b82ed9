#!/usr/bin/env python3
"""Benchmark of the FP4 delta-CSR sparse layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1]

A step is one pass of the hot path over one batch: forward Y = X.W,
grad-input dX = W^T-gather of G, and nnz-sampled grad-W, on BASELINE config 1
(8192 x 8192, Poisson(164) row lengths, FP4 delta-CSR, batch 64, synthetic
seeded data).  Inputs are resident in HBM before the timed region; `copies`
independent layer + activation sets (> 512 MiB in total) are rotated so the
256 MiB MALL cannot serve a step from the previous one.

Prints ONE JSON line (rank 0).  `value` is GNNZ/s = stored synapses per step
/ step time.  `roofline` is computed live from per-kernel HIP events
(sili_profile_*) recorded on the stream the kernels run on; `cpu_baseline`
times the CPU port (oracle/, OpenMP, the reference's algorithm) on the
host cores of this box.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", type=int, default=1)
    p.add_argument("--copies", type=int, default=0, help="0 = enough for > 512 MiB")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--verbose", action="store_true")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="only run 3 device-to-device copies of MIB MiB (HBM counter calibration)")
    return p.parse_args()


class Hip:
    """The few HIP runtime calls bench.py needs (events, device sync)."""

    def __init__(self):
        for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                self.lib = C.CDLL(name)
                break
            except OSError:
                continue
        L = self.lib
        L.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        L.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        L.hipEventSynchronize.argtypes = [C.c_void_p]
        L.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        L.hipEventDestroy.argtypes = [C.c_void_p]

    def event(self):
        e = C.c_void_p()
        assert self.lib.hipEventCreate(C.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.lib.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        assert self.lib.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert self.lib.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return float(ms.value)

    def sync(self):
        assert self.lib.hipDeviceSynchronize() == 0

    def copy_probe(self, mib):
        """Device-to-device copies of a known size: the runtime's blit kernel
        reads and writes exactly `mib` MiB each, which scales the FETCH_SIZE /
        WRITE_SIZE counters to bytes."""
        L = self.lib
        L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        L.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        L.hipFree.argtypes = [C.c_void_p]
        n = mib << 20
        a, b = C.c_void_p(), C.c_void_p()
        assert L.hipMalloc(C.byref(a), n) == 0 and L.hipMalloc(C.byref(b), n) == 0
        assert L.hipMemset(a, 1, n) == 0
        for _ in range(3):
            assert L.hipMemcpy(b, a, n, 3) == 0  # hipMemcpyDeviceToDevice
        self.sync()
        assert L.hipFree(a) == 0 and L.hipFree(b) == 0
        return n


class CAbi:
    """ctypes view of include/sili_hip.h (the boundary bench.py measures)."""

    class ProfEntry(C.Structure):
        _fields_ = [("name", C.c_char * 56), ("count", C.c_int64), ("total_ms", C.c_double),
                    ("min_ms", C.c_double), ("max_ms", C.c_double)]

    def __init__(self, path):
        L = C.CDLL(path)
        vp = C.c_void_p
        L.sili_last_error.restype = C.c_char_p
        L.sili_forward_dense.argtypes = [vp, vp, C.c_int64, vp, vp]
        L.sili_backward_dense.argtypes = [vp, vp, vp, C.c_int64, vp, vp, vp, C.c_float, vp]
        L.sili_sampled_gradw.argtypes = [vp, vp, vp, C.c_int64, vp, vp, vp]
        L.sili_device_alloc.argtypes = [vp, C.c_size_t, C.POINTER(vp)]
        L.sili_device_free.argtypes = [vp, vp]
        L.sili_memcpy_h2d.argtypes = [vp, vp, vp, C.c_size_t]
        L.sili_stream.restype = vp
        L.sili_stream.argtypes = [vp]
        L.sili_profile_enable.argtypes = [vp, C.c_int]
        L.sili_profile_read.argtypes = [vp, C.POINTER(CAbi.ProfEntry), C.c_int, C.POINTER(C.c_int)]
        self.L = L

    def ck(self, rc):
        if rc != 0:
            raise RuntimeError(f"sili error {rc}: {self.L.sili_last_error().decode()}")

    def alloc(self, h, nbytes):
        p = C.c_void_p()
        self.ck(self.L.sili_device_alloc(h, nbytes, C.byref(p)))
        return p

    def upload(self, h, arr):
        arr = np.ascontiguousarray(arr)
        p = self.alloc(h, arr.nbytes)
        self.ck(self.L.sili_memcpy_h2d(h, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes))
        return p

    def profile(self, h):
        n = C.c_int()
        buf = (CAbi.ProfEntry * 64)()
        self.ck(self.L.sili_profile_read(h, buf, 64, C.byref(n)))
        return {buf[i].name.decode(): (buf[i].count, buf[i].total_ms) for i in range(n.value)}


def measured_traffic(label, config):
    """HBM-side bytes per launch of kernel `label`, from the committed
    rocprofv3 --pmc summary of this workload (FETCH_SIZE and WRITE_SIZE
    scaled by a copy kernel of known size).  None when no summary exists."""
    path = os.path.join(ROOT, "profiles", f"c{config}_step_pmc_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes" and f[1] == label:
            return int(f[2])
    return None


def algorithmic(info, n_in, n_out, B):
    """Algorithmic bytes per launch of each kernel (per-unit figures:
    Bv = 1 B/synapse, Bi = exact ULEB bytes, Bp = 8 B/row, Bs = 4 B per
    row/col scale, activations 4 B per element)."""
    nnz = info["nnz_scattered"]
    Bv, Bi, Bp, Bs = nnz, info["index_bytes"], 8 * (n_in + 1), 4 * (n_in + n_out)
    return {
        "fwd:gather": Bv + Bi + Bp + Bs + 4 * B * n_in + 4 * B * n_out,
        "bwd:gather": Bv + Bi + Bp + Bs + 4 * B * n_out + 4 * B * n_in,
        "bwd:sddmm": Bi + Bp + 4 * B * n_in + 4 * B * n_out + 4 * nnz,
        # fused grad-input + grad-W: W (values, index, row starts, scales),
        # gT and xT read once, dX and GW written once
        "bwd:gather_gradw": Bv + Bi + Bp + Bs + 4 * B * n_out + 4 * B * n_in + 4 * B * n_in + 4 * nnz,
        "fwd:transpose": 8 * B * n_in,
        "bwd:transpose": 8 * B * n_out,
    }


def cpu_baseline(wl, seconds):
    """The CPU port (oracle/: the reference's algorithm, OpenMP, per-thread
    private outputs + serial reduce) on this host, same workload."""
    from oracle import HostLayer, have_ref
    threads = os.cpu_count() or 1
    H = HostLayer(wl.n_in, wl.n_out).load_csr(wl.ptrs, wl.cols, w=wl.q).set_scales(wl.value_scale)
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        H.forward_dense(wl.x, threads=threads)
        H.backward_dense(wl.x, wl.g, threads=threads)
        H.sampled_gradw(wl.x, wl.g, threads=threads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() > t_end or len(times) >= 50:
            break
    med = float(np.median(times))
    out = {"value": round(wl.nnz / med / 1e9, 4), "unit": "GNNZ/s", "cores": threads, "kind": "port",
           "sample": f"full config-{wl.name[1:]} step (fwd + grad-input + sampled grad-W), "
                     f"{len(times)} reps, median {med * 1e3:.1f} ms/step"}
    if have_ref():
        from oracle import RefLayer
        R = RefLayer(wl.n_in, wl.n_out, wl.ptrs, wl.cols, wl.q).set_scales(wl.value_scale)
        R.compact()
        rt = []
        t_end = time.perf_counter() + seconds / 2
        while True:
            t0 = time.perf_counter()
            R.forward_dense(wl.x, threads=threads)
            R.backward_dense(wl.x, wl.g, threads=threads)
            rt.append(time.perf_counter() - t0)
            if time.perf_counter() > t_end or len(rt) >= 30:
                break
        out["reference_fwd_bwd_ms"] = round(float(np.median(rt)) * 1e3, 2)
        out["reference_note"] = ("the reference's own disldo_forward + disldo_backward(lr=0) built from "
                                 "its headers (oracle/_ref); it has no standalone grad-W")
    return out


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the layer is sharded by output "
                                   "columns only on paper, no multi-GPU path is built -- run with --gpus 1"}))
        sys.exit(2)
    if a.copy_probe:
        n = Hip().copy_probe(a.copy_probe)
        print(json.dumps({"copy_probe_bytes": n, "copies": 3}), flush=True)
        return
    import sili__new_amd as hip
    from sili__new_amd.synth import make_config

    wl = make_config(a.config)
    B, n_in, n_out = wl.batch, wl.n_in, wl.n_out
    api = CAbi(hip.LIB_PATH)
    rt = Hip()

    # one layer + activation set per copy, all driven on copy 0's stream
    per_copy = None
    layers, bufs = [], []
    copies = a.copies
    t_build = time.perf_counter()
    while True:
        L = hip.SparseLinearLayer(n_in, n_out, wl.nnz)
        L.load_weights(wl.ptrs, wl.cols, wl.q)
        L.set_value_scales(wl.value_scale)
        L.forward_dense(wl.x[:1])  # flushes scales, sizes workspaces
        h = C.c_void_p(L.handle)
        info = L.info()
        x = api.upload(h, wl.x)
        g = api.upload(h, wl.g)
        y = api.alloc(h, 4 * B * n_out)
        dx = api.alloc(h, 4 * B * n_in)
        gw = api.alloc(h, 4 * max(1, info["nnz_scattered"]))
        layers.append((L, h))
        bufs.append((x, g, y, dx, gw))
        if per_copy is None:
            # weights (both orientations) + activations + outputs + workspaces
            per_copy = 2 * (info["nnz_scattered"] + info["index_bytes"]) + 4 * B * (3 * n_in + 3 * n_out) \
                + 4 * info["nnz_scattered"]
            if copies <= 0:
                copies = max(2, int(np.ceil(512 * 2**20 / per_copy)) + 1)
        if len(layers) >= copies:
            break
    t_build = time.perf_counter() - t_build
    stream = api.L.sili_stream(layers[0][1])

    def step(i):
        (_, h), (x, g, y, dx, gw) = layers[i % copies], bufs[i % copies]
        api.ck(api.L.sili_forward_dense(h, x, B, y, stream))
        # x = NULL: backward reads the forward's stored input (feature-major
        # copy), as the reference's backward_dense reads its last_input
        api.ck(api.L.sili_backward_dense(h, None, g, B, dx, gw, None, 0.0, stream))

    for i in range(a.warmup):
        step(i)
    rt.sync()

    # timed region: exactly K steps, bracketed by device syncs
    e0, e1 = rt.event(), rt.event()
    rt.sync()
    rt.record(e0, stream)
    t0 = time.perf_counter()
    for i in range(a.steps):
        step(i)
    rt.record(e1, stream)
    rt.sync()
    wall = time.perf_counter() - t0
    ms = rt.elapsed_ms(e0, e1)
    ms_step = ms / a.steps

    # warm (cache-resident) rate: a single copy, same step count
    w0, w1 = rt.event(), rt.event()
    rt.sync()
    rt.record(w0, stream)
    for i in range(a.steps):
        step(0)
    rt.record(w1, stream)
    rt.sync()
    warm_ms_step = rt.elapsed_ms(w0, w1) / a.steps

    # profiled pass (same steps): per-kernel HIP events on the launch stream
    for _, h in layers:
        api.ck(api.L.sili_profile_enable(h, 1))
    p0, p1 = rt.event(), rt.event()
    rt.record(p0, stream)
    for i in range(a.steps):
        step(i)
    rt.record(p1, stream)
    rt.sync()
    prof_ms_step = rt.elapsed_ms(p0, p1) / a.steps
    kern = {}
    for _, h in layers:
        for name, (cnt, tot) in api.profile(h).items():
            c0, t0_ = kern.get(name, (0, 0.0))
            kern[name] = (c0 + cnt, t0_ + tot)
        api.ck(api.L.sili_profile_enable(h, 0))
    info = layers[0][0].info()
    alg = algorithmic(info, n_in, n_out, B)
    dom = max(kern.items(), key=lambda kv: kv[1][1])
    dom_name, (dom_cnt, dom_tot) = dom
    dom_avg_ms = dom_tot / dom_cnt
    dom_bytes = alg.get(dom_name)
    achieved = dom_bytes / (dom_avg_ms * 1e-3) / 1e9 if dom_bytes else None

    nnz = info["nnz_scattered"]
    # one step's algorithmic bytes: forward + grad-input + sampled grad-W,
    # each op counted as if run alone (the fused backward moves less)
    step_bytes = alg["fwd:gather"] + alg["bwd:gather"] + alg["bwd:sddmm"]
    gnnz = nnz / (ms_step * 1e-3) / 1e9
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9
    flops = 3 * 2 * nnz * B

    out = {
        "metric": "FP4 delta-CSR SpMM GNNZ/s + achieved HBM GB/s (% of peak), fwd+bwd",
        "value": round(gnnz, 4),
        "unit": "GNNZ/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": f"config {a.config}: {n_in}x{n_out} FP4 delta-CSR, Poisson(164) rows, batch {B}; "
                        "step = forward + grad-input + nnz-sampled grad-W",
            "n_in": n_in, "n_out": n_out, "batch": B, "nnz": nnz, "index_bytes": info["index_bytes"],
            "copies_rotated": copies, "rotation_mib": round(copies * per_copy / 2**20, 1),
        },
        "achieved_gbs": round(step_gbs, 2),
        "pct_hbm_peak": round(100.0 * step_gbs / HBM_PEAK_GBS, 3),
        "gflops": round(flops / (ms_step * 1e-3) / 1e9, 2),
        "warm_ms_per_step": round(warm_ms_step, 5),
        "warm_value": round(nnz / (warm_ms_step * 1e-3) / 1e9, 4),
        "wall_s_timed": round(wall, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": dom_name,
            "achieved": round(achieved, 2) if achieved else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 5) if achieved else None,
            "traffic": measured_traffic(dom_name, a.config),
            "avg_launch_ms": round(dom_avg_ms, 5),
            "algorithmic_bytes": dom_bytes,
        },
        "kernels_ms_per_step": {k: round(v[1] / a.steps, 5) for k, v in kern.items()},
        "profiled_ms_per_step": round(prof_ms_step, 5),
    }
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(wl, a.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    if a.verbose:
        print(f"build {t_build:.1f}s copies {copies}", file=sys.stderr)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
