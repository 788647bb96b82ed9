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
host cores of this box, in child processes that never touch the GPU, at the
host share's thread count and at one thread.
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
    p.add_argument("--no-configs", action="store_true",
                   help="config 1: leave out the summary of configs 2, 3 and 4 timed after the line's own step")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--synapto-reps", type=int, default=5, help="config 3: timed synaptogenesis steps")
    p.add_argument("--c4-batches", default="1,8,128", help="config 4: token batches to time")
    p.add_argument("--synap-cycles", type=int, default=0,
                   help="config 1: also time N cycles of the reference's synaptogenesis policy "
                        "(build_probes + synap_step)")
    p.add_argument("--train-lr", type=float, default=0.0,
                   help="config 1: the backward carries the optimizer update at this learning rate "
                        "(stochastic re-quantization, as the reference's SparseLinearLayer)")
    p.add_argument("--verbose", action="store_true")
    p.add_argument("--index-decode", type=int, default=0, metavar="G",
                   help="only time decoding every column of the config-4 q layer from the ULEB128 stream and "
                        "from a FOR index of group size G")
    p.add_argument("--sparse-sweep", action="store_true",
                   help="only time the sparse-input forward of the config-2 layer at several input densities, "
                        "pushed from the canonical store and gathered through the shadow store")
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
        L.sili_forward_sparse.argtypes = [vp, vp, vp, vp, C.c_int64, C.c_int64, vp, vp]
        L.sili_backward_sparse.argtypes = [vp, vp, vp, vp, vp, C.c_int64, C.c_int64, vp, C.c_float, vp]
        L.sili_device_alloc.argtypes = [vp, C.c_size_t, C.POINTER(vp)]
        L.sili_device_free.argtypes = [vp, vp]
        L.sili_memcpy_h2d.argtypes = [vp, vp, vp, C.c_size_t]
        L.sili_stream.restype = vp
        L.sili_stream.argtypes = [vp]
        L.sili_profile_enable.argtypes = [vp, C.c_int]
        L.sili_profile_read.argtypes = [vp, C.POINTER(CAbi.ProfEntry), C.c_int, C.POINTER(C.c_int)]
        L.sili_device_free.argtypes = [vp, vp]
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


def uleb_row_bytes(ptrs, cols):
    """Exact ULEB128 bytes of every row (deltas restart at 0 per row)."""
    ptrs = np.asarray(ptrs, np.int64)
    cols = np.asarray(cols, np.int64)
    prev = np.zeros(len(cols), np.int64)
    if len(cols):
        prev[1:] = cols[:-1]
        starts = ptrs[:-1][np.diff(ptrs) > 0]
        prev[starts] = 0
    d = cols - prev
    lens = np.ones(len(cols), np.int64)
    for k in (7, 14, 21, 28):
        lens += d >= (1 << k)
    csum = np.concatenate([[0], np.cumsum(lens)])
    return csum[ptrs[1:]] - csum[ptrs[:-1]]


def algorithmic(info, n_in, n_out, B, wl=None):
    """Algorithmic bytes per launch of each kernel (per-unit figures:
    Bv = 1 B/synapse, Bi = exact ULEB bytes, Bp = 8 B/row, Bs = 4 B per
    row/col scale, activations 4 B per element; block4: 16 B/tile + exact
    block-index bytes + 8 B per block row)."""
    nnz = info["nnz_scattered"]
    Bv, Bi, Bp, Bs = nnz, info["index_bytes"], 8 * (n_in + 1), 4 * (n_in + n_out)
    out = {
        "fwd:gather": Bv + Bi + Bp + Bs + 4 * B * n_in + 4 * B * n_out,
        "bwd:gather": Bv + Bi + Bp + Bs + 4 * B * n_out + 4 * B * n_in,
        "bwd:sddmm": Bi + Bp + 4 * B * n_in + 4 * B * n_out + 4 * nnz,
        # fused grad-input + grad-W: W (values, index, row starts, scales),
        # gT and xT read once, dX and GW written once
        "bwd:gather_gradw": Bv + Bi + Bp + Bs + 4 * B * n_out + 4 * B * n_in + 4 * B * n_in + 4 * nnz,
        "fwd:transpose": 8 * B * n_in,
        "bwd:transpose": 8 * B * n_out,
        # optimizer update over the canonical store: value bytes read and
        # written, index, row starts (byte + element), the row's scale and its
        # RMSprop state read and written (vs, importance, step: 12 B), output
        # scales, xT and gT read, dX written
        "bwd:train_rows": 2 * Bv + Bi + Bp + 2 * 12 * n_in + 4 * n_out + 4 * B * n_in + 4 * B * n_out
                          + 4 * B * n_in,
        # shadow value bytes refreshed through the kept permutation
        "bwd:train_shadow": 4 * nnz + nnz + nnz,
    }
    # batch-1 byte-split kernels move the same algorithmic bytes as the gather
    for op in ("fwd", "bwd"):
        for k in ("stream", "stream_lds"):
            out[f"{op}:{k}"] = out[f"{op}:gather"]
    T = info.get("n_tiles", 0)
    if T:
        bi = info.get("block_index_bytes", 0)
        Bt_in = 16 * T + bi + 8 * ((n_in + 3) // 4 + 1)
        Bt_out = 16 * T + bi + 8 * ((n_out + 3) // 4 + 1)
        out["fwd:gather_b4"] = Bt_out + Bs + 4 * B * n_in + 4 * B * n_out
        out["bwd:gather_b4"] = Bt_in + Bs + 4 * B * n_out + 4 * B * n_in
        out["bwd:sddmm_b4"] = (Bt_in - 16 * T) + 4 * B * n_in + 4 * B * n_out + 4 * 16 * T
        # optimizer update of the tiles: tile bytes read and written, block
        # index and row starts, xT and gT read, dX read and written, the
        # rows' scales and RMSprop state read and written, output scales
        out["bwd:train_b4"] = (Bt_in + 16 * T) + 4 * B * n_in + 4 * B * n_out + 8 * B * n_in \
            + 2 * 12 * n_in + 4 * n_out
    if wl is not None and wl.x_ptrs is not None and wl.cols is not None:
        # sparse-input forward: value + index bytes of the rows any batch row
        # activates, row starts, scales, the input CSR and the dense output
        active = np.zeros(n_in, bool)
        active[np.asarray(wl.x_idx, np.int64)] = True
        rb = uleb_row_bytes(wl.ptrs, wl.cols)
        rl = np.diff(np.asarray(wl.ptrs, np.int64))
        s_act = int((rb[active] + rl[active]).sum())
        out["fwd_sparse:gather"] = s_act + Bp + Bs + 8 * len(wl.x_idx) + 4 * (B + 1) + 4 * B * n_out
    return out


STEP_DOC = {
    0: "step = forward (batch 1)",
    1: "step = forward + grad-input + nnz-sampled grad-W",
    2: "step = sparse-input forward (10% active inputs per batch row) + grad-input",
    3: "step = block4 forward + grad-input + nnz-sampled grad-W (every slot)",
}


def workload_text(cfg, wl):
    shapes = {0: "205 distinct columns per row", 1: "Poisson(164) rows", 2: "Zipf(1.2) rows, 1% density",
              3: "block4 tiles at 3% block density, every slot live"}
    fmt = "FP4 block4" if cfg == 3 else "FP4 delta-CSR"
    return f"config {cfg}: {wl.n_in}x{wl.n_out} {fmt}, {shapes[cfg]}, batch {wl.batch}; {STEP_DOC[cfg]}"


def build_copy(cfg, wl, hip, api):
    """One layer plus its device-resident activations for config `cfg`."""
    B, n_in, n_out = wl.batch, wl.n_in, wl.n_out
    n_tiles = 0 if wl.tile_br is None else len(wl.tile_br)
    L = hip.SparseLinearLayer(n_in, n_out, max(1, wl.nnz + 16 * n_tiles))
    if wl.cols is not None:
        L.load_weights(wl.ptrs, wl.cols, wl.q)
    if wl.tile_br is not None:
        L.load_block4_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes)
    L.set_value_scales(wl.value_scale)
    L.forward_dense(wl.x[:1])  # flushes scales, sizes workspaces
    h = C.c_void_p(L.handle)
    info = L.info()
    d = {"L": L, "h": h, "info": info, "x": api.upload(h, wl.x.astype(np.float32)),
         "y": api.alloc(h, 4 * B * n_out)}
    if cfg != 0:
        d["g"] = api.upload(h, wl.g.astype(np.float32))
        d["dx"] = api.alloc(h, 4 * B * n_in)
    if cfg == 1:
        d["gws"] = api.alloc(h, 4 * max(1, info["nnz_scattered"]))
    if cfg == 3:
        d["gwb"] = api.alloc(h, 4 * 16 * max(1, info["n_tiles"]))
    if cfg == 2:
        d["xp"] = api.upload(h, np.asarray(wl.x_ptrs, np.int32))
        d["xi"] = api.upload(h, np.asarray(wl.x_idx, np.int32))
        d["xv"] = api.upload(h, np.asarray(wl.x_vals, np.float32))
        d["nnz_x"] = len(wl.x_idx)
    # weights (both orientations) + activations + outputs + workspaces
    d["bytes"] = (2 * (info["nnz_scattered"] + info["index_bytes"]) + 2 * 16 * info["n_tiles"]
                  + 4 * B * (3 * n_in + 3 * n_out) + 4 * info["nnz_scattered"] + 4 * 16 * info["n_tiles"])
    return d


def release_pool(api, pool):
    """Free every copy's device buffers, then its layer (sili_destroy through
    the binding object's destructor), in that order."""
    for d in pool:
        for k in ("x", "y", "g", "dx", "gws", "gwb", "xp", "xi", "xv"):
            if k in d:
                api.ck(api.L.sili_device_free(d["h"], d[k]))
        d.clear()
    pool.clear()


def make_step(cfg, api, B, stream, train_lr=0.0):
    L = api.L

    def step(d):
        h = d["h"]
        if cfg == 2:
            api.ck(L.sili_forward_sparse(h, d["xp"], d["xi"], d["xv"], d["nnz_x"], B, d["y"], stream))
            api.ck(L.sili_backward_dense(h, d["x"], d["g"], B, d["dx"], None, None, 0.0, stream))
            return
        api.ck(L.sili_forward_dense(h, d["x"], B, d["y"], stream))
        if cfg == 1:
            # x = NULL: backward reads the forward's stored input (feature-major
            # copy), as the reference's backward_dense reads its last_input
            if train_lr:
                api.ck(L.sili_backward_dense(h, None, d["g"], B, d["dx"], None, None, train_lr, stream))
            else:
                api.ck(L.sili_backward_dense(h, None, d["g"], B, d["dx"], d["gws"], None, 0.0, stream))
        elif cfg == 3:
            if train_lr:
                api.ck(L.sili_backward_dense(h, None, d["g"], B, d["dx"], None, None, train_lr, stream))
            else:
                api.ck(L.sili_backward_dense(h, None, d["g"], B, d["dx"], None, d["gwb"], 0.0, stream))
    return step


def _time_reps(step, seconds, max_reps, min_reps=2):
    """Wall time of `step` repeated for about `seconds` (at least min_reps,
    at most max_reps): (best, median) in seconds, reps."""
    times = []
    t_end = time.perf_counter() + seconds
    while True:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_reps or (len(times) >= min_reps and time.perf_counter() > t_end):
            break
    return float(np.min(times)), float(np.median(times)), len(times)


def cpu_child_run(spec):
    """Child-process side of the CPU baseline: builds the workload on the host
    (no GPU is touched in this process) and times the CPU port (oracle/: the
    reference's algorithm -- static row split, per-thread private outputs,
    serial reduce) at spec["threads"] OpenMP threads."""
    from oracle import HostLayer
    from sili__new_amd.synth import make_config
    cfg, threads, seconds = spec["cfg"], spec["threads"], spec["seconds"]
    lr = spec.get("lr", 0.0)
    if cfg == 4:
        z = np.load(spec["layer_file"])
        H = HostLayer(int(z["n_in"]), int(z["n_out"]))
        H.load_encoded(z["row_byte_start"], z["row_elem_start"], z["idx"], z["val"])
        H.set_scales(z["value_scale"])
        x = z["x"]
        best, med, reps = _time_reps(lambda: H.forward_dense(x, threads=threads), seconds, 50)
        units = int(z["nnz"])
        sample = f"forward of the q layer ({units} synapses, 5120x204800) at batch 1"
    else:
        wl = make_config(cfg, scale=spec.get("scale", 1.0))
        ptrs = wl.ptrs if wl.ptrs is not None else np.zeros(wl.n_in + 1, np.int32)
        cols = wl.cols if wl.cols is not None else np.zeros(0, np.int32)
        q = wl.q if wl.q is not None else np.zeros(0, np.float32)
        H = HostLayer(wl.n_in, wl.n_out).load_csr(ptrs, cols, w=q)
        if wl.tile_br is not None:
            H.load_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes)
        H.set_scales(wl.value_scale)
        x, B = wl.x.astype(np.float32), wl.batch
        g = None if wl.g is None else wl.g.astype(np.float32)
        if lr:
            # the update's restatement runs on one thread (its batch steps
            # form a dependent chain per synapse, as in the reference)
            threads = 1

            def step():
                H.forward_dense(x, threads=1)
                H.backward_train(x, g, lr)
            sample = f"full config-{cfg} training step (forward + backward with the update, lr {lr})"
        else:
            def step():
                if cfg == 0:
                    H.forward_dense(x, threads=threads)
                elif cfg == 2:
                    H.forward_sparse(wl.x_ptrs, wl.x_idx, wl.x_vals, B, threads=threads)
                    H.backward_dense(x, g, threads=threads)
                else:
                    H.forward_dense(x, threads=threads)
                    H.backward_dense(x, g, threads=threads)
                    H.sampled_gradw(x, g, threads=threads)
            sample = f"full config-{cfg} step ({STEP_DOC[cfg][7:]})"
        best, med, reps = _time_reps(step, seconds, 50, min_reps=spec.get("min_reps", 2))
        units = len(cols) + (0 if wl.tile_br is None else 16 * len(wl.tile_br))
        if spec.get("scale", 1.0) != 1.0:
            sample += f" at scale {spec['scale']} ({wl.n_in}x{wl.n_out}, {units} synapses)"
    out = {"value": round(units / med / 1e9, 6), "best_value": round(units / best / 1e9, 6), "unit": "GNNZ/s",
           "cores": threads, "kind": "port", "median_ms": round(med * 1e3, 3), "best_ms": round(best * 1e3, 3),
           "sample": f"{sample}, {reps} reps"}
    if cfg == 3 and not lr and spec.get("synapto") and wl.cand_r is not None:
        t0 = time.perf_counter()
        H.synapto_step(0.01, wl.cand_r, wl.cand_c, wl.cand_v)
        out["synapto_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_host():
    """What the host reports beside its model name (the VMs of the pool name
    only the family): clock, CPUs online and usable by this process, load
    averages when the baseline ran -- the context of the baseline's spread."""
    out = {}
    try:
        mhz = [float(l.split(":", 1)[1]) for l in open("/proc/cpuinfo") if l.startswith("cpu MHz")]
        if mhz:
            out["cpu_mhz"] = round(sum(mhz) / len(mhz), 1)
    except (OSError, ValueError):
        pass
    out["cpus_online"] = os.cpu_count()
    try:
        out["cpus_usable"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    try:
        out["loadavg"] = [round(v, 2) for v in os.getloadavg()]
    except OSError:
        pass
    return out


def cpu_baseline(cfg, seconds, lr=0.0, layer_file=None):
    """The CPU baseline, timed in child processes (nothing of the GPU process's
    state, and no GPU, in them) with OMP_NUM_THREADS pinned: at the host
    share's thread count (OMP_NUM_THREADS, else the core count) and at one
    thread.  `value` is the multi-thread median; best-of-reps beside it."""
    import subprocess
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)

    def child(t, **extra):
        spec = {"cfg": cfg, "threads": t, "seconds": seconds, "lr": lr, "layer_file": layer_file, **extra}
        print(f"cpu baseline: config {cfg}, {t} thread(s) {extra or ''}", file=sys.stderr, flush=True)
        env = dict(os.environ, OMP_NUM_THREADS=str(t))
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", json.dumps(spec)], env=env,
                           capture_output=True, text=True, timeout=170)
        if r.returncode != 0:
            raise RuntimeError(f"CPU baseline child exited {r.returncode}: {r.stderr[-400:]}")
        return json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])

    runs = {}
    try:
        runs[threads] = child(threads, synapto=True)
        if threads > 1:
            # one thread: the full workload when about 16x the multi-thread
            # step fits the budget, else a smaller instance of the same config
            # (work ~ scale^2 for configs 1-3)
            est = runs[threads]["median_ms"] * 1e-3 * threads
            scale = 1.0
            while cfg in (1, 2, 3) and est * scale * scale > 2.5 * seconds and scale > 1.0 / 16:
                scale /= 2
            runs[1] = child(1, min_reps=1, scale=scale) if scale != 1.0 else child(1, min_reps=1)
    except (RuntimeError, subprocess.TimeoutExpired) as e:
        if not runs:
            return {"error": str(e)[-400:]}
    out = dict(runs[max(runs)])
    out["cpu_model"] = cpu_model()
    out["host"] = cpu_host()
    out["isolated"] = "child process per thread count, OMP_NUM_THREADS pinned"
    if 1 in runs and max(runs) > 1:
        out["one_thread"] = {k: runs[1][k] for k in ("value", "best_value", "median_ms", "best_ms", "sample")}
    return out


def time_synapto(hip, wl, reps):
    """GPU bulk synaptogenesis on config 3: prune 1% by |w|, regrow at fresh
    seeded candidates, rebuild both stores; wall time of the synchronous call
    (candidate upload included)."""
    from sili__new_amd.synth import SEED0, Stream
    n_tiles = len(wl.tile_br)
    L = hip.SparseLinearLayer(wl.n_in, wl.n_out, 16 * n_tiles + 1024)
    L.load_block4_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes)
    L.set_value_scales(wl.value_scale)
    L.synchronize()
    cands = [(wl.cand_r, wl.cand_c, wl.cand_v)]
    m = len(wl.cand_r)
    for i in range(1, reps + 1):
        st = Stream(SEED0 + 3, 100 + i)
        cands.append((st.integers(m, wl.n_in).astype(np.int32), st.integers(m, wl.n_out).astype(np.int32),
                      Stream(SEED0 + 3, 200 + i).normal(m, 0.01)))
    L.synapto_step(0.01, *cands[0])  # warm-up (allocations, code objects)
    times, stats = [], None
    for i in range(1, reps + 1):
        t0 = time.perf_counter()
        stats = L.synapto_step(0.01, *cands[i])
        times.append((time.perf_counter() - t0) * 1e3)
    return {"ms_median": round(float(np.median(times)), 3), "ms_min": round(min(times), 3), "reps": reps,
            "last_stats": stats}


def time_synap_policy(hip, wl, reps, seconds):
    """The reference's synaptogenesis cycle as DISLDOLayer.synaptogenesis
    runs it (sili/sparse_rnn.py:216-219): build_probes(4) + synap_step, on
    config 1 after one backward fills the activity accumulators.  Wall time
    per cycle on the GPU layer (host decisions, device edit and rebuild), and
    the reference's own functions (oracle/_ref) on the same layer."""
    from oracle import RefLayer, have_ref
    L = hip.SparseLinearLayerDeterministic(wl.n_in, wl.n_out, 2 * wl.nnz + 4096)
    L.load_weights(wl.ptrs, wl.cols, wl.q)
    L.expand_headroom(1.0)  # the rows' room the reference layer below is built with
    L.set_value_scales(wl.value_scale)
    x, g = wl.x.astype(np.float32), wl.g.astype(np.float32)
    L.forward_dense(x)
    L.backward_dense(g, 0.0)
    ai, ag = L.neuron_input_accum.copy(), L.neuron_grad_accum.copy()
    L.synchronize()
    cutoff, max_rw = 0.3, 200
    L.build_probes(4)
    L.synap_step(cutoff, max_rw)  # warm-up
    times, t_probe, edits = [], [], 0
    for i in range(reps):
        n0 = L.info()["nnz_scattered"]
        t0 = time.perf_counter()
        L.build_probes(4)
        t1 = time.perf_counter()
        L.synap_step(cutoff, max_rw)
        L.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
        t_probe.append((t1 - t0) * 1e3)
        edits += L.info()["nnz_scattered"] != n0
    out = {"gpu_ms_median": round(float(np.median(times)), 3), "gpu_ms_min": round(min(times), 3), "reps": reps,
           "build_probes_ms_median": round(float(np.median(t_probe)), 3),
           "cycles_that_edited": edits,
           "cycle": "build_probes(4) + synap_step(importance_cutoff 0.3, max_row_weights 200)"}
    # the same cycle after a call that may change the accumulators (as a
    # training step's backward does): build_probes stages them again
    times_r = []
    for i in range(reps):
        L.forward_dense(x[:1])  # untimed; ends the validity of the staged accumulators
        L.synchronize()
        t0 = time.perf_counter()
        L.build_probes(4)
        L.synap_step(cutoff, max_rw)
        L.synchronize()
        times_r.append((time.perf_counter() - t0) * 1e3)
    out["gpu_ms_median_restaged"] = round(float(np.median(times_r)), 3)
    out["restaged_note"] = ("each cycle after an untimed forward_dense, so build_probes re-reads the "
                            "accumulators; gpu_ms_median: back-to-back cycles, which keep them")
    # FoldedLayer's sweep (sili/sparse_rnn.py:1206-1212): build_probes once,
    # synap_step on every row, then the next entry point writes the edits;
    # deferred (one flush for the sweep) and patched per call
    def sweep():
        t0 = time.perf_counter()
        L.build_probes(4)
        for _ in range(wl.n_in):
            L.synap_step(cutoff, max_rw)
        L.synchronize()
        return (time.perf_counter() - t0) * 1e3
    out["sweep_rows"] = wl.n_in
    out["sweep_ms_deferred"] = round(min(sweep() for _ in range(2)), 2)
    os.environ["SILI_POLICY_DEFER"] = "0"
    try:
        out["sweep_ms_patch_per_call"] = round(sweep(), 2)
    finally:
        del os.environ["SILI_POLICY_DEFER"]
    if have_ref():
        R = RefLayer(wl.n_in, wl.n_out, wl.ptrs, wl.cols, wl.q, blank_fraction=1.0)
        rt, cur = [], 0
        t_end = time.perf_counter() + seconds
        try:
            while len(rt) < reps and time.perf_counter() < t_end:
                t0 = time.perf_counter()
                R.build_probes(ai, ag, 4)
                _, cur = R.synap_row_step(cur, cutoff, max_rw)
                rt.append((time.perf_counter() - t0) * 1e3)
        except RuntimeError as e:  # a row out of its reserved space
            out["reference_error"] = str(e)
        if rt:
            out["reference_ms_median"] = round(float(np.median(rt)), 4)
            if "reference_error" not in out:
                t0 = time.perf_counter()
                try:
                    R.build_probes(ai, ag, 4)
                    for _ in range(wl.n_in):
                        _, cur = R.synap_row_step(cur, cutoff, max_rw)
                    out["reference_sweep_ms"] = round((time.perf_counter() - t0) * 1e3, 2)
                except RuntimeError as e:
                    out["reference_error"] = str(e)
        out["reference_note"] = "the reference's delta_csr_build_probes + delta_csr_synap_row_step, one host thread"
    return out


# config 4: the 7 layer shapes of a folded 40 x Mistral-24B-like block stack
# (SURVEY 8(d)): (name, n_in, n_out); 10% of each kept, |N(0, 0.02)| tail above
# its 95th percentile, per-row FP4 scales, decode forward at batch 1 / 8 / 128
C4_LAYERS = [("q", 5120, 204800), ("k", 5120, 204800), ("v", 5120, 204800), ("o", 5120, 204800),
             ("gate", 5120, 1310720), ("up", 5120, 1310720), ("down", 32768, 204800)]
C4_BATCHES = (1, 8, 128)


def run_config4(a, hip, api, rt):
    from sili__new_amd.synth import SEED0, Stream
    t_build = time.perf_counter()
    layers = []
    for i, (name, n_in, n_out) in enumerate(C4_LAYERS):
        L = hip.SparseLinearLayer(n_in, n_out, 1)
        nnz = L.load_synthetic(SEED0 + 4 + 1000 * i, 0.1, 0.02, 0.95)
        h = C.c_void_p(L.handle)
        info = L.info()
        layers.append({"name": name, "L": L, "h": h, "n_in": n_in, "n_out": n_out, "nnz": nnz, "info": info})
    t_build = time.perf_counter() - t_build
    nnz_total = sum(d["nnz"] for d in layers)
    stream = api.L.sili_stream(layers[0]["h"])
    results = {}
    for B in [int(b) for b in a.c4_batches.split(",")]:
        for i, d in enumerate(layers):
            x = Stream(SEED0 + 4, 10 + 100 * B + i).normal(B * d["n_in"]).astype(np.float32)
            d["x"] = api.upload(d["h"], x)
            d["y"] = api.alloc(d["h"], 4 * B * d["n_out"])

        def step():
            for d in layers:
                api.ck(api.L.sili_forward_dense(d["h"], d["x"], B, d["y"], stream))
        steps = max(3, a.steps // (10 if B == 1 else 50 if B == 8 else 200))
        for _ in range(max(1, a.warmup // 5)):
            step()
        rt.sync()
        e0, e1 = rt.event(), rt.event()
        rt.record(e0, stream)
        for _ in range(steps):
            step()
        rt.record(e1, stream)
        rt.sync()
        ms = rt.elapsed_ms(e0, e1) / steps
        for d in layers:
            api.ck(api.L.sili_profile_enable(d["h"], 1))
        step()
        rt.sync()
        kern = {}  # per step (one profiled step; an op may take several launches)
        for d in layers:
            for name, (cnt, tot) in api.profile(d["h"]).items():
                kern[f"{d['name']}:{name}"] = tot
            api.ck(api.L.sili_profile_enable(d["h"], 0))
        # algorithmic bytes per layer forward (SURVEY 8(d) dense-input fwd)
        alg = {}
        for d in layers:
            info = d["info"]
            alg[d["name"]] = (info["nnz_scattered"] + info["index_bytes"] + 8 * (d["n_out"] + 1)
                              + 4 * (d["n_in"] + d["n_out"]) + 4 * B * (d["n_in"] + d["n_out"]))
        step_bytes = sum(alg.values())
        gath = {k: v for k, v in kern.items() if k.split(":")[-1] in ("gather", "stream", "stream_lds", "gather_staged")}
        dom = max(gath.items(), key=lambda kv: kv[1])
        dom_layer = dom[0].split(":")[0]
        ach = alg[dom_layer] / (dom[1] * 1e-3) / 1e9
        results[B] = {"ms_per_step": round(ms, 4), "gnnz_s": round(nnz_total / (ms * 1e-3) / 1e9, 3),
                      "achieved_gbs": round(step_bytes / (ms * 1e-3) / 1e9, 2),
                      "pct_hbm_peak": round(100 * step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                      "steps": steps, "kernels_ms": {k: round(v, 4) for k, v in kern.items()},
                      "layer_algorithmic_bytes": alg,
                      "dominant": {"kernel": dom[0], "op_ms": round(dom[1], 4),
                                   "algorithmic_bytes": alg[dom_layer], "achieved_gbs": round(ach, 2),
                                   "frac": round(ach / HBM_PEAK_GBS, 4)}}
        for d in layers:
            api.ck(api.L.sili_device_free(d["h"], d["x"]))
            api.ck(api.L.sili_device_free(d["h"], d["y"]))
    b_main = 1 if 1 in results else min(results)  # the line's batch: 1 unless not run
    r1 = results[b_main]
    out = {
        "metric": "FP4 delta-CSR SpMM GNNZ/s + achieved HBM GB/s (% of peak), fwd+bwd",
        "value": r1["gnnz_s"], "unit": "GNNZ/s", "n_gpus": 1, "steps": r1["steps"], "warmup": a.warmup,
        "ms_per_step": r1["ms_per_step"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (seeded, generated on the device)",
        "config": {"workload": "config 4: folded 40-block Mistral-24B-like stack, 7 FP4 delta-CSR layers "
                               "(q,k,v,o 5120x204800; gate,up 5120x1310720; down 32768x204800) at 10% density; "
                               f"step = decode forward of all 7 layers at batch {b_main} (every batch run below)",
                   "nnz": nnz_total, "layers": {d["name"]: d["nnz"] for d in layers},
                   "index_bytes": sum(d["info"]["index_bytes"] for d in layers)},
        "achieved_gbs": r1["achieved_gbs"], "pct_hbm_peak": r1["pct_hbm_peak"],
        "roofline": {"bound": "hbm", "kernel": r1["dominant"]["kernel"], "achieved": r1["dominant"]["achieved_gbs"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": r1["dominant"]["frac"],
                     "traffic": measured_traffic(r1["dominant"]["kernel"], 4) if b_main == 1 else None,
                     "op_ms": r1["dominant"]["op_ms"],
                     "algorithmic_bytes": r1["dominant"]["algorithmic_bytes"]},
        "batches": {str(B): r for B, r in results.items()},
        "build_s": round(t_build, 2),
    }
    cpu = None if a.no_cpu_baseline else cpu_baseline_c4(layers[0], a.cpu_seconds)
    for d in layers:  # released while the HIP runtime is fully alive
        d.clear()
    layers.clear()
    out["cpu_baseline"] = cpu
    return out


def run_index_decode(a, hip, api, rt):
    """Column decode of the config-4 q layer (5120 x 204800, ~105 M
    synapses): the ULEB128 stream (wave-parallel varint decode) against the
    FOR index (every column = group start + offset), the latter by its
    lane-per-slot decoder ("for") and by its thread-per-group one.
    Algorithmic bytes: what each decoder must read plus 4 bytes written per
    column."""
    from sili__new_amd.synth import SEED0
    G = a.index_decode
    n_in, n_out = 5120, 204800
    L = hip.SparseLinearLayer(n_in, n_out, 1)
    nnz = L.load_synthetic(SEED0 + 4, 0.1, 0.02, 0.95)
    L.build_for_index(G)
    info = L.info()
    h = C.c_void_p(L.handle)
    for_bytes = len(L.export_for_index()["bytes"])
    cols = api.alloc(h, 4 * nnz)
    stream = api.L.sili_stream(h)
    api.L.sili_decode_columns.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
    out = {"workload": f"config-4 q layer {n_in}x{n_out}, {nnz} synapses; decode every column",
           "group_size": G, "nnz": nnz, "index_bytes": info["index_bytes"], "for_bytes": for_bytes}
    ngroups = None
    for use_for, name in ((0, "uleb"), (1, "for"), (2, "for_thread_per_group")):
        for _ in range(3):
            api.ck(api.L.sili_decode_columns(h, cols, use_for, stream))
        rt.sync()
        api.ck(api.L.sili_profile_enable(h, 1))
        reps = 20
        for _ in range(reps):
            api.ck(api.L.sili_decode_columns(h, cols, use_for, stream))
        rt.sync()
        prof = api.profile(h)
        api.ck(api.L.sili_profile_enable(h, 0))
        (cnt, tot), = [v for k, v in prof.items() if k.startswith("index:")]
        ms = tot / cnt
        if use_for:
            ngroups = -(-nnz // G)  # at least; rows' short last groups add a few
            read = for_bytes + 12 * ngroups
        else:
            read = info["index_bytes"] + 32 * info["n_segments"]
        alg = read + 4 * nnz
        out[name] = {"ms": round(ms, 4), "gcols_s": round(nnz / (ms * 1e-3) / 1e9, 2),
                     "algorithmic_bytes": alg, "achieved_gbs": round(alg / (ms * 1e-3) / 1e9, 1)}
    api.ck(api.L.sili_device_free(h, cols))
    print(json.dumps(out), flush=True)


def run_sparse_sweep(a, hip, api, rt):
    """forward_sparse on the config-2 layer (16384 x 16384, Zipf rows,
    batch 32) at input densities 0.5-10 %: the push kernel (work ~ the active
    synapse visits) against the densify + shadow gather (work ~ nnz * B),
    each forced with SILI_PUSH, device buffers in place, one layer copy."""
    from sili__new_amd.synth import Stream, make_config
    wl = make_config(2)
    B, n_in, n_out = wl.batch, wl.n_in, wl.n_out
    L = hip.SparseLinearLayer(n_in, n_out, wl.nnz)
    L.load_weights(wl.ptrs, wl.cols, wl.q)
    L.set_value_scales(wl.value_scale)
    h = C.c_void_p(L.handle)
    stream = api.L.sili_stream(h)
    y = api.alloc(h, 4 * B * n_out)
    out = {"workload": f"config-2 layer {n_in}x{n_out}, {wl.nnz} synapses, batch {B}; forward_sparse",
           "densities": {}}
    rng = Stream(SEED_SWEEP, 3)
    for dens in (0.005, 0.01, 0.03, 0.1):
        keep = rng.u64(B * n_in).reshape(B, n_in) % 1000 < int(dens * 1000)
        xp = np.concatenate([[0], np.cumsum(keep.sum(1))]).astype(np.int32)
        xi = np.nonzero(keep)[1].astype(np.int32)
        xv = np.abs(rng.normal(len(xi))).astype(np.float32) + 0.01
        dp, di, dv = api.upload(h, xp), api.upload(h, xi), api.upload(h, xv)
        row = {"active_inputs": int(len(xi)),
               "synapse_visits": int(np.diff(wl.ptrs)[xi].sum())}
        for mode, name in (("2", "push"), ("0", "gather")):
            os.environ["SILI_PUSH"] = mode
            for _ in range(3):
                api.ck(api.L.sili_forward_sparse(h, dp, di, dv, len(xi), B, y, stream))
            rt.sync()
            api.ck(api.L.sili_profile_enable(h, 1))
            reps = 20
            for _ in range(reps):
                api.ck(api.L.sili_forward_sparse(h, dp, di, dv, len(xi), B, y, stream))
            rt.sync()
            prof = api.profile(h)
            api.ck(api.L.sili_profile_enable(h, 0))
            row[name + "_us"] = round(sum(tot for k, (cnt, tot) in prof.items()
                                          if k.startswith("fwd_sparse:")) / reps * 1e3, 2)
            row[name + "_kernels_us"] = {k: round(tot / reps * 1e3, 2) for k, (cnt, tot) in prof.items()}
        os.environ.pop("SILI_PUSH", None)
        for k in (dp, di, dv):
            api.ck(api.L.sili_device_free(h, k))
        out["densities"][f"{dens:g}"] = row
    api.ck(api.L.sili_device_free(h, y))
    print(json.dumps(out), flush=True)


SEED_SWEEP = 20261290


def cpu_baseline_c4(d, seconds):
    """The CPU port's forward over the q layer at batch 1 (exported from the
    device to a temporary file the child process loads): a bounded sample of
    the config-4 step."""
    import tempfile
    from sili__new_amd.synth import SEED0, Stream
    L = d["L"]
    ex = L.export_scattered()
    x = Stream(SEED0 + 4, 7).normal(d["n_in"]).astype(np.float32)[None, :]
    fd, path = tempfile.mkstemp(suffix=".npz", prefix="sili_c4q_")
    os.close(fd)
    try:
        np.savez(path, n_in=d["n_in"], n_out=d["n_out"], nnz=d["nnz"], row_byte_start=ex["row_byte_start"],
                 row_elem_start=ex["row_elem_start"], idx=ex["idx"], val=ex["val"],
                 value_scale=np.asarray(L.get_value_scales(), np.float32), x=x)
        del ex
        return cpu_baseline(4, seconds, layer_file=path)
    finally:
        os.unlink(path)


def main():
    if len(sys.argv) == 3 and sys.argv[1] == "--cpu-child":
        print(json.dumps(cpu_child_run(json.loads(sys.argv[2]))), flush=True)
        return
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the layer is sharded by input "
                                   "rows only on paper, no multi-GPU path is built -- run with --gpus 1"}))
        sys.exit(2)
    if a.copy_probe:
        n = Hip().copy_probe(a.copy_probe)
        print(json.dumps({"copy_probe_bytes": n, "copies": 3}), flush=True)
        return
    import sili__new_amd as hip

    if a.index_decode:
        run_index_decode(a, hip, CAbi(hip.LIB_PATH), Hip())
        return
    if a.sparse_sweep:
        run_sparse_sweep(a, hip, CAbi(hip.LIB_PATH), Hip())
        return
    cfg = a.config
    api, rt = CAbi(hip.LIB_PATH), Hip()
    if cfg == 4:
        out = run_config4(a, hip, api, rt)
    else:
        out = run_layer_config(a, hip, api, rt, cfg, a.steps, a.warmup, a.train_lr,
                               synapto_reps=a.synapto_reps, cpu=not a.no_cpu_baseline)
    if cfg == 1 and not a.train_lr and not a.no_configs:
        out["configs"] = other_configs(a, hip, api, rt)
    print(json.dumps(out), flush=True)


def run_layer_config(a, hip, api, rt, cfg, steps, warmup, train_lr, synapto_reps=0, cpu=True):
    """One step of config 0-3 over rotated layer copies: the bench line."""
    from sili__new_amd.synth import make_config
    wl = make_config(cfg)
    B, n_in, n_out = wl.batch, wl.n_in, wl.n_out

    # one layer + activation set per copy, all driven on copy 0's stream;
    # enough copies (> 512 MiB) that the 256 MiB MALL cannot serve a step
    # from the previous one
    copies = a.copies
    t_build = time.perf_counter()
    pool = [build_copy(cfg, wl, hip, api)]
    per_copy = pool[0]["bytes"]
    if copies <= 0:
        copies = max(2, int(np.ceil(512 * 2**20 / per_copy)) + 1)
    while len(pool) < copies:
        pool.append(build_copy(cfg, wl, hip, api))
    t_build = time.perf_counter() - t_build
    stream = api.L.sili_stream(pool[0]["h"])
    if train_lr and cfg not in (1, 3):
        print(json.dumps({"error": "--train-lr applies to configs 1 and 3 only"}))
        sys.exit(2)
    run = make_step(cfg, api, B, stream, train_lr)

    def step(i):
        run(pool[i % copies])

    # set-up: each copy's first call sizes its workspaces (and, with the
    # optimizer update, allocates its optimizer state); then W warmup steps
    for d in pool:
        run(d)
    rt.sync()
    for i in range(warmup):
        step(i)
    rt.sync()

    # timed region: exactly K steps, bracketed by device syncs
    e0, e1 = rt.event(), rt.event()
    rt.sync()
    rt.record(e0, stream)
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    rt.record(e1, stream)
    rt.sync()
    wall = time.perf_counter() - t0
    ms_step = rt.elapsed_ms(e0, e1) / steps

    # warm (cache-resident) rate: a single copy, same step count
    w0, w1 = rt.event(), rt.event()
    rt.sync()
    rt.record(w0, stream)
    for i in range(steps):
        step(0)
    rt.record(w1, stream)
    rt.sync()
    warm_ms_step = rt.elapsed_ms(w0, w1) / steps

    # profiled pass (same steps): per-kernel times from the dispatches' own
    # begin/end stamps, on the stream the kernels run on
    for d in pool:
        api.ck(api.L.sili_profile_enable(d["h"], 1))
    p0, p1 = rt.event(), rt.event()
    rt.record(p0, stream)
    for i in range(steps):
        step(i)
    rt.record(p1, stream)
    rt.sync()
    prof_ms_step = rt.elapsed_ms(p0, p1) / steps
    kern = {}
    for d in pool:
        for name, (cnt, tot) in api.profile(d["h"]).items():
            c0, t0_ = kern.get(name, (0, 0.0))
            kern[name] = (c0 + cnt, t0_ + tot)
        api.ck(api.L.sili_profile_enable(d["h"], 0))
    info = pool[0]["L"].info()
    alg = algorithmic(info, n_in, n_out, B, wl)
    dom_name, (dom_cnt, dom_tot) = max(kern.items(), key=lambda kv: kv[1][1])
    # one op may take several launches (column-block passes): time per op
    launches = dom_cnt / steps
    dom_avg_ms = dom_tot / steps

    nnz_s, n_tiles = info["nnz_scattered"], info["n_tiles"]
    units = nnz_s + 16 * n_tiles  # stored synapses (scattered + block4 slots)
    if cfg == 3 and train_lr:
        dom_bytes = alg.get(dom_name)
        achieved = dom_bytes / (dom_avg_ms * 1e-3) / 1e9 if dom_bytes else None
        roof = {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 2) if achieved else None,
                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5) if achieved else None,
                "traffic": None, "avg_op_ms": round(dom_avg_ms, 5), "launches_per_op": launches,
                "algorithmic_bytes": dom_bytes,
                "slot_steps_per_s": round(16 * n_tiles * B / (dom_avg_ms * 1e-3), 1),
                "note": ("k_train_b4 runs each tile slot's batch steps as a dependent chain of VALU "
                         "instructions (as k_train_rows per synapse): bound by instruction issue, not HBM")}
        step_bytes = alg["fwd:gather_b4"] + alg["bwd:train_b4"]
        flops = 2 * 2 * units * B
    elif cfg == 3:
        # FP32-compute bound: 2 flops per slot per batch column
        dom_flops = 2 * 16 * n_tiles * B
        achieved = dom_flops / (dom_avg_ms * 1e-3) / 1e12
        roof = {"bound": "fp32-valu", "kernel": dom_name, "achieved": round(achieved, 3), "peak": FP32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK_TFLOPS, 5),
                "traffic": measured_traffic(dom_name, cfg), "avg_op_ms": round(dom_avg_ms, 5),
                "launches_per_op": launches,
                "algorithmic_flops": dom_flops, "algorithmic_bytes": alg.get(dom_name),
                "note": ("fp32 vector FMA work: the MFMA variants lose on every op "
                         "(profiles/c3_block4_mfma_vs_valu.md); peak is MI355X dense fp32")}
        step_bytes = alg["fwd:gather_b4"] + alg["bwd:gather_b4"] + alg["bwd:sddmm_b4"]
        flops = 3 * 2 * units * B
    else:
        dom_bytes = alg.get(dom_name)
        achieved = dom_bytes / (dom_avg_ms * 1e-3) / 1e9 if dom_bytes else None
        roof = {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 2) if achieved else None,
                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 5) if achieved else None,
                "traffic": None if train_lr else measured_traffic(dom_name, cfg), "avg_op_ms": round(dom_avg_ms, 5),
                "launches_per_op": launches, "algorithmic_bytes": dom_bytes}
        if dom_name == "bwd:train_rows":
            # one synapse's batch steps are a dependent chain of ~80 VALU
            # instructions each (correctly rounded sqrt and division, clamps,
            # fp64 gradient terms): the kernel is bound by instruction issue
            steps = nnz_s * B
            roof["synapse_steps_per_s"] = round(steps / (dom_avg_ms * 1e-3), 1)
            roof["note"] = ("k_train_rows is bound by VALU issue (~80 instructions per synapse per batch step, "
                            "4 cycles per 64-lane instruction per SIMD), not by HBM")
        if cfg == 0:
            step_bytes = alg["fwd:gather"]
            flops = 2 * units * B
        elif cfg == 2:
            step_bytes = alg["fwd_sparse:gather"] + alg["bwd:gather"]
            flops = 2 * int(np.diff(wl.ptrs)[np.asarray(wl.x_idx)].sum()) + 2 * units * B
        elif train_lr:
            step_bytes = alg["fwd:gather"] + alg["bwd:train_rows"] + alg["bwd:train_shadow"]
            flops = 2 * 2 * units * B
        else:
            # forward + grad-input + sampled grad-W, each op counted as if run
            # alone (the fused backward moves less)
            step_bytes = alg["fwd:gather"] + alg["bwd:gather"] + alg["bwd:sddmm"]
            flops = 3 * 2 * units * B
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9

    workload = workload_text(cfg, wl)
    if train_lr:
        workload = workload.replace("grad-input + nnz-sampled grad-W",
                                    f"backward with the optimizer update (lr {train_lr}, stochastic rounding)")
    out = {
        "metric": "FP4 delta-CSR SpMM GNNZ/s + achieved HBM GB/s (% of peak), fwd+bwd",
        "value": round(units / (ms_step * 1e-3) / 1e9, 4),
        "unit": "GNNZ/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "n_in": n_in, "n_out": n_out, "batch": B, "nnz": units, "nnz_scattered": nnz_s,
            "n_tiles": n_tiles, "index_bytes": info["index_bytes"],
            "copies_rotated": copies, "rotation_mib": round(copies * per_copy / 2**20, 1),
        },
        "achieved_gbs": round(step_gbs, 2),
        "pct_hbm_peak": round(100.0 * step_gbs / HBM_PEAK_GBS, 3),
        "gflops": round(flops / (ms_step * 1e-3) / 1e9, 2),
        "warm_ms_per_step": round(warm_ms_step, 5),
        "warm_value": round(units / (warm_ms_step * 1e-3) / 1e9, 4),
        "wall_s_timed": round(wall, 4),
        "roofline": roof,
        "kernels_ms_per_step": {k: round(v[1] / steps, 5) for k, v in kern.items()},
        "profiled_ms_per_step": round(prof_ms_step, 5),
    }
    # the layers and their device buffers are released here, while the HIP
    # runtime is fully alive (not at interpreter teardown)
    release_pool(api, pool)
    rt.sync()
    if cfg == 3 and synapto_reps > 0:
        out["synapto_gpu"] = time_synapto(hip, wl, synapto_reps)
    if cfg == 1 and a.synap_cycles > 0:
        out["synap_policy"] = time_synap_policy(hip, wl, a.synap_cycles, a.cpu_seconds)
    out["cpu_baseline"] = cpu_baseline(cfg, a.cpu_seconds, lr=train_lr) if cpu else None
    if a.verbose:
        print(f"build {t_build:.1f}s copies {copies}", file=sys.stderr)
    return out


def time_binding(hip, steps=50, warmup=5):
    """Config 1 through the pybind module the way FoldedLayer / DISLDOLayer
    call it (sili/sparse_rnn.py:1004-1212): numpy arrays in, numpy arrays out,
    so every call copies its input to the device and its output back.  Wall
    time per step of forward_dense + backward_dense(lr 0), and of each call."""
    from sili__new_amd.synth import make_config
    wl = make_config(1)
    L = hip.SparseLinearLayer(wl.n_in, wl.n_out, wl.nnz)
    L.load_weights(wl.ptrs, wl.cols, wl.q)
    L.set_value_scales(wl.value_scale)
    x = np.ascontiguousarray(wl.x, dtype=np.float32)
    g = np.ascontiguousarray(wl.g, dtype=np.float32)
    def run(xin, gin):
        for _ in range(warmup):
            L.forward_dense(xin)
            L.backward_dense(gin, 0.0)
        tf = tb = 0.0
        for _ in range(steps):
            t0 = time.perf_counter()
            L.forward_dense(xin)
            t1 = time.perf_counter()
            L.backward_dense(gin, 0.0)
            t2 = time.perf_counter()
            tf += t1 - t0
            tb += t2 - t1
        return {"ms_per_step": round((tf + tb) * 1e3 / steps, 4), "fwd_ms": round(tf * 1e3 / steps, 4),
                "bwd_ms": round(tb * 1e3 / steps, 4)}

    host_bytes = 4 * (x.size + g.size + wl.batch * (wl.n_out + wl.n_in))
    out = {"workload": "config 1 forward_dense + backward_dense(lr 0) through the pybind module, numpy in and "
                       "out (grad-input only: the module's backward returns dx); inputs either ordinary numpy "
                       "arrays or arrays the module returned (page-locked, as a chained layer's input is)",
           "steps": steps, "host_bytes_per_step": host_bytes}
    out["numpy_inputs"] = run(x, g)
    # arrays the module returned: its outputs live in page-locked blocks
    xp = L.forward_dense(x)
    gp = L.backward_dense(g, 0.0)
    out["module_arrays_as_inputs"] = run(xp, gp)
    return out


def other_configs(a, hip, api, rt):
    """Configs 2, 3 (with its synaptogenesis step) and 4 (batches 1, 8, 128)
    timed as config 1 is (rotated copies, HIP events over the timed steps,
    the dominant kernel's algorithmic rate from the profiled pass), at fewer
    steps; a summary of each line."""
    res = {}
    for cfg, steps in ((2, 100), (3, 20)):
        t0 = time.perf_counter()
        o = run_layer_config(a, hip, api, rt, cfg, steps, 5, 0.0, synapto_reps=10 if cfg == 3 else 0, cpu=False)
        r = o["roofline"]
        res[str(cfg)] = {"workload": o["config"]["workload"], "value": o["value"], "unit": o["unit"],
                         "ms_per_step": o["ms_per_step"], "steps": o["steps"],
                         "warm_ms_per_step": o["warm_ms_per_step"],
                         "dominant": {k: r.get(k) for k in ("kernel", "bound", "achieved", "unit", "peak", "frac",
                                                           "avg_op_ms")},
                         "kernels_ms_per_step": o["kernels_ms_per_step"], "wall_s": round(time.perf_counter() - t0, 1)}
        if cfg == 3:
            res["3"]["synapto_gpu"] = o["synapto_gpu"]
    t0 = time.perf_counter()
    a4 = argparse.Namespace(**vars(a))
    a4.c4_batches, a4.steps, a4.warmup, a4.no_cpu_baseline = "1,8,128", 200, 5, True
    o = run_config4(a4, hip, api, rt)
    res["4"] = {"workload": o["config"]["workload"], "nnz": o["config"]["nnz"],
                "batches": {b: {"ms_per_step": r["ms_per_step"], "gnnz_s": r["gnnz_s"], "steps": r["steps"],
                                "pct_hbm_peak": r["pct_hbm_peak"], "dominant": r["dominant"]}
                            for b, r in o["batches"].items()},
                "build_s": o["build_s"], "wall_s": round(time.perf_counter() - t0, 1)}
    res["binding"] = time_binding(hip)
    return res


if __name__ == "__main__":
    main()
