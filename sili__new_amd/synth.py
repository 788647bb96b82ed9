"""Seeded synthetic workloads for the FP4 delta-CSR layer (host, numpy).

One counter-based generator (splitmix64 keyed by (seed, stream, counter)) so
every consumer -- GPU tests, the CPU oracle checks, bench.py -- draws the
same matrices.  Seeds are 20261201 + config index.  Normals are Box-Muller
in float64 rounded to float32; Poisson and truncated Zipf row lengths use
inverse-CDF tables.

Weights follow the reference's per-row FP4 recipe (sili/sparse_rnn.py:
1022-1033): s_r = fl32(max|w_row| / 6), q = fl32(w / s_r); the layer stores
fp4_encode(q) and value_scale[r] = s_r, output_scale = 1.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

SEED0 = 20261201
FP4_MAX = 6.0

_M64 = (1 << 64) - 1


def splitmix64(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


class Stream:
    """Counter-based stream: value i = splitmix64(key + i)."""

    def __init__(self, seed: int, stream: int):
        k = splitmix64(np.array([(seed * 0x100000001B3 + stream) & _M64], dtype=np.uint64))[0]
        self.key = np.uint64(k)
        self.counter = 0

    def u64(self, n: int) -> np.ndarray:
        c = np.arange(self.counter, self.counter + n, dtype=np.uint64)
        self.counter += n
        with np.errstate(over="ignore"):
            return splitmix64(c + self.key)

    def uniform(self, n: int) -> np.ndarray:
        """float64 in [0, 1)."""
        return (self.u64(n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def normal(self, n: int, sigma: float = 1.0) -> np.ndarray:
        u1 = 1.0 - self.uniform(n)          # (0, 1]
        u2 = self.uniform(n)
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        return (z * sigma).astype(np.float32)

    def integers(self, n: int, hi: int) -> np.ndarray:
        """uniform ints in [0, hi) (multiply-shift, bias < 2^-32)."""
        u = self.u64(n) >> np.uint64(32)
        return ((u * np.uint64(hi)) >> np.uint64(32)).astype(np.int64)


def poisson_lengths(st: Stream, n: int, mean: float) -> np.ndarray:
    kmax = int(mean + 20 * math.sqrt(mean) + 20)
    k = np.arange(kmax + 1)
    logp = k * math.log(mean) - mean - np.array([math.lgamma(i + 1) for i in k])
    cdf = np.cumsum(np.exp(logp))
    cdf /= cdf[-1]
    return np.searchsorted(cdf, st.uniform(n), side="right").astype(np.int64)


def zipf_lengths(st: Stream, n: int, a: float, kmax: int) -> np.ndarray:
    k = np.arange(1, kmax + 1, dtype=np.float64)
    cdf = np.cumsum(k ** (-a))
    cdf /= cdf[-1]
    return (np.searchsorted(cdf, st.uniform(n), side="right") + 1).astype(np.int64)


def distinct_columns(st: Stream, lengths: np.ndarray, ncols: int) -> tuple[np.ndarray, np.ndarray]:
    """Per row, `lengths[r]` distinct uniform columns in [0, ncols), sorted.

    Draws candidates in counter order and keeps each row's first distinct
    ones; rows that come up short are redrawn with more candidates."""
    rows = len(lengths)
    lengths = np.minimum(lengths, ncols)
    out_cols = [None] * rows
    todo = np.arange(rows)
    factor = 1.3
    while len(todo):
        want = lengths[todo]
        m = (want * factor + 64).astype(np.int64)
        if ncols <= 4 * 1024 * 1024:
            m = np.minimum(m, ncols * 8)
        row_of = np.repeat(todo, m)
        draws = st.integers(int(m.sum()), ncols)
        order = np.arange(len(draws))
        key = row_of.astype(np.int64) * ncols + draws
        uniq, first = np.unique(key, return_index=True)
        urow = uniq // ncols
        # rank of each unique entry among its row's uniques, by first draw
        srt = np.lexsort((first, urow))
        urow_s, ucol_s = urow[srt], (uniq % ncols)[srt]
        start = np.searchsorted(urow_s, urow_s, side="left")
        rank = np.arange(len(urow_s)) - start
        need = lengths[urow_s]
        keep = rank < need
        got = np.bincount(urow_s[keep], minlength=rows)
        short = []
        kr, kc = urow_s[keep], ucol_s[keep]
        bounds = np.searchsorted(kr, todo, side="left"), np.searchsorted(kr, todo, side="right")
        for i, r in enumerate(todo):
            if got[r] < lengths[r]:
                short.append(r)
                continue
            out_cols[r] = np.sort(kc[bounds[0][i]:bounds[1][i]])
        todo = np.array(short, dtype=np.int64)
        factor *= 2.0
        del order
    ptrs = np.zeros(rows + 1, dtype=np.int64)
    ptrs[1:] = np.cumsum(lengths)
    cols = np.concatenate([c for c in out_cols]) if rows else np.zeros(0, np.int64)
    return ptrs.astype(np.int32), cols.astype(np.int32)


def per_row_quantize(ptrs: np.ndarray, w: np.ndarray, n_rows: int) -> tuple[np.ndarray, np.ndarray]:
    """sili/sparse_rnn.py:1022-1033: s_r = fl32(max|w|/6), q = fl32(w / s_r)."""
    q = w.astype(np.float32).copy()
    s = np.ones(n_rows, dtype=np.float32)
    lens = np.diff(ptrs)
    nz = np.nonzero(lens)[0]
    if len(nz):
        mx = np.maximum.reduceat(np.abs(q), ptrs[:-1][nz].astype(np.int64))
        for r, m in zip(nz, mx):
            if m > 0.0:
                s[r] = np.float32(float(m) / FP4_MAX)
        row_of = np.repeat(np.arange(n_rows), lens)
        q = (q / s[row_of]).astype(np.float32)
    return q, s


@dataclass
class Workload:
    name: str
    n_in: int
    n_out: int
    batch: int
    ptrs: np.ndarray | None = None       # scattered absolute CSR (quantizer inputs)
    cols: np.ndarray | None = None
    q: np.ndarray | None = None
    value_scale: np.ndarray | None = None
    x: np.ndarray | None = None          # dense [B, n_in]
    g: np.ndarray | None = None          # dense [B, n_out]
    x_ptrs: np.ndarray | None = None     # sparse input CSR
    x_idx: np.ndarray | None = None
    x_vals: np.ndarray | None = None
    tile_br: np.ndarray | None = None    # block4 tiles
    tile_bc: np.ndarray | None = None
    tile_bytes: np.ndarray | None = None
    cand_r: np.ndarray | None = None     # synaptogenesis candidates
    cand_c: np.ndarray | None = None
    cand_v: np.ndarray | None = None
    meta: dict = field(default_factory=dict)

    @property
    def nnz(self) -> int:
        return 0 if self.cols is None else int(len(self.cols))


def make_config(idx: int, scale: float = 1.0, batch: int | None = None) -> Workload:
    """BASELINE configs 0..3 (0-based).  `scale` < 1 shrinks the matrix side
    (tests); densities and distributions stay the same."""
    seed = SEED0 + idx
    if idx == 0:
        n = max(8, int(4096 * scale))
        per_row = max(1, int(round(205 * n / 4096)))
        st = Stream(seed, 1)
        lengths = np.full(n, per_row, dtype=np.int64)
        ptrs, cols = distinct_columns(st, lengths, n)
        w = Stream(seed, 2).normal(len(cols), 0.02)
        q, s = per_row_quantize(ptrs, w, n)
        B = batch or 1
        x = Stream(seed, 3).normal(B * n).reshape(B, n)
        return Workload("c0", n, n, B, ptrs, cols, q, s, x=x)
    if idx == 1:
        n = max(16, int(8192 * scale))
        mean = 164.0 * n / 8192
        lengths = poisson_lengths(Stream(seed, 1), n, mean)
        ptrs, cols = distinct_columns(Stream(seed, 2), lengths, n)
        w = Stream(seed, 3).normal(len(cols), 0.02)
        q, s = per_row_quantize(ptrs, w, n)
        B = batch or 64
        x = Stream(seed, 4).normal(B * n).reshape(B, n)
        g = Stream(seed, 5).normal(B * n).reshape(B, n)
        return Workload("c1", n, n, B, ptrs, cols, q, s, x=x, g=g)
    if idx == 2:
        n = max(64, int(16384 * scale))
        kmax = max(1, int(4096 * n / 16384))
        L = zipf_lengths(Stream(seed, 1), n, 1.2, kmax)
        alpha = 0.01 * n * n / float(L.sum())
        L = np.clip(np.rint(alpha * L), 1, kmax).astype(np.int64)
        ptrs, cols = distinct_columns(Stream(seed, 2), L, n)
        w = Stream(seed, 3).normal(len(cols), 0.02)
        q, s = per_row_quantize(ptrs, w, n)
        B = batch or 32
        per = max(1, int(round(0.1 * n)))
        xp, xi = distinct_columns(Stream(seed, 4), np.full(B, per, dtype=np.int64), n)
        xv = np.abs(Stream(seed, 5).normal(len(xi)))
        g = Stream(seed, 6).normal(B * n).reshape(B, n)
        x = np.zeros((B, n), dtype=np.float32)
        x[np.repeat(np.arange(B), np.diff(xp)), xi] = xv
        return Workload("c2", n, n, B, ptrs, cols, q, s, x=x, g=g, x_ptrs=xp, x_idx=xi, x_vals=xv,
                        meta={"zipf_a": 1.2, "density": len(cols) / float(n * n)})
    if idx == 3:
        n = max(16, int(16384 * scale))
        nb = n // 4
        n_tiles = int(round(0.03 * nb * nb))
        st = Stream(seed, 1)
        # distinct uniform tile positions
        keys = np.unique(st.integers(int(n_tiles * 1.2) + 64, nb * nb))
        keys = keys[splitmix64(keys.astype(np.uint64) + np.uint64(seed)).argsort(kind="stable")][:n_tiles]
        keys.sort()
        br, bc = (keys // nb).astype(np.int32), (keys % nb).astype(np.int32)
        w = Stream(seed, 2).normal(len(keys) * 16, 0.02).reshape(-1, 16)  # slot order lj*4+li
        # per-row scale over every slot of the row (row = 4*br + li)
        li = np.tile(np.arange(16) % 4, (len(keys), 1))
        rows = (br[:, None] * 4 + li).ravel()
        amax = np.zeros(n, dtype=np.float32)
        np.maximum.at(amax, rows, np.abs(w).ravel())
        s = np.ones(n, dtype=np.float32)
        nzr = amax > 0
        s[nzr] = (amax[nzr].astype(np.float64) / FP4_MAX).astype(np.float32)
        qv = (w.ravel() / s[rows]).astype(np.float32)
        from .codec import fp4_encode_np
        codes = fp4_encode_np(qv).reshape(-1, 16)
        tile_bytes = (codes | np.uint8(1 << 4)).astype(np.uint8)  # importance code 1: every slot live
        B = batch or 256
        x = Stream(seed, 3).normal(B * n).reshape(B, n)
        g = Stream(seed, 4).normal(B * n).reshape(B, n)
        n_syn = len(keys) * 16
        k = int(round(0.01 * n_syn))
        cst = Stream(seed, 5)
        m = 2 * k + 64
        cr = cst.integers(m, n).astype(np.int32)
        cc = cst.integers(m, n).astype(np.int32)
        cv = Stream(seed, 6).normal(m, 0.01)
        return Workload("c3", n, n, B, value_scale=s, x=x, g=g, tile_br=br, tile_bc=bc,
                        tile_bytes=tile_bytes.ravel(), cand_r=cr, cand_c=cc, cand_v=cv,
                        meta={"n_tiles": len(keys), "prune_k": k})
    raise ValueError(f"unknown config {idx}")
