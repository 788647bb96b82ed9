"""Shared helpers for the parity tests."""
from __future__ import annotations

import numpy as np

# fp32 outputs: |gpu - oracle| <= REL * sum|terms| + ABS  (order of summation only)
REL = 1e-5
ABS = 1e-30


def assert_close_terms(got, want, bound, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bound = np.asarray(bound, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = np.abs(got - want)
    lim = REL * bound + ABS
    bad = ~(err <= lim)
    # identical non-finite values count as equal
    both_nan = np.isnan(got) & np.isnan(want)
    same_inf = np.isinf(got) & (got == want)
    bad &= ~(both_nan | same_inf)
    if bad.any():
        i = np.flatnonzero(bad)[:5]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tolerance; first {i}: "
                             f"got {got.ravel()[i]} want {want.ravel()[i]} bound {bound.ravel()[i]}")


def host_layer(wl):
    from oracle import HostLayer
    H = HostLayer(wl.n_in, wl.n_out)
    if wl.cols is not None:
        H.load_csr(wl.ptrs, wl.cols, w=wl.q)
    if wl.tile_br is not None:
        H.load_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes)
    H.set_scales(wl.value_scale)
    return H


def gpu_layer(hip, wl, max_weights=None):
    n = wl.nnz + (0 if wl.tile_br is None else 16 * len(wl.tile_br))
    L = hip.SparseLinearLayer(wl.n_in, wl.n_out, max_weights or max(n, 1))
    if wl.cols is not None:
        L.load_weights(wl.ptrs, wl.cols, wl.q)
    if wl.tile_br is not None:
        L.load_block4_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes)
    L.set_value_scales(wl.value_scale)
    return L
