"""Short rows packed several to a wave by the float4 gather.

Rows that are one work item of at most 28 index bytes are gathered up to 16
to a wave (the column scan restarting at each row's first byte, each entry
scaled by its own row's scale, one lane group per row).  The layers here have
skewed row lengths in both orientations (many empty and one-entry rows, a few
rows long enough to be split into several work items), so the canonical
store's grad-input gather and the shadow store's forward gather both take the
packed path next to the one-row-per-wave path.  Checked against the dense
double-precision product with the device's fp32 weights (the same oracle
decode as the other parity tests) for every batch the float4 shapes cover
(4..64 columns), with rank-1 and rank-2 scales, a NaN weight code and
non-finite inputs, and with the packing switched off (SILI_SHORT_ROWS=0).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import HostLayer
from tests.util import assert_close_terms

pytestmark = pytest.mark.gpu


def _skewed_layer(rng, n_in, n_out):
    """Row lengths drawn from a heavy tail (half the rows 0-2 entries, a few
    thousands long) over columns drawn from a skewed distribution, so that
    many shadow rows are short as well."""
    u = rng.random(n_in)
    lens = np.where(u < 0.15, 0, np.where(u < 0.55, rng.integers(1, 3, n_in),
                    np.where(u < 0.8, rng.integers(3, 12, n_in),
                             np.where(u < 0.97, rng.integers(12, 60, n_in), rng.integers(200, 2000, n_in)))))
    colp = 1.0 / (np.arange(n_out) + 50.0) ** 0.8
    colp /= colp.sum()
    perm = rng.permutation(n_out)
    cols_l = []
    for n in lens:
        c = rng.choice(n_out, size=min(int(n), n_out), replace=False, p=colp[perm])
        cols_l.append(np.sort(c))
    ptrs = np.concatenate([[0], np.cumsum([len(c) for c in cols_l])]).astype(np.int32)
    cols = np.concatenate(cols_l).astype(np.int32)
    q = rng.normal(0, 2, len(cols)).astype(np.float32)
    return ptrs, cols, q


def _dense(ptrs, cols, q, n_in, n_out):
    return HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q).dense().astype(np.float64)


@pytest.mark.parametrize("rank", [1, 2])
def test_short_rows_both_orientations(hip, rank, monkeypatch):
    rng = np.random.default_rng(7100 + rank)
    n_in, n_out = 6000, 20000
    ptrs, cols, q = _skewed_layer(rng, n_in, n_out)
    D = _dense(ptrs, cols, q, n_in, n_out)
    L = hip.SparseLinearLayer(n_in, n_out, len(cols) + 64)
    L.load_weights(ptrs, cols, q)
    L.set_scale_rank(rank)
    vs = rng.uniform(0.25, 2.0, n_in * rank).astype(np.float32)
    os_ = rng.uniform(0.25, 2.0, n_out * rank).astype(np.float32)
    L.set_value_scales(vs)
    L.set_output_scales(os_)
    S = vs.reshape(n_in, rank).astype(np.float64) @ os_.reshape(n_out, rank).astype(np.float64).T
    W = D * S.astype(np.float32).astype(np.float64)
    for mode in ("1", "0"):
        monkeypatch.setenv("SILI_SHORT_ROWS", mode)
        L.load_weights(ptrs, cols, q)  # a fresh store: the split is built on first use
        L.set_value_scales(vs)
        L.set_output_scales(os_)
        for B in (4, 8, 12, 16, 24, 32, 48, 64):
            x = rng.normal(size=(B, n_in)).astype(np.float32)
            X = x.astype(np.float64)
            y = L.forward_dense(x)
            assert_close_terms(y, X @ W, np.abs(X) @ np.abs(W), f"fwd rank {rank} B{B} short={mode}")
            g = rng.normal(size=(B, n_out)).astype(np.float32)
            G = g.astype(np.float64)
            dx = L.backward_dense(g, 0.0)
            assert_close_terms(dx, G @ W.T, np.abs(G) @ np.abs(W.T), f"dx rank {rank} B{B} short={mode}")
        info = L.info()
        if mode == "1":
            # both orientations packed their short rows
            assert info["short_rows_canonical"] > 1024, info
            assert info["short_rows_shadow"] > 1024, info
        else:
            assert info["short_rows_canonical"] == 0 and info["short_rows_shadow"] == 0, info
    monkeypatch.delenv("SILI_SHORT_ROWS")


def test_short_rows_sparse_paths_and_nonfinite(hip):
    """The sparse-input forward and the sparse-gradient dx (the +0.0 skip
    rules), a NaN weight code in a short row and non-finite inputs."""
    rng = np.random.default_rng(7200)
    n_in, n_out = 5000, 16000
    ptrs, cols, q = _skewed_layer(rng, n_in, n_out)
    # the value bytes, with one NaN code (8) in a one-entry row
    byts = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q).val[:len(cols)].copy()
    r = int(np.flatnonzero(np.diff(ptrs) == 1)[3])
    byts[ptrs[r]] = 0x80 | (byts[ptrs[r]] & 0x0F)
    L = hip.SparseLinearLayer(n_in, n_out, len(cols) + 64)
    L.load_weight_bytes(ptrs, cols, byts)
    vs = rng.uniform(0.25, 2.0, n_in).astype(np.float32)
    L.set_value_scales(vs)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, bytes_=byts).set_scales(vs)
    assert L.info()["has_nonfinite"]
    for B in (8, 32, 64):
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        x[rng.random(x.shape) < 0.9] = 0.0
        x[1, 5] = np.inf
        x[2, 9] = np.nan
        y = L.forward_dense(x)
        assert_close_terms(y, H.forward_dense(x), H.forward_dense(x, absmode=True), f"nonfinite fwd B{B}")
        xp = np.concatenate([[0], np.cumsum((x != 0).sum(1))]).astype(np.int32)
        xi = np.nonzero(x)[1].astype(np.int32)
        xv = x[x != 0].astype(np.float32)
        ys = L.forward_sparse(xp, xi, xv, B)
        assert_close_terms(ys, H.forward_sparse(xp, xi, xv, B), H.forward_sparse(xp, xi, xv, B, absmode=True),
                           f"sparse fwd B{B}")
        g = rng.normal(size=(B, n_out)).astype(np.float32)
        dx = L.backward_dense(g, 0.0)
        assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0], f"dx B{B}")
        g[rng.random(g.shape) < 0.8] = 0.0
        gp = np.concatenate([[0], np.cumsum((g != 0).sum(1))]).astype(np.int32)
        gi = np.nonzero(g)[1].astype(np.int32)
        gv = g[g != 0].astype(np.float32)
        dxs = L.backward_sparse(x, gp, gi, gv, B, 0.0)
        assert_close_terms(dxs, H.backward_sparse(x, gp, gi, gv, B)[0],
                           H.backward_sparse(x, gp, gi, gv, B, absmode=True)[0], f"sparse dx B{B}")
    info = L.info()
    assert info["short_rows_canonical"] > 1024 and info["short_rows_shadow"] > 1024, info
