"""GPU: the sparse-input forward over the active (batch row, input row)
pairs (csrc/push.hip; sisldo_forward, sisldo_ops.hpp:198-551) against the
oracle's restatement, on the cases its work split and LDS tables have to get
right: skewed rows longer than a block's share, batch rows shared by several
blocks and batch rows owned by one, empty batch rows, explicit zeros meeting
NaN weights, active-row lists longer than one LDS table, scales of rank 1
and 2, and layers that also hold block4 tiles.
The profiler confirms the push kernel ran; the default dispatch by input
density is checked at the end."""
import numpy as np
import pytest

from oracle import HostLayer
from test_gpu_stream import kernels_run
from util import assert_close_terms

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def push_always(monkeypatch):
    """Push whenever the layer allows it (by default only inputs with < 2 %
    active (batch row, input row) pairs are pushed)."""
    monkeypatch.setenv("SILI_PUSH", "2")
    yield


def skewed_layer(rng, n_in, n_out, mean, long_rows=3):
    lens = np.minimum(rng.zipf(1.6, n_in) * int(mean), n_out).astype(np.int64)
    lens[rng.random(n_in) < 0.1] = 0
    lens[rng.choice(n_in, long_rows, replace=False)] = min(n_out, 900)
    cols = [np.sort(rng.choice(n_out, size=int(k), replace=False)) for k in lens]
    ptrs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    idx = np.concatenate(cols).astype(np.int32)
    w = rng.normal(0, 2, len(idx)).astype(np.float32)
    return ptrs, idx, w


def sparse_x(rng, B, n_in, density, empty_rows=(1,)):
    # the binding takes each batch row's indices strictly increasing (as the
    # module's dense_to_csr / dense_to_top_k_csr produce them)
    ptrs, idx, vals = [0], [], []
    for b in range(B):
        k = 0 if b in empty_rows else max(1, int(rng.binomial(n_in, density)))
        r = np.sort(rng.choice(n_in, size=k, replace=False))
        v = rng.normal(0, 1, len(r)).astype(np.float32)
        if len(v) > 3:
            v[3] = 0.0  # an explicit zero
        idx.extend(r.tolist())
        vals.extend(v.tolist())
        ptrs.append(len(idx))
    return np.array(ptrs, np.int32), np.array(idx, np.int32), np.array(vals, np.float32)


def check(hip, L, H, xp, xi, xv, B, what):
    y = None

    def run():
        nonlocal y
        y = L.forward_sparse(xp, xi, xv, B)
    names = kernels_run(hip, L, run)
    assert any(n.endswith("push") for n in names), f"{what}: the push kernel did not run ({names})"
    assert_close_terms(y, H.forward_sparse(xp, xi, xv, B), H.forward_sparse(xp, xi, xv, B, absmode=True), what)
    return y


@pytest.mark.parametrize("B", [1, 3, 32, 300])
def test_push_matches_oracle(hip, B):
    rng = np.random.default_rng(40 + B)
    n_in, n_out = 700, 1500
    ptrs, idx, w = skewed_layer(rng, n_in, n_out, 6)
    L = hip.SparseLinearLayer(n_in, n_out, len(idx) + 64)
    L.load_weights(ptrs, idx, w)
    vs = rng.uniform(0.5, 2.0, n_in).astype(np.float32)
    os_ = rng.uniform(0.5, 2.0, n_out).astype(np.float32)
    L.set_value_scales(vs)
    L.set_output_scales(os_)
    H = HostLayer(n_in, n_out).load_csr(ptrs, idx, w=w)
    H.set_scales(vs, os_)
    for density in (0.1, 0.5):
        xp, xi, xv = sparse_x(rng, B, n_in, density)
        check(hip, L, H, xp, xi, xv, B, f"B {B} density {density}")


def test_push_rank2_scales(hip):
    rng = np.random.default_rng(5)
    n_in, n_out, rank = 120, 300, 2
    ptrs, idx, w = skewed_layer(rng, n_in, n_out, 4, long_rows=1)
    L = hip.SparseLinearLayer(n_in, n_out, len(idx) + 64)
    L.load_weights(ptrs, idx, w)
    L.set_scale_rank(rank)
    vs = rng.uniform(0.5, 2.0, n_in * rank).astype(np.float32)
    os_ = rng.uniform(0.5, 2.0, n_out * rank).astype(np.float32)
    L.set_value_scales(vs)
    L.set_output_scales(os_)
    # sisldo_forward reads component 0 of each scale whatever the rank,
    # stored * (vs[r, 0] * os[c, 0]) (sisldo_ops.hpp:302-306): on a dense
    # reference of the decoded codes (unit scales)
    dense = HostLayer(n_in, n_out).load_csr(ptrs, idx, w=w).dense().astype(np.float64)
    S = np.outer(vs[::rank], os_[::rank]).astype(np.float32).astype(np.float64)
    xp, xi, xv = sparse_x(rng, 8, n_in, 0.2)
    X = np.zeros((8, n_in), np.float64)
    for b in range(8):
        X[b, xi[xp[b]:xp[b + 1]]] = xv[xp[b]:xp[b + 1]]
    want = X @ (dense * S)
    bound = np.abs(X) @ np.abs(dense * S)
    assert_close_terms(L.forward_sparse(xp, xi, xv, 8), want, bound, "rank 2")
    # and the oracle's restatement agrees
    H = HostLayer(n_in, n_out, rank).load_csr(ptrs, idx, w=w).set_scales(vs, os_)
    assert_close_terms(L.forward_sparse(xp, xi, xv, 8), H.forward_sparse(xp, xi, xv, 8),
                       H.forward_sparse(xp, xi, xv, 8, absmode=True), "rank 2 vs oracle")


def test_push_nan_weight_meets_explicit_zero(hip):
    n_in, n_out = 4, 6
    ptrs = np.array([0, 2, 3, 4, 5], np.int32)
    cols = np.array([1, 4, 2, 0, 5], np.int32)
    byts = np.array([0x80, 0x20, 0x30, 0x40, 0x50], np.uint8)  # row 0, col 1: code 8 (NaN)
    L = hip.SparseLinearLayer(n_in, n_out, 64)
    L.load_weight_bytes(ptrs, cols, byts)
    # batch row 0 holds row 0 as an explicit zero; batch row 1 does not hold it
    xp = np.array([0, 2, 3], np.int32)
    xi = np.array([0, 2, 3], np.int32)
    xv = np.array([0.0, 1.5, -2.0], np.float32)
    y = L.forward_sparse(xp, xi, xv, 2)
    assert np.isnan(y[0, 1]) and not np.isnan(y[0, 4])  # 0 * NaN, 0 * 1.0
    assert not np.isnan(y[1]).any()
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, bytes_=byts)
    want = H.forward_sparse(xp, xi, xv, 2)
    assert np.array_equal(np.isnan(y), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_allclose(y[ok], want[ok], rtol=1e-6)


def test_push_long_active_lists(hip):
    """A batch row with more active entries than one LDS table holds (several
    table passes); a layer too wide for a block's LDS keeps the gather path."""
    rng = np.random.default_rng(9)
    n_in, n_out = 9000, 70000
    lens = rng.integers(0, 6, n_in)
    cols = [np.sort(rng.choice(n_out, size=int(k), replace=False)) for k in lens]
    ptrs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    idx = np.concatenate(cols).astype(np.int32)
    w = rng.normal(0, 2, len(idx)).astype(np.float32)
    L = hip.SparseLinearLayer(n_in, n_out, len(idx) + 64)
    L.load_weights(ptrs, idx, w)
    H = HostLayer(n_in, n_out).load_csr(ptrs, idx, w=w)
    B = 2
    r0 = np.sort(rng.permutation(n_in)[:8500])
    r1 = np.sort(rng.permutation(n_in)[:300])
    xp = np.array([0, len(r0), len(r0) + len(r1)], np.int32)
    xi = np.concatenate([r0, r1]).astype(np.int32)
    xv = rng.normal(0, 1, len(xi)).astype(np.float32)
    # 70000 outputs do not fit a block's LDS: the gather path serves this layer
    y = L.forward_sparse(xp, xi, xv, B)
    assert_close_terms(y, H.forward_sparse(xp, xi, xv, B), H.forward_sparse(xp, xi, xv, B, absmode=True), "wide")
    # a narrower layer of the same rows takes the push, over several table passes
    n_out2 = 30000
    keep = idx < n_out2
    rows = np.repeat(np.arange(n_in), lens)[keep]
    ptrs2 = np.concatenate([[0], np.cumsum(np.bincount(rows, minlength=n_in))]).astype(np.int32)
    L2 = hip.SparseLinearLayer(n_in, n_out2, int(keep.sum()) + 64)
    L2.load_weights(ptrs2, idx[keep], w[keep])
    H2 = HostLayer(n_in, n_out2).load_csr(ptrs2, idx[keep], w=w[keep])
    check(hip, L2, H2, xp, xi, xv, B, "long active lists")


def test_push_with_block4_tiles(hip):
    from train_util import add_tiles, make_train_case
    c = add_tiles(make_train_case(60, 90, 0.05, 61), seed=61)
    L = hip.SparseLinearLayer(60, 90, 60 * 90)
    L.load_weights_with_importance(c["ptrs"], c["cols"], c["w"], c["imp"])
    L.load_block4_tiles(c["br"], c["bc"], c["tiles"])
    L.set_value_scales(c["vs"])
    H = HostLayer(60, 90).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    H.set_scales(np.asarray(c["vs"], np.float32))
    rng = np.random.default_rng(2)
    for B in (1, 5, 64):
        xp, xi, xv = sparse_x(rng, B, 60, 0.3)
        check(hip, L, H, xp, xi, xv, B, f"tiles B {B}")


def test_push_dispatch_by_density(hip, monkeypatch):
    monkeypatch.setenv("SILI_PUSH", "1")
    rng = np.random.default_rng(12)
    n_in, n_out = 2000, 3000
    ptrs, idx, w = skewed_layer(rng, n_in, n_out, 5)
    L = hip.SparseLinearLayer(n_in, n_out, len(idx) + 64)
    L.load_weights(ptrs, idx, w)
    H = HostLayer(n_in, n_out).load_csr(ptrs, idx, w=w)
    for density, pushed in ((0.01, True), (0.1, False)):
        xp, xi, xv = sparse_x(rng, 16, n_in, density)
        y = None

        def run():
            nonlocal y
            y = L.forward_sparse(xp, xi, xv, 16)
        names = kernels_run(hip, L, run)
        assert any(n.endswith("push") for n in names) == pushed, (density, names)
        assert_close_terms(y, H.forward_sparse(xp, xi, xv, 16), H.forward_sparse(xp, xi, xv, 16, absmode=True),
                           f"density {density}")
