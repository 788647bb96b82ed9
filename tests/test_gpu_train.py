"""GPU: backward with the optimizer update (learning_rate != 0) against the
oracle's restatement (pinned to the reference's own disldo_backward in
test_train_oracle.py): deterministic re-quantization bit-exact, scales and
their optimizer state exact at batch 1, dx within the condition-aware bar;
stochastic re-quantization checked per synapse (the code brackets the
pre-rounding value) and statistically (unbiased), and reproducible per seed."""
import numpy as np
import pytest

from sili__new_amd.codec import fp4_decode_np
from train_util import (B4_CASES, TRAIN_CASES, add_tiles, b4_reserve_like_device, check_b4_reservations, dx_bound,
                        host_layer, make_train_case, split_opts)
from util import assert_close_terms

pytestmark = pytest.mark.gpu


# the reference's layer classes per update variant: (deterministic, stochastic)
CLASSES = {"plain": ("SparseLinearLayerDeterministic", "SparseLinearLayer"),
           "resync": ("SparseLinearLayerResyncDeterministic", "SparseLinearLayerResync"),
           "noscale": ("SparseLinearLayerNoScaleDeterministic", "SparseLinearLayerNoScale")}


def gpu_layer(hip, c, deterministic=True, variant="plain", extra=0):
    cls = getattr(hip, CLASSES[variant][0 if deterministic else 1])
    L = cls(c["n_in"], c["n_out"], len(c["cols"]) + 64 + extra)
    L.load_weights_with_importance(c["ptrs"], c["cols"], c["w"], c["imp"])
    if c["rank"] > 1:
        L.set_scale_rank(c["rank"])
    L.set_value_scales(c["vs"])
    if c["os_trainable"] or c["rank"] > 1:
        L.set_output_scales(c["os"])
    if c["is"] is not None:
        for r in range(c["n_in"]):
            L.set_importance_scale_raw(r, float(c["is"][r]))
        for col in range(c["n_out"]):
            L.set_output_importance_scale_raw(col, float(c["ois"][col]))
    return L


def check_state(L, H, exact, what, vs_rtol=1e-6):
    vs = L.get_value_scales()
    st = L.get_scale_state()
    if exact:
        assert np.array_equal(vs, H.value_scale), what + ": value_scale"
        assert np.array_equal(st["vs_importance"], H.vs_importance), what + ": vs_importance"
        assert np.array_equal(st["vs_momentum"], H.vs_momentum), what + ": vs_momentum"
    else:
        np.testing.assert_allclose(vs, H.value_scale, rtol=vs_rtol, atol=0, err_msg=what)
        np.testing.assert_allclose(st["vs_importance"], H.vs_importance, rtol=1e-5, atol=0, err_msg=what)
        np.testing.assert_allclose(st["vs_momentum"], H.vs_momentum, rtol=1e-5, atol=0, err_msg=what)
    assert np.array_equal(st["vs_step"], H.vs_step), what + ": vs_step"
    assert np.array_equal(st["os_step"], H.os_step), what + ": os_step"
    os_ = np.array([L.get_output_scale_k(c, k) for c in range(H.n_out) for k in range(H.rank)], np.float32)
    np.testing.assert_allclose(os_, H.output_scale, rtol=0 if exact else 1e-5, atol=0, err_msg=what)
    np.testing.assert_allclose(st["os_importance"], H.os_importance, rtol=0 if exact else 1e-5, atol=0,
                               err_msg=what)


@pytest.mark.parametrize("variant", list(CLASSES))
@pytest.mark.parametrize("case", range(len(TRAIN_CASES)))
def test_deterministic_update_matches_oracle(hip, case, variant):
    n_in, n_out, dens, seed, B, lr, opts = TRAIN_CASES[case]
    lopts, copts = split_opts(opts)
    c = make_train_case(n_in, n_out, dens, seed, **lopts)
    H, L = host_layer(c), gpu_layer(hip, c, variant=variant)
    rng = c["rng"]
    for step in range(3):
        what = f"case {case} {variant} step {step}"
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dy = rng.normal(size=(B, n_out)).astype(np.float32)
        bound = dx_bound(H, dy, lr)
        L.forward_dense(x)
        dxg = L.backward_dense(dy, lr, **copts)
        dxh, _, _ = H.backward_train(x, dy, lr, variant=variant, **copts)
        val = L.export_scattered()["val"]
        assert np.array_equal(val, H.val[:H.nnz]), what + ": value bytes"
        assert_close_terms(dxg, dxh, bound, what + ": dx")
        check_state(L, H, B == 1, what)
        # the forward after the update reads the refreshed shadow
        x2 = rng.normal(size=(2, n_in)).astype(np.float32)
        assert_close_terms(L.forward_dense(x2), H.forward_dense(x2), H.forward_dense(x2, absmode=True),
                           what + ": forward after update")


@pytest.mark.parametrize("B", [1, 8])
def test_update_then_stream_and_segment_forward(hip, B):
    """A store large enough for the stream kernels: after an update, the
    forward at batch 1 rebuilds its stream copy from the new value bytes."""
    c = make_train_case(400, 3000, 0.4, 21)
    H, L = host_layer(c), gpu_layer(hip, c)
    x = c["rng"].normal(size=(B, 400)).astype(np.float32)
    dy = c["rng"].normal(size=(B, 3000)).astype(np.float32)
    x1 = c["rng"].normal(size=(1, 400)).astype(np.float32)
    L.forward_dense(x1)  # builds the stream copy before the update
    L.forward_dense(x)
    L.backward_dense(dy, 0.05)
    H.backward_train(x, dy, 0.05)
    assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz])
    for xs in (x1, x):
        assert_close_terms(L.forward_dense(xs), H.forward_dense(xs), H.forward_dense(xs, absmode=True), "fwd")


def bracket(v):
    """The representable FP4 values below and above v (clamped at +-6)."""
    tab = fp4_decode_np(np.arange(16))
    t = np.sort(np.unique(tab[np.isfinite(tab)]))
    v = np.clip(v, t[0], t[-1])
    hi = t[np.searchsorted(t, v, side="left").clip(0, len(t) - 1)]
    lo = t[(np.searchsorted(t, v, side="right") - 1).clip(0, len(t) - 1)]
    return lo, hi


@pytest.mark.parametrize("variant", ["plain", "resync"])
def test_stochastic_update_brackets_and_is_unbiased(hip, variant):
    c = make_train_case(400, 500, 0.1, 31)
    H, L = host_layer(c), gpu_layer(hip, c, deterministic=False, variant=variant)
    L.seed_stochastic_rounding(1234)
    x = c["rng"].normal(size=(1, 400)).astype(np.float32)
    dy = c["rng"].normal(size=(1, 500)).astype(np.float32)
    L.forward_dense(x)
    L.backward_dense(dy, 0.05)
    H.backward_train(x, dy, 0.05, variant=variant)
    tab = fp4_decode_np(np.arange(16))
    val = L.export_scattered()["val"]
    for what, v, code in (("weight", H.last_quant[:H.nnz], val >> 4), ("importance", H.last_imp[:H.nnz], val & 15)):
        got = tab[code]
        lo, hi = bracket(v)
        assert np.all((got == lo) | (got == hi)), what + ": a code outside its bracket"
        gap = hi - lo
        inside = gap > 0
        err = (got[inside] - np.clip(v, -6, 6)[inside]) / gap[inside]
        # unbiased rounding: mean error within ~6 standard errors of 0
        assert abs(err.mean()) < 3.0 / np.sqrt(inside.sum()), (what, err.mean(), inside.sum())
        assert 0.1 < np.mean(got[inside] == hi[inside]) < 0.9, what


def test_stochastic_update_reproducible_per_seed(hip):
    c = make_train_case(200, 300, 0.1, 41)
    x = c["rng"].normal(size=(2, 200)).astype(np.float32)
    dy = c["rng"].normal(size=(2, 300)).astype(np.float32)
    out = []
    for seed in (7, 7, 8):
        L = gpu_layer(hip, c, deterministic=False)
        L.seed_stochastic_rounding(seed)
        for _ in range(2):
            L.forward_dense(x)
            L.backward_dense(dy, 0.05)
        out.append(L.export_scattered()["val"])
    assert np.array_equal(out[0], out[1])
    assert not np.array_equal(out[0], out[2])
    hip.seed_fp4_stochastic_rng(99)  # the module-wide seed reaches every layer's next update
    res = []
    for _ in range(2):
        L = gpu_layer(hip, c, deterministic=False)
        L.forward_dense(x)
        L.backward_dense(dy, 0.05)
        res.append(L.export_scattered()["val"])
        hip.seed_fp4_stochastic_rng(99)
    assert np.array_equal(res[0], res[1])


def _sorted_tiles(br, bc, tiles, n_out):
    bcs = (n_out + 3) // 4
    o = np.argsort(np.asarray(br, np.int64) * bcs + np.asarray(bc, np.int64), kind="stable")
    return np.asarray(br)[o], np.asarray(bc)[o], np.asarray(tiles).reshape(-1, 16)[o]


@pytest.mark.parametrize("case", range(len(B4_CASES)))
def test_block4_update_matches_oracle(hip, case):
    """Layers holding block4 tiles (linear_disldo.hpp:962-1951): tile bytes
    and value bytes bit-exact, scales as in the scattered cases, dx within
    the bar (a tile row's dx terms are summed in a per-wave LDS row buffer,
    then added to the scattered rows' dx once per row and batch step)."""
    from train_util import dx_bound_tiles, tile_opts
    n_in, n_out, dens, seed, B, lr, opts, variant = B4_CASES[case]
    lopts, copts = split_opts(opts)
    c = add_tiles(make_train_case(n_in, n_out, dens, seed, **lopts), seed=case, **tile_opts(opts))
    H = host_layer(c)
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    cls = getattr(hip, CLASSES[variant][0])
    mw = len(c["cols"]) + 16 * len(c["br"]) + 64
    L = cls(n_in, n_out, mw)
    L.load_weights_with_importance(c["ptrs"], c["cols"], c["w"], c["imp"])
    L.load_block4_tiles(c["br"], c["bc"], c["tiles"])
    # the rows reserve their tiles' stored bytes: tiles that grow in the
    # update lose slots in the write-back, on both sides
    b4_reserve_like_device(L, H, mw)
    if c["rank"] > 1:
        L.set_scale_rank(c["rank"])
    L.set_value_scales(c["vs"])
    if c["os_trainable"] or c["rank"] > 1:
        L.set_output_scales(c["os"])
    if c["is"] is not None:
        for r in range(n_in):
            L.set_importance_scale_raw(r, float(c["is"][r]))
        for col in range(n_out):
            L.set_output_importance_scale_raw(col, float(c["ois"][col]))
    tiles0 = c["tiles"].copy()
    rng = c["rng"]
    for step in range(3):
        what = f"block4 case {case} {variant} step {step}"
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dy = rng.normal(size=(B, n_out)).astype(np.float32)
        bound = dx_bound(H, dy, lr) + dx_bound_tiles(H, dy, lr)
        L.forward_dense(x)
        dxg = L.backward_dense(dy, lr, **copts)
        dxh, _, _ = H.backward_train(x, dy, lr, variant=variant, **copts)
        assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz]), what + ": value bytes"
        ex = L.export_block4()
        gb, gc, gt = _sorted_tiles(ex["br"], ex["bc"], ex["tiles"], n_out)
        hb, hc, ht = _sorted_tiles(H.tile_br, H.tile_bc, H.tiles[:16 * H.n_tiles], n_out)
        assert np.array_equal(gb, hb) and np.array_equal(gc, hc), what + ": tile set"
        assert np.array_equal(gt, ht), what + ": tile bytes"
        check_b4_reservations(L, H, what)
        assert_close_terms(dxg, dxh, bound, what + ": dx")
        # batch > 1: the fp64 row sums are associated per synapse on the GPU,
        # per batch step in the oracle; the last-bit differences compound over
        # the steps and the block rows' second scale step
        check_state(L, H, B == 1, what, vs_rtol=1e-5)
        # the forward after the update reads the refreshed block4 shadow
        x2 = rng.normal(size=(2, n_in)).astype(np.float32)
        assert_close_terms(L.forward_dense(x2), H.forward_dense(x2), H.forward_dense(x2, absmode=True),
                           what + ": forward after update")
    assert (H.tiles[:len(tiles0)] != tiles0).sum() > 4, "the tiles barely changed"


def test_update_rejects_oversize_batch(hip):
    c = make_train_case(20, 16, 0.3, 5)
    L2 = gpu_layer(hip, c)
    xb = np.ones((1025, 20), np.float32)
    L2.forward_dense(xb)
    with pytest.raises(ValueError):
        L2.backward_dense(np.ones((1025, 16), np.float32), 0.05)


@pytest.mark.parametrize("case", range(len(TRAIN_CASES)))
def test_sparse_update_matches_oracle(hip, case):
    """backward_sparse with the update (sisldo_ops.hpp:589-848) against the
    IEEE restatement: value bytes exact (round to nearest whatever the layer's
    rounding setting: the default, stochastic class is used), value scales and
    their state exact at batch 1, dx within the bar; the forward afterwards
    reads the refreshed shadow."""
    from train_util import dx_bound_sparse, sparse_dy
    n_in, n_out, dens, seed, B, lr, opts = TRAIN_CASES[case]
    lopts, copts = split_opts(opts)
    c = make_train_case(n_in, n_out, dens, seed, **lopts)
    H, L = host_layer(c), gpu_layer(hip, c, deterministic=False)
    rng = c["rng"]
    for step in range(3):
        what = f"case {case} step {step}"
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dp, di, dv, dense = sparse_dy(rng, B, n_out)
        bound = dx_bound_sparse(H, dense, lr)
        dxg = L.backward_sparse(x, dp, di, dv, B, lr, **copts)
        dxh, _, _ = H.backward_sparse_train(x, dp, di, dv, B, lr, **copts)
        assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz]), what + ": value bytes"
        assert_close_terms(dxg, dxh, bound, what + ": dx")
        vs = L.get_value_scales()
        st = L.get_scale_state()
        if B == 1:
            assert np.array_equal(vs, H.value_scale), what + ": value_scale"
            assert np.array_equal(st["vs_importance"], H.vs_importance), what + ": vs_importance"
        else:
            np.testing.assert_allclose(vs, H.value_scale, rtol=1e-6, atol=0, err_msg=what)
            np.testing.assert_allclose(st["vs_importance"], H.vs_importance, rtol=1e-5, atol=0, err_msg=what)
        assert np.array_equal(st["vs_step"], H.vs_step), what + ": vs_step"
        x2 = rng.normal(size=(2, n_in)).astype(np.float32)
        assert_close_terms(L.forward_dense(x2), H.forward_dense(x2), H.forward_dense(x2, absmode=True),
                           what + ": forward after update")


def test_sparse_update_default_learning_rate(hip):
    """backward_sparse's default learning_rate is 0.01 (sili/cpu_backend.cpp:590)."""
    from train_util import sparse_dy
    c = make_train_case(80, 60, 0.2, 12)
    H, L = host_layer(c), gpu_layer(hip, c)
    x = c["rng"].normal(size=(4, 80)).astype(np.float32)
    dp, di, dv, _ = sparse_dy(c["rng"], 4, 60)
    L.backward_sparse(x, dp, di, dv, 4)
    H.backward_sparse_train(x, dp, di, dv, 4, 0.01)
    assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz])


def _splitmix64(z):
    M = (1 << 64) - 1
    z = (z + 0x9E3779B97F4A7C15) & M
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)


@pytest.mark.parametrize("case", range(len(B4_CASES)))
def test_block4_sparse_update_matches_oracle(hip, case):
    """backward_sparse with the update on layers holding block4 tiles
    (sisldo_ops.hpp:848-1100): the reference rounds the tiles stochastically
    in every layer class; the GPU draws splitmix64(call seed + 2 id), which
    the oracle replays (draw_mode 1; its other draw mode is pinned exactly to
    the reference's own draws).  Value bytes and tile bytes bit-exact, the
    value scales as the scattered sparse update (exact at batch 1), dx within
    the bar."""
    from train_util import dx_bound_sparse, dx_bound_tiles, sparse_dy, tile_opts
    n_in, n_out, dens, seed, B, lr, opts, _ = B4_CASES[case]
    lopts, copts = split_opts(opts)
    c = add_tiles(make_train_case(n_in, n_out, dens, seed, **lopts), seed=case, **tile_opts(opts))
    H = host_layer(c)
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    L = gpu_layer(hip, c, deterministic=(case % 2 == 0), extra=16 * len(c["br"]))
    L.load_block4_tiles(c["br"], c["bc"], c["tiles"])
    b4_reserve_like_device(L, H, len(c["cols"]) + 64 + 16 * len(c["br"]))
    s0 = 977 + case
    L.seed_stochastic_rounding(s0)
    tiles0 = c["tiles"].copy()
    rng = c["rng"]
    for step in range(3):
        what = f"block4 sparse case {case} step {step}"
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dp, di, dv, dense = sparse_dy(rng, B, n_out, density=0.6)
        bound = dx_bound_sparse(H, dense, lr) + dx_bound_tiles(H, dense, lr, sparse=True)
        dxg = L.backward_sparse(x, dp, di, dv, B, lr, **copts)
        call_seed = _splitmix64(s0 ^ _splitmix64(step + 1))
        dxh, _, _ = H.backward_sparse_train(x, dp, di, dv, B, lr, draw_mode=1, draw_seed=call_seed, **copts)
        assert np.array_equal(L.export_scattered()["val"], H.val[:H.nnz]), what + ": value bytes"
        ex = L.export_block4()
        gb, gc, gt = _sorted_tiles(ex["br"], ex["bc"], ex["tiles"], n_out)
        hb, hc, ht = _sorted_tiles(H.tile_br, H.tile_bc, H.tiles[:16 * H.n_tiles], n_out)
        assert np.array_equal(gb, hb) and np.array_equal(gc, hc), what + ": tile set"
        assert np.array_equal(gt, ht), what + ": tile bytes"
        check_b4_reservations(L, H, what)
        assert_close_terms(dxg, dxh, bound, what + ": dx")
        vs, st = L.get_value_scales(), L.get_scale_state()
        if B == 1:
            assert np.array_equal(vs, H.value_scale), what + ": value_scale"
            assert np.array_equal(st["vs_importance"], H.vs_importance), what + ": vs_importance"
        else:
            np.testing.assert_allclose(vs, H.value_scale, rtol=1e-5, atol=0, err_msg=what)
            np.testing.assert_allclose(st["vs_importance"], H.vs_importance, rtol=1e-5, atol=0, err_msg=what)
        assert np.array_equal(st["vs_step"], H.vs_step), what + ": vs_step"
        x2 = rng.normal(size=(2, n_in)).astype(np.float32)
        assert_close_terms(L.forward_dense(x2), H.forward_dense(x2), H.forward_dense(x2, absmode=True),
                           what + ": forward after update")
    assert (H.tiles[:len(tiles0)] != tiles0).sum() > 4, "the tiles barely changed"
