"""CPU: the oracle's backward with the optimizer update against the
reference's own compiled disldo_backward, deterministic variant
(oracle/_ref, this container), over several calls of each seeded case.

The reference's build (its setup.py flags: -O3 -ffast-math on an FMA target)
contracts a*b+c into FMAs.  The restatement is compiled twice:
  - contracted, as the reference is: codes, dx, scales and their state match
    the reference exactly, except one last-place difference in the second
    moment of rows without synapses (the reference's compiler also
    re-associates (1 - beta2) * g * g there), held to 1e-6 relative;
  - IEEE, every expression as written (the build the GPU is checked against):
    codes match the reference exactly, fp32 results to the last places."""
import numpy as np
import pytest

from oracle import have_ref
from train_util import B4_CASES, TRAIN_CASES, dx_bound, host_layer, make_train_case, ref_layer, split_opts
from util import assert_close_terms

pytestmark = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (no reference tree)")


VARIANTS = ["plain", "resync", "noscale"]


def _run(case, contracted, variant="plain"):
    n_in, n_out, dens, seed, B, lr, opts = TRAIN_CASES[case]
    lopts, copts = split_opts(opts)
    c = make_train_case(n_in, n_out, dens, seed, **lopts)
    H, R = host_layer(c), ref_layer(c)
    rng = c["rng"]
    for step in range(3):
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dy = rng.normal(size=(B, n_out)).astype(np.float32)
        bound = dx_bound(H, dy, lr)
        outs_h = H.backward_train(x, dy, lr, contracted=contracted, variant=variant, **copts)
        outs_r = R.backward_train(x, dy, lr, variant=variant, **copts)
        _, _, _, vr = R.export()
        st = R.get_train_state(c["rank"])
        yield step, lopts, bound, H, outs_h, vr, st, outs_r


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("case", range(len(TRAIN_CASES)))
def test_backward_train_matches_reference(case, variant):
    """The contracted restatement against the reference: exact."""
    for step, lopts, bound, H, (dxh, aih, agh), vr, st, (dxr, air, agr) in _run(case, True, variant):
        assert np.array_equal(H.val[:len(vr)], vr), f"codes differ at step {step}"
        if variant == "resync":
            # true-units weights: -ffast-math re-associates the product chain
            # of the weight and both scales differently in the two sources
            assert_close_terms(dxh, dxr, bound, f"dx at step {step}")
        else:
            assert np.array_equal(dxh, dxr), f"dx differs at step {step}"
        assert np.array_equal(aih, air) and np.array_equal(agh, agr)
        assert np.array_equal(H.value_scale, st["value_scale"]), f"value_scale differs at step {step}"
        assert np.array_equal(H.output_scale, st["output_scale"]), f"output_scale differs at step {step}"
        assert np.array_equal(H.vs_step, st["vs_step"]) and np.array_equal(H.os_step, st["os_step"])
        assert np.array_equal(H.os_importance, st["os_importance"])
        assert np.array_equal(H.vs_momentum, st["vs_momentum"])
        np.testing.assert_allclose(H.vs_importance, st["vs_importance"], rtol=1e-6, atol=0)
        if lopts.get("empty_rows", 0) == 0:
            assert np.array_equal(H.vs_importance, st["vs_importance"])


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("case", range(len(TRAIN_CASES)))
def test_ieee_restatement_against_reference(case, variant):
    """The IEEE restatement (the GPU's checker) against the reference: codes
    exact; dx, scales and state within fp32 rounding of the contractions."""
    for step, _, bound, H, (dxh, aih, agh), vr, st, (dxr, air, agr) in _run(case, False, variant):
        what = f"case {case} {variant} step {step}"
        assert np.array_equal(H.val[:len(vr)], vr), what + ": codes"
        assert_close_terms(dxh, dxr, bound, what + ": dx")
        assert np.array_equal(aih, air) and np.array_equal(agh, agr)
        for k in ("value_scale", "output_scale", "vs_momentum", "vs_importance", "os_importance"):
            np.testing.assert_allclose(getattr(H, k), st[k], rtol=1e-5, atol=1e-30, err_msg=what + ": " + k)
        assert np.array_equal(H.vs_step, st["vs_step"]) and np.array_equal(H.os_step, st["os_step"])


def test_learning_rate_zero_is_plain_backward():
    """lr = 0 changes nothing and gives backward_dense's dx."""
    c = make_train_case(70, 50, 0.1, 11)
    H = host_layer(c)
    val0, vs0 = H.val.copy(), H.value_scale.copy()
    x = c["rng"].normal(size=(3, 70)).astype(np.float32)
    dy = c["rng"].normal(size=(3, 50)).astype(np.float32)
    dx, _, _ = H.backward_train(x, dy, 0.0)
    dx0, _, _ = H.backward_dense(x, dy, threads=1)
    assert np.array_equal(H.val, val0) and np.array_equal(H.value_scale, vs0)
    assert np.array_equal(H.vs_step, np.zeros_like(H.vs_step))
    np.testing.assert_allclose(dx, dx0, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("contracted", [True, False])
@pytest.mark.parametrize("case", range(len(TRAIN_CASES)))
def test_backward_sparse_train_matches_reference(case, contracted):
    """backward_sparse with the update (sisldo_ops.hpp:589-848): codes and the
    value scales' state exact (both builds); dx exact for the build compiled
    like the reference, within the fp32 bar for the IEEE one."""
    from train_util import dx_bound_sparse, sparse_dy
    n_in, n_out, dens, seed, B, lr, opts = TRAIN_CASES[case]
    lopts, copts = split_opts(opts)
    c = make_train_case(n_in, n_out, dens, seed, **lopts)
    H, R = host_layer(c), ref_layer(c)
    rng = c["rng"]
    for step in range(3):
        what = f"case {case} step {step}"
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dp, di, dv, dense = sparse_dy(rng, B, n_out)
        bound = dx_bound_sparse(H, dense, lr)
        dxh, aih, agh = H.backward_sparse_train(x, dp, di, dv, B, lr, contracted=contracted, **copts)
        dxr, air, agr = R.backward_sparse_train(x, dp, di, dv, B, lr, **copts)
        _, _, _, vr = R.export()
        st = R.get_train_state(c["rank"])
        assert np.array_equal(H.val[:len(vr)], vr), what + ": codes"
        if contracted:
            assert np.array_equal(dxh, dxr), what + ": dx"
        else:
            assert_close_terms(dxh, dxr, bound, what + ": dx")
        assert np.array_equal(aih, air) and np.array_equal(agh, agr)
        for k in ("value_scale", "vs_importance", "vs_step"):
            if contracted:
                assert np.array_equal(getattr(H, k), st[k]), what + ": " + k
            else:
                np.testing.assert_allclose(getattr(H, k), st[k], rtol=1e-5, atol=1e-30, err_msg=what + ": " + k)


# (n_in, n_out, scattered density, seed, batch, lr, options, variant): odd
# output widths give edge tiles (the scalar path), the rest 4-lane tiles
@pytest.mark.parametrize("case", range(len(B4_CASES)))
def test_block4_update_matches_reference(case):
    """Layers holding block4 tiles (linear_disldo.hpp:962-1951): the tiles'
    update, with the reference's rows given room for dense tiles (no
    eviction).  Contracted build exact on codes, tile bytes and scale state
    (dx within the bar: the 4-lane sums are re-associated by -ffast-math)."""
    from train_util import add_tiles, dx_bound_tiles, tile_opts
    n_in, n_out, dens, seed, B, lr, opts, variant = B4_CASES[case]
    lopts, copts = split_opts(opts)
    c = add_tiles(make_train_case(n_in, n_out, dens, seed, **lopts), seed=case, **tile_opts(opts))
    assert len(c["br"]) > 0 and ((c["bc"] * 4 + 4 > n_out).any() or n_out % 4 == 0)
    tiles0 = c["tiles"].copy()
    H, R = host_layer(c), ref_layer(c)
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    for t in range(len(c["br"])):
        R.put_tile(int(c["br"][t]), int(c["bc"][t]), c["tiles"][16 * t:16 * t + 16])
    R.block4_headroom(0.2, 16 * max(64, int(np.bincount(c["br"]).max())))
    rng = c["rng"]
    for step in range(3):
        what = f"case {case} {variant} step {step}"
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dy = rng.normal(size=(B, n_out)).astype(np.float32)
        bound = dx_bound(H, dy, lr) + dx_bound_tiles(H, dy, lr)
        dxh, _, _ = H.backward_train(x, dy, lr, contracted=True, variant=variant, **copts)
        dxr, _, _ = R.backward_train(x, dy, lr, variant=variant, **copts)
        _, _, _, vr = R.export()
        br, bc, tr = R.export_tiles()
        st = R.get_train_state(c["rank"])
        assert np.array_equal(H.val[:len(vr)], vr), what + ": codes"
        assert np.array_equal(H.tile_br, br) and np.array_equal(H.tile_bc, bc), what + ": tile set"
        assert np.array_equal(H.tiles[:len(tr)], tr), what + ": tile bytes"
        assert_close_terms(dxh, dxr, bound, what + ": dx")
        for k in ("value_scale", "output_scale", "vs_importance", "os_importance"):
            assert np.array_equal(getattr(H, k), st[k]), what + ": " + k
        assert np.array_equal(H.vs_step, st["vs_step"]) and np.array_equal(H.os_step, st["os_step"]), what
    assert (H.tiles[:len(tiles0)] != tiles0).sum() > 4, "the tiles barely changed"


@pytest.mark.parametrize("case", range(len(B4_CASES)))
def test_block4_sparse_update_matches_reference(case):
    """backward_sparse with the update on layers holding block4 tiles
    (sisldo_ops.hpp:848-1100): the reference rounds the tiles stochastically
    through its per-thread xorshift64*, reseeded before every call; the oracle
    replays the same draws in the same order (draw_mode 0).  Codes, tile
    bytes and the value scales' state exact (contracted build), dx within the
    bar."""
    from train_util import add_tiles, dx_bound_sparse, dx_bound_tiles, sparse_dy, tile_opts
    n_in, n_out, dens, seed, B, lr, opts, _ = B4_CASES[case]
    lopts, copts = split_opts(opts)
    c = add_tiles(make_train_case(n_in, n_out, dens, seed, **lopts), seed=case, **tile_opts(opts))
    tiles0 = c["tiles"].copy()
    H, R = host_layer(c), ref_layer(c)
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    for t in range(len(c["br"])):
        R.put_tile(int(c["br"][t]), int(c["bc"][t]), c["tiles"][16 * t:16 * t + 16])
    R.block4_headroom(0.2, 16 * max(64, int(np.bincount(c["br"]).max())))
    rng = c["rng"]
    for step in range(3):
        what = f"block4 sparse case {case} step {step}"
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        dp, di, dv, dense = sparse_dy(rng, B, n_out, density=0.6)
        bound = dx_bound_sparse(H, dense, lr) + dx_bound_tiles(H, dense, lr, sparse=True)
        dseed = 1000 * case + step + 1
        dxh, _, _ = H.backward_sparse_train(x, dp, di, dv, B, lr, contracted=True, draw_mode=0, draw_seed=dseed,
                                            **copts)
        dxr, _, _ = R.backward_sparse_train(x, dp, di, dv, B, lr, draw_seed=dseed, **copts)
        _, _, _, vr = R.export()
        br, bc, tr = R.export_tiles()
        st = R.get_train_state(c["rank"])
        assert np.array_equal(H.val[:len(vr)], vr), what + ": codes"
        assert np.array_equal(H.tile_br, br) and np.array_equal(H.tile_bc, bc), what + ": tile set"
        assert np.array_equal(H.tiles[:len(tr)], tr), what + ": tile bytes"
        assert_close_terms(dxh, dxr, bound, what + ": dx")
        for k in ("value_scale", "vs_importance", "vs_step"):
            assert np.array_equal(getattr(H, k), st[k]), what + ": " + k
    assert (H.tiles[:len(tiles0)] != tiles0).sum() > 4, "the tiles barely changed"


# the block4 cases whose tiles grow past rows reserved to their content
EVICTING_CASES = (0, 1, 2, 3, 4)


def _tight_pair(case, slack):
    """Host and reference layers of block4 case `case` whose block rows
    reserve their tiles' stored bytes plus `slack` (block4_expand_headroom(0,
    slack)), so tiles that grow in the update outgrow their rows."""
    from train_util import add_tiles, tile_opts
    n_in, n_out, dens, seed, B, lr, opts, variant = B4_CASES[case]
    lopts, copts = split_opts(opts)
    c = add_tiles(make_train_case(n_in, n_out, dens, seed, **lopts), seed=case, **tile_opts(opts))
    H, R = host_layer(c), ref_layer(c)
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    for t in range(len(c["br"])):
        R.put_tile(int(c["br"][t]), int(c["bc"][t]), c["tiles"][16 * t:16 * t + 16])
    R.block4_headroom(0.0, slack)
    (_, _, ta, _, _, _), _ = R.block4_reservations()
    H.b4_alloc = np.array(ta, np.uint64)
    H.b4_flags = R.export_tiles_packed()[0][:len(c["br"])].copy()
    return c, H, R, B, lr, variant, copts


def _same_tiles(H, R, what):
    br, bc, tr = R.export_tiles()
    assert np.array_equal(H.tile_br, br) and np.array_equal(H.tile_bc, bc), what + ": tile set"
    assert np.array_equal(H.tiles[:len(tr)], tr), what + ": tile bytes"
    assert np.array_equal(H.b4_flags[:len(br)], R.export_tiles_packed()[0][:len(br)]), what + ": tile_is_sparse"
    _, ctr = R.block4_reservations()
    assert (H.b4_counters[1], H.b4_counters[2]) == (ctr[1], ctr[2]), what + ": merge overflow counters"


@pytest.mark.parametrize("slack", [0, 3])
@pytest.mark.parametrize("case", range(len(B4_CASES)))
def test_block4_update_eviction_matches_reference(case, slack):
    """The dense update on block rows with little room: tiles that grow past
    their row's reserved bytes lose their lowest-|true importance| live slots
    (Block4Store::merge_row_workspace, block4.hpp:1367-1462; called at
    linear_disldo.hpp:1865-1878).  Tile bytes, tile_is_sparse and the
    overflow counters exact against the reference, dx within the bar."""
    from train_util import dx_bound_tiles
    c, H, R, B, lr, variant, copts = _tight_pair(case, slack)
    rng = c["rng"]
    for step in range(3):
        what = f"case {case} slack {slack} step {step}"
        x = rng.normal(size=(B, c["n_in"])).astype(np.float32)
        dy = rng.normal(size=(B, c["n_out"])).astype(np.float32)
        bound = dx_bound(H, dy, lr) + dx_bound_tiles(H, dy, lr)
        dxh, _, _ = H.backward_train(x, dy, lr, contracted=True, variant=variant, **copts)
        dxr, _, _ = R.backward_train(x, dy, lr, variant=variant, **copts)
        _same_tiles(H, R, what)
        assert_close_terms(dxh, dxr, bound, what + ": dx")
    if slack == 0 and case in EVICTING_CASES:
        assert H.b4_counters[0] > 0, "nothing was evicted"


@pytest.mark.parametrize("slack", [0, 3])
@pytest.mark.parametrize("case", range(len(B4_CASES)))
def test_block4_sparse_update_eviction_matches_reference(case, slack):
    """The sparse-gradient update on block rows with little room: the write-
    back with eviction after every (batch row, block row)
    (sisldo_ops.hpp:1036-1052), the reference's seeded draws replayed."""
    from train_util import dx_bound_sparse, dx_bound_tiles, sparse_dy
    c, H, R, B, lr, _, copts = _tight_pair(case, slack)
    rng = c["rng"]
    for step in range(3):
        what = f"sparse case {case} slack {slack} step {step}"
        x = rng.normal(size=(B, c["n_in"])).astype(np.float32)
        dp, di, dv, dense = sparse_dy(rng, B, c["n_out"], density=0.6)
        bound = dx_bound_sparse(H, dense, lr) + dx_bound_tiles(H, dense, lr, sparse=True)
        dseed = 7000 * case + step + 1
        dxh, _, _ = H.backward_sparse_train(x, dp, di, dv, B, lr, contracted=True, draw_mode=0, draw_seed=dseed,
                                            **copts)
        dxr, _, _ = R.backward_sparse_train(x, dp, di, dv, B, lr, draw_seed=dseed, **copts)
        _same_tiles(H, R, what)
        assert_close_terms(dxh, dxr, bound, what + ": dx")
    if slack == 0 and case in EVICTING_CASES:
        assert H.b4_counters[0] > 0, "nothing was evicted"
