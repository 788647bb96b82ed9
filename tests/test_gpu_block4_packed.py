"""GPU: the reference's block4 tile encoding on the device store
(tile_is_sparse, sparse-packed tile bytes, Block4View) against its
restatement (oracle.TileEncodingState / pack_tiles, pinned to the compiled
reference in tests/test_block4_packed_oracle.py): after loads at several
switch points, after dense and sparse-gradient updates, and over the
reference policy's and the bulk step's structural edits."""
import numpy as np
import pytest

from oracle import SWITCH_POINT, TileEncodingState, pack_tiles, tile_live

pytestmark = pytest.mark.gpu


def _sorted(ex, n_out):
    bcs = (n_out + 3) // 4
    o = np.argsort(np.asarray(ex["br"], np.int64) * bcs + ex["bc"], kind="stable")
    assert np.array_equal(o, np.arange(len(o))), "export is in canonical order"
    return ex["br"], ex["bc"], np.asarray(ex["tiles"]).reshape(-1, 16)


def check(L, S, what):
    ex = L.export_block4()
    br, bc, tiles = _sorted(ex, L.n_outputs)
    pk = L.export_block4_packed()
    want = S.flags(br, bc)
    assert np.array_equal(pk["tile_is_sparse"], want), what + ": tile_is_sparse"
    assert np.array_equal(pk["tile_data"], pack_tiles(tiles, want)), what + ": tile bytes"
    # row starts: each block row's tiles, back to back
    lens = np.where(want == 1, 1 + (tile_live(tiles) + 1) // 2 + tile_live(tiles), 16)
    rows = np.bincount(br, weights=lens, minlength=(L.n_inputs + 3) // 4).astype(np.uint64)
    assert np.array_equal(pk["tile_byte_start"], np.concatenate([[0], np.cumsum(rows)]).astype(np.uint64))
    v = L.block4
    assert v.tiles == len(br) and v.synapses == int(tile_live(tiles).sum())
    assert v.used_bytes == len(pk["tile_data"])
    # alloc_bytes: the rows' reserved tile bytes, which hold their content
    assert v.alloc_bytes == int(np.sum(L.export_block4_layout()["ta"])) >= v.used_bytes
    assert v.dropped_growth_events == v.row_merge_overflow_events == v.row_merge_overflow_bytes_dropped == 0
    return br, bc, tiles


@pytest.mark.parametrize("sp", [None, 4, 0, 10])
def test_load_encoding_and_view(hip, sp):
    rng = np.random.default_rng(11)
    n_in, n_out = 36, 44
    keys = np.sort(rng.choice(9 * 11, 40, replace=False))
    br, bc = (keys // 11).astype(np.int32), (keys % 11).astype(np.int32)
    tiles = np.zeros((40, 16), np.uint8)
    for t in range(40):
        live = rng.choice(16, t % 17, replace=False)
        tiles[t, live] = rng.integers(1, 256, len(live))
    L = hip.SparseLinearLayer(n_in, n_out, 16 * 40)
    assert L.block4.switch_point == SWITCH_POINT
    if sp is not None:
        L.block4.switch_point = sp
    L.load_block4_tiles(br, bc, tiles.ravel())
    S = TileEncodingState(SWITCH_POINT if sp is None else sp)
    S.load(br, bc, tiles)
    check(L, S, f"load sp={sp}")
    with pytest.raises(ValueError):
        L.block4.switch_point = 11
    # a switch-point change alone re-encodes nothing (as the reference's setter)
    L.block4.switch_point = 3
    check(L, S, "after setting switch_point")


def test_load_dense_codes_encoding(hip):
    import os
    G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
    n_in, n_out = (int(v) for v in G["ldc_n"])
    L = hip.SparseLinearLayer(n_in, n_out, n_in * n_out)
    L.load_dense_codes(G["ldc_wc"], G["ldc_ic"])
    ex = L.export_block4()
    S = TileEncodingState()
    S.load(ex["br"], ex["bc"], ex["tiles"])
    check(L, S, "load_dense_codes")


def test_updates_reencode(hip):
    from test_gpu_train import gpu_layer
    from train_util import B4_CASES, add_tiles, make_train_case, sparse_dy, split_opts, tile_opts
    flips = 0
    for case in (0, 1, 7):
        n_in, n_out, dens, seed, B, lr, opts, variant = B4_CASES[case]
        lopts, copts = split_opts(opts)
        c = add_tiles(make_train_case(n_in, n_out, dens, seed, **lopts), seed=case, **tile_opts(opts))
        L = gpu_layer(hip, c, variant=variant, extra=1024 * len(c["br"]))
        L.load_block4_tiles(c["br"], c["bc"], c["tiles"])
        # rows with room for all their tiles dense: no slot is evicted
        L.expand_block4_headroom(15.0)
        S = TileEncodingState()
        ex = L.export_block4()
        S.load(ex["br"], ex["bc"], ex["tiles"])
        br, bc, tiles = check(L, S, f"case {case} load")
        rng = c["rng"]
        for step in range(3):
            x = rng.normal(size=(B, n_in)).astype(np.float32)
            dy = rng.normal(size=(B, n_out)).astype(np.float32)
            L.forward_dense(x)
            L.backward_dense(dy, 2.0 * lr, **copts)
            before = S.flags(br, bc)
            ex = L.export_block4()
            S.reencode(ex["br"], ex["bc"], ex["tiles"])
            br, bc, tiles = check(L, S, f"case {case} dense update {step}")
            flips += int((before != S.flags(br, bc)).sum())
            dp, di, dv, dense = sparse_dy(rng, B, n_out, density=0.2)
            L.backward_sparse(x, dp, di, dv, B, 2.0 * lr, **copts)
            nz = np.any(dense != 0, axis=0)
            dirty = np.array([nz[4 * b:4 * b + 4].any() for b in bc])
            before = S.flags(br, bc)
            ex = L.export_block4()
            S.reencode(ex["br"], ex["bc"], ex["tiles"], which=dirty)
            br, bc, tiles = check(L, S, f"case {case} sparse update {step}")
            flips += int((before != S.flags(br, bc)).sum())
    assert flips > 0


def test_policy_and_bulk_edits(hip):
    from test_gpu_synap_policy import feed_accumulators, gpu_policy_layer
    from test_synap_policy_oracle import policy_case
    frozen = 0
    for seed in range(3):
        c = policy_case(seed, tile_density=0.3)
        L = gpu_policy_layer(hip, c)
        S = TileEncodingState()
        ex = L.export_block4()
        S.load(ex["br"], ex["bc"], ex["tiles"])
        check(L, S, f"seed {seed} load")
        rng = c["rng"]
        for it in range(30):
            if it % 3 == 0:
                feed_accumulators(L, rng, c["n_in"], c["n_out"])
                L.build_probes(int(rng.integers(1, 7)))
            b = L.export_block4()
            before = (b["br"], b["bc"], b["tiles"])
            L.synap_step(float(rng.choice([0.6, 1.2, 2.5, 6.5])), int(rng.integers(2, 30)), int(rng.integers(1, 9)))
            a = L.export_block4()
            S.structural(before, (a["br"], a["bc"], a["tiles"]))
            br, bc, tiles = check(L, S, f"seed {seed} call {it}")
            frozen += int(((S.flags(br, bc) == 0) & (tile_live(tiles) <= SWITCH_POINT)).sum())
        # the bulk magnitude-prune step follows the same rules
        b = L.export_block4()
        before = (b["br"], b["bc"], b["tiles"])
        cr = rng.integers(0, c["n_in"], 60).astype(np.int32)
        cc = rng.integers(0, c["n_out"], 60).astype(np.int32)
        cv = rng.normal(0, 1.0, 60).astype(np.float32)
        L.synapto_step(0.2, cr, cc, cv)
        a = L.export_block4()
        S.structural(before, (a["br"], a["bc"], a["tiles"]))
        check(L, S, f"seed {seed} bulk step")
    assert frozen > 0, "no dense tile with <= switch_point live slots arose"
