"""CPU: the reference's sparse-packed block4 tiles (block4.hpp:332-388,
tile_is_sparse, switch_point) against the restatement the device store is
checked with (oracle.TileEncodingState + oracle.pack_tiles): after loads
at several switch points, after the dense and the sparse-gradient optimizer
updates, and over the reference's synaptogenesis policy (removals leave a
dense tile dense; inserts and promotions re-encode)."""
import numpy as np
import pytest

from oracle import RefLayer, TileEncodingState, have_ref, pack_tiles, sparse_pack_tile, tile_live

pytestmark = pytest.mark.skipif(not have_ref(), reason="reference build (oracle/_ref) absent")


def test_sparse_pack_layout_kats():
    # block4.hpp:340-383: [count][ceil(count/2) position bytes, even index in
    # the high nibble][count values]
    t = np.zeros(16, np.uint8)
    assert sparse_pack_tile(t) == bytes([0])
    t[3], t[7], t[12] = 0x21, 0x05, 0xF3
    assert sparse_pack_tile(t) == bytes([3, 0x37, 0xC0, 0x21, 0x05, 0xF3])


def _ref_tiles(n_in, n_out, br, bc, tiles, sp=None):
    R = RefLayer(n_in, n_out, np.zeros(n_in + 1, np.int32), np.zeros(0, np.int32), np.zeros(0, np.float32))
    if sp is not None:
        R.switch_point(sp)
    for t in range(len(br)):
        R.put_tile(int(br[t]), int(bc[t]), tiles[t])
    return R


def _check(R, S, what):
    br, bc, tiles = R.export_tiles()
    flags, packed, used = R.export_tiles_packed()
    want = S.flags(br, bc)
    assert np.array_equal(flags, want), what + ": tile_is_sparse"
    assert np.array_equal(packed, pack_tiles(tiles, want)), what + ": stored bytes"
    return br, bc, tiles


@pytest.mark.parametrize("sp", [None, 4, 0, 10])
def test_load_encoding(sp):
    rng = np.random.default_rng(7)
    n_in, n_out = 36, 44
    keys = rng.choice(9 * 11, 40, replace=False)
    br, bc = (keys // 11).astype(np.int32), (keys % 11).astype(np.int32)
    tiles = np.zeros((40, 16), np.uint8)
    for t in range(40):  # live counts 0 .. 16
        live = rng.choice(16, t % 17, replace=False)
        tiles[t, live] = rng.integers(1, 256, len(live))
    R = _ref_tiles(n_in, n_out, br, bc, tiles, sp)
    assert R.switch_point() == (10 if sp is None else sp)
    S = TileEncodingState(R.switch_point())
    b, c, t = R.export_tiles()
    S.load(b, c, t)
    _check(R, S, f"load sp={sp}")
    assert sorted(set(tile_live(t))) == list(range(17))


def test_updates_reencode_the_tiles_they_touch():
    from train_util import B4_CASES, add_tiles, make_train_case, ref_layer, sparse_dy, split_opts, tile_opts
    for case in (0, 1, 7):
        n_in, n_out, dens, seed, B, lr, opts, variant = B4_CASES[case]
        lopts, copts = split_opts(opts)
        c = add_tiles(make_train_case(n_in, n_out, dens, seed, **lopts), seed=case, **tile_opts(opts))
        R = ref_layer(c)
        for t in range(len(c["br"])):
            R.put_tile(int(c["br"][t]), int(c["bc"][t]), c["tiles"][16 * t:16 * t + 16])
        R.block4_headroom(0.2, 16 * max(64, int(np.bincount(c["br"]).max())))
        S = TileEncodingState()
        br, bc, tiles = R.export_tiles()
        S.load(br, bc, tiles)
        _check(R, S, f"case {case} load")
        rng = c["rng"]
        flips = 0
        for step in range(3):
            x = rng.normal(size=(B, n_in)).astype(np.float32)
            dy = rng.normal(size=(B, n_out)).astype(np.float32)
            R.backward_train(x, dy, 2.0 * lr, variant=variant, **copts)
            before = S.flags(br, bc)
            br, bc, tiles = R.export_tiles()
            S.reencode(br, bc, tiles)
            flips += int((before != S.flags(br, bc)).sum())
            _check(R, S, f"case {case} dense update {step}")
            dp, di, dv, dense = sparse_dy(rng, B, n_out, density=0.2)
            R.backward_sparse_train(x, dp, di, dv, B, 2.0 * lr, draw_seed=step + 1, **copts)
            nz = np.any(dense != 0, axis=0)  # columns with a nonzero dy in some batch row
            dirty = np.array([nz[4 * b:4 * b + 4].any() for b in bc])
            before = S.flags(br, bc)
            br, bc, tiles = R.export_tiles()
            S.reencode(br, bc, tiles, which=dirty)
            flips += int((before != S.flags(br, bc)).sum())
            _check(R, S, f"case {case} sparse update {step}")
        assert flips > 0, f"case {case}: no tile changed its encoding"


def test_policy_edits_keep_dense_tiles_dense():
    from test_synap_policy_oracle import accum, layers, policy_case
    seen_frozen = 0
    for seed in range(4):
        c = policy_case(seed, tile_density=0.3)
        H, R = layers(c)
        S = TileEncodingState()
        br, bc, tiles = R.export_tiles()
        S.load(br, bc, tiles)
        _check(R, S, f"seed {seed} load")
        rng = c["rng"]
        cur = 0
        for it in range(40):
            if it % 3 == 0:
                ai, ag = accum(rng, c["n_in"]) + 1.0, accum(rng, c["n_out"]) + 1.0  # probe scores >= 1
                R.build_probes(ai, ag, int(rng.integers(1, 7)))
            cutoff = float(rng.choice([0.6, 1.2, 2.5, 6.5]))
            before = R.export_tiles()
            _, cur = R.synap_row_step(cur, cutoff, int(rng.integers(2, 30)), int(rng.integers(1, 9)), 1e-3)
            after = R.export_tiles()
            S.structural(before, after)
            _check(R, S, f"seed {seed} call {it}")
            live = tile_live(after[2])
            seen_frozen += int(((S.flags(after[0], after[1]) == 0) & (live <= 10)).sum())
    assert seen_frozen > 0, "no dense tile with <= switch_point live slots arose"
