"""CPU: the oracle's restatement of the reference's synaptogenesis policy
(delta_csr_build_probes, delta_csr_synap_row_step) against the reference's
own compiled functions (oracle/_ref), over random call sequences: probes
(shared and per-row top-k, accumulators with ties), removals by importance
cutoff and by capacity, the prune cap, inserts, block4 promotion and
demotion, out_degree bookkeeping.  Structure compared byte for byte after
every call."""
import numpy as np
import pytest

from oracle import HostLayer, have_ref

pytestmark = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (no reference tree)")


def policy_case(seed, n_in=24, n_out=40, density=0.15, tile_density=0.08):
    """Scattered synapses with importances over the FP4 range, plus block4
    tiles (2-16 live slots each) outside the scattered positions."""
    rng = np.random.default_rng(seed)
    brs, bcs = (n_in + 3) // 4, (n_out + 3) // 4
    keys = np.flatnonzero(rng.random(brs * bcs) < tile_density)
    br, bc = (keys // bcs).astype(np.int32), (keys % bcs).astype(np.int32)
    tiles = np.zeros((len(keys), 16), np.uint8)
    cover = np.zeros((n_in, n_out), bool)
    for t, (a, b) in enumerate(zip(br, bc)):
        live = rng.random(16) < rng.uniform(0.2, 0.9)
        live[rng.integers(16)] = live[rng.integers(16)] = True
        for s in np.flatnonzero(live):
            lj, li = divmod(int(s), 4)
            r, c = a * 4 + li, b * 4 + lj
            if r < n_in and c < n_out:
                w = rng.integers(1, 16)
                w = 3 if w == 8 else w
                tiles[t, s] = (rng.integers(0, 8) << 4) | w
                cover[r, c] = True
    mask = (rng.random((n_in, n_out)) < density) & ~cover
    mask[np.arange(n_in), rng.integers(0, n_out, n_in)] |= ~cover[np.arange(n_in), rng.integers(0, n_out, n_in)]
    mask &= ~cover
    for r in range(n_in):
        if not mask[r].any():
            free = np.flatnonzero(~cover[r])
            mask[r, free[0]] = True
    ptrs = np.concatenate([[0], np.cumsum(mask.sum(1))]).astype(np.int32)
    cols = np.nonzero(mask)[1].astype(np.int32)
    w = rng.normal(0, 2, len(cols)).astype(np.float32)
    imp = rng.choice([0.0, 0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 6.0], len(cols)).astype(np.float32)
    return dict(n_in=n_in, n_out=n_out, ptrs=ptrs, cols=cols, w=w, imp=imp, br=br, bc=bc,
                tiles=tiles.ravel(), rng=rng)


def layers(c):
    from oracle import RefLayer
    H = HostLayer(c["n_in"], c["n_out"]).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    H.load_tiles(c["br"], c["bc"], c["tiles"])
    R = RefLayer(c["n_in"], c["n_out"], c["ptrs"], c["cols"], c["w"], c["imp"], blank_fraction=8.0)
    for t in range(len(c["br"])):
        R.put_tile(int(c["br"][t]), int(c["bc"][t]), c["tiles"][16 * t:16 * t + 16])
    return H, R


def accum(rng, n):
    """Activity accumulators with ties (repeated values and zeros)."""
    return (rng.integers(0, 6, n) * 0.5).astype(np.float32)


def assert_same(H, R, what):
    bs, es, idx, val = R.export()
    assert np.array_equal(H.row_elem_start, es), what + ": elem_start"
    assert np.array_equal(H.row_byte_start, bs), what + ": byte_start"
    assert np.array_equal(H.idx[:len(idx)], idx) and np.array_equal(H.val[:len(val)], val), what + ": bytes"
    br, bc, t = R.export_tiles()
    assert np.array_equal(H.tile_br, br) and np.array_equal(H.tile_bc, bc), what + ": tile positions"
    assert np.array_equal(H.tiles[:len(t)], t), what + ": tile bytes"
    assert np.array_equal(H.out_deg, R.out_degree()), what + ": out_degree"


@pytest.mark.parametrize("seed", range(6))
def test_synap_policy_matches_reference(seed):
    c = policy_case(seed)
    H, R = layers(c)
    rng = c["rng"]
    H.out_deg = np.bincount(c["cols"], minlength=c["n_out"]).astype(np.int32)
    assert np.array_equal(H.out_deg, R.out_degree())
    cur = 0
    changed = 0
    for it in range(60):
        what = f"seed {seed} call {it}"
        if it % 3 == 0:
            k = int(rng.integers(0, 7))
            per_row = bool(rng.integers(0, 2))
            ai, ag = accum(rng, c["n_in"]), accum(rng, c["n_out"])
            H.build_probes(ai, ag, k, per_row)
            R.build_probes(ai, ag, k, per_row)
            pr, pc, pv, has = R.get_probes()
            assert H.probe_nnz == len(pr), what + ": probe count"
            assert np.array_equal(H.probes[0][:H.probe_nnz], pr) and np.array_equal(H.probes[1][:H.probe_nnz], pc)
            assert np.array_equal(H.probes[2][:H.probe_nnz], pv), what + ": probe scores"
            assert (len(H.probes[0]) > 0) == has, what + ": probe vectors"
        if (it // 12) % 2 == 0:  # growth phase: low cutoff, room to grow
            cutoff, max_rw = float(rng.choice([0.0, 0.3])), int(rng.integers(10, 30))
        else:                    # pruning phase
            cutoff, max_rw = float(rng.choice([0.6, 1.2, 2.5])), int(rng.integers(2, 12))
        max_prune = int(rng.integers(1, 9))
        eps = float(rng.choice([1e-3, 0.75]))
        before = H.val[:H.nnz].copy(), H.n_tiles
        did_h = H.synap_step(cutoff, max_rw, max_prune, eps)
        did_r, cur = R.synap_row_step(cur, cutoff, max_rw, max_prune, eps)
        assert did_h == did_r and H.synap_cursor == cur, what + ": return / cursor"
        assert_same(H, R, what)
        changed += (H.nnz != len(before[0])) or (H.n_tiles != before[1])
    assert changed > 5, "the sequence made too few structural changes to test anything"


def test_removal_after_demotion_is_skipped():
    """A tile row holding two live slots, both below the cutoff: the first
    removal (highest column first) demotes the tile, which moves the other
    slot to the scattered store; the second removal then finds no tile and
    leaves it (delta_csr_memory.hpp:1183-1212), while out_degree still drops."""
    from oracle import RefLayer
    n_in, n_out = 8, 12
    ptrs = np.array([0, 1, 2, 3, 4, 5, 6, 7, 8], np.int32)
    cols = np.array([11, 11, 11, 11, 11, 11, 11, 11], np.int32)
    w = np.full(8, 1.0, np.float32)
    imp = np.full(8, 6.0, np.float32)
    tile = np.zeros(16, np.uint8)
    tile[0 * 4 + 1] = 0x03  # row 1, col 4: importance code 0, weight 1.5
    tile[2 * 4 + 1] = 0x02  # row 1, col 6: importance code 0, weight 1.0
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=w, imp=imp).load_tiles([0], [1], tile)
    R = RefLayer(n_in, n_out, ptrs, cols, w, imp, blank_fraction=8.0)
    R.put_tile(0, 1, tile)
    # the reference's out_degree after a load counts the scattered synapses only
    H.out_deg = R.out_degree().copy()
    did_h, nxt_h = H.synap_row_step(1, 1.0, 30, 8, 1e-3)
    did_r, nxt_r = R.synap_row_step(1, 1.0, 30, 8, 1e-3)
    assert did_h and did_r and nxt_h == nxt_r == 2
    assert_same(H, R, "demote edge")
    # removing col 6 left one live slot: the tile was demoted, moving col 4 to
    # the scattered store, where the removal aimed at the tile slot missed it
    cols_after = H.decode_cols()
    r1 = cols_after[int(H.row_elem_start[1]):int(H.row_elem_start[2])]
    assert 4 in r1 and 6 not in r1 and H.n_tiles == 0
    assert H.out_deg[4] == 0 and H.out_deg[6] == 0


def test_empty_row_without_probes_returns_false():
    from oracle import RefLayer
    ptrs = np.array([0, 0, 2], np.int32)
    cols = np.array([1, 3], np.int32)
    w = np.ones(2, np.float32)
    H = HostLayer(2, 5).load_csr(ptrs, cols, w=w)
    R = RefLayer(2, 5, ptrs, cols, w, blank_fraction=8.0)
    H.out_deg = R.out_degree()
    assert H.synap_row_step(0, 0.5, 4) == (False, 1)
    assert R.synap_row_step(0, 0.5, 4) == (False, 1)
    assert_same(H, R, "empty row")


@pytest.mark.parametrize("case", ["scattered_low", "tile_low", "both_low"])
def test_synapse_stored_twice(case):
    """A synapse held both in its row and in a live tile slot (a load that
    puts a tile over a scattered synapse, or an update that makes a zero slot
    live): each removal takes the copy its entry names, the row's or the
    tile's (delta_csr_memory.hpp:1183-1225)."""
    from oracle import RefLayer
    n_in, n_out = 4, 12
    ptrs = np.array([0, 0, 3, 3, 3], np.int32)
    cols = np.array([2, 5, 9], np.int32)  # row 1
    w = np.array([1.0, -1.5, 2.0], np.float32)
    imp_s, imp_t = {"scattered_low": (0.0, 6.0), "tile_low": (6.0, 0.0), "both_low": (0.0, 0.5)}[case]
    imp = np.array([6.0, imp_s, 6.0], np.float32)
    tile = np.zeros(16, np.uint8)
    imp_code = {0.0: 0, 0.5: 1, 6.0: 7}[imp_t]
    tile[1 * 4 + 1] = (imp_code << 4) | 0x3  # (row 1, col 5): the same synapse in the tile
    tile[2 * 4 + 1] = 0x72                   # (row 1, col 6)
    tile[3 * 4 + 0] = 0x71                   # (row 0, col 7)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=w, imp=imp).load_tiles([0], [1], tile)
    R = RefLayer(n_in, n_out, ptrs, cols, w, imp, blank_fraction=8.0)
    R.put_tile(0, 1, tile)
    H.out_deg = R.out_degree().copy()
    did_h, nxt_h = H.synap_row_step(1, 1.0, 30, 8, 1e-3)
    did_r, nxt_r = R.synap_row_step(1, 1.0, 30, 8, 1e-3)
    assert did_h == did_r and nxt_h == nxt_r
    assert_same(H, R, case)
    r1 = H.decode_cols()[int(H.row_elem_start[1]):int(H.row_elem_start[2])]
    slot = int(H.tiles[1 * 4 + 1])
    assert (5 in r1) == (case == "tile_low"), case + ": the row's copy"
    assert (slot != 0) == (case == "scattered_low"), case + ": the tile's copy"
