"""GPU: the policy's row patches (csrc/patch.hip) against a full rebuild.
The same sequence of reference-policy calls (build_probes, synap_step,
synap_row_step) runs on two layers: one applies each call's edit as a row
patch of the stores, the other through the bulk pipeline, which rebuilds
every store (SILI_POLICY_PATCH=0).  After every call the internal stores --
canonical and shadow, scattered and block4, work items, split-row lists, the
shadow permutations -- are the same byte for byte (sili_debug_store_digest),
calls return and raise the same, and the layers compute the same.  Cases:
promotion and demotion of tiles, rows long enough to split into several work
items in either orientation, a layer that keeps the shadow permutation
(after an update), and a full sweep of synap_step over every row
(FoldedLayer's, sili/sparse_rnn.py:1206-1212) -- compared after every call
(each flush then writes one block row) and compared only after the sweep
(one flush writes every block row the sweep edited)."""
import numpy as np
import pytest

from test_gpu_synap_policy import feed_accumulators, gpu_policy_layer
from test_synap_policy_oracle import accum, policy_case

pytestmark = pytest.mark.gpu


def call(monkeypatch, patch, f, *args):
    monkeypatch.setenv("SILI_POLICY_PATCH", "1" if patch else "0")
    try:
        return f(*args), None
    except RuntimeError as e:
        return None, str(e)


def same_state(A, B, what):
    da, db = A._store_digest(), B._store_digest()
    names = ["canonical", "shadow", "block4", "block4 shadow", "shadow permutation", "block4 permutation"]
    bad = [names[i] for i in range(6) if da[i] != db[i]]
    if bad:
        detail = []
        ea, eb = A.export_block4(), B.export_block4()
        ka = {(int(r), int(c)): bytes(ea["tiles"][16 * i:16 * i + 16]) for i, (r, c) in enumerate(zip(ea["br"], ea["bc"]))}
        kb = {(int(r), int(c)): bytes(eb["tiles"][16 * i:16 * i + 16]) for i, (r, c) in enumerate(zip(eb["br"], eb["bc"]))}
        for k in sorted(set(ka) | set(kb)):
            if ka.get(k) != kb.get(k):
                detail.append(f"tile {k}: patch {ka.get(k, b'').hex()} rebuild {kb.get(k, b'').hex()}")
        pa, pb = A.export_block4_packed(), B.export_block4_packed()
        if not np.array_equal(pa["tile_is_sparse"], pb["tile_is_sparse"]):
            diff = np.flatnonzero(pa["tile_is_sparse"] != pb["tile_is_sparse"]) if len(pa["tile_is_sparse"]) == \
                len(pb["tile_is_sparse"]) else "lengths"
            detail.append(f"tile_is_sparse differs at {diff}")
        sa, sb = A.export_scattered(), B.export_scattered()
        for k in ("row_byte_start", "row_elem_start", "idx", "val"):
            if not np.array_equal(sa[k], sb[k]):
                detail.append(f"scattered {k} differs")
        assert not bad, f"{what}: {', '.join(bad)} differ; " + "; ".join(detail[:12])


def run_sequence(hip, monkeypatch, c, calls, seed, train_first=False, sweep=False):
    A, B = gpu_policy_layer(hip, c), gpu_policy_layer(hip, c)
    rng = np.random.default_rng(seed)
    n_in, n_out = c["n_in"], c["n_out"]
    if train_first:
        for L in (A, B):
            r = np.random.default_rng(seed + 1)
            x = r.normal(size=(4, n_in)).astype(np.float32)
            dy = r.normal(size=(4, n_out)).astype(np.float32)
            L.forward_dense(x)
            L.backward_dense(dy, 0.05)
        assert A._store_digest()[4] != 0, "the update keeps the shadow permutation"
    same_state(A, B, "start")
    raised = 0
    for it in range(calls):
        what = f"seed {seed} call {it}"
        if it % 3 == 0 or sweep and it % n_in == 0:
            k = int(rng.integers(2, 9))
            s = int(rng.integers(0, 1 << 30))
            for L in (A, B):
                feed_accumulators(L, np.random.default_rng(s), n_in, n_out)
            per_row = bool(rng.integers(0, 2))
            call(monkeypatch, True, A.build_probes, k, per_row)
            call(monkeypatch, False, B.build_probes, k, per_row)
        cutoff = float(rng.choice([0.0, 0.3, 0.6, 1.2]))
        max_rw = int(rng.integers(2, 40))
        max_prune = int(rng.integers(0, 9))
        if not sweep and it % 5 == 4:
            row = int(rng.integers(0, 2 * n_in))
            ra = call(monkeypatch, True, A.synap_row_step, row, cutoff, max_rw, max_prune, 1e-3)
            rb = call(monkeypatch, False, B.synap_row_step, row, cutoff, max_rw, max_prune, 1e-3)
        else:
            ra = call(monkeypatch, True, A.synap_step, cutoff, max_rw, max_prune, 1e-3)
            rb = call(monkeypatch, False, B.synap_step, cutoff, max_rw, max_prune, 1e-3)
        assert ra == rb, what + ": result"
        raised += ra[1] is not None
        same_state(A, B, what)
        if it % 7 == 6:
            x = rng.normal(size=(3, n_in)).astype(np.float32)
            np.testing.assert_allclose(A.forward_dense(x), B.forward_dense(x), rtol=1e-6, atol=1e-6)
            dy = rng.normal(size=(3, n_out)).astype(np.float32)
            np.testing.assert_allclose(A.backward_dense(dy, 0.0), B.backward_dense(dy, 0.0), rtol=1e-6, atol=1e-6)
    return raised


@pytest.mark.parametrize("seed", range(4))
def test_patch_matches_rebuild_with_tiles(hip, monkeypatch, seed):
    run_sequence(hip, monkeypatch, policy_case(seed), 45, seed)


@pytest.mark.parametrize("shape", [(12, 2400, 0.3), (2400, 12, 0.3)])
def test_patch_matches_rebuild_split_rows(hip, monkeypatch, shape):
    """Rows of > 508 index bytes (several work items) in the canonical store
    (wide) or in the shadow (tall)."""
    n_in, n_out, density = shape
    c = policy_case(70, n_in=n_in, n_out=n_out, density=density, tile_density=0.01)
    run_sequence(hip, monkeypatch, c, 24, 70)


def test_patch_matches_rebuild_kept_permutation(hip, monkeypatch):
    run_sequence(hip, monkeypatch, policy_case(81, n_in=40, n_out=64), 30, 81, train_first=True)


def test_patch_matches_rebuild_full_sweep(hip, monkeypatch):
    c = policy_case(90, n_in=36, n_out=50, density=0.12, tile_density=0.06)
    run_sequence(hip, monkeypatch, c, 2 * 36, 90, sweep=True)


@pytest.mark.parametrize("case", ["tiles", "trained", "large"])
def test_deferred_sweep_matches_rebuild(hip, monkeypatch, case):
    """synap_step over every row with nothing else in between: the edits of
    all block rows stay pending on the host and are written in one flush
    (the changed canonical rows and block rows patched, both shadows rebuilt
    from them) when another entry point runs -- here the digest.  Calls
    return as the rebuilding layer's do; the final stores are the same."""
    shape = {"tiles": (36, 50, 0.12, 0.06), "trained": (40, 64, 0.1, 0.05), "large": (200, 300, 0.05, 0.02)}[case]
    n_in, n_out, density, tile_density = shape
    c = policy_case(95, n_in=n_in, n_out=n_out, density=density, tile_density=tile_density)
    A, B = gpu_policy_layer(hip, c), gpu_policy_layer(hip, c)
    rng = np.random.default_rng(95)
    if case == "trained":
        for L in (A, B):
            r = np.random.default_rng(96)
            L.forward_dense(r.normal(size=(4, n_in)).astype(np.float32))
            L.backward_dense(r.normal(size=(4, n_out)).astype(np.float32), 0.05)
    for sweep in range(2):
        s = int(rng.integers(0, 1 << 30))
        for L in (A, B):
            feed_accumulators(L, np.random.default_rng(s), n_in, n_out)
        k = int(rng.integers(3, 9))
        call(monkeypatch, True, A.build_probes, k)
        call(monkeypatch, False, B.build_probes, k)
        cutoff, max_rw, max_prune = [(0.3, 30, 4), (1.2, 8, 6)][sweep]
        for i in range(n_in):
            ra = call(monkeypatch, True, A.synap_step, cutoff, max_rw, max_prune, 1e-3)
            rb = call(monkeypatch, False, B.synap_step, cutoff, max_rw, max_prune, 1e-3)
            assert ra == rb, f"sweep {sweep} step {i}"
        same_state(A, B, f"after sweep {sweep}")
        x = rng.normal(size=(3, n_in)).astype(np.float32)
        np.testing.assert_allclose(A.forward_dense(x), B.forward_dense(x), rtol=1e-6, atol=1e-6)
