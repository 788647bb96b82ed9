"""GPU: gathers in column-block passes (the gathered operand, columns x batch
fp32, exceeds one XCD's 4 MiB L2: each pass gathers a <= 2 MiB slice; pass 0
stores, later passes add) against the CPU oracle, in both orientations, with
rows long enough to be split into several work items inside a block."""
import numpy as np
import pytest

from oracle import HostLayer
from tests.test_gpu_stream import kernel_counts, make_pair, transpose_rows
from tests.util import assert_close_terms

pytestmark = pytest.mark.gpu


def synthetic(hip, n_in, n_out, keep, seed):
    L = hip.SparseLinearLayer(n_in, n_out, 1)
    L.load_synthetic(seed, keep, 0.02, 0.5)
    ex = L.export_scattered()
    H = HostLayer(n_in, n_out).load_encoded(ex["row_byte_start"], ex["row_elem_start"], ex["idx"], ex["val"])
    H.set_scales(np.asarray(L.get_value_scales(), np.float32))
    return H, L


@pytest.mark.parametrize("B,passes", [(32, 1), (64, 1), (128, 4), (256, 8)])
def test_forward_column_blocks(hip, monkeypatch, B, passes):
    # shadow columns = n_in = 16384: operand 64 KiB per batch column
    # (batches 65..128 take the staged-input gather unless it is switched off)
    monkeypatch.setenv("SILI_STAGED", "0")
    H, L = synthetic(hip, 16384, 300, 0.4, 99)
    x = np.random.default_rng(B).normal(size=(B, 16384)).astype(np.float32)
    counts = kernel_counts(hip, L, lambda: assert_close_terms(
        L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), f"colblock fwd B{B}"))
    assert counts.get("fwd:gather") == passes, counts


def test_forward_staged_at_batch_128(hip):
    """By default batch 128 stages the input in LDS: one launch, no passes."""
    H, L = synthetic(hip, 16384, 300, 0.4, 97)
    x = np.random.default_rng(7).normal(size=(128, 16384)).astype(np.float32)
    counts = kernel_counts(hip, L, lambda: assert_close_terms(
        L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), "staged fwd B128"))
    assert counts.get("fwd:gather_staged") == 1 and "fwd:gather" not in counts, counts


def test_forward_column_blocks_off(hip, monkeypatch):
    monkeypatch.setenv("SILI_COLBLOCK", "0")
    monkeypatch.setenv("SILI_STAGED", "0")
    H, L = synthetic(hip, 16384, 300, 0.4, 98)
    x = np.random.default_rng(5).normal(size=(128, 16384)).astype(np.float32)
    counts = kernel_counts(hip, L, lambda: assert_close_terms(
        L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), "no colblock fwd"))
    assert counts.get("fwd:gather") == 1, counts


def test_backward_column_blocks_designed_rows(hip):
    """Canonical orientation (dx = W^T g gathers gT, 20000 columns x 64):
    short, empty and long rows, multi-byte deltas, 3 passes, twice in a row."""
    rng = np.random.default_rng(3)
    n_out = 20000
    rows = []
    for r in range(400):
        k = [0, 1, 5, 40, 300, 2500, 9000][r % 7]
        rows.append(np.sort(rng.choice(n_out, size=k, replace=False)))
    H, L = make_pair(hip, rows, n_out)
    for rep in range(2):
        x = rng.normal(size=(64, len(rows))).astype(np.float32)
        g = rng.normal(size=(64, n_out)).astype(np.float32)

        def run():
            L.forward_dense(x)
            dx = L.backward_dense(g, 0.0)
            assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0],
                               f"colblock dx {rep}")
        counts = kernel_counts(hip, L, run)
        assert counts.get("bwd:gather") == 3, counts


@pytest.mark.parametrize("n_in,n_out,op", [(16383, 301, "fwd"), (301, 16383, "bwd")])
def test_block4_column_blocks(hip, monkeypatch, n_in, n_out, op):
    """Block4 gathers (plus scattered synapses outside the tiles) in column-block
    passes: forward over a 16383-wide input, grad-input over a 16383-wide
    gradient, batch 128 (8 MB operand: 4 passes of 2 MiB slices), edge tiles
    at the last block."""
    monkeypatch.setenv("SILI_COLBLOCK_B4_MB", "2")
    from tests.test_gpu_parity import _edge_block4_layer
    br, bc, tiles, ptrs, cols, q, vs = _edge_block4_layer(n_in, n_out, 7, density=0.05)
    H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q).load_tiles(br, bc, tiles).set_scales(vs)
    L = hip.SparseLinearLayer(n_in, n_out, len(cols) + 16 * len(br) + 64)
    L.load_weights(ptrs, cols, q)
    L.load_block4_tiles(br, bc, tiles)
    L.set_value_scales(vs)
    rng = np.random.default_rng(8)
    x = rng.normal(size=(128, n_in)).astype(np.float32)
    g = rng.normal(size=(128, n_out)).astype(np.float32)

    def run():
        y = L.forward_dense(x)
        assert_close_terms(y, H.forward_dense(x), H.forward_dense(x, absmode=True), "b4 colblock fwd")
        dx = L.backward_dense(g, 0.0)
        assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0], "b4 colblock dx")
    counts = kernel_counts(hip, L, run)
    assert counts.get(f"{op}:gather_b4") == 4, counts
