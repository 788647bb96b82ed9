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
def test_forward_column_blocks(hip, B, passes):
    # shadow columns = n_in = 16384: operand 64 KiB per batch column
    H, L = synthetic(hip, 16384, 300, 0.4, 99)
    x = np.random.default_rng(B).normal(size=(B, 16384)).astype(np.float32)
    counts = kernel_counts(hip, L, lambda: assert_close_terms(
        L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), f"colblock fwd B{B}"))
    assert counts.get("fwd:gather") == passes, counts


def test_forward_column_blocks_off(hip, monkeypatch):
    monkeypatch.setenv("SILI_COLBLOCK", "0")
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
