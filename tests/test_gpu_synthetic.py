"""GPU: the device generator of seeded synthetic layers (config 4 workloads)
and the forward pass over them, checked against the CPU oracle on the
exported store -- at a small size and at the full size of a config-4 layer."""
import numpy as np
import pytest

from oracle import HostLayer
from tests.util import assert_close_terms

pytestmark = pytest.mark.gpu

M64 = (1 << 64) - 1


def fmix64(k):
    k = k.astype(np.uint64)
    k ^= k >> np.uint64(33)
    k *= np.uint64(0xff51afd7ed558ccd)
    k ^= k >> np.uint64(33)
    k *= np.uint64(0xc4ceb9fe1a85ec53)
    k ^= k >> np.uint64(33)
    return k


def kept_mask(seed, n_in, n_out, keep_prob):
    """The generator's keep rule restated: high word of
    fmix64(seed ^ r*K1 ^ c*K2) below keep_prob * 2^32."""
    with np.errstate(over="ignore"):
        r = np.arange(n_in, dtype=np.uint64)[:, None] * np.uint64(0x9E3779B97F4A7C15)
        c = np.arange(n_out, dtype=np.uint64)[None, :] * np.uint64(0xD1B54A32D192ED03)
        h = fmix64(np.uint64(seed) ^ r ^ c)
    thr = np.uint64(min(4294967295, int(keep_prob * 4294967296.0)))
    return (h >> np.uint64(32)) < thr


def exported(L, n_in, n_out):
    ex = L.export_scattered()
    H = HostLayer(n_in, n_out).load_encoded(ex["row_byte_start"], ex["row_elem_start"], ex["idx"], ex["val"])
    H.set_scales(np.asarray(L.get_value_scales(), np.float32))
    return H


@pytest.mark.parametrize("n_in,n_out,keep,tail", [(96, 333, 0.13, 0.95), (40, 2000, 0.1, 0.5)])
def test_structure_follows_the_hash_and_row_recipe(hip, n_in, n_out, keep, tail):
    seed = 12345
    L = hip.SparseLinearLayer(n_in, n_out, 1)
    nnz = L.load_synthetic(seed, keep, 0.02, tail)
    H = exported(L, n_in, n_out)
    assert np.all(np.isfinite(H.value_scale)) and not L.info()["has_nonfinite"]
    mask = kept_mask(seed, n_in, n_out, keep)
    assert nnz == int(mask.sum()) == H.nnz
    p = H.row_elem_start.astype(np.int64)
    assert np.array_equal(np.diff(p), mask.sum(1))
    assert np.array_equal(H.decode_cols(), np.nonzero(mask)[1])
    # per-row recipe: the row maximum quantizes to +-6 (code 7 / 15)
    codes = H.val[:H.nnz] >> 4
    for r in range(n_in):
        seg = codes[p[r]:p[r + 1]]
        if len(seg):
            assert (seg & 7).max() == 7
    assert not np.any(codes == 8)


@pytest.mark.parametrize("batch", [1, 8, 128])
def test_forward_on_synthetic_layer(hip, batch):
    n_in, n_out = 512, 4096
    L = hip.SparseLinearLayer(n_in, n_out, 1)
    L.load_synthetic(777, 0.1, 0.02, 0.95)
    H = exported(L, n_in, n_out)
    x = np.random.default_rng(batch).normal(size=(batch, n_in)).astype(np.float32)
    assert_close_terms(L.forward_dense(x), H.forward_dense(x), H.forward_dense(x, absmode=True), "synthetic fwd")


@pytest.mark.parametrize("batch", [1, 8])
def test_config4_q_layer_full_size(hip, batch):
    """One config-4 layer at its full size (5120 x 204800, ~105 M synapses)."""
    n_in, n_out = 5120, 204800
    L = hip.SparseLinearLayer(n_in, n_out, 1)
    nnz = L.load_synthetic(20261205, 0.1, 0.02, 0.95)
    assert abs(nnz / (n_in * n_out) - 0.1) < 0.001
    H = exported(L, n_in, n_out)
    # every weight finite (an infinite row scale would make rows NaN on both sides)
    assert np.all(np.isfinite(H.value_scale)) and not L.info()["has_nonfinite"]
    x = np.random.default_rng(3).normal(size=(batch, n_in)).astype(np.float32)
    y = L.forward_dense(x)
    assert np.all(np.isfinite(y))
    assert_close_terms(y, H.forward_dense(x, threads=16), H.forward_dense(x, absmode=True, threads=16), "c4 q fwd")
