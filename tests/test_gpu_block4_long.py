"""GPU: block4 gathers over long block rows with multi-byte block-column
deltas (a chunk of 64 index bytes then holds fewer than 64 tiles, and a tile's
last byte can sit at a lane past the chunk's tile count), in every kernel
variant the launch knobs select, against the CPU oracle."""
import numpy as np
import pytest

from oracle import HostLayer
from tests.test_gpu_parity import _edge_block4_layer
from tests.util import assert_close_terms

pytestmark = pytest.mark.gpu

VARIANTS = [
    {},                                               # default: 16 lanes per tile, 2 in flight
    {"SILI_B4_BL": "8", "SILI_B4_U": "4"},
    {"SILI_B4_BL": "32", "SILI_B4_U": "4"},
    {"SILI_B4_BL": "64", "SILI_B4_U": "2"},           # one tile per wave step
    {"SILI_B4_BL": "64", "SILI_B4_U": "8"},
    {"SILI_B4_MFMA": "1", "SILI_B4_MFMA_U": "1"},     # v_mfma_f32_4x4x1f32
    {"SILI_B4_MFMA": "1", "SILI_B4_MFMA_U": "4"},
]


@pytest.fixture(scope="module")
def layers(hip):
    out = {}
    for n_in, n_out in ((16383, 301), (301, 16383)):
        br, bc, tiles, ptrs, cols, q, vs = _edge_block4_layer(n_in, n_out, 17, density=0.05)
        H = HostLayer(n_in, n_out).load_csr(ptrs, cols, w=q).load_tiles(br, bc, tiles).set_scales(vs)
        L = hip.SparseLinearLayer(n_in, n_out, len(cols) + 16 * len(br) + 64)
        L.load_weights(ptrs, cols, q)
        L.load_block4_tiles(br, bc, tiles)
        L.set_value_scales(vs)
        out[(n_in, n_out)] = (H, L)
    return out


def test_design_has_multibyte_block_deltas(layers):
    """The 301 x 16383 layer's canonical block rows span 4096 block columns at
    5 % density: some block-column deltas take two ULEB bytes."""
    H, _ = layers[(301, 16383)]
    assert np.any(H.bidx >= 0x80)


@pytest.mark.parametrize("colblock", ["0", "1"])
@pytest.mark.parametrize("variant", range(len(VARIANTS)))
@pytest.mark.parametrize("B", [4, 8, 64, 128])
def test_long_block_rows(hip, layers, monkeypatch, variant, B, colblock):
    monkeypatch.setenv("SILI_COLBLOCK", colblock)
    monkeypatch.setenv("SILI_COLBLOCK_B4_MB", "2")  # batches 64 / 128: 2 / 4 block4 passes
    for k, v in VARIANTS[variant].items():
        monkeypatch.setenv(k, v)
    rng = np.random.default_rng(B * 10 + variant)
    for (n_in, n_out), (H, L) in layers.items():
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        g = rng.normal(size=(B, n_out)).astype(np.float32)
        y = L.forward_dense(x)
        assert_close_terms(y, H.forward_dense(x), H.forward_dense(x, absmode=True), f"fwd {n_in}x{n_out} B{B}")
        dx = L.backward_dense(g, 0.0)
        assert_close_terms(dx, H.backward_dense(x, g)[0], H.backward_dense(x, g, absmode=True)[0],
                           f"dx {n_in}x{n_out} B{B}")
