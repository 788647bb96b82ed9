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
    {},                                               # default: 16 lanes per tile, 2 in flight (32 at B >= 128,
                                                      # batch chunks on their own XCDs)
    {"SILI_B4_WIDE": "0"},                            # 16 lanes per tile at every batch
    {"SILI_B4_XCDQ": "0"},                            # batch chunks in launch order
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


@pytest.mark.parametrize("B", [4, 64, 128, 256])
def test_sampled_gradw_by_column_range(hip, layers, monkeypatch, B):
    """The block4 sampled grad-W over runs of tiles by column range (range x
    on XCD x) gives what the store's own work items give, bit for bit, for
    any number of ranges (0: the work items; the default takes 8 when gT
    exceeds 4 MiB, as it does here from batch 64 on), and matches the
    oracle."""
    rng = np.random.default_rng(B)
    for (n_in, n_out), (H, L) in layers.items():
        x = rng.normal(size=(B, n_in)).astype(np.float32)
        g = rng.normal(size=(B, n_out)).astype(np.float32)
        got = {}
        for K in ["0", "1", "3", "8", "16", None]:
            if K is None:
                monkeypatch.delenv("SILI_SDDMM_RANGES", raising=False)
            else:
                monkeypatch.setenv("SILI_SDDMM_RANGES", K)
            got[K] = L.sampled_gradw(x, g)[1]
        for K, gb in got.items():
            assert np.array_equal(gb.view(np.uint32), got["0"].view(np.uint32)), f"{n_in}x{n_out} B{B} ranges {K}"
        gb_o = H.sampled_gradw(x, g)[1]
        assert_close_terms(got[None], gb_o, H.sampled_gradw(x, g, absmode=True)[1], f"gw {n_in}x{n_out} B{B}")


def test_sampled_gradw_ranges_follow_structure(hip, monkeypatch):
    """The tiles' column ranges are rebuilt after the structure changes: a
    bulk synaptogenesis step and a new set of tiles, each followed by the
    grad-W by ranges and by the store's work items (equal bit for bit)."""
    n_in, n_out = 301, 16383
    br, bc, tiles, ptrs, cols, q, vs = _edge_block4_layer(n_in, n_out, 23, density=0.05)
    L = hip.SparseLinearLayer(n_in, n_out, 4 * (len(cols) + 16 * len(br)) + 4096)
    L.load_weights(ptrs, cols, q)
    L.load_block4_tiles(br, bc, tiles)
    rng = np.random.default_rng(5)
    B = 64
    x = rng.normal(size=(B, n_in)).astype(np.float32)
    g = rng.normal(size=(B, n_out)).astype(np.float32)

    def both(what):
        monkeypatch.setenv("SILI_SDDMM_RANGES", "8")
        a = L.sampled_gradw(x, g)[1]
        monkeypatch.setenv("SILI_SDDMM_RANGES", "0")
        b = L.sampled_gradw(x, g)[1]
        assert a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32)), what
        return a

    n0 = both("loaded").shape[0]
    e = np.zeros(0, np.int32)
    L.synapto_step(0.3, e, e, np.zeros(0, np.float32))  # prunes slots, demotes tiles
    both("after a synaptogenesis step")
    br2, bc2, tiles2, *_ = _edge_block4_layer(n_in, n_out, 29, density=0.03)
    L.load_block4_tiles(br2, bc2, tiles2)
    assert both("after new tiles").shape[0] != n0
