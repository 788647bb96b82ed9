"""GPU: the FOR index (the reference prototype's group frame-of-reference
format, prototypes/for_delta_encoding) built on the device from the
canonical store: exported bytes equal the oracle's restatement (pinned to
the prototype's own encoder in tests/test_for_oracle.py) for every group
size, and every column decodes from it exactly as from the ULEB128 stream;
a structural rebuild drops it."""
import numpy as np
import pytest

import oracle
from sili__new_amd.synth import make_config
from tests.util import gpu_layer

pytestmark = pytest.mark.gpu


def _layer(hip, n_in, n_out, rows):
    ptrs = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    cols = np.concatenate([np.asarray(r, np.int32) for r in rows]) if sum(map(len, rows)) else np.zeros(0, np.int32)
    w = np.linspace(-5, 5, max(1, len(cols))).astype(np.float32)[:len(cols)]
    L = hip.SparseLinearLayer(n_in, n_out, max(1, len(cols)))
    L.load_weights(ptrs, cols, w)
    return L, ptrs, cols


def _check(L, ptrs, cols, G, what):
    L.build_for_index(G)
    ex = L.export_for_index()
    rs, b = oracle.for_encode_rows(ptrs, cols, G)
    assert np.array_equal(ex["row_byte_start"], rs), what + ": row starts"
    assert np.array_equal(ex["bytes"], b), what + ": bytes"
    assert np.array_equal(L.decode_columns(1), cols), what + ": FOR decode (lane per slot)"
    assert np.array_equal(L.decode_columns(2), cols), what + ": FOR decode (thread per group)"
    assert np.array_equal(L.decode_columns(0), cols), what + ": ULEB decode"


@pytest.mark.parametrize("G", [8, 16, 32, 64])
def test_for_index_designed_rows(hip, G):
    rng = np.random.default_rng(G)
    rows = [[], [0], [5], list(range(64)), list(np.cumsum(rng.integers(1, 300, 50))),
            [3, 70000, 70001, 4_999_999], [], list(np.sort(rng.choice(5_000_000, 1000, replace=False)))]
    for n in (15, 16, 17, 33):
        rows.append(list(np.sort(rng.choice(4096, n, replace=False))))
    L, ptrs, cols = _layer(hip, len(rows), 5_000_000, rows)
    _check(L, ptrs, cols, G, f"designed G{G}")


@pytest.mark.parametrize("cfg,scale", [(1, 0.25), (2, 0.25), (0, 1.0)])
def test_for_index_config_layers(hip, cfg, scale):
    wl = make_config(cfg, scale=scale)
    L = gpu_layer(hip, wl)
    for G in (16, 64):
        _check(L, wl.ptrs, wl.cols, G, f"c{cfg} G{G}")


def test_for_index_dropped_on_rebuild(hip):
    wl = make_config(1, scale=0.125)
    L = gpu_layer(hip, wl)
    L.build_for_index(16)
    assert np.array_equal(L.decode_columns(True), wl.cols)
    rng = np.random.default_rng(1)
    cr = rng.integers(0, wl.n_in, 200).astype(np.int32)
    cc = rng.integers(0, wl.n_out, 200).astype(np.int32)
    cv = rng.normal(0, 0.01, 200).astype(np.float32)
    L.synapto_step(0.01, cr, cc, cv)
    with pytest.raises(ValueError):
        L.decode_columns(True)
    L.build_for_index(16)
    ex = L.export_scattered()
    H = oracle.HostLayer(wl.n_in, wl.n_out).load_encoded(ex["row_byte_start"], ex["row_elem_start"], ex["idx"],
                                                         ex["val"])
    assert np.array_equal(L.decode_columns(True), H.decode_cols())
