"""CPU: the restatement of the group frame-of-reference (FOR) index encoding
(oracle.for_encode_row) against the reference prototype's own encoder
(prototypes/for_delta_encoding/for_encoding_bench.cpp, compiled in place) and
against its decode rule (every column = group start + its offset)."""
import numpy as np
import pytest

from oracle import for_encode_row, have_ref, ref_for_encode


def _decode(b, n, G):
    """The prototype's decode (for_encoding_bench.cpp:72-96), restated."""
    out, pos, carry = [], 0, 0
    for _ in range((n + G - 1) // G):
        w = (1, 2, 4)[b[pos]]
        pos += 1
        offs = [int.from_bytes(b[pos + w * k:pos + w * (k + 1)], "little") for k in range(G)]
        pos += G * w
        out.extend(carry + o for o in offs)
        carry = out[-1]
    assert pos == len(b)
    return out[:n]


def _rows(rng):
    yield np.array([], np.int64)
    yield np.array([0], np.int64)
    yield np.array([5], np.int64)
    yield np.arange(0, 64)                     # tier 0 everywhere, exact groups
    yield np.cumsum(rng.integers(1, 300, 50))  # tier 1 groups
    yield np.array([3, 70000, 70001, 5000000])  # tier 2
    for n in (1, 15, 16, 17, 33, 100, 1000):
        yield np.sort(rng.choice(1 << 20, size=n, replace=False))


@pytest.mark.parametrize("G", [8, 16, 32, 64])
def test_for_encoding_round_trip_and_tiers(G):
    rng = np.random.default_rng(G)
    for cols in _rows(rng):
        b = for_encode_row(cols, G)
        # _decode walks every group and checks it ends exactly at the last byte
        assert _decode(b, len(cols), G) == [int(c) for c in cols]
    # tier boundaries: largest offset 255 -> 1 byte, 256 -> 2, 65536 -> 4
    assert for_encode_row([255], G)[0] == 0 and for_encode_row([256], G)[0] == 1
    assert for_encode_row([65535], G)[0] == 1 and for_encode_row([65536], G)[0] == 2


@pytest.mark.skipif(not have_ref(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("G", [8, 16, 32, 64])
def test_for_encoding_matches_reference_prototype(G):
    rng = np.random.default_rng(100 + G)
    for cols in _rows(rng):
        if len(cols) == 0:
            continue
        assert for_encode_row(cols, G) == ref_for_encode(cols, G), (G, len(cols))
