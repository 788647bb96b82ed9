"""CPU: the restatements of the module's CSR utilities (oracle.dense_to_csr,
oracle.dense_to_top_k_csr) pinned by the reference's own tests and, for the
top-k conversion, against the reference's compiled top_k_csr (csr.hpp)."""
import numpy as np
import pytest

from oracle import dense_to_csr, dense_to_top_k_csr, have_ref, ref_top_k_csr


def test_dense_to_csr_reference_kats():
    # tests/unit/python/test_sili.py TestDenseToCsr
    x = np.array([[1.0, 0.0, 2.0], [0.0, 3.0, 0.0]], dtype=np.float32)
    p, i, v = dense_to_csr(x, 0.0)
    assert p.tolist() == [0, 2, 3] and i.tolist() == [0, 2, 1]
    np.testing.assert_array_equal(v, [1.0, 2.0, 3.0])
    p, i, v = dense_to_csr(np.array([[0.001, 1.0]], np.float32), 0.01)
    assert i.tolist() == [1]
    # the keep rule is strict on both sides and never keeps NaN
    p, i, v = dense_to_csr(np.array([0.5, -0.5, 0.50001, np.nan, -np.inf], np.float32), 0.5)
    assert p.tolist() == [0, 2] and i.tolist() == [2, 4]


def test_top_k_reference_kat():
    # tests/unit/test_csr_union.cpp:124-160: a global budget by magnitude
    x = np.array([[-9.0, 1.0, 2.0, -3.0, 0.5], [1.0, -8.0, 7.0, 0.2, -0.1]], np.float32)
    p, i, v = dense_to_top_k_csr(x, 4)
    got = {(r, int(c)) for r in range(2) for c in i[p[r]:p[r + 1]]}
    assert got == {(0, 0), (1, 1), (1, 2), (0, 3)}
    assert p.tolist() == [0, 2, 4] and i.tolist() == [0, 3, 1, 2]
    np.testing.assert_array_equal(v, [-9.0, -3.0, -8.0, 7.0])


@pytest.mark.skipif(not have_ref(), reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("rows,cols,k,threads", [(1, 100, 7, 1), (4, 33, 20, 3), (32, 512, 1000, 4),
                                                 (8, 64, 10_000, 2), (16, 300, 1, 4)])
def test_top_k_matches_reference(rows, cols, k, threads):
    rng = np.random.default_rng(rows * 1000 + k)
    # distinct magnitudes: the cut is fixed whatever the partial sorts' order
    mag = rng.permutation(rows * cols).astype(np.float32) * np.float32(0.25) + np.float32(0.125)
    x = (mag * np.where(rng.random(rows * cols) < 0.5, -1, 1)).astype(np.float32).reshape(rows, cols)
    p, i, v = dense_to_top_k_csr(x, k)
    rp, ri, rv = ref_top_k_csr(x, k, threads)
    assert np.array_equal(p, rp) and np.array_equal(i, ri) and np.array_equal(v, rv)


def test_top_k_zero_budget_is_empty():
    # k = 0 (the reference's top_k_csr is not called with it here: its COO to
    # CSR conversion leaves no index vectors for an empty selection)
    p, i, v = dense_to_top_k_csr(np.ones((3, 5), np.float32), 0)
    assert p.tolist() == [0, 0, 0, 0] and len(i) == 0 and len(v) == 0
