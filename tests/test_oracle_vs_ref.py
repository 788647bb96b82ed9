"""CPU: the oracle against the reference's own compiled headers (oracle/_ref)
on seeded configuration-shaped layers.  Runs where the reference tree is
present (this container); the committed golden fixtures cover the GPU box."""
import numpy as np
import pytest

from oracle import HostLayer, RefLayer, have_ref
from sili__new_amd.synth import make_config
from util import assert_close_terms

pytestmark = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (no reference tree)")


@pytest.mark.parametrize("idx,scale,batch", [(0, 0.0625, 3), (1, 0.0625, 8), (2, 0.03125, 4)])
def test_structure_and_dense_paths(idx, scale, batch):
    wl = make_config(idx, scale=scale, batch=batch)
    H = HostLayer(wl.n_in, wl.n_out).load_csr(wl.ptrs, wl.cols, w=wl.q).set_scales(wl.value_scale)
    R = RefLayer(wl.n_in, wl.n_out, wl.ptrs, wl.cols, wl.q).set_scales(wl.value_scale)
    R.compact()
    bs, es, idx_b, val = R.export()
    assert np.array_equal(bs, H.row_byte_start) and np.array_equal(es, H.row_elem_start)
    assert np.array_equal(idx_b, H.idx[:H.index_bytes]) and np.array_equal(val, H.val[:H.nnz])
    x = wl.x.astype(np.float32)
    g = wl.g if wl.g is not None else np.random.default_rng(idx).normal(size=(batch, wl.n_out)).astype(np.float32)
    assert_close_terms(H.forward_dense(x), R.forward_dense(x), H.forward_dense(x, absmode=True), "fwd")
    dx, ai, ag = H.backward_dense(x, g)
    rdx, rai, rag = R.backward_dense(x, g)
    adx, aai, aag = H.backward_dense(x, g, absmode=True)
    assert_close_terms(dx, rdx, adx, "dx")
    assert_close_terms(ai, rai, aai, "acc_in")
    assert_close_terms(ag, rag, aag, "acc_grad")


def test_sparse_paths():
    wl = make_config(2, scale=0.03125, batch=4)
    H = HostLayer(wl.n_in, wl.n_out).load_csr(wl.ptrs, wl.cols, w=wl.q).set_scales(wl.value_scale)
    R = RefLayer(wl.n_in, wl.n_out, wl.ptrs, wl.cols, wl.q).set_scales(wl.value_scale)
    R.compact()
    B = wl.batch
    y = H.forward_sparse(wl.x_ptrs, wl.x_idx, wl.x_vals, B)
    assert_close_terms(y, R.forward_sparse(wl.x_ptrs, wl.x_idx, wl.x_vals, B),
                       H.forward_sparse(wl.x_ptrs, wl.x_idx, wl.x_vals, B, absmode=True), "sparse fwd")
    rng = np.random.default_rng(7)
    dp = np.concatenate([[0], np.cumsum(np.full(B, 9))]).astype(np.int32)
    di = np.concatenate([np.sort(rng.choice(wl.n_out, 9, replace=False)) for _ in range(B)]).astype(np.int32)
    dv = rng.normal(size=len(di)).astype(np.float32)
    x = wl.x.astype(np.float32)
    got = H.backward_sparse(x, dp, di, dv, B)
    want = R.backward_sparse(x, dp, di, dv, B)
    bound = H.backward_sparse(x, dp, di, dv, B, absmode=True)
    for a, b, c, what in zip(got, want, bound, ("dx", "acc_in", "acc_grad")):
        assert_close_terms(a, b, c, what)


def test_block4_store_and_forward():
    wl = make_config(3, scale=0.03125, batch=5)
    H = HostLayer(wl.n_in, wl.n_out).load_tiles(wl.tile_br, wl.tile_bc, wl.tile_bytes).set_scales(wl.value_scale)
    R = RefLayer(wl.n_in, wl.n_out, np.zeros(wl.n_in + 1, np.int32), np.zeros(0, np.int32),
                 np.zeros(0, np.float32)).set_scales(wl.value_scale)
    tb = wl.tile_bytes.reshape(-1, 16)
    for k in range(len(wl.tile_br)):
        R.put_tile(wl.tile_br[k], wl.tile_bc[k], tb[k])
    R.compact()
    br, bc, t = R.export_tiles()
    assert np.array_equal(br, H.tile_br) and np.array_equal(bc, H.tile_bc)
    assert np.array_equal(t, H.tiles[:16 * H.n_tiles])
    x = wl.x.astype(np.float32)
    assert_close_terms(H.forward_dense(x), R.forward_dense(x), H.forward_dense(x, absmode=True), "b4 fwd")
    dx, ai, ag = H.backward_dense(x, wl.g)
    rdx, rai, rag = R.backward_dense(x, wl.g)
    assert_close_terms(dx, rdx, H.backward_dense(x, wl.g, absmode=True)[0], "b4 dx")
