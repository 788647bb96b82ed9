"""Seeded layers for the tests of backward with the optimizer update."""
import numpy as np

from oracle import HostLayer


def make_train_case(n_in, n_out, density, seed, rank=1, empty_rows=0, os_trainable=False, imp_scales=False):
    """Random scattered layer with weights across the FP4 range, importances,
    value scales (and, when asked, trainable output scales and importance
    scales); rows [0, empty_rows) hold no synapse."""
    rng = np.random.default_rng(seed)
    # rank > 1 sets output-scale components, which marks the output scales
    # trainable (set_output_scale_raw_k, delta_csr_types.hpp:1217-1222)
    os_trainable = bool(os_trainable or rank > 1)
    ptrs, cols = [0], []
    for r in range(n_in):
        if r >= empty_rows:
            k = max(1, int(rng.binomial(n_out, density)))
            cols.extend(np.sort(rng.choice(n_out, size=min(k, n_out), replace=False)).tolist())
        ptrs.append(len(cols))
    c = dict(n_in=n_in, n_out=n_out, rank=rank, os_trainable=os_trainable,
             ptrs=np.array(ptrs, np.int32), cols=np.array(cols, np.int32))
    nnz = len(cols)
    c["w"] = rng.normal(0.0, 1.5, size=nnz).astype(np.float32)
    c["imp"] = np.abs(rng.normal(0.0, 1.0, size=nnz)).astype(np.float32)
    vs = np.zeros(n_in * rank, np.float32)
    vs[::rank] = rng.uniform(0.5, 1.5, n_in)
    for k in range(1, rank):
        vs[k::rank] = rng.uniform(0.0, 0.3, n_in)
    os_ = np.zeros(n_out * rank, np.float32)
    os_[::rank] = rng.uniform(0.5, 1.5, n_out) if (os_trainable or rank > 1) else 1.0
    for k in range(1, rank):
        os_[k::rank] = rng.uniform(0.0, 0.3, n_out)
    c["vs"], c["os"] = vs, os_
    c["is"] = rng.uniform(0.5, 2.0, n_in).astype(np.float32) if imp_scales else None
    c["ois"] = rng.uniform(0.5, 2.0, n_out).astype(np.float32) if imp_scales else None
    c["rng"] = rng
    return c


def host_layer(c):
    H = HostLayer(c["n_in"], c["n_out"], c["rank"]).load_csr(c["ptrs"], c["cols"], w=c["w"], imp=c["imp"])
    H.set_scales(c["vs"], c["os"])
    H.output_scale_trainable = bool(c["os_trainable"])
    H.importance_scale = c["is"]
    H.output_importance_scale = c["ois"]
    return H


def ref_layer(c):
    from oracle import RefLayer
    R = RefLayer(c["n_in"], c["n_out"], c["ptrs"], c["cols"], c["w"], c["imp"])
    R.set_scales(c["vs"], c["os"] if (c["os_trainable"] or c["rank"] > 1) else None, c["rank"])
    # set_output_scale_raw marks the output scales trainable; keep the case's choice
    R.set_train_state(os_trainable=int(c["os_trainable"]))
    if c["is"] is not None:
        R.set_importance_scales(c["is"], c["ois"])
    return R


# (n_in, n_out, density, seed, batch, lr, options)
TRAIN_CASES = [
    (64, 48, 0.2, 1, 1, 0.05, {}),
    (64, 48, 0.2, 2, 4, 0.05, {}),
    (200, 300, 0.05, 3, 1, 0.1, {}),
    (100, 80, 0.1, 4, 2, 0.05, dict(lr_per_row_nnz=True)),
    (100, 80, 0.1, 5, 1, 0.05, dict(damp_by_importance=False)),
    (100, 80, 0.1, 6, 3, 0.05, dict(os_trainable=True)),
    (60, 50, 0.1, 7, 2, 0.05, dict(empty_rows=10)),
    (80, 64, 0.15, 8, 1, 0.05, dict(rank=2, os_trainable=True)),
    (90, 70, 0.1, 9, 2, 0.2, dict(imp_scales=True)),
    (40, 600, 0.3, 10, 1, 0.05, {}),  # rows longer than one 64-byte decode chunk
    # batches the GPU kernels take 8 steps at a time (a partial last group at 12 and 36)
    (100, 80, 0.1, 13, 12, 0.05, {}),
    (64, 200, 0.2, 14, 64, 0.02, dict(os_trainable=True)),
    (50, 60, 0.2, 15, 36, 0.05, dict(rank=2, imp_scales=True)),
]
LAYER_OPTS = ("rank", "empty_rows", "os_trainable", "imp_scales")


def split_opts(opts):
    layer = {k: v for k, v in opts.items() if k in LAYER_OPTS}
    call = {k: v for k, v in opts.items() if k not in LAYER_OPTS and k not in TILE_OPTS}
    return layer, call


def tile_opts(opts):
    return {k: v for k, v in opts.items() if k in TILE_OPTS}


def dx_bound_tiles(H, dy, lr, max_abs_delta=2.0, sparse=False):
    """dx_bound (dense update) or dx_bound_sparse (sparse update) over the
    block4 tile slots of H: sum over each tile row's slots of |w| * |dy|,
    |w| bounded over the call as for scattered synapses."""
    from sili__new_amd.codec import fp4_decode_np
    dy = np.atleast_2d(dy)
    B = dy.shape[0]
    T = np.zeros((H.n_in, B))
    if H.n_tiles == 0:
        return T.T
    tiles = H.tiles[:16 * H.n_tiles].reshape(-1, 16)
    s = np.arange(16)
    rows = (np.asarray(H.tile_br, np.int64)[:, None] * 4 + s % 4).ravel()
    cols = (np.asarray(H.tile_bc, np.int64)[:, None] * 4 + s // 4).ravel()
    ok = (rows < H.n_in) & (cols < H.n_out)
    rows, cols = rows[ok], cols[ok]
    q0 = fp4_decode_np(tiles.ravel()[ok] & 0xF).astype(np.float64)
    q0[~np.isfinite(q0)] = 6.0
    vs = H.value_scale.reshape(H.n_in, H.rank).astype(np.float64)
    os_ = H.output_scale.reshape(H.n_out, H.rank).astype(np.float64)
    S = np.abs(vs[rows] * os_[cols]).sum(1)
    mag = 6.0 * S if sparse else (np.abs(q0) + B * abs(lr) * max_abs_delta) * S
    np.add.at(T, rows, (np.abs(dy[:, cols].astype(np.float64)) * mag).T)
    return T.T


def dx_bound(H, dy, lr, max_abs_delta=2.0):
    """sum over a row's synapses of |w| * |dy| with |w| bounded over the whole
    call: each batch step moves a weight code by at most lr * max_abs_delta,
    so |quant| <= |code before| + B * lr * max_abs_delta.  Taken before the
    update (the scales are those the call's dx uses)."""
    from sili__new_amd.codec import fp4_decode_np
    dy = np.atleast_2d(dy)
    B = dy.shape[0]
    cols = H.decode_cols()
    rows = np.repeat(np.arange(H.n_in), np.diff(H.row_elem_start.astype(np.int64)))
    q0 = fp4_decode_np(H.val[:len(cols)] >> 4).astype(np.float64)
    vs = H.value_scale.reshape(H.n_in, H.rank).astype(np.float64)
    os_ = H.output_scale.reshape(H.n_out, H.rank).astype(np.float64)
    S = np.abs(vs[rows] * os_[cols]).sum(1)
    mag = (np.abs(q0) + B * abs(lr) * max_abs_delta) * S
    T = np.zeros((H.n_in, B))
    np.add.at(T, rows, (np.abs(dy[:, cols].astype(np.float64)) * mag).T)
    return T.T


def sparse_dy(rng, B, n_out, density=0.3):
    """A sparse dy CSR (strictly increasing indices per batch row), with some
    explicit zeros and an empty batch row when B > 2; also its dense form."""
    ptrs, idx, vals = [0], [], []
    for b in range(B):
        if B > 2 and b == 1:
            ptrs.append(len(idx))
            continue
        cols = np.flatnonzero(rng.random(n_out) < density)
        v = rng.normal(size=len(cols)).astype(np.float32)
        v[rng.random(len(cols)) < 0.05] = 0.0
        idx.extend(cols.tolist())
        vals.extend(v.tolist())
        ptrs.append(len(idx))
    ptrs, idx, vals = np.array(ptrs, np.int32), np.array(idx, np.int32), np.array(vals, np.float32)
    dense = np.zeros((B, n_out), np.float32)
    for b in range(B):
        dense[b, idx[ptrs[b]:ptrs[b + 1]]] = vals[ptrs[b]:ptrs[b + 1]]
    return ptrs, idx, vals, dense


def dx_bound_sparse(H, dy_dense, lr, max_step=None):
    """sum over a row's synapses of |w| * |dy|, |w| bounded over the call.
    Each step moves a weight by |-lr * g| / (sqrt(imp) + eps) and re-quantizes,
    so the bound takes the largest code (6) for every synapse: coarse but safe."""
    from sili__new_amd.codec import fp4_decode_np  # noqa: F401
    dy = np.atleast_2d(dy_dense)
    B = dy.shape[0]
    cols = H.decode_cols()
    rows = np.repeat(np.arange(H.n_in), np.diff(H.row_elem_start.astype(np.int64)))
    vs = H.value_scale.reshape(H.n_in, H.rank)[:, 0].astype(np.float64)
    os_ = H.output_scale.reshape(H.n_out, H.rank)[:, 0].astype(np.float64)
    mag = 6.0 * np.abs(vs[rows] * os_[cols])
    T = np.zeros((H.n_in, B))
    np.add.at(T, rows, (np.abs(dy[:, cols].astype(np.float64)) * mag).T)
    return T.T


def add_tiles(c, tile_density=0.3, seed=0, tile_gap=None):
    """Block4 tiles over the windows of c that hold no scattered synapse (all
    16 slots coded, some empty), edge windows included.  tile_gap = (a, b):
    every other block row holds no tile in block columns [a, b), so its next
    tile's block-column delta takes a multi-byte ULEB128."""
    rng = np.random.default_rng(1000 + seed)
    n_in, n_out = c["n_in"], c["n_out"]
    brs, bcs = (n_in + 3) // 4, (n_out + 3) // 4
    used = np.zeros((brs, bcs), bool)
    for r in range(n_in):
        for col in c["cols"][c["ptrs"][r]:c["ptrs"][r + 1]]:
            used[r // 4, col // 4] = True
    if tile_gap is not None:
        used[::2, tile_gap[0]:tile_gap[1]] = True
    keys = [k for k in np.flatnonzero(rng.random(brs * bcs) < tile_density) if not used.flat[k]]
    if n_out % 4:  # at least one edge tile (columns past n_out in the window)
        free = [b * bcs + bcs - 1 for b in range(brs) if not used[b, bcs - 1]]
        if free and free[0] not in keys:
            keys = sorted(keys + [free[0]])
    br = np.array([k // bcs for k in keys], np.int32)
    bc = np.array([k % bcs for k in keys], np.int32)
    codes_w = rng.integers(0, 16, (len(keys), 16))
    codes_w[codes_w == 8] = 3
    codes_i = rng.integers(0, 8, (len(keys), 16))
    tiles = ((codes_i << 4) | codes_w).astype(np.uint8)
    tiles[rng.random(tiles.shape) < 0.25] = 0
    for t, (a, b) in enumerate(zip(br, bc)):  # slots outside the layer stay 0
        for s in range(16):
            lj, li = divmod(s, 4)
            if a * 4 + li >= n_in or b * 4 + lj >= n_out:
                tiles[t, s] = 0
    c["br"], c["bc"], c["tiles"] = br, bc, tiles.ravel()
    return c


# block4 update cases: (n_in, n_out, density, seed, batch, lr, options, variant);
# odd widths give edge tiles.  The wide cases hold > 64 tiles per block row
# (block rows over several 64-byte decode windows), block-column gaps of 140
# (two-byte deltas) and batches past the kernels' 64-step LDS row passes.
B4_CASES = [
    (40, 37, 0.05, 21, 1, 0.3, {}, "plain"),
    (44, 50, 0.05, 22, 3, 0.3, {}, "plain"),
    (36, 30, 0.05, 23, 8, 0.2, dict(rank=2), "plain"),
    (40, 37, 0.05, 24, 2, 0.3, {}, "resync"),
    (40, 37, 0.05, 25, 2, 0.3, {}, "noscale"),
    (64, 61, 0.05, 26, 12, 0.1, dict(imp_scales=True, lr_per_row_nnz=True), "plain"),
    (33, 45, 0.05, 27, 1, 0.5, dict(damp_by_importance=False), "plain"),
    (24, 1030, 0.01, 28, 256, 0.004, dict(tile_density=0.5, tile_gap=(60, 200)), "plain"),
    (24, 1030, 0.01, 29, 1024, 0.001, dict(tile_density=0.5, tile_gap=(60, 200)), "plain"),
    (20, 1027, 0.01, 30, 100, 0.01, dict(tile_density=0.5, tile_gap=(61, 201)), "resync"),
]
TILE_OPTS = ("tile_density", "tile_gap")


def b4_reserve_like_device(L, H, max_weights):
    """Give the oracle layer H the block4 reservations and tile encoding that
    L's load_block4_tiles left (tiles placed one by one in canonical order,
    oracle.block4_put_layer), checking the device holds the same; the
    updates' write-back then evicts on both alike."""
    from oracle import block4_put_layer
    T, flags = block4_put_layer(H.n_in, max_weights, H.tile_br, H.tile_bc, H.tiles[:16 * H.n_tiles])
    H.b4res = T.M
    H.b4_flags = flags.copy() if len(flags) else np.zeros(1, np.uint8)
    check_b4_reservations(L, H, "load")


def check_b4_reservations(L, H, what):
    """The device's block4 reservations, tile_is_sparse and write-back
    counters against the oracle's."""
    d = L.export_block4_layout()
    M = H.b4res
    assert list(d["ia"]) == M.ia and list(d["ea"]) == M.ea and list(d["ta"]) == M.ta, what + ": reservations"
    assert d["dropped_growth_events"] == M.dropped, what + ": dropped growth events"
    assert (d["evicted"], d["row_merge_overflow_events"], d["row_merge_overflow_bytes_dropped"]) == \
        tuple(H.b4_counters), what + ": write-back counters"
    if H.n_tiles:
        assert np.array_equal(L.export_block4_packed()["tile_is_sparse"], H.b4_flags[:H.n_tiles]), \
            what + ": tile_is_sparse"
