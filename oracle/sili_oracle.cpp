// sili_oracle.cpp -- CPU restatement of the reference's FP4 delta-CSR sparse
// layer (TEST INFRASTRUCTURE ONLY: see sili_oracle.h).
//
// Written from the reference's documented semantics; each function names the
// reference file:line it follows.  Parallel loops mirror the reference's
// OpenMP structure (static row split, per-thread private outputs, serial
// reduce -- linear_disldo.hpp:91-125) so the timed CPU baseline runs the same
// algorithm the reference does.
#include "sili_oracle.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <map>
#include <numeric>
#include <unordered_set>
#include <vector>
#include <omp.h>

namespace {

constexpr int TILE = 4;          // block4.hpp:15-27 (SILI_BLOCK4_TILE_SIZE)
constexpr int TILE_SLOTS = 16;
constexpr int PROMOTE_MIN_LIVE = 2;  // block4.hpp:19-21

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// fp4quant.hpp:68-84 -- E2M1, bias 1, code 8 repurposed as NaN 0x7FC00000.
inline float fp4_dec(uint32_t code) {
    const uint32_t s = (code >> 3) & 1u, e = (code >> 1) & 3u, m = code & 1u;
    uint32_t bits;
    if (e == 0) bits = m ? (0x3F000000u | (s << 31)) : (s ? 0x7FC00000u : 0u);
    else        bits = (s << 31) | ((e + 126u) << 23) | (m << 22);
    return u2f(bits);
}

// fp4quant.hpp:86-121 -- nearest, ties away from zero via the carry trick,
// saturate at 6, NaN -> 0, |v| < 0.25 -> 0 (never the NaN slot).
inline uint8_t fp4_enc(float v) {
    const uint32_t bits = f2u(v);
    const uint32_t sign = bits & 0x80000000u, a = bits & 0x7FFFFFFFu;
    uint32_t mag;
    if (a > 0x7F800000u) return 0;
    if (a < 0x3E800000u) mag = 0;
    else if (a < 0x3F400000u) mag = 1;
    else if (a < 0x3F800000u) mag = 2;
    else {
        uint32_t r = a + (1u << 21);
        if (r > 0x40C00000u) r = 0x40C00000u;
        mag = (((r >> 23) & 0xFFu) - 126u) << 1 | ((r >> 22) & 1u);
    }
    if (mag == 0) return 0;
    return uint8_t((sign ? 8u : 0u) | mag);
}

// delta_csr_types.hpp:217-241
inline size_t uleb_enc(uint32_t v, uint8_t *out) {
    size_t n = 0;
    do {
        uint8_t b = uint8_t(v & 0x7Fu);
        v >>= 7;
        if (v) b |= 0x80u;
        out[n++] = b;
    } while (v);
    return n;
}
inline size_t uleb_len(uint32_t v) {
    size_t n = 1;
    while (v >= 0x80u) { v >>= 7; ++n; }
    return n;
}
inline uint32_t uleb_dec(const uint8_t *buf, uint64_t &pos) {
    uint32_t r = 0;
    int sh = 0;
    uint8_t b;
    do {
        b = buf[pos++];
        r |= uint32_t(b & 0x7Fu) << sh;
        sh += 7;
    } while (b & 0x80u);
    return r;
}

// delta_csr_types.hpp:1206-1240 -- S(r,c) = sum_k vs[r,k]*os[c,k], accumulated
// from 0.  Components k >= 1 use the contracted (fma) form a -ffast-math
// -march=native build of the reference produces; rank 1 is exact either way.
inline float scale_rc(const OracleLayer *L, int64_t r, int64_t c) {
    const int rk = L->rank;
    float s = L->value_scale[r * rk] * L->output_scale[c * rk];
    for (int k = 1; k < rk; ++k)
        s = std::fma(L->value_scale[r * rk + k], L->output_scale[c * rk + k], s);
    return s;
}
// Component-0-only scale (sisldo_ops.hpp:302-305, 527-531).
inline float vs0(const OracleLayer *L, int64_t r) { return L->value_scale[r * L->rank]; }
inline float os0(const OracleLayer *L, int64_t c) { return L->output_scale[c * L->rank]; }

inline float maybe_abs(float v, int absmode) { return absmode ? std::fabs(v) : v; }

struct TileRef { int64_t br, bc, t; };

// Walk the block4 store row by row (block4.hpp:1103-1131, linear_disldo.hpp:164-197).
std::vector<TileRef> collect_tiles(const OracleLayer *L) {
    std::vector<TileRef> v;
    if (L->n_tiles <= 0) return v;
    v.reserve(size_t(L->n_tiles));
    const int64_t brows = (L->n_in + TILE - 1) / TILE;
    for (int64_t br = 0; br < brows; ++br) {
        uint64_t pos = L->brow_byte_start[br];
        uint32_t bc = 0;
        for (uint64_t t = L->brow_tile_start[br]; t < L->brow_tile_start[br + 1]; ++t) {
            bc += uleb_dec(L->bidx, pos);
            v.push_back({br, int64_t(bc), int64_t(t)});
        }
    }
    return v;
}

// Stored length of a tile (block4_stored_tile_len, block4.hpp:340-345).
uint64_t b4_tile_len(const uint8_t *td, bool sparse) {
    uint64_t live = 0;
    for (int s = 0; s < 16; ++s) live += td[s] != 0;
    return sparse ? 1 + (live + 1) / 2 + live : 16;
}
uint8_t b4_encode_flag(const uint8_t *td, uint32_t sp) {
    uint32_t live = 0;
    for (int s = 0; s < 16; ++s) live += td[s] != 0;
    return live <= sp ? 1 : 0;
}

// Block4Store::merge_row_workspace (block4.hpp:1367-1462) for the block row
// holding tiles tl[k0, k1): eviction by lowest |true importance| until the
// row's stored bytes fit its reservation, then the whole-tile clamp's
// counters.
void b4_merge_row(const OracleLayer *L, uint8_t *tiles, const std::vector<TileRef> &tl, int64_t k0, int64_t k1,
                  const OracleTrainState *S, OracleB4Merge *M) {
    if (k0 >= k1) return;
    const int64_t br = tl[size_t(k0)].br;
    const uint64_t alloc = M->tile_alloc[br];
    auto len_of = [&](int64_t k) {
        const int64_t t = tl[size_t(k)].t;
        return b4_tile_len(tiles + 16 * t, M->tile_sparse[t] != 0);
    };
    uint64_t used = 0;
    for (int64_t k = k0; k < k1; ++k) used += len_of(k);
    while (used > alloc) {
        double best = -1.0;
        int64_t bk = -1;
        int bslot = 0;
        for (int64_t k = k0; k < k1; ++k) {
            const uint8_t *td = tiles + 16 * tl[size_t(k)].t;
            for (int li = 0; li < TILE; ++li)
                for (int lj = 0; lj < TILE; ++lj) {
                    const uint8_t byte = td[lj * TILE + li];
                    if (byte == 0) continue;
                    const int64_t row = br * TILE + li, col = tl[size_t(k)].bc * TILE + lj;
                    const float is = (S->importance_scale && row < L->n_in) ? S->importance_scale[row] : 1.0f;
                    const float ois =
                        (S->output_importance_scale && col < L->n_out) ? S->output_importance_scale[col] : 1.0f;
                    const double a = std::fabs(static_cast<double>(fp4_dec(byte >> 4)) * static_cast<double>(is) *
                                               static_cast<double>(ois));
                    if (best < 0.0 || a < best) {
                        best = a;
                        bk = k;
                        bslot = lj * TILE + li;
                    }
                }
        }
        if (bk < 0) break;  // nothing live left
        const int64_t t = tl[size_t(bk)].t;
        const uint64_t before = len_of(bk);
        tiles[16 * t + bslot] = 0;
        M->tile_sparse[t] = b4_encode_flag(tiles + 16 * t, M->switch_point);
        used = used - before + len_of(bk);
        ++M->evicted;
    }
    uint64_t fit_pos = 0;
    int64_t fit = 0;
    for (int64_t k = k0; k < k1; ++k) {
        const uint64_t tlen = len_of(k);
        if (fit_pos + tlen > alloc) break;
        fit_pos += tlen;
        ++fit;
    }
    if (fit < k1 - k0) {
        ++M->overflow_events;
        M->overflow_bytes += used - fit_pos;
    }
}

int nthreads_of(int threads) { return threads > 0 ? threads : 1; }

}  // namespace

extern "C" {

float oracle_fp4_decode(uint8_t code) { return fp4_dec(code & 0xFu); }
uint8_t oracle_fp4_encode(float v) { return fp4_enc(v); }
void oracle_fp4_encode_array(const float *v, int64_t n, uint8_t *out) {
    for (int64_t i = 0; i < n; ++i) out[i] = fp4_enc(v[i]);
}
size_t oracle_uleb_encode(uint32_t v, uint8_t *out) { return uleb_enc(v, out); }
uint32_t oracle_uleb_decode(const uint8_t *buf, uint64_t *pos) { return uleb_dec(buf, *pos); }

int64_t oracle_csr_index_bytes(int64_t rows, const int32_t *ptrs, const int32_t *idx) {
    int64_t total = 0;
    for (int64_t r = 0; r < rows; ++r) {
        uint32_t prev = 0;
        for (int64_t i = ptrs[r]; i < ptrs[r + 1]; ++i) {
            total += int64_t(uleb_len(uint32_t(idx[i]) - prev));
            prev = uint32_t(idx[i]);
        }
    }
    return total;
}

// delta_csr_memory.hpp:16-93 followed by sisldo_ops.hpp:44-96 (compact): the
// compacted stream is the concatenation of each row's canonical ULEB bytes;
// value bytes are (fp4_encode(w) << 4) | fp4_encode(imp).
int oracle_csr_encode_bytes(int64_t rows, const int32_t *ptrs, const int32_t *idx,
                            const uint8_t *bytes, uint64_t *row_byte_start,
                            uint64_t *row_elem_start, uint8_t *idx_out,
                            uint8_t *val_out) {
    uint64_t bpos = 0;
    for (int64_t r = 0; r < rows; ++r) {
        row_byte_start[r] = bpos;
        row_elem_start[r] = uint64_t(ptrs[r]);
        uint32_t prev = 0;
        for (int64_t i = ptrs[r]; i < ptrs[r + 1]; ++i) {
            const uint32_t c = uint32_t(idx[i]);
            if (i > ptrs[r] && c <= prev) return -1;  // strictly increasing required
            bpos += uleb_enc(c - prev, idx_out + bpos);
            prev = c;
            val_out[i] = bytes[i];
        }
    }
    row_byte_start[rows] = bpos;
    row_elem_start[rows] = uint64_t(ptrs[rows]);
    return 0;
}

int oracle_csr_encode(int64_t rows, const int32_t *ptrs, const int32_t *idx,
                      const float *w, const float *imp, uint64_t *row_byte_start,
                      uint64_t *row_elem_start, uint8_t *idx_out, uint8_t *val_out) {
    const int64_t nnz = ptrs[rows];
    std::vector<uint8_t> bytes(size_t(std::max<int64_t>(nnz, 1)));
    for (int64_t i = 0; i < nnz; ++i)
        bytes[size_t(i)] = uint8_t((fp4_enc(w[i]) << 4) | fp4_enc(imp ? imp[i] : 0.0f));
    return oracle_csr_encode_bytes(rows, ptrs, idx, bytes.data(), row_byte_start,
                                   row_elem_start, idx_out, val_out);
}

// delta_csr_memory.hpp:95-123 (delta_csr_to_absolute), columns only.
int oracle_csr_decode(int64_t rows, const uint64_t *row_byte_start,
                      const uint64_t *row_elem_start, const uint8_t *idx,
                      int32_t *cols_out) {
    for (int64_t r = 0; r < rows; ++r) {
        uint64_t pos = row_byte_start[r];
        uint32_t col = 0;
        for (uint64_t e = row_elem_start[r]; e < row_elem_start[r + 1]; ++e) {
            col += uleb_dec(idx, pos);
            cols_out[e] = int32_t(col);
        }
        if (pos != row_byte_start[r + 1]) return -1;
    }
    return 0;
}

// delta_csr_memory.hpp:127-213 (delta_csr_combined_to_absolute): scattered
// entries plus live (byte != 0) block4 slots, per row sorted by column.
int64_t oracle_combined_to_absolute(const OracleLayer *L, int32_t *ptrs, int32_t *idx,
                                    float *w, float *imp) {
    struct E { uint32_t c; float w, imp; };
    const auto tiles = collect_tiles(L);
    // tiles grouped by block row, in bc order already
    std::vector<size_t> tb((L->n_in + TILE - 1) / TILE + 1, 0);
    for (const auto &t : tiles) tb[size_t(t.br) + 1]++;
    for (size_t i = 1; i < tb.size(); ++i) tb[i] += tb[i - 1];
    int64_t flat = 0;
    if (ptrs) ptrs[0] = 0;
    std::vector<E> row;
    for (int64_t r = 0; r < L->n_in; ++r) {
        row.clear();
        uint64_t pos = L->row_byte_start[r];
        uint32_t col = 0;
        for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
            col += uleb_dec(L->idx, pos);
            row.push_back({col, fp4_dec(L->val[e] >> 4), fp4_dec(L->val[e] & 0xFu)});
        }
        if (L->n_tiles > 0) {
            const int64_t br = r / TILE, li = r % TILE;
            for (size_t k = tb[size_t(br)]; k < tb[size_t(br) + 1]; ++k) {
                const uint8_t *td = L->tiles + 16 * tiles[k].t;
                for (int lj = 0; lj < TILE; ++lj) {
                    const uint8_t b = td[lj * TILE + li];
                    const int64_t c = tiles[k].bc * TILE + lj;
                    if (b == 0 || c >= L->n_out) continue;
                    row.push_back({uint32_t(c), fp4_dec(b & 0xFu), fp4_dec(b >> 4)});
                }
            }
        }
        std::stable_sort(row.begin(), row.end(), [](const E &a, const E &b) { return a.c < b.c; });
        for (const auto &e : row) {
            if (idx) idx[flat] = int32_t(e.c);
            if (w) w[flat] = e.w;
            if (imp) imp[flat] = e.imp;
            ++flat;
        }
        if (ptrs) ptrs[r + 1] = int32_t(flat);
    }
    return flat;
}

void oracle_dense_weights(const OracleLayer *L, float *W) {
    std::fill(W, W + L->n_in * L->n_out, 0.0f);
    for (int64_t r = 0; r < L->n_in; ++r) {
        uint64_t pos = L->row_byte_start[r];
        uint32_t col = 0;
        for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
            col += uleb_dec(L->idx, pos);
            W[r * L->n_out + col] = fp4_dec(L->val[e] >> 4) * scale_rc(L, r, col);
        }
    }
    for (const auto &t : collect_tiles(L)) {
        const uint8_t *td = L->tiles + 16 * t.t;
        for (int li = 0; li < TILE; ++li)
            for (int lj = 0; lj < TILE; ++lj) {
                const int64_t r = t.br * TILE + li, c = t.bc * TILE + lj;
                if (r >= L->n_in || c >= L->n_out) continue;
                W[r * L->n_out + c] = fp4_dec(td[lj * TILE + li] & 0xFu) * scale_rc(L, r, c);
            }
    }
}

// linear_disldo.hpp:68-345 (disldo_forward).  Scattered pass skips exact-zero
// inputs (:114); block4 pass does 4-term dots per output column (:297-326).
void oracle_forward_dense(const OracleLayer *L, const float *x, int64_t batch, float *y,
                          int threads, int absmode) {
    const int nt = nthreads_of(threads);
    const int64_t n_in = L->n_in, n_out = L->n_out;
    const size_t ost = size_t(batch * n_out);
    std::vector<float> t_out(size_t(nt) * ost, 0.0f);
#pragma omp parallel num_threads(nt)
    {
        float *mo = t_out.data() + size_t(omp_get_thread_num()) * ost;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n_in; ++r) {
            uint64_t pos = L->row_byte_start[r];
            uint32_t col = 0;
            for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
                col += uleb_dec(L->idx, pos);
                const float w = maybe_abs(fp4_dec(L->val[e] >> 4) * scale_rc(L, r, col), absmode);
                for (int64_t b = 0; b < batch; ++b) {
                    const float iv = maybe_abs(x[b * n_in + r], absmode);
                    if (iv == 0.0f) continue;
                    mo[b * n_out + col] += w * iv;
                }
            }
        }
    }
    for (int t = 0; t < nt; ++t)
        for (size_t i = 0; i < ost; ++i) y[i] += t_out[size_t(t) * ost + i];
    if (L->n_tiles <= 0) return;
    const auto tiles = collect_tiles(L);
    std::fill(t_out.begin(), t_out.end(), 0.0f);
#pragma omp parallel num_threads(nt)
    {
        float *mo = t_out.data() + size_t(omp_get_thread_num()) * ost;
#pragma omp for schedule(static)
        for (int64_t ti = 0; ti < int64_t(tiles.size()); ++ti) {
            const auto &t = tiles[size_t(ti)];
            const uint8_t *td = L->tiles + 16 * t.t;
            for (int lj = 0; lj < TILE; ++lj) {
                const int64_t col = t.bc * TILE + lj;
                if (col >= n_out) continue;
                float w4[TILE];
                int64_t ri[TILE];
                for (int li = 0; li < TILE; ++li) {
                    const int64_t row = t.br * TILE + li;
                    if (row < n_in) {
                        w4[li] = maybe_abs(fp4_dec(td[lj * TILE + li] & 0xFu) * scale_rc(L, row, col), absmode);
                        ri[li] = row;
                    } else { w4[li] = 0.0f; ri[li] = 0; }
                }
                for (int64_t b = 0; b < batch; ++b) {
                    float acc = 0.0f;
                    for (int li = 0; li < TILE; ++li)
                        acc += w4[li] * maybe_abs(x[b * n_in + ri[li]], absmode);
                    mo[b * n_out + col] += acc;
                }
            }
        }
    }
    for (int t = 0; t < nt; ++t)
        for (size_t i = 0; i < ost; ++i) y[i] += t_out[size_t(t) * ost + i];
}

// linear_disldo.hpp:462-2113 at learning_rate == 0: accumulators (:515-520),
// scattered dx (:884 with quant = stored code, cw = quant*S), block4 dx
// (:1617/1662/1701), per-thread dx buffers reduced serially (:2044-2049).
void oracle_backward_dense(const OracleLayer *L, const float *x, const float *dy,
                           int64_t batch, float *dx, float *acc_in, float *acc_grad,
                           int threads, int absmode) {
    const int nt = nthreads_of(threads);
    const int64_t n_in = L->n_in, n_out = L->n_out;
    if (acc_in && acc_grad) {
        for (int64_t b = 0; b < batch; ++b) {
            for (int64_t r = 0; r < n_in; ++r) acc_in[r] += std::fabs(x[b * n_in + r]);
            for (int64_t c = 0; c < n_out; ++c) acc_grad[c] += std::fabs(dy[b * n_out + c]);
        }
    }
    const size_t dst = size_t(batch * n_in);
    std::vector<float> t_dx(size_t(nt) * dst, 0.0f);
    const auto tiles = collect_tiles(L);
    std::vector<size_t> tb((n_in + TILE - 1) / TILE + 1, 0);
    for (const auto &t : tiles) tb[size_t(t.br) + 1]++;
    for (size_t i = 1; i < tb.size(); ++i) tb[i] += tb[i - 1];
#pragma omp parallel num_threads(nt)
    {
        float *mdx = t_dx.data() + size_t(omp_get_thread_num()) * dst;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n_in; ++r) {
            uint64_t pos = L->row_byte_start[r];
            uint32_t col = 0;
            for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
                col += uleb_dec(L->idx, pos);
                const float cw = maybe_abs(fp4_dec(L->val[e] >> 4) * scale_rc(L, r, col), absmode);
                for (int64_t b = 0; b < batch; ++b)
                    mdx[b * n_in + r] += cw * maybe_abs(dy[b * n_out + col], absmode);
            }
        }
        // block4 rows: per tile row li, 4-wide dot over lj (hsum of w*dy)
#pragma omp for schedule(static)
        for (int64_t br = 0; br < int64_t(tb.size()) - 1; ++br) {
            for (size_t k = tb[size_t(br)]; k < tb[size_t(br) + 1]; ++k) {
                const auto &t = tiles[k];
                const uint8_t *td = L->tiles + 16 * t.t;
                for (int li = 0; li < TILE; ++li) {
                    const int64_t row = br * TILE + li;
                    if (row >= n_in) continue;
                    float w4[TILE];
                    bool ok[TILE];
                    for (int lj = 0; lj < TILE; ++lj) {
                        const int64_t col = t.bc * TILE + lj;
                        ok[lj] = col < n_out;
                        w4[lj] = ok[lj] ? maybe_abs(fp4_dec(td[lj * TILE + li] & 0xFu) * scale_rc(L, row, col), absmode) : 0.0f;
                    }
                    for (int64_t b = 0; b < batch; ++b) {
                        float hs = 0.0f;
                        for (int lj = 0; lj < TILE; ++lj)
                            if (ok[lj]) hs += w4[lj] * maybe_abs(dy[b * n_out + t.bc * TILE + lj], absmode);
                        mdx[b * n_in + row] += hs;
                    }
                }
            }
        }
    }
    for (int t = 0; t < nt; ++t)
        for (size_t i = 0; i < dst; ++i) dx[i] += t_dx[size_t(t) * dst + i];
}

// sisldo_ops.hpp:198-551 (sisldo_forward).  Scattered weights use
// stored*(vs0*os0) (:302-306); block4 windows skip dead slots and use
// (dec*vs0)*os0 (:527-531).  Inputs must be sorted within each batch row.
void oracle_forward_sparse(const OracleLayer *L, const int32_t *ptrs, const int32_t *idx,
                           const float *vals, int64_t batch, float *y, int threads,
                           int absmode) {
    const int nt = nthreads_of(threads);
    const int64_t n_out = L->n_out;
    const size_t ost = size_t(batch * n_out);
    std::vector<float> t_out(size_t(nt) * ost, 0.0f);
    // Scattered: per batch row, split the (active row, element) work evenly.
#pragma omp parallel num_threads(nt)
    {
        float *mo = t_out.data() + size_t(omp_get_thread_num()) * ost;
        for (int64_t b = 0; b < batch; ++b) {
#pragma omp for schedule(static)
            for (int64_t i = ptrs[b]; i < ptrs[b + 1]; ++i) {
                const int64_t r = idx[i];
                const float v = maybe_abs(vals[i], absmode);
                uint64_t pos = L->row_byte_start[r];
                uint32_t col = 0;
                const float vsr = vs0(L, r);
                for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
                    col += uleb_dec(L->idx, pos);
                    const float w = maybe_abs(fp4_dec(L->val[e] >> 4) * (vsr * os0(L, col)), absmode);
                    mo[b * n_out + col] += w * v;
                }
            }
        }
    }
    for (int t = 0; t < nt; ++t)
        for (size_t i = 0; i < ost; ++i) y[i] += t_out[size_t(t) * ost + i];
    if (L->n_tiles <= 0) return;
    const auto tiles = collect_tiles(L);
    std::vector<size_t> tb((L->n_in + TILE - 1) / TILE + 1, 0);
    for (const auto &t : tiles) tb[size_t(t.br) + 1]++;
    for (size_t i = 1; i < tb.size(); ++i) tb[i] += tb[i - 1];
    for (int64_t b = 0; b < batch; ++b) {
        int64_t i = ptrs[b];
        while (i < ptrs[b + 1]) {
            const int64_t br = idx[i] / TILE, lo = br * TILE, hi = lo + TILE;
            float local[TILE] = {0, 0, 0, 0};
            int64_t j = i;
            while (j < ptrs[b + 1] && idx[j] < hi) { local[idx[j] - lo] = maybe_abs(vals[j], absmode); ++j; }
            for (size_t k = tb[size_t(br)]; k < tb[size_t(br) + 1]; ++k) {
                const auto &t = tiles[k];
                const uint8_t *td = L->tiles + 16 * t.t;
                for (int lj = 0; lj < TILE; ++lj) {
                    const int64_t col = t.bc * TILE + lj;
                    if (col >= n_out) continue;
                    float acc = 0.0f;
                    for (int li = 0; li < TILE; ++li) {
                        const int64_t row = br * TILE + li;
                        if (row >= L->n_in) continue;
                        const uint8_t byte = td[lj * TILE + li];
                        if (byte == 0) continue;
                        const float wt = maybe_abs(fp4_dec(byte & 0xFu) * vs0(L, row) * os0(L, col), absmode);
                        acc += wt * local[li];
                    }
                    y[b * n_out + col] += acc;
                }
            }
            i = j;
        }
    }
}

// sisldo_ops.hpp:589-1104 (disldo_backward_sparse_grad) at lr == 0: per row a
// merge-join against the sorted sparse dy; weight = stored*(vs0*os0); block4
// slots skip dy == 0 and use dec*vs0*os0.
void oracle_backward_sparse(const OracleLayer *L, const float *x, const int32_t *dptrs,
                            const int32_t *didx, const float *dvals, int64_t batch,
                            float *dx, float *acc_in, float *acc_grad, int threads,
                            int absmode) {
    const int nt = nthreads_of(threads);
    const int64_t n_in = L->n_in, n_out = L->n_out;
    if (acc_in && acc_grad) {
        for (int64_t b = 0; b < batch; ++b)
            for (int64_t r = 0; r < n_in; ++r) acc_in[r] += std::fabs(x[b * n_in + r]);
        for (int64_t b = 0; b < batch; ++b)
            for (int64_t j = dptrs[b]; j < dptrs[b + 1]; ++j) acc_grad[didx[j]] += std::fabs(dvals[j]);
    }
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t og0 = dptrs[b], og1 = dptrs[b + 1];
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t r = 0; r < n_in; ++r) {
            uint64_t pos = L->row_byte_start[r];
            uint32_t col = 0;
            int64_t og = og0;
            float acc = 0.0f;
            const float vsr = vs0(L, r);
            for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
                col += uleb_dec(L->idx, pos);
                const float w = maybe_abs(fp4_dec(L->val[e] >> 4) * (vsr * os0(L, col)), absmode);
                while (og < og1 && didx[og] < int32_t(col)) ++og;
                if (og >= og1 || didx[og] != int32_t(col)) continue;
                acc += w * maybe_abs(dvals[og], absmode);
            }
            dx[b * n_in + r] += acc;
        }
    }
    if (L->n_tiles <= 0) return;
    const auto tiles = collect_tiles(L);
    std::vector<size_t> tb((n_in + TILE - 1) / TILE + 1, 0);
    for (const auto &t : tiles) tb[size_t(t.br) + 1]++;
    for (size_t i = 1; i < tb.size(); ++i) tb[i] += tb[i - 1];
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t og0 = dptrs[b], og1 = dptrs[b + 1];
#pragma omp parallel for num_threads(nt) schedule(static)
        for (int64_t br = 0; br < int64_t(tb.size()) - 1; ++br) {
            float dxa[TILE] = {0, 0, 0, 0};
            int64_t og = og0;
            for (size_t k = tb[size_t(br)]; k < tb[size_t(br) + 1]; ++k) {
                const auto &t = tiles[k];
                const int64_t lo = t.bc * TILE, hi = lo + TILE;
                while (og < og1 && didx[og] < lo) ++og;
                float dl[TILE] = {0, 0, 0, 0};
                bool any = false;
                for (int64_t p = og; p < og1 && didx[p] < hi; ++p) { dl[didx[p] - lo] = maybe_abs(dvals[p], absmode); any = true; }
                if (!any) continue;
                const uint8_t *td = L->tiles + 16 * t.t;
                for (int li = 0; li < TILE; ++li) {
                    const int64_t row = br * TILE + li;
                    if (row >= n_in) continue;
                    for (int lj = 0; lj < TILE; ++lj) {
                        if (dl[lj] == 0.0f) continue;
                        const int64_t col = lo + lj;
                        if (col >= n_out) continue;
                        const float w = maybe_abs(fp4_dec(td[lj * TILE + li] & 0xFu) * vs0(L, row) * os0(L, col), absmode);
                        dxa[li] += w * dl[lj];
                    }
                }
            }
            for (int li = 0; li < TILE; ++li)
                if (br * TILE + li < n_in) dx[b * n_in + br * TILE + li] += dxa[li];
        }
    }
}

// Explicit nnz-sampled grad-W.  The reference never materialises it: it is
// the g = dy*x consumed per (synapse, b) by disldo_backward's optimizer
// (linear_disldo.hpp:811-882).  GW[e] = sum_b x[b,r(e)] * dy[b,c(e)].
void oracle_sampled_gradw(const OracleLayer *L, const float *x, const float *dy,
                          int64_t batch, float *gw_scattered, float *gw_tiles,
                          int threads, int absmode) {
    const int nt = nthreads_of(threads);
    const int64_t n_in = L->n_in, n_out = L->n_out;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < n_in; ++r) {
        uint64_t pos = L->row_byte_start[r];
        uint32_t col = 0;
        for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
            col += uleb_dec(L->idx, pos);
            double s = 0.0;
            for (int64_t b = 0; b < batch; ++b)
                s += double(maybe_abs(x[b * n_in + r], absmode)) * double(maybe_abs(dy[b * n_out + col], absmode));
            gw_scattered[e] = float(s);
        }
    }
    if (L->n_tiles <= 0 || !gw_tiles) return;
    const auto tiles = collect_tiles(L);
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t ti = 0; ti < int64_t(tiles.size()); ++ti) {
        const auto &t = tiles[size_t(ti)];
        for (int lj = 0; lj < TILE; ++lj)
            for (int li = 0; li < TILE; ++li) {
                const int64_t r = t.br * TILE + li, c = t.bc * TILE + lj;
                double s = 0.0;
                if (r < n_in && c < n_out)
                    for (int64_t b = 0; b < batch; ++b)
                        s += double(maybe_abs(x[b * n_in + r], absmode)) * double(maybe_abs(dy[b * n_out + c], absmode));
                gw_tiles[16 * t.t + lj * TILE + li] = float(s);
            }
    }
}

// ---------------------------------------------------------------------------
// Bulk synaptogenesis (magnitude prune + candidate regrow).  The selection
// policy is new (no reference equivalent); the structural rules follow the
// reference:
//   - removing a block4 slot zeroes its byte, and a tile whose live count
//     drops below 2 is demoted to scattered (delta_csr_memory.hpp:1203-1225,
//     949-999; demoted bytes requantize dec->enc, i.e. code 8 -> 0);
//   - an insert whose 4x4 window already holds a tile writes into the tile
//     (delta_csr_memory.hpp:620-646); otherwise it is a scattered insert, and a
//     window that then holds >= 2 scattered synapses is promoted into a tile
//     (delta_csr_memory.hpp:648-700).
// Phase order: select -> prune -> demote -> insert -> promote -> rebuild.
int oracle_synapto_step(const OracleLayer *L, float prune_frac, const int32_t *cand_r,
                        const int32_t *cand_c, const float *cand_v, const float *cand_score,
                        int64_t n_cand, int default_imp_code, int32_t *out_ptrs,
                        int32_t *out_cols, uint8_t *out_bytes, int32_t *out_tile_br,
                        int32_t *out_tile_bc, uint8_t *out_tile_bytes,
                        OracleSynaptoStats *stats) {
    const int64_t n_in = L->n_in, n_out = L->n_out;
    struct Syn { uint32_t absw; int64_t r, c; int64_t where; };  // where>=0: scattered elem; <0: -(tile*16+slot)-1
    std::vector<Syn> all;
    // scattered
    std::vector<int32_t> cols(size_t(L->row_elem_start[n_in]));
    if (oracle_csr_decode(n_in, L->row_byte_start, L->row_elem_start, L->idx, cols.data()) != 0) return -1;
    for (int64_t r = 0; r < n_in; ++r)
        for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
            const int64_t c = cols[e];
            const float w = fp4_dec(L->val[e] >> 4) * scale_rc(L, r, c);
            all.push_back({f2u(w) & 0x7FFFFFFFu, r, c, int64_t(e)});
        }
    const auto tiles = collect_tiles(L);
    std::vector<std::vector<uint8_t>> tdata(tiles.size(), std::vector<uint8_t>(16));
    for (size_t k = 0; k < tiles.size(); ++k) {
        std::memcpy(tdata[k].data(), L->tiles + 16 * tiles[k].t, 16);
        for (int lj = 0; lj < TILE; ++lj)
            for (int li = 0; li < TILE; ++li) {
                const uint8_t b = tdata[k][lj * TILE + li];
                const int64_t r = tiles[k].br * TILE + li, c = tiles[k].bc * TILE + lj;
                if (b == 0 || r >= n_in || c >= n_out) continue;
                const float w = fp4_dec(b & 0xFu) * scale_rc(L, r, c);
                all.push_back({f2u(w) & 0x7FFFFFFFu, r, c, -(int64_t(k) * 16 + lj * TILE + li) - 1});
            }
    }
    const int64_t N = int64_t(all.size());
    const int64_t k_prune = std::min<int64_t>(N, int64_t(std::llround(double(prune_frac) * double(N))));
    // k smallest by (|w| bits, r, c)
    std::vector<size_t> order(all.size());
    std::iota(order.begin(), order.end(), size_t(0));
    auto less = [&](size_t a, size_t b) {
        const Syn &x = all[a], &y = all[b];
        if (x.absw != y.absw) return x.absw < y.absw;
        if (x.r != y.r) return x.r < y.r;
        return x.c < y.c;
    };
    if (k_prune > 0 && k_prune < N)
        std::nth_element(order.begin(), order.begin() + k_prune, order.end(), less);
    std::vector<char> s_removed(cols.size(), 0);
    std::vector<char> tile_touched(tiles.size(), 0);
    // pruned (r,c) set for the "not just-pruned" regrow rule
    std::vector<std::pair<int64_t, int64_t>> pruned_rc;
    for (int64_t i = 0; i < k_prune; ++i) {
        const Syn &s = all[order[size_t(i)]];
        pruned_rc.push_back({s.r, s.c});
        if (s.where >= 0) s_removed[size_t(s.where)] = 1;
        else {
            const int64_t q = -s.where - 1;
            tdata[size_t(q / 16)][size_t(q % 16)] = 0;
            tile_touched[size_t(q / 16)] = 1;
        }
    }
    std::sort(pruned_rc.begin(), pruned_rc.end());
    // scattered survivors per row: map row -> sorted (col, byte)
    std::vector<std::vector<std::pair<int64_t, uint8_t>>> rows{size_t(n_in)};
    for (int64_t r = 0; r < n_in; ++r)
        for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e)
            if (!s_removed[e]) rows[size_t(r)].push_back({cols[e], L->val[e]});
    // demote touched tiles with live < 2
    std::vector<char> tile_alive(tiles.size(), 1);
    int64_t n_demoted = 0;
    auto requant = [](uint8_t code) -> uint8_t { return code == 8 ? 0 : code; };
    for (size_t k = 0; k < tiles.size(); ++k) {
        if (!tile_touched[k]) continue;
        int live = 0;
        for (int s = 0; s < 16; ++s) live += tdata[k][size_t(s)] != 0;
        if (live >= PROMOTE_MIN_LIVE) continue;
        tile_alive[k] = 0;
        ++n_demoted;
        for (int lj = 0; lj < TILE; ++lj)
            for (int li = 0; li < TILE; ++li) {
                const uint8_t b = tdata[k][size_t(lj * TILE + li)];
                const int64_t r = tiles[k].br * TILE + li, c = tiles[k].bc * TILE + lj;
                if (b == 0 || r >= n_in || c >= n_out) continue;
                const uint8_t sb = uint8_t((requant(b & 0xFu) << 4) | requant(b >> 4));
                auto &row = rows[size_t(r)];
                row.insert(std::lower_bound(row.begin(), row.end(), std::make_pair(c, uint8_t(0))), {c, sb});
            }
    }
    // tile lookup by window after demotion
    auto win_key = [&](int64_t br, int64_t bc) { return br * ((n_out + TILE - 1) / TILE) + bc; };
    std::vector<std::pair<int64_t, size_t>> tile_index;  // (window key, tile k)
    for (size_t k = 0; k < tiles.size(); ++k)
        if (tile_alive[k]) tile_index.push_back({win_key(tiles[k].br, tiles[k].bc), k});
    std::sort(tile_index.begin(), tile_index.end());
    auto find_tile = [&](int64_t br, int64_t bc) -> int64_t {
        const int64_t key = win_key(br, bc);
        auto it = std::lower_bound(tile_index.begin(), tile_index.end(), std::make_pair(key, size_t(0)));
        if (it != tile_index.end() && it->first == key) return int64_t(it->second);
        return -1;
    };
    auto stored = [&](int64_t r, int64_t c) -> bool {
        const auto &row = rows[size_t(r)];
        auto it = std::lower_bound(row.begin(), row.end(), std::make_pair(c, uint8_t(0)));
        if (it != row.end() && it->first == c) return true;
        const int64_t k = find_tile(r / TILE, c / TILE);
        return k >= 0 && tdata[size_t(k)][size_t((c % TILE) * TILE + (r % TILE))] != 0;
    };
    // inserts: candidates in list order, first k_pruned valid ones
    int64_t n_grown = 0;
    std::vector<std::pair<int64_t, int64_t>> accepted;   // sorted set of accepted (r,c)
    std::vector<int64_t> touched_windows;
    for (int64_t i = 0; i < n_cand && n_grown < k_prune; ++i) {
        const int64_t r = cand_r[i], c = cand_c[i];
        if (r < 0 || r >= n_in || c < 0 || c >= n_out) continue;
        if (std::binary_search(pruned_rc.begin(), pruned_rc.end(), std::make_pair(r, c))) continue;
        if (std::binary_search(accepted.begin(), accepted.end(), std::make_pair(r, c))) continue;
        if (stored(r, c)) continue;
        accepted.insert(std::lower_bound(accepted.begin(), accepted.end(), std::make_pair(r, c)), {r, c});
        ++n_grown;
        const float S = scale_rc(L, r, c);
        const uint8_t wc = fp4_enc(cand_v[i] / S);
        const uint8_t ic = cand_score ? fp4_enc(cand_score[i]) : uint8_t(default_imp_code & 0xF);
        const int64_t k = find_tile(r / TILE, c / TILE);
        if (k >= 0) {
            tdata[size_t(k)][size_t((c % TILE) * TILE + (r % TILE))] = uint8_t((ic << 4) | wc);
        } else {
            auto &row = rows[size_t(r)];
            row.insert(std::lower_bound(row.begin(), row.end(), std::make_pair(c, uint8_t(0))),
                       {c, uint8_t((wc << 4) | ic)});
            touched_windows.push_back(win_key(r / TILE, c / TILE));
        }
    }
    // promote windows that received a scattered insert and now hold >= 2
    std::sort(touched_windows.begin(), touched_windows.end());
    touched_windows.erase(std::unique(touched_windows.begin(), touched_windows.end()), touched_windows.end());
    const int64_t bcols = (n_out + TILE - 1) / TILE;
    struct NewTile { int64_t br, bc; uint8_t d[16]; };
    std::vector<NewTile> new_tiles;
    for (const int64_t key : touched_windows) {
        const int64_t br = key / bcols, bc = key % bcols;
        int cnt = 0;
        for (int li = 0; li < TILE; ++li) {
            const int64_t r = br * TILE + li;
            if (r >= n_in) continue;
            const auto &row = rows[size_t(r)];
            for (const auto &e : row) if (e.first >= bc * TILE && e.first < bc * TILE + TILE) ++cnt;
        }
        if (cnt < PROMOTE_MIN_LIVE) continue;
        NewTile nt{br, bc, {0}};
        for (int li = 0; li < TILE; ++li) {
            const int64_t r = br * TILE + li;
            if (r >= n_in) continue;
            auto &row = rows[size_t(r)];
            std::vector<std::pair<int64_t, uint8_t>> keep;
            for (const auto &e : row) {
                if (e.first >= bc * TILE && e.first < bc * TILE + TILE) {
                    const uint8_t b = e.second;
                    nt.d[(e.first - bc * TILE) * TILE + li] = uint8_t(requant(b >> 4) | (requant(b & 0xFu) << 4));
                } else keep.push_back(e);
            }
            row.swap(keep);
        }
        new_tiles.push_back(nt);
    }
    // rebuild outputs
    int64_t flat = 0;
    out_ptrs[0] = 0;
    for (int64_t r = 0; r < n_in; ++r) {
        for (const auto &e : rows[size_t(r)]) {
            out_cols[flat] = int32_t(e.first);
            out_bytes[flat] = e.second;
            ++flat;
        }
        out_ptrs[r + 1] = int32_t(flat);
    }
    struct OutTile { int64_t br, bc; const uint8_t *d; };
    std::vector<OutTile> ot;
    for (size_t k = 0; k < tiles.size(); ++k)
        if (tile_alive[k]) ot.push_back({tiles[k].br, tiles[k].bc, tdata[k].data()});
    for (const auto &t : new_tiles) ot.push_back({t.br, t.bc, t.d});
    std::sort(ot.begin(), ot.end(), [](const OutTile &a, const OutTile &b) {
        return a.br != b.br ? a.br < b.br : a.bc < b.bc;
    });
    for (size_t k = 0; k < ot.size(); ++k) {
        out_tile_br[k] = int32_t(ot[k].br);
        out_tile_bc[k] = int32_t(ot[k].bc);
        std::memcpy(out_tile_bytes + 16 * k, ot[k].d, 16);
    }
    if (stats) {
        stats->n_prune_target = k_prune;
        stats->n_pruned = k_prune;
        stats->n_grown = n_grown;
        stats->n_demoted_tiles = n_demoted;
        stats->n_promoted_tiles = int64_t(new_tiles.size());
        stats->n_scattered = flat;
        stats->n_tiles = int64_t(ot.size());
    }
    return 0;
}

}  // extern "C"

// ---- backward with the optimizer update ------------------------------------
namespace {

// std::max / std::min as the reference calls them (a NaN first operand is
// returned as is).
inline float std_max(float a, float b) { return (a < b) ? b : a; }
inline float std_min(float a, float b) { return (b < a) ? b : a; }

// BoundedRMSpropSynapsePolicy::update_ci (delta_csr_types.hpp:707-712).
inline float bounded_update_ci(float ci, float g, float contrib, float beta2, float min_decay_frac,
                               float max_ci) {
    const float ema = beta2 * ci + (1.0f - beta2) * (g * g + contrib * contrib);
    const float floor_ = min_decay_frac * ci;
    return std_min(std_max(ema, floor_), max_ci);
}

// BoundedRMSpropSynapsePolicy::update_cw (delta_csr_types.hpp:749-758).
inline float bounded_update_cw(float g, float ci, float S, float eff_lr, float eps, bool damp,
                               float max_abs_delta) {
    float raw = damp ? (-g * S) / (std::sqrt(ci) + eps) : (-g * S);
    if (raw > max_abs_delta) raw = max_abs_delta;
    if (raw < -max_abs_delta) raw = -max_abs_delta;
    return eff_lr * raw;
}

// RMSpropScalePolicy::update with its bias-correction counter
// (delta_csr_types.hpp:413-434).
inline void rmsprop_scale_update(float &scale, float &state, float g_agg, float eff_lr, float beta2,
                                 float eps, float contrib_agg, uint32_t &step) {
    if (!std::isfinite(g_agg) || !std::isfinite(contrib_agg)) return;
    const float new_state = beta2 * state + (1.0f - beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
    if (!std::isfinite(new_state)) return;
    float state_hat = new_state;
    ++step;
    const float bias_correction = 1.0f - std::pow(beta2, static_cast<float>(step));
    if (bias_correction > 0.0f) state_hat = new_state / bias_correction;
    if (!std::isfinite(state_hat)) return;
    const float new_scale = scale - eff_lr * g_agg / (std::sqrt(state_hat) + eps);
    if (!std::isfinite(new_scale)) return;
    state = new_state;
    scale = new_scale;
}

}  // namespace

extern "C" {

// linear_disldo.hpp:466-2113 (scattered loop :624-880, dead-row bootstrap
// :1944-2040, dx reduction :2043-2048, output_scale update :2050-2080).
int oracle_backward_train(const OracleLayer *L, uint8_t *val, uint8_t *tiles, OracleTrainState *S,
                          const float *x, const float *dy, int64_t batch, float *dx,
                          float *acc_in, float *acc_grad, const OracleTrainParams *P) {
    if (L->n_tiles > 0 && !tiles) return -1;
    const int64_t n_in = L->n_in, n_out = L->n_out;
    const int rank = L->rank;
    const float lr = P->lr;
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t r = 0; r < n_in; ++r) acc_in[r] += std::fabs(x[b * n_in + r]);
        for (int64_t c = 0; c < n_out; ++c) acc_grad[c] += std::fabs(dy[b * n_out + c]);
    }
    std::vector<float> mdx(size_t(batch * n_in), 0.0f);
    std::vector<float> mcol(size_t(n_out * rank), 0.0f), mcol_c(size_t(n_out * rank), 0.0f);
    float *vs = S->value_scale, *os = S->output_scale;
    const bool deferred = P->variant == 1, no_scale = P->variant == 2;
    // DeferredScaleWrite: each synapse's true-units (cw, ci) and column, stored
    // after the scales are final (linear_disldo.hpp:501-509,783,2090-2112)
    const uint64_t nnz_all = L->row_elem_start[n_in];
    std::vector<float> def_w(deferred ? nnz_all : 0), def_i(deferred ? nnz_all : 0);
    std::vector<uint32_t> def_col(deferred ? nnz_all : 0);
    for (int64_t r = 0; r < n_in; ++r) {
        const uint64_t e0 = L->row_elem_start[r], e1 = L->row_elem_start[r + 1];
        const uint64_t nnz_row = e1 - e0;
        if (nnz_row == 0) continue;
        const float eff_lr = P->lr_per_row_nnz ? lr / static_cast<float>(nnz_row) : lr;
        const float scale_eff_lr = lr / static_cast<float>(nnz_row);
        const float imp_scale = S->importance_scale ? S->importance_scale[r] : 1.0f;
        double sg[4] = {0, 0, 0, 0}, sgc[4] = {0, 0, 0, 0};
        uint64_t pos = L->row_byte_start[r];
        uint32_t col = 0;
        for (uint64_t vb = e0; vb < e1; ++vb) {
            col += uleb_dec(L->idx, pos);
            const float cw_orig = fp4_dec(val[vb] >> 4);
            const float ci_orig = fp4_dec(val[vb] & 0xFu);
            const float out_imp_scale = S->output_importance_scale ? S->output_importance_scale[col] : 1.0f;
            const float combined_imp_scale = imp_scale * out_imp_scale;
            float ci = ci_orig * combined_imp_scale;
            if (deferred) {
                // true-units update under component 0 of both scales
                // (linear_disldo.hpp:687-790)
                const float val_scale = vs[r * rank], out_scale = os[int64_t(col) * rank];
                const float combined_scale = val_scale * out_scale;
                float cw = cw_orig * combined_scale;
                for (int64_t b = 0; b < batch; ++b) {
                    const float iv = x[b * n_in + r];
                    const float dyv = dy[b * n_out + col];
                    const float g = dyv * iv;
                    if (lr != 0.0f) {
                        const float contrib = iv * cw_orig;
                        ci = bounded_update_ci(ci, g, contrib, P->beta2, P->min_decay_frac, P->max_ci);
                        cw += bounded_update_cw(g, ci, 1.0f, eff_lr, P->eps, P->damp_by_importance != 0,
                                                P->max_abs_delta);
                        sg[0] += static_cast<double>(cw_orig) * static_cast<double>(out_scale) * g;
                        mcol[size_t(col) * rank] += cw_orig * val_scale * g;
                        sgc[0] += static_cast<double>(cw_orig) * static_cast<double>(out_scale) * contrib;
                        mcol_c[size_t(col) * rank] += cw_orig * val_scale * contrib;
                    }
                    mdx[size_t(b * n_in + r)] += cw * dyv;
                }
                if (lr != 0.0f) {
                    def_w[vb] = cw;
                    def_i[vb] = ci;
                    def_col[vb] = col;
                }
                continue;
            }
            float Sc = 0.0f;
            for (int k = 0; k < rank; ++k) Sc += vs[r * rank + k] * os[int64_t(col) * rank + k];
            float quant = cw_orig;
            float cw = quant * Sc;
            for (int64_t b = 0; b < batch; ++b) {
                const float iv = x[b * n_in + r];
                const float dyv = dy[b * n_out + col];
                const float g = dyv * iv;
                if (lr != 0.0f) {
                    const float contrib = iv * cw_orig;
                    ci = bounded_update_ci(ci, g, contrib, P->beta2, P->min_decay_frac, P->max_ci);
                    quant += bounded_update_cw(g, ci, Sc, eff_lr, P->eps, P->damp_by_importance != 0,
                                               P->max_abs_delta);
                    cw = quant * Sc;
                    const float qf = (quant == 0.0f) ? P->zero_escape_eps : quant;
                    for (int k = 0; k < rank; ++k) {
                        const float os_k = os[int64_t(col) * rank + k];
                        const float vs_k = vs[r * rank + k];
                        sg[k] += static_cast<double>(qf) * static_cast<double>(os_k) * g;
                        mcol[size_t(col) * rank + k] += qf * vs_k * g;
                        sgc[k] += static_cast<double>(qf) * static_cast<double>(os_k) * contrib;
                        mcol_c[size_t(col) * rank + k] += qf * vs_k * contrib;
                    }
                }
                mdx[size_t(b * n_in + r)] += cw * dyv;
            }
            if (lr != 0.0f) {
                if (S->quant_out) S->quant_out[vb] = quant;
                if (S->imp_out) S->imp_out[vb] = ci / combined_imp_scale;
                val[vb] = uint8_t((fp4_enc(quant) << 4) | fp4_enc(ci / combined_imp_scale));
            }
        }
        // the row's scale step (linear_disldo.hpp:898-925): every component,
        // component 0 alone under DeferredScaleWrite, none under NoScalePolicy
        if (lr != 0.0f && !no_scale) {
            if (deferred) {
                // the reference indexes the scale and its second moment by the
                // row alone here (value_scale[r]: component r % rank of row
                // r / rank once rank > 1), its step counter by (r, 0)
                rmsprop_scale_update(vs[r], S->vs_importance[r], static_cast<float>(sg[0]), scale_eff_lr, P->beta2,
                                     P->eps, static_cast<float>(sgc[0]), S->vs_step[r * rank]);
            } else {
                for (int k = 0; k < rank; ++k) {
                    const int64_t i = r * rank + k;
                    rmsprop_scale_update(vs[i], S->vs_importance[i], static_cast<float>(sg[k]), scale_eff_lr,
                                         P->beta2, P->eps, static_cast<float>(sgc[k]), S->vs_step[i]);
                }
            }
        }
    }
    // block4 tiles (linear_disldo.hpp:962-1951, FP4): every slot of a tile
    // trains (row count n_tiles(br) * 4), after the scattered rows' scale
    // steps, with the same bounded RMSprop step on the code (S = the
    // rank-summed scale) and the zero-escape coefficient.  A tile whose 4
    // columns are all in range takes the reference's 4-lane path: per batch
    // step the row-gradient terms and dx terms of the 4 slots are summed in
    // fp32 lane order ((t0 + t1) + t2) + t3 before the fp64 / fp32
    // accumulation; an edge tile takes the scalar path (fp64 per term).
    // Round to nearest; the block rows' scale step follows (:1923-1951).  The
    // reference also evicts live slots when a block row's compressed tiles
    // outgrow its reserved bytes (block4.hpp merge_row_workspace); that
    // storage-budget rule is not restated (rows are taken to have room).
    std::vector<uint32_t> b4_live(size_t(n_in), 0);
    if (L->n_tiles > 0) {
        const auto tl = collect_tiles(L);
        const int64_t brows = (n_in + TILE - 1) / TILE;
        std::vector<int64_t> nt_br(size_t(brows), 0);
        for (const auto &t : tl) ++nt_br[size_t(t.br)];
        for (int64_t r = 0; r < n_in; ++r) b4_live[size_t(r)] = uint32_t(nt_br[size_t(r / TILE)] * TILE);
        if (lr != 0.0f) {
            std::vector<double> mrow(size_t(n_in * rank), 0.0), mrow_c(size_t(n_in * rank), 0.0);
            for (const auto &t : tl) {
                uint8_t *td = tiles + 16 * t.t;
                const int64_t bc = t.bc;
                const bool full = bc * TILE + TILE <= n_out;
                for (int li = 0; li < TILE; ++li) {
                    const int64_t row = t.br * TILE + li;
                    if (row >= n_in) continue;
                    const uint32_t nnz_row = b4_live[size_t(row)];
                    const float imp_scale = S->importance_scale ? S->importance_scale[row] : 1.0f;
                    const float effective_lr = P->lr_per_row_nnz ? lr / static_cast<float>(nnz_row) : lr;
                    float vs_k[4] = {0, 0, 0, 0};
                    for (int k = 0; k < rank; ++k) vs_k[k] = vs[row * rank + k];
                    float S4[4], cis4[4], q[4], q0[4], ci[4], osk[4][4];
                    bool valid[4];
                    for (int lj = 0; lj < TILE; ++lj) {
                        const int64_t col = bc * TILE + lj;
                        valid[lj] = col < n_out;
                        for (int k = 0; k < 4; ++k) osk[k][lj] = 0.0f;
                        if (!valid[lj]) {
                            S4[lj] = cis4[lj] = q[lj] = q0[lj] = ci[lj] = 0.0f;
                            continue;
                        }
                        const uint8_t b = td[lj * TILE + li];
                        const float ois = S->output_importance_scale ? S->output_importance_scale[col] : 1.0f;
                        float sc = 0.0f;
                        for (int k = 0; k < rank; ++k) sc += vs_k[k] * os[col * rank + k];
                        S4[lj] = sc;
                        cis4[lj] = imp_scale * ois;
                        q[lj] = q0[lj] = fp4_dec(b & 0xFu);
                        ci[lj] = fp4_dec(b >> 4) * cis4[lj];
                        for (int k = 0; k < rank; ++k) osk[k][lj] = os[col * rank + k];
                    }
                    double mr[4] = {0, 0, 0, 0}, mrc[4] = {0, 0, 0, 0};
                    float mc[4][4] = {}, mcc[4][4] = {};
                    for (int64_t b = 0; b < batch; ++b) {
                        const float iv = x[b * n_in + row];
                        float t_dx[4] = {0, 0, 0, 0}, t_r[4][4] = {}, t_rc[4][4] = {};
                        for (int lj = 0; lj < TILE; ++lj) {
                            if (!valid[lj]) continue;
                            const float dyv = dy[b * n_out + bc * TILE + lj];
                            const float g = dyv * iv;
                            const float contrib = q0[lj] * iv;
                            ci[lj] = bounded_update_ci(ci[lj], g, contrib, P->beta2, P->min_decay_frac, P->max_ci);
                            q[lj] += bounded_update_cw(g, ci[lj], S4[lj], effective_lr, P->eps, P->damp_by_importance != 0,
                                                       P->max_abs_delta);
                            const float qf = (q[lj] == 0.0f) ? P->zero_escape_eps : q[lj];
                            for (int k = 0; k < rank; ++k) {
                                if (full) {
                                    t_r[k][lj] = qf * osk[k][lj] * g;
                                    t_rc[k][lj] = qf * osk[k][lj] * contrib;
                                } else {
                                    mr[k] += static_cast<double>(qf) * static_cast<double>(osk[k][lj]) * g;
                                    mrc[k] += static_cast<double>(qf) * static_cast<double>(osk[k][lj]) * contrib;
                                }
                                mc[k][lj] += qf * vs_k[k] * g;
                                mcc[k][lj] += qf * vs_k[k] * contrib;
                            }
                            if (full) t_dx[lj] = (q[lj] * S4[lj]) * dyv;
                            else mdx[size_t(b * n_in + row)] += q[lj] * S4[lj] * dyv;
                        }
                        if (full) {
                            for (int k = 0; k < rank; ++k) {
                                mr[k] += static_cast<double>(((t_r[k][0] + t_r[k][1]) + t_r[k][2]) + t_r[k][3]);
                                mrc[k] += static_cast<double>(((t_rc[k][0] + t_rc[k][1]) + t_rc[k][2]) + t_rc[k][3]);
                            }
                            mdx[size_t(b * n_in + row)] += ((t_dx[0] + t_dx[1]) + t_dx[2]) + t_dx[3];
                        }
                    }
                    for (int k = 0; k < rank; ++k) {
                        mrow[size_t(row * rank + k)] += mr[k];
                        mrow_c[size_t(row * rank + k)] += mrc[k];
                    }
                    for (int lj = 0; lj < TILE; ++lj) {
                        if (!valid[lj]) continue;
                        const int64_t col = bc * TILE + lj;
                        for (int k = 0; k < rank; ++k) {
                            mcol[size_t(col * rank + k)] += mc[k][lj];
                            mcol_c[size_t(col * rank + k)] += mcc[k][lj];
                        }
                        td[lj * TILE + li] = uint8_t((fp4_enc(ci[lj] / cis4[lj]) << 4) | fp4_enc(q[lj]));
                    }
                }
            }
            // the tiles are rewritten through each block row's workspace:
            // re-encoded by live count, then written back with eviction
            // (linear_disldo.hpp:1839-1880)
            if (S->b4) {
                for (const auto &t : tl)
                    S->b4->tile_sparse[t.t] = b4_encode_flag(tiles + 16 * t.t, S->b4->switch_point);
                for (int64_t k0 = 0; k0 < int64_t(tl.size());) {
                    int64_t k1 = k0;
                    while (k1 < int64_t(tl.size()) && tl[size_t(k1)].br == tl[size_t(k0)].br) ++k1;
                    b4_merge_row(L, tiles, tl, k0, k1, S, S->b4);
                    k0 = k1;
                }
            }
            // the block rows' scale step (linear_disldo.hpp:1923-1951): every
            // scale variant, its own finiteness guards
            for (int64_t row = 0; row < n_in; ++row) {
                const uint32_t nnz_row = b4_live[size_t(row)];
                if (nnz_row == 0) continue;
                const float scale_eff_lr = lr / static_cast<float>(nnz_row);
                for (int k = 0; k < rank; ++k) {
                    const double sum = mrow[size_t(row * rank + k)], sum_c = mrow_c[size_t(row * rank + k)];
                    if (sum == 0.0 && sum_c == 0.0) continue;
                    const float g_agg = static_cast<float>(sum), contrib_agg = static_cast<float>(sum_c);
                    if (!std::isfinite(g_agg) || !std::isfinite(contrib_agg)) continue;
                    const int64_t idx = row * rank + k;
                    float &vs_imp = S->vs_importance[idx];
                    const float new_vs_imp = P->beta2 * vs_imp + (1.0f - P->beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
                    if (!std::isfinite(new_vs_imp)) continue;
                    uint32_t &step = S->vs_step[idx];
                    ++step;
                    const float bias_correction = 1.0f - std::pow(P->beta2, static_cast<float>(step));
                    const float vs_imp_hat = bias_correction > 0.0f ? new_vs_imp / bias_correction : new_vs_imp;
                    if (!std::isfinite(vs_imp_hat)) continue;
                    const float new_vs = vs[idx] - scale_eff_lr * g_agg / (std::sqrt(vs_imp_hat) + P->eps);
                    if (!std::isfinite(new_vs)) continue;
                    vs_imp = new_vs_imp;
                    vs[idx] = new_vs;
                }
            }
        }
    }
    // rows with no synapse: a two-moment step on value_scale from
    // g = x[row] * sum_col(os * dy)
    if (lr != 0.0f) {
        auto dead = [&](int64_t r) {
            return L->row_elem_start[r + 1] == L->row_elem_start[r] && b4_live[size_t(r)] == 0;
        };
        bool any_dead = false;
        for (int64_t r = 0; r < n_in && !any_dead; ++r) any_dead = dead(r);
        if (any_dead) {
            std::vector<double> dead_S(size_t(batch * rank), 0.0);
            for (int64_t b = 0; b < batch; ++b)
                for (int k = 0; k < rank; ++k) {
                    double s = 0.0;
                    for (int64_t c = 0; c < n_out; ++c)
                        s += static_cast<double>(os[c * rank + k]) * static_cast<double>(dy[b * n_out + c]);
                    dead_S[size_t(b * rank + k)] = s;
                }
            for (int64_t r = 0; r < n_in; ++r) {
                if (!dead(r)) continue;
                for (int k = 0; k < rank; ++k) {
                    double sum = 0.0;
                    for (int64_t b = 0; b < batch; ++b) {
                        const float iv = x[b * n_in + r];
                        if (iv == 0.0f) continue;
                        sum += static_cast<double>(iv) * dead_S[size_t(b * rank + k)];
                    }
                    if (sum == 0.0) continue;
                    const float g = static_cast<float>(sum);
                    if (!std::isfinite(g)) continue;
                    const int64_t i = r * rank + k;
                    float &m = S->vs_momentum[i];
                    float &v = S->vs_importance[i];
                    const float new_m = P->beta1 * m + (1.0f - P->beta1) * g;
                    const float new_v = P->beta2 * v + (1.0f - P->beta2) * g * g;
                    if (!std::isfinite(new_m) || !std::isfinite(new_v)) continue;
                    const float dead_lr = lr / static_cast<float>(n_out);
                    const float new_vs = vs[i] - dead_lr * new_m / (std::sqrt(new_v) + P->eps);
                    if (!std::isfinite(new_vs)) continue;
                    m = new_m;
                    v = new_v;
                    vs[i] = new_vs;
                }
            }
        }
    }
    for (size_t i = 0; i < mdx.size(); ++i) dx[i] += mdx[i];
    if (lr != 0.0f && S->output_scale_trainable && !no_scale) {
        for (int64_t c = 0; c < n_out; ++c) {
            const int32_t deg = S->out_degree ? S->out_degree[c] : 0;
            if (deg == 0) continue;
            const float col_eff_lr = lr / static_cast<float>(deg);
            for (int k = 0; k < rank; ++k) {
                const int64_t i = c * rank + k;
                const double sum = 0.0 + static_cast<double>(mcol[size_t(i)]);
                const double sum_c = 0.0 + static_cast<double>(mcol_c[size_t(i)]);
                rmsprop_scale_update(os[i], S->os_importance[i], static_cast<float>(sum), col_eff_lr, P->beta2,
                                     P->eps, static_cast<float>(sum_c), S->os_step[i]);
            }
        }
    }
    // DeferredScaleWrite replay under the final scales (linear_disldo.hpp:2090-2112)
    if (deferred && lr != 0.0f) {
        for (int64_t r = 0; r < n_in; ++r) {
            const float fis = S->importance_scale ? S->importance_scale[r] : 1.0f;
            for (uint64_t vb = L->row_elem_start[r]; vb < L->row_elem_start[r + 1]; ++vb) {
                const uint32_t col = def_col[vb];
                const float fois = S->output_importance_scale ? S->output_importance_scale[col] : 1.0f;
                const float final_combined_scale = vs[r * rank] * os[int64_t(col) * rank];
                const float final_combined_imp_scale = fis * fois;
                const float w = def_w[vb] / final_combined_scale;
                const float imp = def_i[vb] / final_combined_imp_scale;
                if (S->quant_out) S->quant_out[vb] = w;
                if (S->imp_out) S->imp_out[vb] = imp;
                val[vb] = uint8_t((fp4_enc(w) << 4) | fp4_enc(imp));
            }
        }
    }
    return 0;
}

}  // extern "C"

namespace {

// The stochastic FP4 encoder with its draw supplied (fp4quant.hpp:238-265):
// top 24 bits -> uniform [0,1) below 1.0, low 22 bits -> dither above.
uint32_t fp4_enc_stoch(float v, uint64_t r) {
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    const uint32_t sign = bits & 0x80000000u, abits = bits & 0x7FFFFFFFu;
    if (abits > 0x7F800000u) return 0u;
    uint32_t mag;
    if (abits >= 0x40C00000u) {
        mag = 7u;
    } else if (abits < 0x3F800000u) {
        float av;
        std::memcpy(&av, &abits, 4);
        const float u01 = static_cast<float>((r >> 40) * (1.0 / 16777216.0));
        if (abits < 0x3F000000u) mag = (u01 < av * 2.0f) ? 1u : 0u;
        else mag = (u01 < av * 2.0f - 1.0f) ? 2u : 1u;
    } else {
        uint32_t rounded = abits + uint32_t(r & 0x3FFFFFu);
        if (rounded > 0x40C00000u) rounded = 0x40C00000u;
        mag = ((((rounded >> 23) & 0xFFu) - 126u) << 1) | ((rounded >> 22) & 1u);
    }
    if (mag == 0u) return 0u;
    return (sign ? 8u : 0u) | mag;
}

uint64_t splitmix64_o(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Draw source of the block4 sparse-gradient update (OracleTrainParams.draw_mode).
struct Draws {
    int mode;
    uint64_t seed, xs;
    explicit Draws(const OracleTrainParams *P)
        : mode(P->draw_mode), seed(P->draw_seed), xs((P->draw_seed ^ 0x9E3779B97F4A7C15ULL) | 1ULL) {}
    uint32_t enc(float v, uint64_t id) {
        if (mode == 1) return fp4_enc_stoch(v, splitmix64_o(seed + id));
        uint32_t bits;
        std::memcpy(&bits, &v, 4);
        const uint32_t a = bits & 0x7FFFFFFFu;
        if (a > 0x7F800000u || a >= 0x40C00000u) return fp4_enc_stoch(v, 0);  // no draw taken
        xs ^= xs >> 12;  // xorshift64* (fp4quant.hpp:196-200)
        xs ^= xs << 25;
        xs ^= xs >> 27;
        return fp4_enc_stoch(v, xs * 0x2545F4914F6CDD1DULL);
    }
};

// The block4 section of disldo_backward_sparse_grad (sisldo_ops.hpp:848-1100).
int sparse_train_b4(const OracleLayer *L, uint8_t *tiles, OracleTrainState *S, const float *x,
                    const int32_t *dptrs, const int32_t *didx, const float *dvals, int64_t batch, float *dx,
                    const OracleTrainParams *P) {
    if (L->n_tiles <= 0) return 0;
    if (!tiles) return -1;
    const int64_t n_in = L->n_in, n_out = L->n_out;
    const int rank = L->rank;
    const float lr = P->lr, beta2 = P->beta2, eps = P->eps;
    float *vs = S->value_scale;
    const float *os = S->output_scale;
    const auto tl = collect_tiles(L);
    const int64_t brows = (n_in + TILE - 1) / TILE;
    std::vector<int64_t> tb(size_t(brows) + 1, 0);
    for (const auto &t : tl) tb[size_t(t.br) + 1]++;
    for (int64_t i = 0; i < brows; ++i) tb[size_t(i) + 1] += tb[size_t(i)];
    std::vector<double> rs(size_t(n_in), 0.0), rsc(size_t(n_in), 0.0);
    std::vector<float> dyrow(static_cast<size_t>(n_out), 0.0f);
    Draws dr(P);
    for (int64_t b = 0; b < batch; ++b) {
        std::fill(dyrow.begin(), dyrow.end(), 0.0f);
        for (int32_t j = dptrs[b]; j < dptrs[b + 1]; ++j) dyrow[size_t(didx[j])] = dvals[j];
        for (int64_t br = 0; br < brows; ++br) {
            const int64_t ntl = tb[size_t(br) + 1] - tb[size_t(br)];
            if (ntl == 0) continue;
            const float nnz_row = static_cast<float>(ntl * TILE);
            float dx_acc[TILE] = {0, 0, 0, 0};
            double rg[TILE] = {0, 0, 0, 0}, rgc[TILE] = {0, 0, 0, 0};
            for (int64_t k = tb[size_t(br)]; k < tb[size_t(br) + 1]; ++k) {
                uint8_t *td = tiles + 16 * tl[size_t(k)].t;
                const int64_t bc = tl[size_t(k)].bc;
                bool dirty = false;
                for (int li = 0; li < TILE; ++li) {
                    const int64_t row = br * TILE + li;
                    if (row >= n_in) continue;
                    const float in_val = x[b * n_in + row];
                    const float val_scale = vs[row * rank];
                    const float imp_scale = S->importance_scale ? S->importance_scale[row] : 1.0f;
                    const float effective_lr = P->lr_per_row_nnz ? lr / nnz_row : lr;
                    for (int lj = 0; lj < TILE; ++lj) {
                        const int64_t col = bc * TILE + lj;
                        if (col >= n_out) continue;
                        const float dy_val = dyrow[size_t(col)];
                        if (dy_val == 0.0f) continue;
                        const uint8_t byte = td[lj * TILE + li];
                        const float w_decoded = fp4_dec(byte & 0xFu);
                        const float out_scale = os[col * rank];
                        const float combined_scale = val_scale * out_scale;
                        const float w = w_decoded * combined_scale;
                        dx_acc[li] += w * dy_val;
                        if (lr == 0.0f) continue;
                        const float ois = S->output_importance_scale ? S->output_importance_scale[col] : 1.0f;
                        const float combined_imp_scale = imp_scale * ois;
                        const float grad = dy_val * in_val;
                        float imp = fp4_dec(byte >> 4) * combined_imp_scale;
                        const float contrib = in_val * w;
                        imp = beta2 * imp + (1.0f - beta2) * (grad * grad + contrib * contrib);
                        const float new_w = w + (P->damp_by_importance ? (-effective_lr * grad) / (std::sqrt(imp) + eps)
                                                                       : (-effective_lr * grad));
                        const uint64_t id = 2ull * ((uint64_t(b) * uint64_t(L->n_tiles) + uint64_t(k)) * 16ull +
                                                    uint64_t(lj * TILE + li));
                        const uint32_t wq = dr.enc(new_w / combined_scale, id);
                        const uint32_t iq = dr.enc(imp / combined_imp_scale, id + 1);
                        td[lj * TILE + li] = uint8_t((iq << 4) | wq);
                        dirty = true;
                        rg[li] += static_cast<double>(w_decoded) * static_cast<double>(out_scale) * (dy_val * in_val);
                        rgc[li] += static_cast<double>(w_decoded) * static_cast<double>(out_scale) *
                                   static_cast<double>(contrib);
                    }
                }
                // a rewritten tile is re-encoded by its live count
                // (commit_dirty_tile_in_workspace, sisldo_ops.hpp:1032-1034)
                if (dirty && S->b4) S->b4->tile_sparse[tl[size_t(k)].t] = b4_encode_flag(td, S->b4->switch_point);
            }
            // the block row's workspace written back (sisldo_ops.hpp:1036-1052)
            if (lr != 0.0f && S->b4) b4_merge_row(L, tiles, tl, tb[size_t(br)], tb[size_t(br) + 1], S, S->b4);
            for (int li = 0; li < TILE; ++li) {
                const int64_t row = br * TILE + li;
                if (row >= n_in) continue;
                dx[b * n_in + row] += dx_acc[li];
                rs[size_t(row)] += rg[li];
                rsc[size_t(row)] += rgc[li];
            }
        }
    }
    if (lr == 0.0f) return 0;
    for (int64_t row = 0; row < n_in; ++row) {
        if (rs[size_t(row)] == 0.0 && rsc[size_t(row)] == 0.0) continue;
        const int64_t br = row / TILE;
        const int64_t nnz_row = (tb[size_t(br) + 1] - tb[size_t(br)]) * TILE;
        if (nnz_row == 0) continue;
        const float scale_eff_lr = lr / static_cast<float>(nnz_row);
        const float g_agg = static_cast<float>(rs[size_t(row)]);
        const float contrib_agg = static_cast<float>(rsc[size_t(row)]);
        float &vs_imp = S->vs_importance[row];
        const float new_vs_imp = beta2 * vs_imp + (1.0f - beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
        uint32_t &step = S->vs_step[row * rank];
        ++step;
        const float bias_correction = 1.0f - std::pow(beta2, static_cast<float>(step));
        const float vs_imp_hat = bias_correction > 0.0f ? new_vs_imp / bias_correction : new_vs_imp;
        vs_imp = new_vs_imp;
        vs[row] -= scale_eff_lr * g_agg / (std::sqrt(vs_imp_hat) + eps);
    }
    return 0;
}

}  // namespace

extern "C" {

// sisldo_ops.hpp:613-1100 (disldo_backward_sparse_grad): the scattered
// section, then the block4 section.
int oracle_backward_sparse_train(const OracleLayer *L, uint8_t *val, uint8_t *tiles, OracleTrainState *S, const float *x,
                                 const int32_t *dptrs, const int32_t *didx, const float *dvals, int64_t batch,
                                 float *dx, float *acc_in, float *acc_grad, const OracleTrainParams *P) {
    if (L->n_tiles > 0 && !tiles) return -1;
    const int64_t n_in = L->n_in;
    const int rank = L->rank;
    const float lr = P->lr, beta2 = P->beta2, eps = P->eps;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t r = 0; r < n_in; ++r) acc_in[r] += std::fabs(x[b * n_in + r]);
    for (int64_t b = 0; b < batch; ++b)
        for (int32_t j = dptrs[b]; j < dptrs[b + 1]; ++j) acc_grad[didx[j]] += std::fabs(dvals[j]);
    if (L->row_elem_start[n_in] == 0) return sparse_train_b4(L, tiles, S, x, dptrs, didx, dvals, batch, dx, P);
    float *vs = S->value_scale;
    const float *os = S->output_scale;
    std::vector<double> sg(size_t(n_in), 0.0), sgc(size_t(n_in), 0.0);
    for (int64_t b = 0; b < batch; ++b) {
        const int32_t og_start = dptrs[b], og_end = dptrs[b + 1];
        for (int64_t r = 0; r < n_in; ++r) {
            const uint64_t e0 = L->row_elem_start[r], e1 = L->row_elem_start[r + 1];
            if (e1 == e0) continue;
            const float in_val = x[b * n_in + r];
            const float effective_lr = P->lr_per_row_nnz ? lr / static_cast<float>(e1 - e0) : lr;
            int32_t og = og_start;
            float dx_accum = 0.0f;
            const float imp_scale = S->importance_scale ? S->importance_scale[r] : 1.0f;
            const float val_scale = vs[r * rank];
            uint64_t pos = L->row_byte_start[r];
            uint32_t col = 0;
            for (uint64_t vb = e0; vb < e1; ++vb) {
                col += uleb_dec(L->idx, pos);
                const float w_stored = fp4_dec(val[vb] >> 4);
                const float out_scale = os[int64_t(col) * rank];
                const float combined_scale = val_scale * out_scale;
                const float w = w_stored * combined_scale;
                // merge with the batch row's sorted gradient columns
                while (og < og_end && didx[og] < static_cast<int32_t>(col)) ++og;
                if (og >= og_end || didx[og] != static_cast<int32_t>(col)) continue;
                const float dy_val = dvals[og];
                dx_accum += w * dy_val;
                if (lr != 0.0f) {
                    const float out_imp_scale =
                        S->output_importance_scale ? S->output_importance_scale[col] : 1.0f;
                    const float combined_imp_scale = imp_scale * out_imp_scale;
                    const float grad = dy_val * in_val;
                    const float stored_imp = fp4_dec(val[vb] & 0xFu);
                    float imp = stored_imp * combined_imp_scale;
                    const float contrib = in_val * w;
                    imp = beta2 * imp + (1.0f - beta2) * (grad * grad + contrib * contrib);
                    const float new_w = w + (P->damp_by_importance ? (-effective_lr * grad) / (std::sqrt(imp) + eps)
                                                                   : (-effective_lr * grad));
                    val[vb] = uint8_t((fp4_enc(new_w / combined_scale) << 4) | fp4_enc(imp / combined_imp_scale));
                    sg[size_t(r)] += static_cast<double>(w_stored) * static_cast<double>(out_scale) * (dy_val * in_val);
                    sgc[size_t(r)] += static_cast<double>(w_stored) * static_cast<double>(out_scale) *
                                      static_cast<double>(contrib);
                }
            }
            dx[b * n_in + r] += dx_accum;
        }
    }
    if (lr != 0.0f) {
        // value_scale[r] and its second moment by the row index, the step
        // counter by (r, 0) (sisldo_ops.hpp:820-846)
        for (int64_t r = 0; r < n_in; ++r) {
            if (sg[size_t(r)] == 0.0 && sgc[size_t(r)] == 0.0) continue;
            const uint64_t nnz_row = L->row_elem_start[r + 1] - L->row_elem_start[r];
            if (nnz_row == 0) continue;
            const float scale_eff_lr = lr / static_cast<float>(nnz_row);
            const float g_agg = static_cast<float>(sg[size_t(r)]);
            const float contrib_agg = static_cast<float>(sgc[size_t(r)]);
            float &vs_imp = S->vs_importance[r];
            const float new_vs_imp = beta2 * vs_imp + (1.0f - beta2) * (g_agg * g_agg + contrib_agg * contrib_agg);
            uint32_t &step = S->vs_step[r * rank];
            ++step;
            const float bias_correction = 1.0f - std::pow(beta2, static_cast<float>(step));
            const float vs_imp_hat = bias_correction > 0.0f ? new_vs_imp / bias_correction : new_vs_imp;
            vs_imp = new_vs_imp;
            vs[r] -= scale_eff_lr * g_agg / (std::sqrt(vs_imp_hat) + eps);
        }
    }
    return sparse_train_b4(L, tiles, S, x, dptrs, didx, dvals, batch, dx, P);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// The reference's synaptogenesis policy: delta_csr_build_probes
// (delta_csr_memory.hpp:1309-1426) and delta_csr_synap_row_step
// (delta_csr_memory.hpp:1021-1264), restated on a mutable host copy of the
// layer with the reference's sequential edit semantics: removals in
// descending column order, a block4 slot removal demoting its tile at once
// when fewer than 2 slots stay live (a later removal aimed at a slot that
// demotion already moved to the scattered store then finds no tile and does
// nothing), inserts one at a time, each followed by the promotion check.
// The orderings use the same std::sort / std::partial_sort calls with the
// same comparators and input order as the reference (tie order included).
namespace {

inline uint64_t uleb_size(uint32_t v) {
    uint64_t n = 1;
    while (v >= 0x80u) {
        v >>= 7;
        ++n;
    }
    return n;
}

struct MutLayer {
    int64_t n_in = 0, n_out = 0;
    std::vector<std::vector<std::pair<uint32_t, uint8_t>>> rows;  // per row, by column: (col, (w<<4)|imp)
    std::map<std::pair<uint32_t, uint32_t>, std::array<uint8_t, 16>> tiles;  // (br, bc) -> slot lj*4+li, (imp<<4)|w
    // per-row reservations of the scattered store (index bytes, elements):
    // the room delta_csr_row_insert_col checks; NULL: unlimited
    const uint64_t *res_b = nullptr, *res_e = nullptr;
    // the block4 store's reservations and tile encoding (NULL: not kept)
    OracleB4Res *b4 = nullptr;
    std::map<std::pair<uint32_t, uint32_t>, uint8_t> flags;  // tile_is_sparse
};

// ---- the block4 store's reservations (block4.hpp:497-946) -------------------
uint64_t b4_total(const uint64_t *v, size_t n) {
    uint64_t s = 0;
    for (size_t i = 0; i < n; ++i) s += v[i];
    return s;
}
struct B4Budget {};  // thrown when a row's growth exceeds a budget

// block row br's use: block-column ULEB128 bytes, tiles, stored tile bytes
void b4_use(const MutLayer &M, uint32_t br, uint64_t &ui, uint64_t &ue, uint64_t &ut) {
    ui = ue = ut = 0;
    uint32_t prev = 0;
    for (auto it = M.tiles.lower_bound({br, 0u}); it != M.tiles.end() && it->first.first == br; ++it) {
        ui += uleb_size(it->first.second - prev);
        prev = it->first.second;
        ++ue;
        ut += b4_tile_len(it->second.data(), M.flags.at(it->first) != 0);
    }
}

// block4_row_shift (block4.hpp:497-617) / block4_grow_last_row (:619-646)
// towards targets (ti, tt, te) for block row br, clamped to its use
void b4_shift(OracleB4Res *R, size_t rows, size_t br, uint64_t ti, uint64_t tt, uint64_t te, uint64_t ui,
              uint64_t ue, uint64_t ut, bool last_row_grows) {
    if (br + 1 >= rows) {
        if (!last_row_grows) return;
        if (ti > R->ia[br]) {
            if (b4_total(R->ia, rows) + (ti - R->ia[br]) > R->idx_budget) throw B4Budget{};
            R->ia[br] = ti;
        }
        if (tt > R->ta[br]) {
            if (b4_total(R->ta, rows) + (tt - R->ta[br]) > R->tile_budget) throw B4Budget{};
            R->ta[br] = tt;
        }
        if (te > R->ea[br]) R->ea[br] = te;
        return;
    }
    ti = std::max(ti, ui);
    tt = std::max(tt, ut);
    te = std::max(te, ue);
    if (R->ia[br] != ti) {
        if (ti > R->ia[br] && b4_total(R->ia, rows) + (ti - R->ia[br]) > R->idx_budget) throw B4Budget{};
        R->ia[br] = ti;
    }
    if (R->ta[br] != tt) {
        if (tt > R->ta[br] && b4_total(R->ta, rows) + (tt - R->ta[br]) > R->tile_budget) throw B4Budget{};
        R->ta[br] = tt;
    }
    if (R->ea[br] != te) R->ea[br] = te;
}

// block4_row_insert_tile's room check and get_or_create's growth
// (block4.hpp:670-771,1170-1183) for a new tile (br, bc); throws B4Budget
void b4_insert_tile(MutLayer &M, uint32_t br, uint32_t bc) {
    OracleB4Res *R = M.b4;
    const size_t rows = size_t((M.n_in + TILE - 1) / TILE);
    uint64_t ui, ue, ut;
    b4_use(M, br, ui, ue, ut);
    auto nx = M.tiles.upper_bound({br, bc});
    uint32_t prev = 0;
    if (nx != M.tiles.begin() && std::prev(nx)->first.first == br) prev = std::prev(nx)->first.second;
    int64_t d = int64_t(uleb_size(bc - prev));
    if (nx != M.tiles.end() && nx->first.first == br)
        d += int64_t(uleb_size(nx->first.second - bc)) - int64_t(uleb_size(nx->first.second - prev));
    const bool fits = !(d > 0 && uint64_t(d) > R->ia[br] - ui) && ue < R->ea[br] && 1 <= R->ta[br] - ut;
    if (fits) return;
    b4_shift(R, rows, br, R->ia[br] + 5, R->ta[br] + 1, R->ea[br] + 1, ui, ue, ut, true);
}

// a sparse tile's handle commit (commit_dirty_sparse_tile, block4.hpp:
// 1226-1290): the tile re-encoded by live count; growth beyond the row's room
// takes the shortfall, beyond the tile budget the commit is dropped
bool b4_commit(MutLayer &M, uint32_t br, uint32_t bc, const std::array<uint8_t, 16> &nt) {
    OracleB4Res *R = M.b4;
    const size_t rows = size_t((M.n_in + TILE - 1) / TILE);
    auto &cur = M.tiles[{br, bc}];
    uint8_t &fl = M.flags[{br, bc}];
    const uint64_t old_len = b4_tile_len(cur.data(), fl != 0);
    const uint8_t nfl = b4_encode_flag(nt.data(), R->switch_point);
    const uint64_t new_len = b4_tile_len(nt.data(), nfl != 0);
    if (new_len > old_len) {
        uint64_t ui, ue, ut;
        b4_use(M, br, ui, ue, ut);
        const uint64_t d = new_len - old_len, room = R->ta[br] - ut;
        if (d > room) {
            const uint64_t shortfall = d - room;
            if (b4_total(R->ta, rows) + shortfall > R->tile_budget) {
                ++R->dropped;
                return false;
            }
            R->ta[br] += shortfall;
        }
    }
    cur = nt;
    fl = nfl;
    return true;
}

// a slot written through a handle: in place in a dense tile, a commit of a
// sparse one
void b4_write_slot(MutLayer &M, uint32_t br, uint32_t bc, uint32_t slot, uint8_t byte) {
    auto &t = M.tiles[{br, bc}];
    if (!M.b4 || M.flags.at({br, bc}) == 0) {
        t[slot] = byte;
        return;
    }
    std::array<uint8_t, 16> nt = t;
    nt[slot] = byte;
    b4_commit(M, br, bc, nt);
}

uint64_t row_index_bytes(const std::vector<std::pair<uint32_t, uint8_t>> &row) {
    uint64_t b = 0;
    uint32_t prev = 0;
    for (const auto &e : row) {
        b += uleb_size(e.first - prev);
        prev = e.first;
    }
    return b;
}

MutLayer load_mut(const OracleLayer *L) {
    MutLayer M;
    M.n_in = L->n_in;
    M.n_out = L->n_out;
    M.rows.resize(size_t(L->n_in));
    for (int64_t r = 0; r < L->n_in; ++r) {
        uint64_t pos = L->row_byte_start[r];
        uint32_t col = 0;
        for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
            col += uleb_dec(L->idx, pos);
            M.rows[size_t(r)].push_back({col, L->val[e]});
        }
    }
    for (const auto &t : collect_tiles(L)) {
        std::array<uint8_t, 16> d;
        std::memcpy(d.data(), L->tiles + 16 * t.t, 16);
        M.tiles[{uint32_t(t.br), uint32_t(t.bc)}] = d;
    }
    return M;
}

// ValueAccessor<FP4BiPacked>::set (fp4quant.hpp:280-467): round to nearest.
inline uint8_t scat_byte(float w, float imp) { return uint8_t((fp4_enc(w) << 4) | fp4_enc(imp)); }

// delta_csr_row_insert_col (delta_csr_memory.hpp:498-585): false when the
// column is already stored, or when the new delta (and the re-encoded next
// one) would exceed the row's reserved bytes, or the row its reserved
// elements -- the reference's unsigned arithmetic included.
bool mut_insert(MutLayer &M, uint32_t r, uint32_t c, float w, float imp) {
    auto &row = M.rows[r];
    auto it = std::lower_bound(row.begin(), row.end(), std::make_pair(c, uint8_t(0)));
    if (it != row.end() && it->first == c) return false;
    if (M.res_b) {
        const uint32_t prev = it == row.begin() ? 0u : (it - 1)->first;
        uint64_t grow = uleb_size(c - prev), shrink = 0;
        if (it != row.end()) {
            grow += uleb_size(it->first - c);
            shrink = uleb_size(it->first - prev);
        }
        const int64_t idx_delta = int64_t(grow) - int64_t(shrink);
        const uint64_t used = row_index_bytes(row);
        if (idx_delta > 0 && uint64_t(idx_delta) > M.res_b[r] - used) return false;
        if (uint64_t(row.size()) >= M.res_e[r]) return false;
    }
    row.insert(it, {c, scat_byte(w, imp)});
    return true;
}

bool mut_remove(MutLayer &M, uint32_t r, uint32_t c) {
    auto &row = M.rows[r];
    auto it = std::lower_bound(row.begin(), row.end(), std::make_pair(c, uint8_t(0)));
    if (it == row.end() || it->first != c) return false;
    row.erase(it);
    return true;
}

// block4_demote_tile (delta_csr_memory.hpp:949-999).  Returns the row whose
// insert failed (the reference throws there), or -1.
int64_t mut_demote(MutLayer &M, uint32_t br, uint32_t bc) {
    auto it = M.tiles.find({br, bc});
    if (it == M.tiles.end()) return -1;
    const auto d = it->second;
    for (uint32_t li = 0; li < TILE; ++li) {
        const uint32_t r = br * TILE + li;
        if (int64_t(r) >= M.n_in) continue;
        for (uint32_t lj = 0; lj < TILE; ++lj) {
            const uint8_t b = d[lj * TILE + li];
            if (b == 0) continue;
            const uint32_t c = bc * TILE + lj;
            if (int64_t(c) >= M.n_out) continue;
            if (!mut_insert(M, r, c, fp4_dec(b & 0xFu), fp4_dec(b >> 4))) return int64_t(r);
        }
    }
    M.flags.erase(it->first);
    M.tiles.erase(it);
    return -1;
}

// block4_maybe_promote (delta_csr_memory.hpp:591-702).
void mut_maybe_promote(MutLayer &M, uint32_t row, uint32_t col) {
    const uint32_t br = row / TILE, bc = col / TILE, li = row % TILE, lj = col % TILE;
    auto tit = M.tiles.find({br, bc});
    if (tit != M.tiles.end()) {
        auto &rw = M.rows[row];
        auto it = std::lower_bound(rw.begin(), rw.end(), std::make_pair(col, uint8_t(0)));
        if (it == rw.end() || it->first != col) return;
        const float w = fp4_dec(it->second >> 4), imp = fp4_dec(it->second & 0xFu);
        b4_write_slot(M, br, bc, lj * TILE + li, uint8_t(fp4_enc(w) | (fp4_enc(imp) << 4)));
        if (M.b4) {  // maybe_compress (block4.hpp:1193-1205)
            uint8_t &fl = M.flags[{br, bc}];
            if (fl == 0 && b4_encode_flag(tit->second.data(), M.b4->switch_point)) fl = 1;
        }
        rw.erase(it);
        return;
    }
    const int64_t row_lo = int64_t(br) * TILE, row_hi = std::min<int64_t>(row_lo + TILE, M.n_in);
    const int64_t col_lo = int64_t(bc) * TILE, col_hi = std::min<int64_t>(col_lo + TILE, M.n_out);
    struct Found { uint32_t r, c; uint8_t b; };
    std::vector<Found> found;
    for (int64_t r = row_lo; r < row_hi; ++r)
        for (const auto &e : M.rows[size_t(r)])
            if (int64_t(e.first) >= col_lo && int64_t(e.first) < col_hi) found.push_back({uint32_t(r), e.first, e.second});
    if (found.size() < size_t(PROMOTE_MIN_LIVE)) return;
    std::array<uint8_t, 16> d{};
    for (const auto &f : found) {
        const float w = fp4_dec(f.b >> 4), imp = fp4_dec(f.b & 0xFu);
        d[(f.c - uint32_t(col_lo)) * TILE + (f.r - uint32_t(row_lo))] = uint8_t(fp4_enc(w) | (fp4_enc(imp) << 4));
    }
    if (M.b4) {
        // get_or_create: a sparse-empty tile (may throw B4Budget), then the
        // handle's commit of its slots
        b4_insert_tile(M, br, bc);
        M.tiles[{br, bc}] = std::array<uint8_t, 16>{};
        M.flags[{br, bc}] = 1;
        b4_commit(M, br, bc, d);
    } else {
        M.tiles[{br, bc}] = d;
    }
    for (const auto &f : found) mut_remove(M, f.r, f.c);
}

int64_t mut_store(const MutLayer &M, int32_t *out_ptrs, int32_t *out_cols, uint8_t *out_bytes, int32_t *out_br,
                  int32_t *out_bc, uint8_t *out_tiles) {
    int64_t flat = 0;
    out_ptrs[0] = 0;
    for (int64_t r = 0; r < M.n_in; ++r) {
        for (const auto &e : M.rows[size_t(r)]) {
            out_cols[flat] = int32_t(e.first);
            out_bytes[flat] = e.second;
            ++flat;
        }
        out_ptrs[r + 1] = int32_t(flat);
    }
    int64_t k = 0;
    for (const auto &t : M.tiles) {
        out_br[k] = int32_t(t.first.first);
        out_bc[k] = int32_t(t.first.second);
        std::memcpy(out_tiles + 16 * k, t.second.data(), 16);
        ++k;
    }
    return k;
}

}  // namespace

extern "C" {

// delta_csr_build_probes (delta_csr_memory.hpp:1309-1426): the probe list in
// the reference's order.  Returns the number of probes written (<= cap), or
// -1 when k <= 0 or the layer is empty (the reference then zeroes the probe
// count and keeps its old index vectors).
int64_t oracle_build_probes(const OracleLayer *L, const float *acc_in, const float *acc_grad, int64_t k,
                            int per_row, int32_t *prow, int32_t *pcol, float *pval, int64_t cap) {
    const size_t n_in = size_t(L->n_in), n_out = size_t(L->n_out);
    if (n_in == 0 || n_out == 0 || k <= 0) return -1;
    const size_t kk_in = std::min(size_t(k), n_in), kk = size_t(k);
    std::vector<size_t> in_idx(n_in);
    std::iota(in_idx.begin(), in_idx.end(), 0);
    std::partial_sort(in_idx.begin(), in_idx.begin() + kk_in, in_idx.end(),
                      [&](size_t a, size_t b) { return acc_in[a] > acc_in[b]; });
    in_idx.resize(kk_in);
    int64_t n = 0;
    auto emit = [&](size_t r, size_t c) {
        if (n < cap) {
            prow[n] = int32_t(r);
            pcol[n] = int32_t(c);
            pval[n] = acc_in[r] * acc_grad[c];
        }
        ++n;
    };
    auto row_cols = [&](size_t r) {
        std::vector<uint32_t> cols;
        uint64_t pos = L->row_byte_start[r];
        uint32_t col = 0;
        for (uint64_t e = L->row_elem_start[r]; e < L->row_elem_start[r + 1]; ++e) {
            col += uleb_dec(L->idx, pos);
            cols.push_back(col);
        }
        return cols;
    };
    if (!per_row) {
        const size_t kk_out = std::min(kk, n_out);
        std::vector<size_t> out_idx(n_out);
        std::iota(out_idx.begin(), out_idx.end(), 0);
        std::partial_sort(out_idx.begin(), out_idx.begin() + kk_out, out_idx.end(),
                          [&](size_t a, size_t b) { return acc_grad[a] > acc_grad[b]; });
        out_idx.resize(kk_out);
        for (size_t r : in_idx) {
            const auto ex = row_cols(r);
            for (size_t c : out_idx)
                if (!std::binary_search(ex.begin(), ex.end(), uint32_t(c))) emit(r, c);
        }
    } else {
        for (size_t r : in_idx) {
            const auto ex = row_cols(r);
            std::vector<size_t> cand;
            for (size_t c = 0; c < n_out; ++c)
                if (!std::binary_search(ex.begin(), ex.end(), uint32_t(c))) cand.push_back(c);
            const size_t kk_row = std::min(kk, cand.size());
            if (kk_row == 0) continue;
            std::partial_sort(cand.begin(), cand.begin() + kk_row, cand.end(),
                              [&](size_t a, size_t b) { return acc_grad[a] > acc_grad[b]; });
            for (size_t i = 0; i < kk_row; ++i) emit(r, cand[i]);
        }
    }
    return n;
}

// delta_csr_synap_row_step on row `row` (already reduced modulo n_in; the
// caller advances its cursor).  probes: the layer's probe list (pnnz entries
// read; has_probes: its index vectors are non-empty).  out_degree [n_out] is
// updated as the reference updates it.  The new structure goes to the out_*
// arrays (capacities: scattered <= nnz + n_probes + 16 * n_tiles, tiles <=
// n_tiles + n_probes); *n_tiles_out receives the tile count.  Returns 1 when
// the reference returns true, 0 when false.
// res_b / res_e [n_in] (may be NULL: unlimited): the rows' reserved index
// bytes and elements.  An insert that does not fit ends the call as the
// reference's throw does (delta_csr_memory.hpp:1236-1250): returns -2, the
// removals and the inserts before it applied, fail[0..4] = probe index,
// column, the row's used bytes, its reserved bytes, insertions skipped.  A
// demotion that does not fit (block4_demote_tile's throw, :983-991) returns
// -3 with the layer as before the call and fail[0..2] = row, br, bc (the
// reference leaves that tile half demoted).
int oracle_synap_row_step2(const OracleLayer *L, int64_t row, const int32_t *prow, const int32_t *pcol,
                           const float *pval, int64_t pnnz, int has_probes, float importance_cutoff,
                           int64_t max_row_weights, int64_t max_prune_per_step, float importance_eps,
                           int32_t *out_degree, int32_t *out_ptrs, int32_t *out_cols, uint8_t *out_bytes,
                           int32_t *out_br, int32_t *out_bc, uint8_t *out_tiles, int64_t *n_tiles_out,
                           const uint64_t *res_b, const uint64_t *res_e, int64_t *fail, OracleB4Res *b4) {
    MutLayer M = load_mut(L);
    M.res_b = res_b;
    M.res_e = res_b ? res_e : nullptr;
    M.b4 = b4;
    if (b4) {
        int64_t k = 0;
        for (const auto &t : M.tiles) M.flags[t.first] = b4->flags_in[k++];
    }
    const MutLayer M0 = M;
    std::vector<int32_t> deg0(out_degree, out_degree + L->n_out);
    const size_t rows4 = size_t((L->n_in + TILE - 1) / TILE);
    std::vector<uint64_t> ia0, ea0, ta0;
    const uint64_t dropped0 = b4 ? b4->dropped : 0;
    if (b4) {
        ia0.assign(b4->ia, b4->ia + rows4);
        ea0.assign(b4->ea, b4->ea + rows4);
        ta0.assign(b4->ta, b4->ta + rows4);
    }
    auto finish = [&](int ret) {
        *n_tiles_out = mut_store(M, out_ptrs, out_cols, out_bytes, out_br, out_bc, out_tiles);
        if (b4) {
            int64_t k = 0;
            for (const auto &t : M.tiles) b4->flags_out[k++] = M.flags.at(t.first);
        }
        return ret;
    };
    if (M.n_in == 0) return finish(0);
    const uint32_t r = uint32_t(row), br = r / TILE, li = r % TILE;
    const size_t n_scattered = M.rows[r].size();
    std::vector<uint32_t> b4_bc, b4_lj;
    for (const auto &t : M.tiles) {
        if (t.first.first != br) continue;
        for (uint32_t lj = 0; lj < TILE; ++lj) {
            if (t.second[lj * TILE + li] == 0) continue;
            const uint32_t col = t.first.second * TILE + lj;
            if (int64_t(col) >= M.n_out) continue;
            b4_bc.push_back(t.first.second);
            b4_lj.push_back(lj);
        }
    }
    const size_t n_exist = n_scattered + b4_bc.size();
    if (n_exist == 0 && !has_probes) return finish(0);
    std::vector<uint32_t> exist_cols(n_exist);
    std::vector<float> exist_imp(n_exist);
    std::vector<bool> exist_is_b4(n_exist, false);
    for (size_t k = 0; k < n_scattered; ++k) {
        exist_cols[k] = M.rows[r][k].first;
        exist_imp[k] = fp4_dec(M.rows[r][k].second & 0xFu);
    }
    for (size_t j = 0; j < b4_bc.size(); ++j) {
        const size_t k = n_scattered + j;
        const uint8_t b = M.tiles[{br, b4_bc[j]}][b4_lj[j] * TILE + li];
        exist_cols[k] = b4_bc[j] * TILE + b4_lj[j];
        exist_imp[k] = fp4_dec(b >> 4);
        exist_is_b4[k] = true;
    }
    std::vector<uint32_t> probe_cols;
    std::vector<float> probe_scores;
    for (int64_t p = 0; p < pnnz; ++p)
        if (int64_t(prow[p]) == int64_t(r)) {
            probe_cols.push_back(uint32_t(pcol[p]));
            probe_scores.push_back(pval[p]);
        }
    std::vector<size_t> by_imp(n_exist);
    std::iota(by_imp.begin(), by_imp.end(), 0);
    std::sort(by_imp.begin(), by_imp.end(), [&](size_t a, size_t b) { return exist_imp[a] < exist_imp[b]; });
    struct RemoveEntry { uint32_t col; bool is_b4; };
    std::vector<RemoveEntry> to_remove;
    const size_t max_rw = size_t(max_row_weights), max_prune = size_t(max_prune_per_step);
    for (size_t rank = 0; rank < n_exist && to_remove.size() < max_prune; ++rank) {
        const size_t k = by_imp[rank];
        const size_t keep = n_exist - to_remove.size();
        if (std::max(exist_imp[k], importance_eps) < importance_cutoff || keep > max_rw)
            to_remove.push_back({exist_cols[k], exist_is_b4[k]});
    }
    std::sort(to_remove.begin(), to_remove.end(), [](const RemoveEntry &a, const RemoveEntry &b) { return a.col > b.col; });
    {
        std::unordered_set<uint32_t> exist_set(exist_cols.begin(), exist_cols.end());
        std::vector<size_t> pidx(probe_cols.size());
        std::iota(pidx.begin(), pidx.end(), 0);
        std::sort(pidx.begin(), pidx.end(), [&](size_t a, size_t b) { return probe_scores[a] > probe_scores[b]; });
        std::vector<uint32_t> add_cols;
        std::vector<float> add_scores;
        const size_t slots = max_rw - (n_exist - to_remove.size());
        for (size_t p : pidx) {
            if (add_cols.size() >= slots) break;
            if (!exist_set.count(probe_cols[p])) {
                add_cols.push_back(probe_cols[p]);
                add_scores.push_back(probe_scores[p]);
            }
        }
        probe_cols = std::move(add_cols);
        probe_scores = std::move(add_scores);
    }
    for (const auto &re : to_remove) {
        if (re.is_b4) {
            const uint32_t bc = re.col / TILE, lj = re.col % TILE;
            bool should_demote = false;
            auto it = M.tiles.find({br, bc});
            if (it != M.tiles.end() && it->second[lj * TILE + li] != 0) {
                b4_write_slot(M, br, bc, lj * TILE + li, 0);
                int live = 0;
                for (uint8_t b : it->second) live += b != 0;
                should_demote = live < PROMOTE_MIN_LIVE;
            }
            if (should_demote) {
                const int64_t fr = mut_demote(M, br, bc);
                if (fr >= 0) {
                    M = M0;
                    std::copy(deg0.begin(), deg0.end(), out_degree);
                    if (b4) {  // the layer as before, reservations included
                        std::copy(ia0.begin(), ia0.end(), b4->ia);
                        std::copy(ea0.begin(), ea0.end(), b4->ea);
                        std::copy(ta0.begin(), ta0.end(), b4->ta);
                        b4->dropped = dropped0;
                    }
                    if (fail) {
                        fail[0] = fr;
                        fail[1] = br;
                        fail[2] = bc;
                    }
                    return finish(-3);
                }
            }
        } else {
            mut_remove(M, r, re.col);
        }
        if (out_degree[re.col] > 0) --out_degree[re.col];
    }
    for (size_t i = 0; i < probe_cols.size(); ++i) {
        if (!mut_insert(M, r, probe_cols[i], 0.0f, probe_scores[i])) {
            if (fail) {
                fail[0] = int64_t(i);
                fail[1] = probe_cols[i];
                fail[2] = int64_t(row_index_bytes(M.rows[r]));
                fail[3] = res_b ? int64_t(res_b[r]) : -1;
                fail[4] = int64_t(probe_cols.size() - i);
            }
            return finish(-2);
        }
        ++out_degree[probe_cols[i]];
        try {
            mut_maybe_promote(M, r, probe_cols[i]);
        } catch (const B4Budget &) {
            if (fail) fail[0] = int64_t(i);
            return finish(-4);
        }
    }
    return finish(1);
}

int oracle_synap_row_step(const OracleLayer *L, int64_t row, const int32_t *prow, const int32_t *pcol,
                          const float *pval, int64_t pnnz, int has_probes, float importance_cutoff,
                          int64_t max_row_weights, int64_t max_prune_per_step, float importance_eps,
                          int32_t *out_degree, int32_t *out_ptrs, int32_t *out_cols, uint8_t *out_bytes,
                          int32_t *out_br, int32_t *out_bc, uint8_t *out_tiles, int64_t *n_tiles_out,
                          const uint64_t *res_b, const uint64_t *res_e, int64_t *fail) {
    return oracle_synap_row_step2(L, row, prow, pcol, pval, pnnz, has_probes, importance_cutoff, max_row_weights,
                                  max_prune_per_step, importance_eps, out_degree, out_ptrs, out_cols, out_bytes,
                                  out_br, out_bc, out_tiles, n_tiles_out, res_b, res_e, fail, nullptr);
}

}  // extern "C"
