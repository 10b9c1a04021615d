// Pieces shared by the fused single-step and multi-step kernels:
//   * the logit-processor prologue (grammar mask, repetition / frequency / presence penalties over
//     decode-count histograms plus the drafted-token history, logit bias, temperature), evaluated
//     per element in fp32 and rounded to bf16 after every processor exactly where the reference's
//     PyTorch path rounds (reference core/naive.py:131-268; kernel counterpart ops/prologue.py);
//   * the tile stage (greedy tile argmax or exact tile top-128 into the scratch row);
//   * the row merge of the tiles' candidates into the sorted top-128;
//   * top-k / top-p / min-p truncation in the reference's order (core/naive.py:270-328).
#pragma once

#include "ss_philox.h"
#include "ss_select.h"

namespace ss {

constexpr uint32_t IND_GRAMMAR = 0x001, IND_MULT = 0x002, IND_FREQ = 0x004, IND_PRES = 0x008,
                   IND_BIAS = 0x010, IND_TEMP = 0x020, IND_GREEDY = 0x040, IND_TOPK = 0x080,
                   IND_TOPP = 0x100, IND_MINP = 0x200, IND_TOPLOGPROBS = 0x400,
                   IND_SVGD = 0x800;

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct SampleSmem {
    SelectSmem sel;
    uint64_t cand[SS_K];
    int32_t idx[SS_K];
    int32_t hist[64];
    uint32_t red[SS_WAVES];
};

// Request state of one logit row, uniform over the workgroup. Row pointers are already offset to
// the request's slot (and timestep for the grammar).
struct RowState {
    uint32_t ind;
    const uint16_t *logits;
    const int32_t *d2t;
    const uint32_t *grammar;
    const int32_t *ctx;
    const int32_t *dec;
    const uint16_t *bias;
    float rep, freq, pres, temp;
    int nhist;  // drafted tokens of the history staged in SampleSmem::hist
};

__device__ __forceinline__ int tile_col(int j) {  // column offset of element j inside a tile
    return (j >> 2) * (SS_BLOCK * 4) + (int)threadIdx.x * 4 + (j & 3);
}

// One element through the processor chain. x is bf16-exact on entry and on exit.
__device__ __forceinline__ float process_element(float x, const RowState &rs, int tcol,
                                                 uint32_t gword, int32_t dec, int32_t ctx,
                                                 uint32_t braw, const int32_t *hist) {
    const uint32_t ind = rs.ind;
    if (ind & IND_GRAMMAR) {
        if (rs.grammar && !((gword >> (tcol & 31)) & 1u)) x = -INFINITY;
    }
    if ((ind & (IND_MULT | IND_FREQ | IND_PRES)) && rs.dec) {
        // The history never counts token 0: the reference pads the history with 0 and then
        // restores the original count of token 0 (core/naive.py:179-203).
        if (tcol != 0) {
            for (int h = 0; h < rs.nhist; ++h) dec += (hist[h] == tcol);
        }
        if ((ind & IND_MULT) && rs.ctx) {
            if (dec + ctx > 0) x = rbf(x < 0.0f ? x * rs.rep : x / rs.rep);
        }
        if (ind & IND_FREQ) x = rbf(x - rbf((float)dec) * rs.freq);
        if (ind & IND_PRES) x = rbf(x - (dec > 0 ? rs.pres : 0.0f));
    }
    if ((ind & IND_BIAS) && rs.bias) x = rbf(x + bf2f(braw));
    if (ind & IND_TEMP) x = rbf(x / rs.temp);
    return x;
}

// Streams one tile of one row through the prologue and returns the elements' keys (0 = absent).
// VEC: vocabulary and every row base are 4-element aligned, so a 4-column chunk is either fully
// inside the vocabulary or fully outside, and planes load as 8 / 16-byte vectors.
template <int E, bool VEC>
__device__ __forceinline__ void prologue_keys(const RowState &rs, int col0, int V,
                                              const int32_t *hist, uint32_t (&keys)[E]) {
    constexpr int NCH = E / 4;
    const uint32_t ind = rs.ind;
    const bool any_proc = (ind & 0x3Fu) != 0;
    const bool use_g = (ind & IND_GRAMMAR) && rs.grammar;
    const bool use_rep = (ind & (IND_MULT | IND_FREQ | IND_PRES)) && rs.dec;
    const bool use_ctx = use_rep && (ind & IND_MULT) && rs.ctx;
    const bool use_bias = (ind & IND_BIAS) && rs.bias;
    const bool remap = rs.d2t != nullptr && (ind & 0x1Fu);

    uint32_t lg[E];
    int tcol[E];
    uint32_t gw[E];
    int32_t dc[E], cc[E];
    uint32_t bs[E];

    // Logits: 8-byte vector per chunk when aligned, streamed with non-temporal loads.
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = col0 + tile_col(4 * c);
        if (VEC) {
            u32x2 w = col < V ? __builtin_nontemporal_load((const u32x2 *)(rs.logits + col))
                              : u32x2{0u, 0u};
            lg[4 * c + 0] = w.x & 0xffffu;
            lg[4 * c + 1] = w.x >> 16;
            lg[4 * c + 2] = w.y & 0xffffu;
            lg[4 * c + 3] = w.y >> 16;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                lg[4 * c + i] = col + i < V ? (uint32_t)rs.logits[col + i] : 0xff80u;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) tcol[4 * c + i] = col + i;
    }
    if (any_proc) {
        if (remap) {
#pragma unroll
            for (int j = 0; j < E; ++j) tcol[j] = tcol[j] < V ? rs.d2t[tcol[j]] : 0;
        }
        if (use_g) {
#pragma unroll
            for (int j = 0; j < E; ++j) {
                if (!remap && VEC && (j & 3)) {
                    gw[j] = gw[j & ~3];
                } else {
                    gw[j] = (col0 + tile_col(j) < V) ? rs.grammar[tcol[j] >> 5] : 0xffffffffu;
                }
            }
        }
        if (use_rep) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int col = col0 + tile_col(4 * c);
                if (VEC && !remap) {
                    i32x4 d = col < V ? __builtin_nontemporal_load((const i32x4 *)(rs.dec + col))
                                      : i32x4{0, 0, 0, 0};
                    dc[4 * c + 0] = d.x; dc[4 * c + 1] = d.y; dc[4 * c + 2] = d.z; dc[4 * c + 3] = d.w;
                    if (use_ctx) {
                        i32x4 q = col < V ? __builtin_nontemporal_load((const i32x4 *)(rs.ctx + col))
                                          : i32x4{0, 0, 0, 0};
                        cc[4 * c + 0] = q.x; cc[4 * c + 1] = q.y; cc[4 * c + 2] = q.z; cc[4 * c + 3] = q.w;
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool ok = col + i < V;
                        dc[4 * c + i] = ok ? rs.dec[tcol[4 * c + i]] : 0;
                        if (use_ctx) cc[4 * c + i] = ok ? rs.ctx[tcol[4 * c + i]] : 0;
                    }
                }
            }
        }
        if (use_bias) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int col = col0 + tile_col(4 * c);
                if (VEC && !remap) {
                    u32x2 b = col < V ? __builtin_nontemporal_load((const u32x2 *)(rs.bias + col))
                                      : u32x2{0u, 0u};
                    bs[4 * c + 0] = b.x & 0xffffu; bs[4 * c + 1] = b.x >> 16;
                    bs[4 * c + 2] = b.y & 0xffffu; bs[4 * c + 3] = b.y >> 16;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        bs[4 * c + i] = col + i < V ? (uint32_t)rs.bias[tcol[4 * c + i]] : 0u;
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const bool ok = col0 + tile_col(j) < V;
        float x = bf2f(lg[j]);
        if (any_proc) {
            x = process_element(x, rs, tcol[j], use_g ? gw[j] : 0xffffffffu, use_rep ? dc[j] : 0,
                                use_ctx ? cc[j] : 0, use_bias ? bs[j] : 0u, hist);
        }
        keys[j] = ok ? key16(f2bf(x)) : 0u;
    }
}

// Tile stage. Greedy rows store one u32 per tile: (key << 16) | (0xffff - column offset), whose
// maximum picks the lowest column among equal maxima. Other rows store their exact top-128 as
// (key << 16) | column offset, in column order, at scratch[tile * 128 ...].
template <int E>
__device__ __forceinline__ void tile_stage(SampleSmem &sm, bool greedy, const uint32_t (&keys)[E],
                                           uint32_t *scr, int tile) {
    if (greedy) {
        uint32_t best = 0;
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const uint32_t c = keys[j] ? ((keys[j] << 16) | (0xffffu - (uint32_t)tile_col(j))) : 0u;
            best = best > c ? best : c;
        }
        best = wave_max_u32(best);
        if (lane_id() == 0) sm.red[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t b = sm.red[0];
            for (int w = 1; w < SS_WAVES; ++w) b = b > sm.red[w] ? b : sm.red[w];
            scr[tile] = b;
        }
        return;
    }
    auto load = [&](int, uint32_t(&out)[E]) {
#pragma unroll
        for (int j = 0; j < E; ++j) out[j] = keys[j];
    };
    uint32_t thi, margin;
    int level;
    radix_threshold<E, 16>(sm.sel, 1, load, (uint32_t)SS_K, thi, level, margin);
    compact<E, 4>(sm.sel, 1, load, thi, level, margin, [&](uint32_t pos, int, int j) {
        if (pos < (uint32_t)SS_K) scr[tile * SS_K + (int)pos] = (keys[j] << 16) | (uint32_t)tile_col(j);
    });
}

// Greedy merge over the tiles' maxima (wave 0): the largest value, lowest column on ties.
__device__ __forceinline__ int greedy_merge(const uint32_t *scr, int tiles, int block_n, int V) {
    uint64_t best = 0;
    for (int t = lane_id(); t < tiles; t += 64) {
        const uint32_t c = scr[t];
        const uint64_t c64 = ((uint64_t)(c >> 16) << 32) | ((uint64_t)(0xffffu - (uint32_t)t) << 16) |
                             (uint64_t)(c & 0xffffu);
        best = best > c64 ? best : c64;
    }
    best = wave_max_u64(best);
    const int tile = (int)(0xffffu - (uint32_t)((best >> 16) & 0xffffu));
    const int off = (int)(0xffffu - (uint32_t)(best & 0xffffu));
    const int idx = tile * block_n + off;
    return idx < V ? idx : V - 1;
}

// Row merge: all threads call; on return wave 0 holds the row's top-128 sorted by (value desc,
// column asc), element e = 2 * lane + i as (v_i, idx_i).
__device__ __forceinline__ void merge_row(SampleSmem &sm, const uint32_t *scr, int tiles,
                                          int block_n, int V, float &v0, float &v1, int &i0,
                                          int &i1) {
    constexpr int EM = 16;
    const int ncand = tiles * SS_K;
    const int nsc = (ncand + SS_BLOCK * EM - 1) / (SS_BLOCK * EM);
    auto load = [&](int sc, uint32_t(&out)[EM]) {
#pragma unroll
        for (int j = 0; j < EM; ++j) {
            const int p = order_pos<EM, 4>(sc, j);
            out[j] = p < ncand ? (scr[p] >> 16) : 0u;
        }
    };
    uint32_t thi, margin;
    int level;
    radix_threshold<EM, 16>(sm.sel, nsc, load, (uint32_t)SS_K, thi, level, margin);
    compact<EM, 4>(sm.sel, nsc, load, thi, level, margin, [&](uint32_t pos, int sc, int j) {
        if (pos >= (uint32_t)SS_K) return;
        const int p = order_pos<EM, 4>(sc, j);
        const uint32_t c = scr[p];
        const int idx = (p / SS_K) * block_n + (int)(c & 0xffffu);
        sm.cand[pos] = ((uint64_t)(c >> 16) << 8) | (uint64_t)(127u - pos);
        sm.idx[pos] = idx < V ? idx : V - 1;  // only an absent-element sentinel can exceed V
    });
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        uint64_t c0 = sm.cand[2 * lane], c1 = sm.cand[2 * lane + 1];
        wave_sort128_desc(c0, c1);
        v0 = bf2f(unkey16((uint32_t)(c0 >> 8)));
        v1 = bf2f(unkey16((uint32_t)(c1 >> 8)));
        i0 = sm.idx[127 - (int)(c0 & 0x7fu)];
        i1 = sm.idx[127 - (int)(c1 & 0x7fu)];
    }
}

// exp(v - m) for both elements of the lane and the wave-wide sum. m is element 0 (the maximum).
__device__ __forceinline__ float exp_parts(float v0, float v1, float &m, float &x0, float &x1) {
    m = __shfl(v0, 0, 64);
    x0 = expf(v0 - m);
    x1 = expf(v1 - m);
    return wave_sum_f32(x0 + x1);
}

// top-k -> top-p -> min-p on the sorted top-128 (wave 0), each on the values left by the
// previous one, as in reference core/naive.py:270-328 (applied in that order by
// `thread_first(values, self.top_k, self.top_p, self.min_p)`, core/naive.py:338).
__device__ __forceinline__ void truncate(uint32_t ind, int32_t topk, float topp, float minp,
                                         float &v0, float &v1) {
    const int e0 = 2 * lane_id(), e1 = e0 + 1;
    if (ind & IND_TOPK) {
        if (e0 >= topk) v0 = -INFINITY;
        if (e1 >= topk) v1 = -INFINITY;
    }
    if (ind & IND_TOPP) {
        // softmax in fp32 (x * (1 / sum)), cumulative sum accumulated in fp64 and compared in
        // fp32 against p; position 0 is always kept.
        float m, x0, x1;
        const float s = exp_parts(v0, v1, m, x0, x1);
        const float inv = 1.0f / s;
        const float p0 = x0 * inv, p1 = x1 * inv;
        const double inc = wave_inclusive_sum_f64((double)p0 + (double)p1);
        double exc = __shfl_up(inc, 1, 64);
        if (lane_id() == 0) exc = 0.0;
        const double c0 = exc + (double)p0, c1 = c0 + (double)p1;
        if (e0 > 0 && (float)c0 > topp) v0 = -INFINITY;
        if ((float)c1 > topp) v1 = -INFINITY;
    }
    if (ind & IND_MINP) {
        // bf16 softmax, masked where the rounded probability is below bf16(min_p * p_max).
        float m, x0, x1;
        const float s = exp_parts(v0, v1, m, x0, x1);
        const float inv = 1.0f / s;
        const float s0 = rbf(x0 * inv), s1 = rbf(x1 * inv);
        const float lower = rbf(minp * __shfl(s0, 0, 64));
        if (s0 < lower) v0 = -INFINITY;
        if (s1 < lower) v1 = -INFINITY;
    }
}

// First element (lowest sorted position) holding the maximum of z over the wave's 128 elements.
__device__ __forceinline__ int wave_argmax_first(float z0, float z1) {
    const int e0 = 2 * lane_id();
    const uint64_t a = ((uint64_t)key32(__float_as_uint(z0)) << 32) | (uint32_t)(127 - e0);
    const uint64_t b = ((uint64_t)key32(__float_as_uint(z1)) << 32) | (uint32_t)(126 - e0);
    const uint64_t best = wave_max_u64(a > b ? a : b);
    return 127 - (int)(best & 0xffffffffu);
}

}  // namespace ss
