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

typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 b2v __attribute__((ext_vector_type(2)));

// Rounds two fp32 values to bf16 (round-to-nearest-even, v_cvt_pk_bf16_f32) in place.
__device__ __forceinline__ void round_pair(float &a, float &b) {
    const f2v v = {a, b};
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2v));
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xffff0000u);
}

template <int E>
__device__ __forceinline__ void round_all(float (&x)[E]) {
#pragma unroll
    for (int j = 0; j < E; j += 2) round_pair(x[j], x[j + 1]);
}

// Divisor state of a per-row constant d: rcp = RN(1/d); `exact` is false when d is 0, infinite or
// NaN, where the plain IEEE quotient is used instead.
struct Divisor {
    float d, rcp;
    bool fast;
};

__device__ __forceinline__ Divisor make_divisor(float d) {
    Divisor v;
    v.d = d;
    v.rcp = 1.0f / d;
    v.fast = d != 0.0f && __builtin_isfinite(d) && __builtin_isfinite(v.rcp) && v.rcp != 0.0f;
    return v;
}

// bf16(x / d) for a bf16-exact x: q0 = x * RN(1/d) is within 2 ulp of x / d and one FMA
// correction brings it within 0.5 ulp + 2^-24 ulp. Because x and d carry 8 significant bits,
// x / d is either exactly representable (then the corrected quotient equals it) or at least
// ~2^-17 (relative) away from every bf16 rounding boundary, so the bf16 rounding of the result is
// that of the correctly rounded fp32 quotient, which is what torch's `div` computes.
__device__ __forceinline__ float div_exact_bf16(float x, const Divisor &v) {
    if (!v.fast) return x / v.d;
    const float q0 = x * v.rcp;
    const float r = __builtin_fmaf(-q0, v.d, x);
    const float q1 = __builtin_fmaf(r, v.rcp, q0);
    return __builtin_isinf(x) ? q0 : q1;
}

// Order-preserving 16-bit key of a bf16-exact float (-0 folded onto +0).
__device__ __forceinline__ uint32_t key_of(float x) {
    const uint32_t u = __float_as_uint(x + 0.0f);
    const uint32_t flip = (uint32_t)((int32_t)u >> 31) | 0x80000000u;
    return (u ^ flip) >> 16;
}

// Streams one tile of one row through the processor chain and returns the keys (0 = absent).
// The chain runs processor by processor over all E elements, so every indicator test is a
// uniform branch taken once per tile, and each processor ends with one packed bf16 rounding --
// the rounding points of the reference's PyTorch path (core/naive.py:131-268): grammar mask,
// multiplicative penalty (x < 0 ? x * r : x / r where context + decode counts > 0), frequency
// penalty x - bf16(count) * f (one rounding, as torch's addcmul), presence penalty, logit bias,
// temperature.
// VEC: vocabulary and every row base are 4-element aligned, so a 4-column chunk is either fully
// inside the vocabulary or fully outside, and planes load as 8 / 16-byte vectors.
template <int E, bool VEC>
__device__ __forceinline__ void prologue_keys(const RowState &rs, int col0, int V,
                                              const int32_t *hist, uint32_t (&keys)[E]) {
    constexpr int NCH = E / 4;
    const uint32_t ind = rs.ind;
    const bool use_g = (ind & IND_GRAMMAR) && rs.grammar;
    const bool use_rep = (ind & (IND_MULT | IND_FREQ | IND_PRES)) && rs.dec;
    const bool use_mult = use_rep && (ind & IND_MULT) && rs.ctx;
    const bool use_bias = (ind & IND_BIAS) && rs.bias;
    const bool remap = rs.d2t != nullptr && (use_g || use_rep || use_bias);
    const bool direct = VEC && !remap;

    float x[E];
    bool ok[E];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int col = col0 + tile_col(4 * c);
        if (VEC) {
            const bool in = col < V;
            const u32x2 w = in ? __builtin_nontemporal_load((const u32x2 *)(rs.logits + col))
                               : u32x2{0u, 0u};
            x[4 * c + 0] = __uint_as_float(w.x << 16);
            x[4 * c + 1] = __uint_as_float(w.x & 0xffff0000u);
            x[4 * c + 2] = __uint_as_float(w.y << 16);
            x[4 * c + 3] = __uint_as_float(w.y & 0xffff0000u);
#pragma unroll
            for (int i = 0; i < 4; ++i) ok[4 * c + i] = in;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ok[4 * c + i] = col + i < V;
                x[4 * c + i] = ok[4 * c + i] ? bf2f(rs.logits[col + i]) : 0.0f;
            }
        }
    }

    if (use_g || use_rep || use_bias) {
        int tcol[E];
#pragma unroll
        for (int j = 0; j < E; ++j) tcol[j] = col0 + tile_col(j);
        if (remap) {
#pragma unroll
            for (int j = 0; j < E; ++j) tcol[j] = ok[j] ? rs.d2t[tcol[j]] : 0;
        }
        if (use_g) {
#pragma unroll
            for (int j = 0; j < E; ++j) {
                uint32_t w;
                if (direct) {
                    w = ok[j] ? rs.grammar[(col0 + tile_col(j & ~3)) >> 5] : 0xffffffffu;
                } else {
                    w = ok[j] ? rs.grammar[tcol[j] >> 5] : 0xffffffffu;
                }
                x[j] = ((w >> (tcol[j] & 31)) & 1u) ? x[j] : -INFINITY;
            }
        }
        if (use_rep) {
            int32_t dec[E];
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int col = col0 + tile_col(4 * c);
                if (direct) {
                    const i32x4 d = ok[4 * c] ? __builtin_nontemporal_load((const i32x4 *)(rs.dec + col))
                                              : i32x4{0, 0, 0, 0};
                    dec[4 * c + 0] = d.x; dec[4 * c + 1] = d.y; dec[4 * c + 2] = d.z; dec[4 * c + 3] = d.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) dec[4 * c + i] = ok[4 * c + i] ? rs.dec[tcol[4 * c + i]] : 0;
                }
            }
            if (rs.nhist > 0) {
                // The history never counts token 0: the reference pads the history with 0 and then
                // restores the original count of token 0 (core/naive.py:179-203).
                for (int h = 0; h < rs.nhist; ++h) {
                    const int t = hist[h];
#pragma unroll
                    for (int j = 0; j < E; ++j) dec[j] += (tcol[j] == t && t != 0) ? 1 : 0;
                }
            }
            if (use_mult) {
                const Divisor rep = make_divisor(rs.rep);
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    int32_t ctx[4];
                    const int col = col0 + tile_col(4 * c);
                    if (direct) {
                        const i32x4 q = ok[4 * c] ? __builtin_nontemporal_load((const i32x4 *)(rs.ctx + col))
                                                  : i32x4{0, 0, 0, 0};
                        ctx[0] = q.x; ctx[1] = q.y; ctx[2] = q.z; ctx[3] = q.w;
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) ctx[i] = ok[4 * c + i] ? rs.ctx[tcol[4 * c + i]] : 0;
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int j = 4 * c + i;
                        const float y = x[j] < 0.0f ? x[j] * rs.rep : div_exact_bf16(x[j], rep);
                        x[j] = (dec[j] + ctx[i] > 0) ? y : x[j];
                    }
                }
                round_all(x);
            }
            if (ind & IND_FREQ) {
                float cnt[E];
#pragma unroll
                for (int j = 0; j < E; ++j) cnt[j] = (float)dec[j];
                round_all(cnt);
#pragma unroll
                for (int j = 0; j < E; ++j) x[j] = __builtin_fmaf(-cnt[j], rs.freq, x[j]);
                round_all(x);
            }
            if (ind & IND_PRES) {
#pragma unroll
                for (int j = 0; j < E; ++j) x[j] = x[j] - (dec[j] > 0 ? rs.pres : 0.0f);
                round_all(x);
            }
        }
        if (use_bias) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int col = col0 + tile_col(4 * c);
                if (direct) {
                    const u32x2 b = ok[4 * c] ? __builtin_nontemporal_load((const u32x2 *)(rs.bias + col))
                                              : u32x2{0u, 0u};
                    x[4 * c + 0] += __uint_as_float(b.x << 16);
                    x[4 * c + 1] += __uint_as_float(b.x & 0xffff0000u);
                    x[4 * c + 2] += __uint_as_float(b.y << 16);
                    x[4 * c + 3] += __uint_as_float(b.y & 0xffff0000u);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        x[4 * c + i] += ok[4 * c + i] ? bf2f(rs.bias[tcol[4 * c + i]]) : 0.0f;
                }
            }
            round_all(x);
        }
    }
    if (ind & IND_TEMP) {
        const Divisor t = make_divisor(rs.temp);
#pragma unroll
        for (int j = 0; j < E; ++j) x[j] = div_exact_bf16(x[j], t);
        round_all(x);
    }
#pragma unroll
    for (int j = 0; j < E; ++j) keys[j] = ok[j] ? key_of(x[j]) : 0u;
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

// Selects the row's top-128 among `nsc` blocks of candidates and leaves them, in column order,
// as (key << 8 | 127 - pos) composites and column indices in sm.cand / sm.idx.
template <bool HELD, int EM, class Load, class Cand>
__device__ __forceinline__ void merge_select(SampleSmem &sm, int nsc, Load load, Cand cand,
                                             int block_n, int V) {
    uint32_t thi, margin;
    int level;
    radix_threshold<EM, 16>(sm.sel, nsc, load, (uint32_t)SS_K, thi, level, margin);
    compact<EM, 4>(sm.sel, nsc, load, thi, level, margin, [&](uint32_t pos, int sc, int j) {
        if (pos >= (uint32_t)SS_K) return;
        const int p = order_pos<EM, 4>(sc, j);
        const uint32_t c = cand(sc, j);
        const int idx = (p / SS_K) * block_n + (int)(c & 0xffffu);
        sm.cand[pos] = ((uint64_t)(c >> 16) << 8) | (uint64_t)(127u - pos);
        sm.idx[pos] = idx < V ? idx : V - 1;  // only an absent-element sentinel can exceed V
    });
}

// Row merge: all threads call; on return wave 0 holds the row's top-128 sorted by (value desc,
// column asc), element e = 2 * lane + i as (v_i, idx_i). Up to 4096 candidates are read once
// with 16-byte loads and kept in registers; larger rows stream them from the scratch per pass.
__device__ __forceinline__ void merge_row(SampleSmem &sm, const uint32_t *scr, int tiles,
                                          int block_n, int V, float &v0, float &v1, int &i0,
                                          int &i1) {
    constexpr int EM = 16;
    const int ncand = tiles * SS_K;
    const int nsc = (ncand + SS_BLOCK * EM - 1) / (SS_BLOCK * EM);
    if (nsc == 1) {
        uint32_t held[EM];
#pragma unroll
        for (int c = 0; c < EM / 4; ++c) {
            const int p = order_pos<EM, 4>(0, 4 * c);  // multiple of 4; ncand is a multiple of 128
            const uint4 q = p < ncand ? *(const uint4 *)(scr + p) : make_uint4(0u, 0u, 0u, 0u);
            held[4 * c + 0] = q.x; held[4 * c + 1] = q.y; held[4 * c + 2] = q.z; held[4 * c + 3] = q.w;
        }
        merge_select<true, EM>(
            sm, 1,
            [&](int, uint32_t(&out)[EM]) {
#pragma unroll
                for (int j = 0; j < EM; ++j) out[j] = held[j] >> 16;
            },
            [&](int, int j) { return held[j]; }, block_n, V);
    } else {
        merge_select<false, EM>(
            sm, nsc,
            [&](int sc, uint32_t(&out)[EM]) {
#pragma unroll
                for (int j = 0; j < EM; ++j) {
                    const int p = order_pos<EM, 4>(sc, j);
                    out[j] = p < ncand ? (scr[p] >> 16) : 0u;
                }
            },
            [&](int sc, int j) { return scr[order_pos<EM, 4>(sc, j)]; }, block_n, V);
    }
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
