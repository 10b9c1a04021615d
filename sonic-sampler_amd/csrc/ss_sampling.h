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
    uint32_t surv[2 * SS_K];   // tile stage: candidates that pass the lower bound
    uint32_t runs[4][SS_K];    // row merge: the waves' sorted samples
    int32_t col[4 * SS_K];     // row merge: column of each sample slot
    int32_t flag;
    uint64_t cand[SS_K];
    int32_t idx[SS_K];
    int32_t hist[64];
    uint32_t red[SS_WAVES];
    int32_t tok[SS_K];         // selection: the candidates' tokens (columns, then remapped)
    float noise[SS_K];         // selection: their Gumbel noise
    float qcand[SS_K];         // verification: their draft probabilities
};

// Workgroup memory of the tile kernels (E keys per thread). The members from `run` on are written
// only after the tile stage's first barrier, when every wave has finished its prologue, so a
// grammar row staged for the prologue (stage_grammar) may overlay them (TILE_OVERLAY).
template <int E>
struct TileSmem {
    uint32_t scan[SS_WAVES * 16];  // workgroup scans of up to 16 values per thread
    uint32_t red[SS_WAVES];
    uint32_t cnt[SS_WAVES];       // survivors of each wave
    int32_t hist[64];             // drafted tokens that extend the decode history
    uint32_t run[SS_WAVES][SS_K + 64];  // each wave's survivors, then its sorted run
    uint32_t run2[2][SS_K];       // merge tree: the top-128 of runs (0, 1) and (2, 3)
    // each wave's packed keys, pair i of lane l at [i * 64 + l], read back by the survivors of
    // wave_survivors_masked
    uint32_t keys[SS_WAVES][E / 2 * 64];
};

// Byte offset in TileSmem where a staged grammar row may begin.
constexpr int TILE_OVERLAY = (SS_WAVES * 16 + 2 * SS_WAVES + 64) * 4;
static_assert(TILE_OVERLAY % 16 == 0, "16-byte grammar stores");
static_assert(TILE_OVERLAY == __builtin_offsetof(TileSmem<16>, run), "overlay starts at the runs");

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
    int vt;     // width of the counts / bias / grammar rows (target vocabulary)
    int nhist;  // drafted tokens of the history staged in SampleSmem::hist
    // The row's grammar words staged in workgroup memory (gather layout only), or NULL: the
    // gathers through d2t then read LDS instead of scattered global words.
    const uint32_t *glds;
    // Column of the logits' first column in the target vocabulary (sharded vocabulary: the
    // shard's offset), added to every column that addresses a side plane, d2t or the history.
    int shard;
};

typedef const __attribute__((address_space(3))) uint32_t *lds_cu32p;

// First column of candidate list `l` of a row: lists are the tiles of `per` tiles per shard, shard
// w covering target columns [w * shard, ...), so list l is tile l % per of shard l / per. The
// division is a multiply-high by magic = ceil(2^32 / per), exact for l < 2^16 and 2 <= per < 2^16.
// Unsharded rows use per = the row's tile count, so l / per is 0.
struct ListMap {
    uint32_t magic;
    int per, shard, block_n;
    __device__ __forceinline__ int base(int l) const {
        const int w = (int)__umulhi((uint32_t)l, magic);
        return w * shard + (l - w * per) * block_n;
    }
    // Scratch entry holding greedy list l's composite: a shard's tiles store theirs densely at
    // the start of the shard's slice (tile t of shard w at w * per * 128 + t).
    __device__ __forceinline__ int greedy_entry(int l) const {
        const int w = (int)__umulhi((uint32_t)l, magic);
        return w * per * SS_K + (l - w * per);
    }
};

__host__ __device__ inline ListMap make_list_map(int per, int shard, int block_n) {
    ListMap m;
    m.magic = (uint32_t)((((uint64_t)1 << 32) + (uint64_t)per - 1) / (uint64_t)per);
    m.per = per;
    m.shard = shard;
    m.block_n = block_n;
    return m;
}

// Renumbers workgroup L of a launch of N so that each XCD runs a contiguous range of the new
// numbers: the dispatcher hands consecutive workgroups to the device's 8 XCDs in turn (L % 8), and
// workgroup L becomes number local + the start of XCD L % 8's range, the first N % 8 XCDs taking
// one number more. A bijection on [0, N) for any N; workgroups that share data (the tiles of one
// row) then share an L2.
__device__ __forceinline__ int xcd_grouped(int L, int N) {
    const int q = N >> 3, r = N & 7;
    const int x = L & 7, local = L >> 3;
    return x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
}

__device__ __forceinline__ int tile_col(int j) {  // column offset of element j inside a tile
    return (j >> 2) * (SS_BLOCK * 4) + (int)threadIdx.x * 4 + (j & 3);
}

// The 16-bit keys of a thread's E elements, two per register: element 2i in the low half of p[i],
// element 2i + 1 in the high half. Comparisons with a 16-bit threshold t read a half in place: the
// low half through a 16-bit source select, the high half against (t << 16) | 0xffff.
template <int E>
struct Keys {
    uint32_t p[E / 2];

    __device__ __forceinline__ uint32_t at(int j) const {
        return (j & 1) ? p[j >> 1] >> 16 : p[j >> 1] & 0xffffu;
    }
    __device__ __forceinline__ bool gt(int j, uint32_t t) const {
        return (j & 1) ? p[j >> 1] > ((t << 16) | 0xffffu) : (uint16_t)p[j >> 1] > (uint16_t)t;
    }
    __device__ __forceinline__ bool ge(int j, uint32_t t) const {
        return (j & 1) ? p[j >> 1] >= (t << 16) : (uint16_t)p[j >> 1] >= (uint16_t)t;
    }
    __device__ __forceinline__ bool eq(int j, uint32_t t) const {
        return (j & 1) ? (p[j >> 1] >> 16) == t : (uint16_t)p[j >> 1] == (uint16_t)t;
    }
    // the pair register of element j with element j's key replaced by k
    __device__ __forceinline__ uint32_t with(int j, uint32_t k) const {
        return (j & 1) ? (p[j >> 1] & 0xffffu) | (k << 16) : (p[j >> 1] & 0xffff0000u) | k;
    }
    // (key << 16) | (0xffff - column of element j), from cb = 0xffff - 4 * thread
    __device__ __forceinline__ uint32_t composite(int j, uint32_t cb) const {
        const uint32_t hi = (j & 1) ? (p[j >> 1] & 0xffff0000u) : (p[j >> 1] << 16);
        return (hi | cb) - (uint32_t)((j >> 2) * (SS_BLOCK * 4) + (j & 3));
    }
};

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

// Divisor state of a per-row constant d: rcp = 1/d from v_rcp_f32 (within 1 ulp); `fast` is
// false when d is 0, infinite or NaN or the reciprocal is not a normal number (|d| near the ends
// of the fp32 range), where the plain IEEE quotient is used instead.
struct Divisor {
    float d, rcp;
    bool fast;
};

__device__ __forceinline__ Divisor make_divisor(float d) {
    Divisor v;
    v.d = d;
    v.rcp = __builtin_amdgcn_rcpf(d);
    v.fast = d != 0.0f && __builtin_isfinite(d) && __builtin_isnormal(v.rcp);
    return v;
}

// x / d for bf16 x and d, valid as the input of a bf16 rounding. Both carry 8 significant bits, so
// x / d is either exact with at most 8 significant bits (a bf16 value) or at least 2^-17 (relative)
// away from every bf16 rounding boundary, since a boundary needs 9 significant bits. x * rcp with
// rcp within 1 ulp of 1/d is within 2^-22 of x / d, so its bf16 rounding equals that of torch's
// correctly rounded fp32 quotient.
__device__ __forceinline__ float div_bf16(float x, const Divisor &v) {
    return v.fast ? x * v.rcp : x / v.d;
}

// Order-preserving 16-bit key (key16) of a bf16-exact float: 0x8000 plus the signed magnitude
// of its top 16 bits (negation by xor with the sign mask and subtraction of it).
// Key of bf16 -inf (key_of and packed_keys): every finite or +inf value has a larger one.
constexpr uint32_t KEY_NEG_INF = 0x0080;

__device__ __forceinline__ uint32_t key_of(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t s = (uint32_t)((int32_t)u >> 31);
    const uint32_t m = (u >> 16) & 0x7fffu;
    return ((m ^ s) - s) + 0x8000u;
}

// Raw buffer view of one row: loads past `bytes` return 0 without faulting, so every load below is
// unconditional. Descriptor word 3 for gfx9-family raw buffers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_buffer(const void *p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes < 0x7fffffff ? bytes : 0x7fffffff),
                                             0x00020000);
}

constexpr int NT = 2;  // non-temporal: each plane is read once

typedef short s2v __attribute__((ext_vector_type(2)));
typedef unsigned short u2v __attribute__((ext_vector_type(2)));

// key16 of the two bf16 halves of `u` at once, with packed 16-bit integer operations: with m the
// half's sign mask (0 or 0xffff), (u ^ (m | 0x8000)) - m is u + 0x8000 for a positive half and
// (0x7fff - magnitude) + 1 = 0x8000 - magnitude for a negative one (-0 and +0 both 0x8000). The
// xor-or is one three-input bit operation: three instructions a pair.
__device__ __forceinline__ uint32_t packed_keys(uint32_t u) {
    const uint32_t m = __builtin_bit_cast(uint32_t, __builtin_bit_cast(s2v, u) >> (s2v){15, 15});
    const uint32_t t = u ^ (m | 0x80008000u);
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u2v, t) - __builtin_bit_cast(u2v, m));
}

// bf16 rounding of one value (round-to-nearest-even): converted into the high half of a packed
// pair whose low half is bf16(0) = 0, the register is the rounded value as a float.
__device__ __forceinline__ float rnd(float a) {
    const f2v v = {0.0f, a};
    return __uint_as_float(__builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2v)));
}

// Processor constants of one row, uniform over the workgroup.
struct Chain {
    bool mult, freq, pres, bias, temp;
    float rep, fr, pr;
    Divisor rdiv, tdiv;
};

// The whole processor chain on one element, rounding to bf16 after every processor as the
// reference's PyTorch path does (core/naive.py:131-268): multiplicative penalty (x < 0 ? x * r :
// x / r where context + decode counts > 0), frequency penalty x - bf16(count) * f (one rounding,
// as torch's addcmul), presence penalty, logit bias, temperature.
__device__ __forceinline__ float chain(const Chain &k, float x, int32_t dec, int32_t ctx, float b) {
    if (k.mult && dec + ctx > 0) x = rnd(x < 0.0f ? x * k.rep : div_bf16(x, k.rdiv));
    if (k.freq) x = rnd(__builtin_fmaf(-rnd((float)dec), k.fr, x));
    if (k.pres) x = rnd(x - (dec > 0 ? k.pr : 0.0f));
    if (k.bias) x = rnd(x + b);
    if (k.temp) x = rnd(div_bf16(x, k.tdiv));
    return x;
}

// Branch-free form of `chain` for rows whose divisors have exact reciprocals (Divisor::fast):
// every processor is applied, the ones that are off with neutral parameters (factor 1, penalty
// 0, bias 0, temperature 1). Rounding a bf16-exact value to bf16 is the identity, so the result
// equals that of the gated chain.
struct FastChain {
    bool mult;
    float rep, rrcp, fr, pr, trcp;
};

__device__ __forceinline__ FastChain fast_chain(const Chain &k) {
    FastChain f;
    f.mult = k.mult;
    f.rep = k.rep;
    f.rrcp = k.rdiv.rcp;
    f.fr = k.freq ? k.fr : 0.0f;
    f.pr = k.pres ? k.pr : 0.0f;
    f.trcp = k.temp ? k.tdiv.rcp : 1.0f;
    return f;
}

__device__ __forceinline__ float chain_fast(const FastChain &k, float x, int32_t dec, int32_t ctx,
                                            float b) {
    const float xm = rnd(x < 0.0f ? x * k.rep : x * k.rrcp);
    x = (k.mult && dec + ctx > 0) ? xm : x;
    x = rnd(__builtin_fmaf(-rnd((float)dec), k.fr, x));
    x = rnd(x - (dec > 0 ? k.pr : 0.0f));
    x = rnd(x + b);
    return rnd(x * k.trcp);
}

// Branch-free chain with IEEE divisions, for rows whose divisors have no exact reciprocal (zero,
// infinite, NaN or extreme). Applied to every element it equals the gated chain: for an element
// with zero counts and bias every processor but the temperature is the identity (up to the sign
// of a zero, which keys do not see).
__device__ __forceinline__ float chain_ieee(const Chain &k, float x, int32_t dec, int32_t ctx,
                                            float b) {
    const float xm = rnd(x < 0.0f ? x * k.rep : x / k.rdiv.d);
    x = (k.mult && dec + ctx > 0) ? xm : x;
    x = rnd(__builtin_fmaf(-rnd((float)dec), k.freq ? k.fr : 0.0f, x));
    x = rnd(x - (dec > 0 && k.pres ? k.pr : 0.0f));
    x = rnd(x + b);
    return k.temp ? rnd(x / k.tdiv.d) : x;
}

// Keys of E elements from their (grammar-masked) logits x, decode counts, context counts and
// bias bits. Most elements of a row have zero counts and zero bias; for them every penalty and the
// bias are the identity and the chain reduces to the temperature division, which runs for all
// elements with one multiply each. Elements with a nonzero count or bias (or every element, when a
// non-finite frequency penalty turns 0 * f into NaN) then run the full chain one element position
// at a time, so a wave pays for it only at the positions where one of its lanes holds one. Rows
// whose divisors have no exact reciprocal take the IEEE chain on every element instead. `ok` marks
// elements inside the vocabulary; it can be false only when `partial` is set. x(j) and bb(j) return
// the (grammar-masked) logit and the bias bits of element j; bw(j) is nonzero whenever element j's
// bias is nonzero (it may also be nonzero for a zero bias: the chain is exact for every element).
// maybe_exc is false when no element can have a nonzero count or bias (no penalty or bias plane is
// read) and the chain is not forced on every element: the keys are then the temperature keys.
// pair(j) (j even) is the 32-bit word holding the masked bf16 logits of elements j and j + 1.
template <int E, class XOf, class PairOf, class BiasOf, class BiasWordOf>
__device__ __forceinline__ void finish_keys(const Chain &k, bool all_exc, bool partial, XOf x,
                                            PairOf pair, bool maybe_exc,
                                            const bool (&ok)[E], const int32_t (&dec)[E],
                                            const int32_t (&ctx)[E], BiasOf bb, BiasWordOf bw,
                                            Keys<E> &keys) {
    if ((!k.mult || k.rdiv.fast) && (!k.temp || k.tdiv.fast)) {
        const FastChain f = fast_chain(k);
        if (!k.temp) {
            // no temperature: the keys of the (grammar-masked) bf16 pairs as they are
#pragma unroll
            for (int j = 0; j < E; j += 2) keys.p[j >> 1] = packed_keys(pair(j));
        } else {
#pragma unroll
            for (int j = 0; j < E; j += 2) {
                const f2v v = {x(j) * f.trcp, x(j + 1) * f.trcp};
                keys.p[j >> 1] = packed_keys(__builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2v)));
            }
        }
        // The branch at each element position is on the wave's ballot, so it is uniform: the
        // chain then runs with every lane active and the ballot selects its result.
        if (all_exc) {
#pragma unroll
            for (int j = 0; j < E; ++j)
                keys.p[j >> 1] = keys.with(j, key_of(chain_fast(f, x(j), dec[j], ctx[j], __uint_as_float(bb(j)))));
        } else if (maybe_exc) {
#pragma unroll
            for (int j = 0; j < E; ++j) {
                const uint64_t m = __ballot(((uint32_t)(dec[j] | ctx[j]) | bw(j)) != 0u);
                if (m) {
                    const uint32_t kc = key_of(chain_fast(f, x(j), dec[j], ctx[j], __uint_as_float(bb(j))));
                    keys.p[j >> 1] = lane_select(m, keys.p[j >> 1], keys.with(j, kc));
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < E; j += 2)
            keys.p[j >> 1] = key_of(chain_ieee(k, x(j), dec[j], ctx[j], __uint_as_float(bb(j)))) |
                             (key_of(chain_ieee(k, x(j + 1), dec[j + 1], ctx[j + 1], __uint_as_float(bb(j + 1)))) << 16);
    }
    if (partial) {
#pragma unroll
        for (int j = 0; j < E; j += 2)
            keys.p[j >> 1] = (ok[j] ? keys.p[j >> 1] & 0xffffu : 0u) | (ok[j + 1] ? keys.p[j >> 1] & 0xffff0000u : 0u);
    }
}

// Processor flags of one row.
struct Uses {
    bool g, rep, mult, bias, remap;
};

__device__ __forceinline__ Uses row_uses(const RowState &rs) {
    Uses u;
    u.g = (rs.ind & IND_GRAMMAR) && rs.grammar;
    u.rep = (rs.ind & (IND_MULT | IND_FREQ | IND_PRES)) && rs.dec;
    u.mult = u.rep && (rs.ind & IND_MULT) && rs.ctx;
    u.bias = (rs.ind & IND_BIAS) && rs.bias;
    u.remap = rs.d2t != nullptr && (u.g || u.rep || u.bias);
    return u;
}

__device__ __forceinline__ Chain row_chain(const RowState &rs, const Uses &u, bool &all_exc) {
    Chain k;
    k.mult = u.mult;
    k.freq = u.rep && (rs.ind & IND_FREQ);
    k.pres = u.rep && (rs.ind & IND_PRES);
    k.bias = u.bias;
    k.temp = (rs.ind & IND_TEMP) != 0;
    k.rep = rs.rep;
    k.fr = rs.freq;
    k.pr = rs.pres;
    k.rdiv = make_divisor(rs.rep);
    k.tdiv = make_divisor(rs.temp);
    all_exc = k.freq && !__builtin_isfinite(rs.freq);
    return k;
}

// The logits of one tile as 4-column words (VEC layout). They depend on the row only, so the
// kernels issue them first, before the request state that decides how the other planes are read.
template <int E>
__device__ __forceinline__ void load_logits_vec(const uint16_t *lrow, int col0, int V,
                                                u32x2 (&lw)[E / 4]) {
    const __amdgpu_buffer_rsrc_t lg = row_buffer(lrow, (int64_t)V * 2);
    const int lane4 = (int)threadIdx.x * 4;
#pragma unroll
    for (int c = 0; c < E / 4; ++c)
        lw[c] = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_raw_buffer_load_b64(lg, lane4 * 2, (col0 + c * (SS_BLOCK * 4)) * 2, NT));
}

// Reads at workgroup-uniform addresses through the constant address space, which the compiler
// serves with scalar loads: they wait on the scalar counter, never on the vector loads already in
// flight. Only for data no kernel of the launch writes.
typedef const __attribute__((address_space(4))) uint32_t *const_u32p;

__device__ __forceinline__ int32_t uniform_i32(const int32_t *p, int idx) {
    return (int32_t)*(const_u32p)(uintptr_t)(p + idx);
}

// p[idx] of a 16-bit array, read as the aligned dword holding it (a dword never crosses a page,
// so the 2 bytes beside the element are always mapped).
__device__ __forceinline__ uint32_t uniform_u16(const uint16_t *p, int idx) {
    const uintptr_t addr = (uintptr_t)(p + idx);
    const uint32_t w = *(const_u32p)(addr & ~(uintptr_t)3);
    return (addr & 2) ? (w >> 16) : (w & 0xffffu);
}

// Per-request bf16 parameter p[slot] as fp32, or `dflt` when p is NULL. `any` is a valid array of
// the same length, read instead of a NULL p so that the reads of a request issue unbranched.
__device__ __forceinline__ float param_bf16(const uint16_t *p, const uint16_t *any, int slot,
                                            float dflt) {
    const uint32_t h = uniform_u16(p ? p : any, slot);
    return p ? bf2f(h) : dflt;
}

// Per-request parameters of a row stage, read with one vector load into one register of every
// wave: lane RP_IND the indicator word, RP_TOPK top_k (SS_K when absent), RP_TOPP / RP_MINP the
// fp32 bits of top_p / min_p (1 / 0 when absent), RP_TOPZ the top-logprob count (dflt_topz when
// absent). Read as scalars they would be live across the merge, whose register pressure spills
// each one right after its load, so that the reads would wait one after another.
enum { RP_IND = 0, RP_TOPK = 1, RP_TOPP = 2, RP_MINP = 3, RP_TOPZ = 4 };

__device__ __forceinline__ uint32_t row_params(const uint16_t *ind, const int32_t *topk,
                                               const uint16_t *topp, const uint16_t *minp,
                                               const int32_t *topz, int slot, int dflt_topz) {
    const int lane = lane_id();
    const void *p = lane == RP_IND    ? (const void *)ind
                    : lane == RP_TOPK ? (const void *)topk
                    : lane == RP_TOPP ? (const void *)topp
                    : lane == RP_MINP ? (const void *)minp
                    : lane == RP_TOPZ ? (const void *)topz
                                      : nullptr;
    const bool wide = lane == RP_TOPK || lane == RP_TOPZ;
    uint32_t v = lane == RP_TOPK   ? (uint32_t)SS_K
                 : lane == RP_TOPP ? 0x3f800000u
                 : lane == RP_TOPZ ? (uint32_t)dflt_topz
                                   : 0u;
    if (p) {
        // 16-bit fields as the aligned dword holding them
        const uintptr_t addr = (uintptr_t)p + (uintptr_t)slot * (wide ? 4u : 2u);
        const uint32_t w = *(const uint32_t *)(addr & ~(uintptr_t)3);
        v = wide ? w : (addr & 2) ? (w >> 16) : (w & 0xffffu);
        if (lane == RP_TOPP || lane == RP_MINP) v <<= 16;
    }
    return v;
}

// Direct layout (no d2t remap, vocabulary a multiple of 4, 8 / 16-byte aligned rows): the side
// planes of one tile -- grammar words, decode and context counts, bias -- as loaded words.
template <int E>
struct Planes {
    u32x2 bw[E / 4];
    i32x4 dw[E / 4], cw[E / 4];
    uint32_t gw[E / 4];
};

// Issues every side-plane load of the tile before any loaded word is consumed. A plane that is
// off reads through an empty buffer, which returns zeros without touching memory.
template <int E>
__device__ __forceinline__ void issue_planes(const RowState &rs, const Uses &u, bool on, int col0,
                                             Planes<E> &pl) {
    const int lane4 = (int)threadIdx.x * 4;
    const bool g = on && u.g, rep = on && u.rep, mult = on && u.mult, bias = on && u.bias;
    const __amdgpu_buffer_rsrc_t gb =
        row_buffer(g ? rs.grammar : nullptr, g ? (int64_t)((rs.vt + 31) >> 5) * 4 : 0);
    const __amdgpu_buffer_rsrc_t db = row_buffer(rep ? rs.dec : nullptr, rep ? (int64_t)rs.vt * 4 : 0);
    const __amdgpu_buffer_rsrc_t cb = row_buffer(mult ? rs.ctx : nullptr, mult ? (int64_t)rs.vt * 4 : 0);
    const __amdgpu_buffer_rsrc_t bb = row_buffer(bias ? rs.bias : nullptr, bias ? (int64_t)rs.vt * 2 : 0);
#pragma unroll
    for (int c = 0; c < E / 4; ++c) {
        const int base = col0 + c * (SS_BLOCK * 4);  // uniform, a multiple of 32
        pl.dw[c] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(db, lane4 * 4, base * 4, NT));
        pl.cw[c] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(cb, lane4 * 4, base * 4, NT));
        pl.bw[c] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(bb, lane4 * 2, base * 2, NT));
        pl.gw[c] = __builtin_amdgcn_raw_buffer_load_b32(gb, (lane4 >> 5) * 4, (base >> 5) * 4, 0);
    }
}

template <int E>
__device__ __forceinline__ void direct_keys(const RowState &rs, const Uses &u, int col0, int V,
                                            const int32_t *hist, const u32x2 (&lw_in)[E / 4],
                                            const Planes<E> &pl, Keys<E> &keys) {
    constexpr int NCH = E / 4;
    const int lane4 = (int)threadIdx.x * 4;
    bool all_exc;
    const Chain k = row_chain(rs, u, all_exc);
    // logits and bias stay in their loaded bf16 pairs and are widened where they are used
    u32x2 lw[NCH];
    bool ok[E];
    int32_t dec[E], ctx[E];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        lw[c] = lw_in[c];
        const bool in = col0 + c * (SS_BLOCK * 4) + lane4 < V;
        dec[4 * c + 0] = pl.dw[c].x; dec[4 * c + 1] = pl.dw[c].y; dec[4 * c + 2] = pl.dw[c].z; dec[4 * c + 3] = pl.dw[c].w;
        ctx[4 * c + 0] = pl.cw[c].x; ctx[4 * c + 1] = pl.cw[c].y; ctx[4 * c + 2] = pl.cw[c].z; ctx[4 * c + 3] = pl.cw[c].w;
#pragma unroll
        for (int i = 0; i < 4; ++i) ok[4 * c + i] = in;
    }
    if (u.g) {
        // a masked element becomes bf16 -inf (0xff80) in place
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t g = pl.gw[c] >> (lane4 & 31);
            lw[c].x = (g & 1u) ? lw[c].x : ((lw[c].x & 0xffff0000u) | 0xff80u);
            lw[c].x = (g & 2u) ? lw[c].x : ((lw[c].x & 0x0000ffffu) | 0xff800000u);
            lw[c].y = (g & 4u) ? lw[c].y : ((lw[c].y & 0xffff0000u) | 0xff80u);
            lw[c].y = (g & 8u) ? lw[c].y : ((lw[c].y & 0x0000ffffu) | 0xff800000u);
        }
    }
    if (u.rep && rs.nhist > 0) {
        // The history never counts token 0: the reference pads the history with 0 and then
        // restores the original count of token 0 (core/naive.py:179-203).
        // Offset of the token from the lane's element 0, compared with each element's constant
        // offset (j / 4) * 1024 + j % 4, so no per-element column is kept live.
        const int base = rs.shard + col0 + 4 * (int)threadIdx.x;
        for (int h = 0; h < rs.nhist; ++h) {
            const int t = hist[h];
            if (t == 0) continue;
            const int d = t - base;
#pragma unroll
            for (int j = 0; j < E; ++j) dec[j] += d == (j >> 2) * (SS_BLOCK * 4) + (j & 3) ? 1 : 0;
        }
    }
    auto x = [&](int j) {
        const uint32_t w = (j & 2) ? lw[j >> 2].y : lw[j >> 2].x;
        return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
    };
    auto bb = [&](int j) {
        const uint32_t w = (j & 2) ? pl.bw[j >> 2].y : pl.bw[j >> 2].x;
        return (j & 1) ? (w & 0xffff0000u) : (w << 16);
    };
    // the bias word of the element's pair, shifted so that -0 in the high half does not count
    auto bw = [&](int j) { return ((j & 2) ? pl.bw[j >> 2].y : pl.bw[j >> 2].x) << 1; };
    auto pair = [&](int j) { return (j & 2) ? lw[j >> 2].y : lw[j >> 2].x; };
    finish_keys<E>(k, all_exc, col0 + SS_BLOCK * E > V, x, pair, all_exc || u.rep || u.mult || u.bias, ok,
                   dec, ctx, bb, bw, keys);
}

// Direct layout, row with every side plane off (no grammar, penalty or bias): the keys come from
// the logits alone and no other plane is read.
template <int E>
__device__ __forceinline__ void plain_keys(const RowState &rs, const Uses &u, int col0, int V,
                                           const u32x2 (&lw)[E / 4], Keys<E> &keys) {
    const int lane4 = (int)threadIdx.x * 4;
    bool all_exc;
    const Chain k = row_chain(rs, u, all_exc);
    bool ok[E];
#pragma unroll
    for (int c = 0; c < E / 4; ++c) {
        const bool in = col0 + c * (SS_BLOCK * 4) + lane4 < V;
#pragma unroll
        for (int i = 0; i < 4; ++i) ok[4 * c + i] = in;
    }
    const int32_t zero[E] = {};
    auto x = [&](int j) {
        const uint32_t w = (j & 2) ? lw[j >> 2].y : lw[j >> 2].x;
        return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
    };
    auto none = [](int) { return 0u; };
    auto pair = [&](int j) { return (j & 2) ? lw[j >> 2].y : lw[j >> 2].x; };
    finish_keys<E>(k, false, col0 + SS_BLOCK * E > V, x, pair, false, ok, zero, zero, none, none, keys);
}

// General layout: d2t-remapped columns (gathers through the target vocabulary) or unaligned rows.
// Largest grammar row that stage_grammar copies into workgroup memory, and the 16-byte quads it
// stages for a vt-token vocabulary.
constexpr int SS_STAGE_MAX_WORDS = 8192;

__host__ __device__ __forceinline__ int stage_quads(int vt) { return (((vt + 31) >> 5) + 3) >> 2; }

// The d2t targets of a tile's E columns (GATHER_VEC layout: each 4-column chunk is one 16-byte
// load), for callers that issue them ahead of the prologue.
template <int E>
__device__ __forceinline__ void load_d2t(const RowState &rs, int col0, int V, int32_t (&tcol)[E]) {
    const __amdgpu_buffer_rsrc_t m = row_buffer(rs.d2t, (int64_t)(rs.shard + V) * 4);
    const int lane4 = (int)threadIdx.x * 4;
#pragma unroll
    for (int c = 0; c < E / 4; ++c) {
        const i32x4 t = __builtin_bit_cast(
            i32x4, __builtin_amdgcn_raw_buffer_load_b128(m, lane4 * 4, (rs.shard + col0 + c * (SS_BLOCK * 4)) * 4, 0));
        tcol[4 * c + 0] = t.x; tcol[4 * c + 1] = t.y; tcol[4 * c + 2] = t.z; tcol[4 * c + 3] = t.w;
    }
}

// PRE: the d2t targets of the E columns come in `pre` (load_d2t, issued by the caller before the
// grammar staging's barrier, so that both round trips overlap) instead of being loaded here.
template <int E, bool VEC, bool PRE = false>
__device__ __forceinline__ void gather_keys(const RowState &rs, const Uses &u, int col0, int V,
                                            const int32_t *hist, const u32x2 (&lw)[E / 4],
                                            Keys<E> &keys, const int32_t *pre = nullptr) {
    constexpr int NCH = E / 4;
    const int lane4 = (int)threadIdx.x * 4;
    bool all_exc;
    const Chain k = row_chain(rs, u, all_exc);

    // logits and bias stay in bf16 pairs (element 2i in the low half), as loaded: widened where
    // they are used, they would hold one register per element
    u32x2 lv[NCH];
    bool ok[E];
    const __amdgpu_buffer_rsrc_t lg = row_buffer(rs.logits, (int64_t)V * 2);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int base = col0 + c * (SS_BLOCK * 4);  // uniform
        if (VEC) {
            lv[c] = lw[c];
            const bool in = base + lane4 < V;
#pragma unroll
            for (int i = 0; i < 4; ++i) ok[4 * c + i] = in;
        } else {
            uint32_t h[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[i] = __builtin_amdgcn_raw_buffer_load_b16(lg, (lane4 + i) * 2, base * 2, NT);
                ok[4 * c + i] = base + lane4 + i < V;
            }
            lv[c].x = h[0] | (h[1] << 16);
            lv[c].y = h[2] | (h[3] << 16);
        }
    }

    int32_t dec[E], ctx[E];
    uint32_t bpk[E / 2];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        dec[j] = 0;
        ctx[j] = 0;
    }
#pragma unroll
    for (int i = 0; i < E / 2; ++i) bpk[i] = 0;
    if (u.g || u.rep || u.bias) {
        int tcol[E];
#pragma unroll
        for (int j = 0; j < E; ++j) tcol[j] = rs.shard + col0 + tile_col(j);
        if (u.remap && PRE) {
#pragma unroll
            for (int j = 0; j < E; ++j) tcol[j] = pre[j];
        } else if (u.remap) {
            const __amdgpu_buffer_rsrc_t m = row_buffer(rs.d2t, (int64_t)(rs.shard + V) * 4);
            if (VEC) {
                // the 4 columns of a chunk are consecutive (and V % 4 == 0): one 16-byte load
#pragma unroll
                for (int c = 0; c < NCH; ++c) {
                    const i32x4 t = __builtin_bit_cast(
                        i32x4, __builtin_amdgcn_raw_buffer_load_b128(m, lane4 * 4, (rs.shard + col0 + c * (SS_BLOCK * 4)) * 4, 0));
                    tcol[4 * c + 0] = t.x; tcol[4 * c + 1] = t.y; tcol[4 * c + 2] = t.z; tcol[4 * c + 3] = t.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < E; ++j) tcol[j] = __builtin_amdgcn_raw_buffer_load_b32(m, tcol[j] * 4, 0, 0);
            }
        }
        // a masked element becomes bf16 -inf (0xff80) in place; a column outside the target
        // vocabulary (negative, or at or past it) reads 0 (masked) on either path
        if (u.g && rs.glds) {
            // Staged row (stage_grammar): a column's word index is clamped to that of lim, the
            // first bit of the zero words past the row, and the bits past the vocabulary in its
            // last word are clear, so the lookup needs no range branch. v_bfe reads the low five
            // bits of its offset operand, the column's bit within the word; a signed one-bit field
            // is 0 or all ones, and the pair's two of them select, half by half, between the pair
            // and two -inf halves.
            const lds_cu32p gl = (lds_cu32p)rs.glds;
            const uint32_t wlim = (uint32_t)(stage_quads(rs.vt) * 4);
#pragma unroll
            for (int i = 0; i < E / 2; ++i) {
                const uint32_t t0 = (uint32_t)tcol[2 * i], t1 = (uint32_t)tcol[2 * i + 1];
                const uint32_t w0 = gl[min(__builtin_amdgcn_ubfe(t0, 5u, 27u), wlim)];
                const uint32_t w1 = gl[min(__builtin_amdgcn_ubfe(t1, 5u, 27u), wlim)];
                const uint32_t k0 = (uint32_t)__builtin_amdgcn_sbfe((int)w0, t0, 1u);
                const uint32_t k1 = (uint32_t)__builtin_amdgcn_sbfe((int)w1, t1, 1u);
                const uint32_t keep = (k0 & 0xffffu) | (k1 & 0xffff0000u);
                const uint32_t p = (i & 1) ? lv[i >> 1].y : lv[i >> 1].x;
                const uint32_t m = (p & keep) | (0xff80ff80u & ~keep);
                if (i & 1) lv[i >> 1].y = m; else lv[i >> 1].x = m;
            }
        } else if (u.g) {
            const __amdgpu_buffer_rsrc_t g = row_buffer(rs.grammar, (int64_t)((rs.vt + 31) >> 5) * 4);
#pragma unroll
            for (int j = 0; j < E; ++j) {
                const uint32_t w = (uint32_t)tcol[j] < (uint32_t)rs.vt
                                       ? __builtin_amdgcn_raw_buffer_load_b32(g, (tcol[j] >> 5) * 4, 0, 0) : 0u;
                const bool keep = ((w >> (tcol[j] & 31)) & 1u) != 0u;
                uint32_t p = (j & 2) ? lv[j >> 2].y : lv[j >> 2].x;
                p = keep ? p : (j & 1) ? ((p & 0x0000ffffu) | 0xff800000u) : ((p & 0xffff0000u) | 0xff80u);
                if (j & 2) lv[j >> 2].y = p; else lv[j >> 2].x = p;
            }
        }
        if (u.rep) {
            const __amdgpu_buffer_rsrc_t d = row_buffer(rs.dec, (int64_t)rs.vt * 4);
#pragma unroll
            for (int j = 0; j < E; ++j) dec[j] = __builtin_amdgcn_raw_buffer_load_b32(d, tcol[j] * 4, 0, 0);
            if (rs.nhist > 0) {
                // The history never counts token 0 (core/naive.py:179-203).
                for (int h = 0; h < rs.nhist; ++h) {
                    const int t = hist[h];
#pragma unroll
                    for (int j = 0; j < E; ++j) dec[j] += (tcol[j] == t && t != 0) ? 1 : 0;
                }
            }
        }
        if (u.mult) {
            const __amdgpu_buffer_rsrc_t q = row_buffer(rs.ctx, (int64_t)rs.vt * 4);
#pragma unroll
            for (int j = 0; j < E; ++j) ctx[j] = __builtin_amdgcn_raw_buffer_load_b32(q, tcol[j] * 4, 0, 0);
        }
        if (u.bias) {
            const __amdgpu_buffer_rsrc_t b = row_buffer(rs.bias, (int64_t)rs.vt * 2);
#pragma unroll
            for (int j = 0; j < E; ++j)
                bpk[j >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(b, tcol[j] * 2, 0, 0) << (16 * (j & 1));
        }
    }
    auto x = [&](int j) {
        const uint32_t w = (j & 2) ? lv[j >> 2].y : lv[j >> 2].x;
        return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
    };
    auto bb = [&](int j) { return (j & 1) ? (bpk[j >> 1] & 0xffff0000u) : (bpk[j >> 1] << 16); };
    // the bias word of the element's pair, shifted so that -0 in the high half does not count
    auto bw = [&](int j) { return bpk[j >> 1] << 1; };
    auto pair = [&](int j) { return (j & 2) ? lv[j >> 2].y : lv[j >> 2].x; };
    finish_keys<E>(k, all_exc, col0 + SS_BLOCK * E > V, x, pair, all_exc || u.rep || u.mult || u.bias, ok,
                   dec, ctx, bb, bw, keys);
}

// Quads of workgroup memory a staged grammar row occupies: stage_grammar fills whole blocks of 64
// quads (one wave's load), and the row is followed by at least one quad of zeros.
__host__ __device__ __forceinline__ int stage_region_quads(int vt) {
    const int quads = stage_quads(vt);
    const int blocks = (quads + 63) >> 6;
    return blocks * 64 > quads ? blocks * 64 : quads + 1;
}

// Copies the grammar row of a `vt`-token vocabulary (ceil(vt / 32) words) into workgroup memory
// `dst` (16-byte aligned, 4 * stage_region_quads(vt) words) with direct global-to-LDS loads
// (buffer_load_dwordx4 ... lds): wave w moves quads [256 i + 64 w, 256 i + 64 w + 64) of the row
// into the same quads of `dst` (the wave's LDS base in M0, 16 bytes per lane), for the blocks that
// start inside the row, so the row passes through no vector registers and the loads stay in
// flight while the wave issues its other loads. Words past the row read 0 (the load's range
// check, dword by dword), so every quad of the last block past the row is zero. Nothing waits
// here: each wave calls stage_grammar_finish after its own loads, and the caller synchronizes the
// workgroup before reading `dst`.
__device__ __forceinline__ void stage_grammar(const uint32_t *grammar, int vt, uint32_t *dst) {
    const int words = (vt + 31) >> 5;
    const __amdgpu_buffer_rsrc_t g = row_buffer(grammar, (int64_t)words * 4);
    const int quads = stage_quads(vt);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    typedef __attribute__((address_space(3))) void *lds_vp;
#pragma unroll
    for (int i = 0; i < SS_STAGE_MAX_WORDS / 4 / SS_BLOCK; ++i) {
        const int q0 = i * SS_BLOCK + wave * 64;  // the wave's first quad (uniform)
        if (q0 < quads)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(g, (lds_vp)(dst + 4 * q0), 16, lane_id() * 16, q0 * 16, 0, 0);
    }
}

// Completes a staged grammar row once the calling wave's loads have landed (it waits for them):
// the wave that loaded the row's last word clears its bits past the vocabulary, and when the row
// ends exactly on a 64-quad block, the quad of zeros after it is written. Then every column at or
// past vt, clamped to word 4 * stage_quads(vt), reads a clear bit. All threads call, before the
// workgroup barrier that publishes `dst`.
__device__ __forceinline__ void stage_grammar_finish(int vt, uint32_t *dst) {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's loads (into LDS too) are done
    const int quads = stage_quads(vt);
    const int last = vt >> 5;  // the word holding bit vt
    if ((vt & 31) != 0 && (int)threadIdx.x == ((last >> 2) & (SS_BLOCK - 1) & ~63))
        dst[last] &= (1u << (vt & 31)) - 1u;
    if ((quads & 63) == 0 && threadIdx.x == 0) *(i32x4 *)(dst + 4 * quads) = i32x4{0, 0, 0, 0};
}

// Memory layouts of the prologue, fixed per launch by the host:
//   MODE_DIRECT      no d2t, vocabulary a multiple of 4, 8 / 16-byte aligned rows: vector loads
//                    of every plane, all issued before any is consumed;
//   MODE_GATHER_VEC  d2t given: vector logit loads, per-element gathers through the target vocab;
//   MODE_SCALAR      anything else: per-element loads throughout.
enum { MODE_DIRECT = 0, MODE_GATHER_VEC = 1, MODE_SCALAR = 2 };

// Gather pass H of a tile (elements j + 16 H, 4 H chunks of 1024 columns further) and the passes
// after it. H is a template parameter so that the keys each pass writes keep constant indices: a
// loop over the passes that the compiler leaves rolled (at E = 64 the body is too large to unroll)
// would index the key array at run time and place it in scratch memory.
template <int E, int MODE, int H>
__device__ __forceinline__ void gather_pass(const RowState &rs, const Uses &u, int col0, int V,
                                            const int32_t *hist, const u32x2 (&lw)[E / 4], Keys<E> &keys) {
    if constexpr (H < E / 16) {
        u32x2 lh[4];
        if constexpr (MODE != MODE_SCALAR && E >= 64) {
            load_logits_vec<16>(rs.logits, col0 + 4 * 4 * SS_BLOCK * H, V, lh);
        } else if constexpr (MODE != MODE_SCALAR) {
#pragma unroll
            for (int c = 0; c < 4; ++c) lh[c] = lw[4 * H + c];
        }
        Keys<16> kh;
        gather_keys<16, MODE == MODE_GATHER_VEC>(rs, u, col0 + 4 * 4 * SS_BLOCK * H, V, hist, lh, kh);
#pragma unroll
        for (int i = 0; i < 8; ++i) keys.p[8 * H + i] = kh.p[i];
        gather_pass<E, MODE, H + 1>(rs, u, col0, V, hist, lw, keys);
    }
}

// Streams one tile of one row through the processor chain and returns the keys (0 = absent).
// `lw` holds the tile's logits from load_logits_vec unless MODE is MODE_SCALAR.
// PRE (GATHER_VEC, E <= 32): the d2t targets of the tile's columns come in `pre` (load_d2t).
template <int E, int MODE, bool PRE = false>
__device__ __forceinline__ void prologue_keys(const RowState &rs, int col0, int V,
                                              const int32_t *hist, const u32x2 (&lw)[E / 4],
                                              Keys<E> &keys, const int32_t *pre = nullptr) {
    static_assert(!PRE || (MODE == MODE_GATHER_VEC && E <= 32), "pre-loaded d2t targets: GATHER_VEC, E <= 32");
    const Uses u = row_uses(rs);
    if constexpr (MODE == MODE_DIRECT) {
        if (!(u.g || u.rep || u.mult || u.bias)) {
            plain_keys<E>(rs, u, col0, V, lw, keys);
        } else if constexpr (E >= 32) {
            // The processor chain in 4096-column passes: element j of pass h is element j + 16 h
            // of the tile (4 h chunks of 1024 columns further). Its per-element state for all E
            // elements at once would set the kernel's register allocation, and so its occupancy,
            // for every row (144 VGPRs at E = 32, three waves per SIMD, against 90 for the plain
            // rows alone).
#pragma unroll
            for (int h = 0; h < E / 16; ++h) {
                // at E = 64 a pass reloads its logits with its planes (in the same round of loads):
                // the preloaded ones would stay live through every pass
                u32x2 lh[4];
                if constexpr (E >= 64) {
                    load_logits_vec<16>(rs.logits, col0 + 4 * 4 * SS_BLOCK * h, V, lh);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) lh[c] = lw[4 * h + c];
                }
                Planes<16> pl;
                issue_planes<16>(rs, u, true, rs.shard + col0 + 4 * 4 * SS_BLOCK * h, pl);
                Keys<16> kh;
                direct_keys<16>(rs, u, col0 + 4 * 4 * SS_BLOCK * h, V, hist, lh, pl, kh);
#pragma unroll
                for (int i = 0; i < 8; ++i) keys.p[8 * h + i] = kh.p[i];
            }
        } else {
            Planes<E> pl;
            issue_planes<E>(rs, u, true, rs.shard + col0, pl);
            direct_keys<E>(rs, u, col0, V, hist, lw, pl, keys);
        }
    } else if constexpr ((E >= 32 && MODE == MODE_GATHER_VEC) || E >= 64) {
        // 4096-column passes, as above: the gathered columns and planes of all 32 elements at
        // once would hold 156 VGPRs (three waves per SIMD).
        if constexpr (E >= 64) {
            gather_pass<E, MODE, 0>(rs, u, col0, V, hist, lw, keys);
        } else {
            // two passes, which the compiler unrolls (and schedules in fewer registers than the
            // recursive form: 96 VGPRs against 102 at E = 32)
#pragma unroll
            for (int h = 0; h < E / 16; ++h) {
                u32x2 lh[4];
                if constexpr (MODE != MODE_SCALAR) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) lh[c] = lw[4 * h + c];
                }
                Keys<16> kh;
                gather_keys<16, MODE == MODE_GATHER_VEC, PRE>(rs, u, col0 + 4 * 4 * SS_BLOCK * h, V, hist, lh, kh,
                                                              PRE ? pre + 16 * h : nullptr);
#pragma unroll
                for (int i = 0; i < 8; ++i) keys.p[8 * h + i] = kh.p[i];
            }
        }
    } else {
        gather_keys<E, MODE == MODE_GATHER_VEC, PRE>(rs, u, col0, V, hist, lw, keys, pre);
    }
}

// Workgroup-wide sum of one count per thread. All threads call.
__device__ __forceinline__ uint32_t block_count(uint32_t n, uint32_t *red) {
    n = wave_sum(n);
    if (lane_id() == 0) red[threadIdx.x >> 6] = n;
    __syncthreads();
    uint32_t s = 0;
#pragma unroll
    for (int w = 0; w < SS_WAVES; ++w) s += red[w];
    __syncthreads();
    return s;
}

__device__ __forceinline__ uint32_t mbcnt64(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// A wave's keys as wave_survivors_masked spilled them to workgroup memory (pair i of lane l at
// TileSmem::keys[wave][i * 64 + l]), read through a volatile pointer: every use is a fresh LDS
// read, so the rare exact cut keeps no copy of the keys in registers and does not set the tile
// kernels' register allocation (at E = 32 it would hold 92 VGPRs instead of 57). The pointer is
// in the LDS address space: through a generic one each read is a flat load that waits for all of
// the wave's memory operations (s_waitcnt vmcnt(0)), one full round trip per key pair.
typedef const volatile __attribute__((address_space(3))) uint32_t *lds_cvu32p;

struct SpilledKeys {
    lds_cvu32p p;
    __device__ __forceinline__ uint32_t pair(int i) const { return p[i * 64]; }
    // this lane's count of keys >= t in the high half and of keys > t in the low half (each at
    // most E, so a workgroup sum of them keeps the halves apart)
    template <int E>
    __device__ __forceinline__ uint32_t count_at(uint32_t t) const {
        uint32_t n = 0;
#pragma unroll 4
        for (int i = 0; i < E / 2; ++i) {
            const uint32_t w = pair(i), a = w & 0xffffu, b = w >> 16;
            n += (a >= t ? 0x10000u : 0u) + (a > t ? 1u : 0u) + (b >= t ? 0x10000u : 0u) + (b > t ? 1u : 0u);
        }
        return n;
    }
    // count of this lane's keys k with pred(k)
    template <int E, class Pred>
    __device__ __forceinline__ uint32_t count(Pred pred) const {
        uint32_t n = 0;
#pragma unroll 4
        for (int i = 0; i < E / 2; ++i) {
            const uint32_t w = pair(i);
            n += (pred(w & 0xffffu) ? 1u : 0u) + (pred(w >> 16) ? 1u : 0u);
        }
        return n;
    }
};

// One wave's part of the exact cut: its elements with key > T, and those key == T elements whose
// bit is set in tie_keep, go to the wave's own LDS region as composites (key << 16) |
// (0xffff - column), placed by ballot and mbcnt, and the wave sorts them there in descending order
// (zero padded to 128). The tie rule keeps every wave within 128.
template <int E>
__device__ __forceinline__ void wave_survivors_exact(TileSmem<E> &sm, const SpilledKeys &sk, uint32_t T,
                                                     uint64_t tie_keep) {
    const int lane = lane_id();
    uint32_t *run = sm.run[__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)];
    const uint32_t cb = 0xffffu - 4u * threadIdx.x;  // 0xffff - column of the lane's element 0
    uint32_t cnt = 0;  // wave-uniform
#pragma unroll 2
    for (int j = 0; j < E; ++j) {
        const uint32_t w = sk.pair(j >> 1);
        const uint32_t key = (j & 1) ? w >> 16 : w & 0xffffu;
        const bool p = key > T || ((tie_keep >> j) & 1ull) != 0ull;
        const uint64_t m = __ballot(p);
        uint32_t *at = run + cnt;  // uniform
        if (p && cnt <= (uint32_t)SS_K)
            at[mbcnt64(m)] = ((key << 16) | cb) - (uint32_t)((j >> 2) * (SS_BLOCK * 4) + (j & 3));
        cnt = min(cnt + (uint32_t)__popcll(m), (uint32_t)SS_K + 1u);
    }
    if (cnt <= 64) {
        uint32_t v = lane < (int)cnt ? run[lane] : 0u;
        wave_sort64_desc(v);
        run[lane] = v;
        run[64 + lane] = 0u;
    } else {
        uint32_t a0 = 2 * lane < (int)cnt ? run[2 * lane] : 0u;
        uint32_t a1 = 2 * lane + 1 < (int)cnt ? run[2 * lane + 1] : 0u;
        wave_bitonic128_desc<2>(a0, a1);
        run[2 * lane] = a0;
        run[2 * lane + 1] = a1;
    }
}

// The survivors (key > T) of one wave, unsorted, in the wave's run, without a ballot per element
// position. Every lane builds a bitmask of its surviving elements with packed 16-bit
// operations (bit i: element 2i, bit 16 + i: element 2i + 1), an exclusive scan of the lanes'
// counts gives each lane its first position in the run, and the lane writes its survivors one
// set bit at a time (a lane holds a few), reading each survivor's key back from its keys stored
// in workgroup memory. Returns the wave's survivor count; above 128 the run is left unwritten
// (the caller takes the exact cut, which rewrites every run).
template <int E>
__device__ __forceinline__ uint32_t wave_survivors_masked(TileSmem<E> &sm, const Keys<E> &keys,
                                                          uint32_t T) {
    constexpr int NM = (E / 2 + 15) / 16;  // 32-bit masks of 16 key pairs each
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint32_t *run = sm.run[wave];
    uint32_t *spill = sm.keys[wave];
    const uint32_t tt = T | (T << 16);
    uint32_t mask[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) mask[m] = 0;
#pragma unroll
    for (int i = 0; i < E / 2; ++i) {
        // max(key - T, 0) is nonzero exactly when key > T; its minimum with 1 is that bit. Written
        // as the two packed 16-bit instructions: as C the compiler turns them into a compare and
        // a select per half and a permute (seven instructions a pair instead of two).
        uint32_t d;
        asm("v_pk_sub_u16 %0, %1, %2 clamp\n\tv_pk_min_u16 %0, %0, %3" : "=&v"(d)
            : "v"(keys.p[i]), "v"(tt), "v"(0x00010001u));
        mask[i >> 4] |= d << (i & 15);
        spill[i * 64 + lane] = keys.p[i];
    }
    uint32_t n = 0;
#pragma unroll
    for (int m = 0; m < NM; ++m) n += (uint32_t)__popc(mask[m]);
    const uint32_t inc = wave_inclusive_sum(n);
    const uint32_t total = lane_u32(inc, 63);
    if (total > (uint32_t)SS_K) return total;
    uint32_t pos = inc - n;
    const uint32_t cb = 0xffffu - 4u * threadIdx.x;  // 0xffff - column of the lane's element 0
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        uint32_t mk = mask[m];
        while (mk) {
            const uint32_t b = (uint32_t)__builtin_ctz(mk);
            mk &= mk - 1u;
            const uint32_t i = 16u * (uint32_t)m + (b & 15u), hi = b >> 4;
            const uint32_t key = (spill[i * 64 + lane] >> (hi << 4)) & 0xffffu;
            const uint32_t j = 2u * i + hi;  // element index; its column offset in the tile
            const uint32_t off = (j >> 2) * (SS_BLOCK * 4) + (j & 3u);
            run[pos++] = ((key << 16) | cb) - off;
        }
    }
    return total;
}

// Tile stage. Greedy rows store one u32 per tile: (key << 16) | (0xffff - column offset), whose
// maximum picks the lowest column among equal maxima. Other rows store their exact top-128 as the
// same composites, sorted in descending order (0 for absent entries), at scratch[tile * 128 ...].
//
// The top-128 is found without a selection over the whole tile. Lower bound: per wave, the
// largest multiple of 4, t, such that the lanes' largest and second-largest keys include at least
// 32 keys >= t,
// so the wave holds at least 32 keys >= t; with lo the smallest of the four wave bounds, the tile
// holds at least 128 keys >= lo. Every wave then collects its survivors (keys >= lo: about 160 of
// a 4096-wide tile of unstructured logits, 30-50 per wave) in its own LDS region and sorts them;
// a two-level merge tree keeps the top-128 of the four sorted runs.
//
// When a wave has more than 128 survivors (long runs of equal keys such as the -inf of
// grammar-masked elements, or the tile's high values concentrated in one wave), the tile finds
// the exact 128th key T (the bound itself when the ties sit there, confirmed by one pair of
// counts; otherwise by bisection on workgroup counts) and ranks the keys equal to T in column
// order with one workgroup scan; the waves then collect the elements with key > T and the first
// 128 - #(key > T) of the ties: exactly the first 128 of the stable descending order, so no wave
// can exceed 128.
template <int E>
__device__ __forceinline__ void tile_stage(TileSmem<E> &sm, bool greedy, const Keys<E> &keys,
                                           uint32_t *scr, int tile, int valid) {
    const int lane = lane_id();
    const int wave = (int)threadIdx.x >> 6;
    if (greedy) {
        // an absent element (key 0) has a composite below 0x10000, under that of every element
        // of the vocabulary, and every tile holds at least one such element
        const uint32_t cb = 0xffffu - 4u * threadIdx.x;
        uint32_t best = 0;
#pragma unroll
        for (int j = 0; j < E; ++j) best = max(best, keys.composite(j, cb));
        best = wave_max_u32(best);
        if (lane == 0) sm.red[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t b = sm.red[0];
            for (int w = 1; w < SS_WAVES; ++w) b = b > sm.red[w] ? b : sm.red[w];
            scr[tile] = b;
        }
        return;
    }
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    uint32_t bound = 0;
    if constexpr (E >= 64) {
        // At 64 elements a lane its largest key alone bounds well: the bound is the largest t (to
        // 14 of the 16 key bits) that at least 32 lane maxima reach, so the wave holds at least 32
        // keys >= t. One packed max a pair, one ballot a bisection step.
        u16x2 a1 = {0, 0};
#pragma unroll
        for (int i = 0; i < E / 2; ++i) a1 = __builtin_elementwise_max(a1, __builtin_bit_cast(u16x2, keys.p[i]));
        const uint32_t m1 = max((uint32_t)a1.x, (uint32_t)a1.y);
#pragma unroll
        for (int b = 15; b >= 2; --b) {
            const uint32_t c = bound | (1u << b);
            if (__popcll(__ballot(m1 >= c)) >= 32) bound = c;
        }
    } else {
        // The lane's largest and second-largest key: the two largest of its even and of its odd
        // elements with packed 16-bit max / min, then the two largest of those four. With few
        // elements a lane (and on the partial last tile of a row) the second-largest keeps the
        // bound tight enough that the survivors fit a wave's run.
        u16x2 a1 = {0, 0}, a2 = {0, 0};
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
            const u16x2 v = __builtin_bit_cast(u16x2, keys.p[i]);
            a2 = __builtin_elementwise_max(a2, __builtin_elementwise_min(a1, v));
            a1 = __builtin_elementwise_max(a1, v);
        }
        const uint32_t m1 = max((uint32_t)a1.x, (uint32_t)a1.y);
        const uint32_t m2 = max(min((uint32_t)a1.x, (uint32_t)a1.y), max((uint32_t)a2.x, (uint32_t)a2.y));
        // 14 of the 16 key bits: the bound may sit up to 3 keys low, which only adds a few survivors
#pragma unroll
        for (int b = 15; b >= 2; --b) {
            const uint32_t c = bound | (1u << b);
            if (__popcll(__ballot(m1 >= c)) + __popcll(__ballot(m2 >= c)) >= 32) bound = c;
        }
    }
    // A wave with fewer than 32 keys above -inf among its lanes' largest ones (few tokens admitted
    // by a grammar, or few valid columns on a row's partial last tile) keeps every key above -inf
    // instead: its bound would otherwise drag the tile's down to -inf, and every other wave's
    // masked elements would then survive. The tile then holds at least 128 survivors only if the
    // waves' counts add up to it, which the check after the survivor pass makes. A tile of fewer
    // than 128 valid columns (`valid`) keeps the plain bounds: all of its columns survive.
    if (bound <= KEY_NEG_INF && valid >= SS_K) bound = KEY_NEG_INF + 1;
    if (lane == 0) sm.red[wave] = bound;
    __syncthreads();
    const uint32_t lo = min(min(sm.red[0], sm.red[1]), min(sm.red[2], sm.red[3]));
    // bounds are multiples of 4 but for a floored one, so lo shows whether one was floored; only
    // then can the survivors of a tile of 128 valid columns or more add up to fewer than 128
    const bool floored = lo == KEY_NEG_INF + 1;
    uint32_t T = lo ? lo - 1 : 0u;  // key 0 (absent) never survives
    const uint32_t cnt = wave_survivors_masked<E>(sm, keys, T);
    if (cnt <= 64) {
        uint32_t *run = sm.run[wave];
        uint32_t v = lane < (int)cnt ? run[lane] : 0u;
        wave_sort64_desc(v);
        run[lane] = v;
        run[64 + lane] = 0u;
    } else if (cnt <= (uint32_t)SS_K) {
        uint32_t *run = sm.run[wave];
        uint32_t a0 = 2 * lane < (int)cnt ? run[2 * lane] : 0u;
        uint32_t a1 = 2 * lane + 1 < (int)cnt ? run[2 * lane + 1] : 0u;
        wave_bitonic128_desc<2>(a0, a1);
        run[2 * lane] = a0;
        run[2 * lane + 1] = a1;
    }
    if (lane == 0) sm.cnt[wave] = cnt;
    __syncthreads();
    const uint32_t n0 = sm.cnt[0], n1 = sm.cnt[1], n2 = sm.cnt[2], n3 = sm.cnt[3];
    bool exact = max(max(n0, n1), max(n2, n3)) > (uint32_t)SS_K;
    // Fewer than 128 survivors, all of the keys above -inf: the tile's first 128 are those and
    // then its first 128 - survivors -inf keys in column order. When the tile's first 256 columns
    // (wave 0's elements 0-3, whose keys the survivor pass spilled) hold that many, wave 0 appends
    // them to the merged survivors (`fill`); otherwise the exact cut runs. Every wave counts them
    // from the spill, so the decision is the same in all of them without another barrier.
    bool fill = false;
    uint32_t survivors = 0;
    if (__builtin_expect(floored, 0)) {
        survivors = n0 + n1 + n2 + n3;
        if (survivors < (uint32_t)SS_K) {
            const uint32_t w0 = sm.keys[0][lane], w1 = sm.keys[0][64 + lane];
            const uint32_t k4[4] = {w0 & 0xffffu, w0 >> 16, w1 & 0xffffu, w1 >> 16};
            uint32_t lead = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) lead += (uint32_t)__popcll(__ballot(k4[i] == KEY_NEG_INF));
            fill = lead >= (uint32_t)SS_K - survivors;
            exact = !fill;
        }
    }
    if (__builtin_expect(exact, 0)) {
        // Exact cut, from the spilled keys. T is the 128th key: usually the bound itself (ties at
        // lo), or, when a wave's bound was floored, the -inf key (the tile holds fewer than 128
        // keys above -inf: ties at the -inf of grammar-masked elements); one pair of counts
        // confirms a candidate. Otherwise bisection.
        const SpilledKeys sk{(lds_cvu32p)(sm.keys[wave] + lane)};
        uint32_t above = 0;  // keys > T
        bool found = false;
        const bool few = floored && n0 + n1 + n2 + n3 < (uint32_t)SS_K;
#pragma unroll 1
        for (int i = 0; i < (floored ? 2 : 1) && !found; ++i) {
            const uint32_t cand = floored && (few == (i == 0)) ? KEY_NEG_INF : lo;
            const uint32_t at = block_count(sk.count_at<E>(cand), sm.red);
            if ((at & 0xffffu) < (uint32_t)SS_K && (at >> 16) >= (uint32_t)SS_K) {
                T = cand;
                above = at & 0xffffu;
                found = true;
            }
        }
        if (!found) {
            uint32_t t = 0;  // the largest t with at least 128 keys >= t
#pragma unroll 1
            for (int b = 15; b >= 0; --b) {
                const uint32_t c = t | (1u << b);
                if (block_count(sk.count<E>([&](uint32_t k) { return k >= c; }), sm.red) >= (uint32_t)SS_K) t = c;
            }
            T = t;
            above = block_count(sk.count<E>([&](uint32_t k) { return k > T; }), sm.red);
        }
        // The first `need` keys equal to T in column order (chunk, thread, element) are kept: their
        // ranks come from one workgroup scan of the tie counts per chunk, chunk after chunk (a
        // runtime loop over the spilled keys, so that the counts of all chunks are never live
        // together: as registers they would set the kernel's allocation).
        const uint32_t need = (uint32_t)SS_K - above;
        uint64_t tie_keep = 0;
        uint32_t before = 0;
        // `before` (ties in earlier chunks) is a workgroup total, so every thread leaves the loop
        // together once `need` ties are ranked: with many ties (the -inf of a grammar that admits
        // few tokens) that is usually after the first chunk, and later chunks keep none
#pragma unroll 1
        for (int c = 0; c < E / 4 && before < need; ++c) {
            const uint32_t w0 = sk.pair(2 * c), w1 = sk.pair(2 * c + 1);
            const uint32_t k4[4] = {w0 & 0xffffu, w0 >> 16, w1 & 0xffffu, w1 >> 16};
            uint32_t eq[1] = {(uint32_t)(k4[0] == T) + (k4[1] == T) + (k4[2] == T) + (k4[3] == T)}, tot[1];
            block_exclusive_scan<1>(eq, tot, sm.scan);
            uint32_t r = before + eq[0];  // rank of this thread's first tie in chunk c
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (k4[i] == T) {
                    tie_keep |= (r < need ? 1ull : 0ull) << (4 * c + i);
                    ++r;
                }
            }
            before += tot[0];
        }
        wave_survivors_exact<E>(sm, sk, T, tie_keep);
        __syncthreads();
    }
    if (wave < 2) {
        // runs 2w and 2w+1, the second reversed: the elementwise maximum is a bitonic sequence
        // holding the top-128 of both
        const uint32_t *A = sm.run[2 * wave], *B = sm.run[2 * wave + 1];
        uint32_t a0 = max(A[2 * lane], B[127 - 2 * lane]);
        uint32_t a1 = max(A[2 * lane + 1], B[126 - 2 * lane]);
        wave_bitonic128_desc<128>(a0, a1);
        sm.run2[wave][2 * lane] = a0;
        sm.run2[wave][2 * lane + 1] = a1;
    }
    __syncthreads();
    if (wave == 0) {
        uint32_t c0 = max(sm.run2[0][2 * lane], sm.run2[1][127 - 2 * lane]);
        uint32_t c1 = max(sm.run2[0][2 * lane + 1], sm.run2[1][126 - 2 * lane]);
        wave_bitonic128_desc<128>(c0, c1);
        *(uint2 *)(scr + tile * SS_K + 2 * lane) = make_uint2(c0, c1);
        if (__builtin_expect(fill, 0)) {
            // The merged survivors took positions 0 .. survivors - 1 and zeros the rest; the -inf
            // key of column c = 4 * lane + i (c < 256) with rank r among them overwrites position
            // survivors + r while r < 128 - survivors. Its keys come from the survivor pass's
            // spill (nothing has written over them since). The list's store, which other lanes
            // of the wave made to the same positions, completes before these issue (vmcnt(0)).
            const uint32_t need = (uint32_t)SS_K - survivors;
            const uint32_t w0 = sm.keys[0][lane], w1 = sm.keys[0][64 + lane];
            const uint32_t k4[4] = {w0 & 0xffffu, w0 >> 16, w1 & 0xffffu, w1 >> 16};
            uint32_t r = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) r += mbcnt64(__ballot(k4[i] == KEY_NEG_INF));
            __builtin_amdgcn_s_waitcnt(0x0f70);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (k4[i] == KEY_NEG_INF) {
                    if (r < need)
                        scr[tile * SS_K + survivors + r] = (KEY_NEG_INF << 16) | (0xffffu - (uint32_t)(4 * lane + i));
                    ++r;
                }
            }
        }
    }
}

// Greedy merge over the tiles' maxima (wave 0): the largest value, lowest column on ties.
// `first` is the composite of list `lane`, read ahead by load_samples.
__device__ __forceinline__ int greedy_merge(const uint32_t *scr, int tiles, const ListMap &lm, int V,
                                            uint32_t first) {
    uint64_t best = 0;
    for (int t = lane_id(); t < tiles; t += 64) {
        const uint32_t c = t < 64 ? first : scr[lm.greedy_entry(t)];
        const uint64_t c64 = ((uint64_t)(c >> 16) << 32) | ((uint64_t)(0xffffu - (uint32_t)t) << 16) |
                             (uint64_t)(c & 0xffffu);
        best = best > c64 ? best : c64;
    }
    best = wave_max_u64(best);
    const int tile = (int)(0xffffu - (uint32_t)((best >> 16) & 0xffffu));
    const int off = (int)(0xffffu - (uint32_t)(best & 0xffffu));
    const int idx = lm.base(tile) + off;
    return idx < V ? idx : V - 1;
}

// Selects the row's top-128 among `nsc` blocks of candidates and leaves them, in column order,
// as (key << 8 | 127 - pos) composites and column indices in sm.cand / sm.idx.
template <bool HELD, int EM, class Load, class Cand>
__device__ __forceinline__ void merge_select(SampleSmem &sm, int nsc, Load load, Cand cand,
                                             const ListMap &lm, int V) {
    uint32_t thi, margin;
    int level;
    radix_threshold<EM, 16>(sm.sel, nsc, load, (uint32_t)SS_K, thi, level, margin);
    compact<EM, 4>(sm.sel, nsc, load, thi, level, margin, [&](uint32_t pos, int sc, int j) {
        if (pos >= (uint32_t)SS_K) return;
        const int p = order_pos<EM, 4>(sc, j);
        const uint32_t c = cand(sc, j);
        const int idx = lm.base(p / SS_K) + (int)(0xffffu - (c & 0xffffu));
        sm.cand[pos] = ((uint64_t)(c >> 16) << 8) | (uint64_t)(127u - pos);
        sm.idx[pos] = idx < V ? idx : V - 1;  // only an absent-element sentinel can exceed V
    });
}

// Exact row merge by radix selection over every candidate (any tile order). All threads call; on
// return wave 0 holds the row's top-128 sorted by (value desc, column asc), element
// e = 2 * lane + i as (v_i, idx_i). Up to 4096 candidates are read once with 16-byte loads and
// kept in registers; larger rows stream them from the scratch per pass.
__device__ __forceinline__ void merge_row_radix(SampleSmem &sm, const uint32_t *scr, int tiles,
                                                const ListMap &lm, int V, float &v0, float &v1, int &i0,
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
            [&](int, int j) { return held[j]; }, lm, V);
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
            [&](int sc, int j) { return scr[order_pos<EM, 4>(sc, j)]; }, lm, V);
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

// The merge inputs of one row, read at the start of a row kernel so that their latency overlaps
// the reads of the request state: every thread's two sample slots of merge_row, and for wave 0
// the first unmerged entry of list t = lane (lists from 64 on are read inside the merge).
struct RowSamples {
    uint32_t raw[2];   // list entries of the thread's two elements (0 past the last slot)
    int slot[2];       // their sample slots s = list * kp + position
    int base[2];       // first column of their lists' tiles
    uint32_t next;
    uint32_t greedy;   // wave 0: tile t = lane's greedy composite, had the row been greedy
    int kp;            // merged prefix length of every list
    uint32_t kpm;      // ceil(2^16 / kp): (s * kpm) >> 16 == s / kp for every slot s < 512
};

__device__ __forceinline__ int merge_prefix(int tiles) { return min(SS_K, (4 * SS_K) / tiles); }

// List of sample slot s (< 512).
__device__ __forceinline__ int slot_list(const RowSamples &smp, int s) {
    return (int)(((uint32_t)s * smp.kpm) >> 16);
}

// Run length of whole sorted lists placed in a wave's 128 elements: kp when kp is a power of two
// from 8 to 64 (then 128 / kp lists per wave, odd ones reversed, so that the bitonic network can
// start at merge size 2 kp), else 1 (arbitrary placement, full sort).
__device__ __forceinline__ int merge_run(int kp) {
    return (kp >= 8 && kp <= 64 && (kp & (kp - 1)) == 0) ? kp : 1;
}

// BUF: `scr` is a global scratch row of tiles * 128 words, read by range-checked buffer loads (an
// entry outside the row reads 0), so that every load issues unbranched, ahead of whatever the
// kernel waits for next; else `scr` may be workgroup memory.
template <bool BUF = false>
__device__ __forceinline__ void load_samples(const uint32_t *scr, int tiles, const ListMap &lm,
                                             RowSamples &smp) {
    const int words = tiles * SS_K;
    auto at = [&](bool ok, int w) -> uint32_t {
        if constexpr (BUF) {
            const __amdgpu_buffer_rsrc_t rb = row_buffer(scr, (int64_t)words * 4);
            return __builtin_amdgcn_raw_buffer_load_b32(rb, (ok ? w : words) * 4, 0, 0);
        } else {
            return ok ? scr[w] : 0u;
        }
    };
    const int kp = merge_prefix(tiles);
    smp.kp = kp;
    // above 512 tiles kp is 0: nothing is merged and the exactness check sends the row to the
    // radix merge
    smp.kpm = kp ? (65536u + (uint32_t)kp - 1u) / (uint32_t)kp : 0u;
    const int ns = tiles * kp;  // <= 512
    const int run = merge_run(kp);
    const int wave = (int)threadIdx.x >> 6, lane = lane_id();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        // run > 1: element e = 2 * lane + i of the wave is in run r = e / kp, i.e. list
        // 128 / kp * wave + r; else any placement. With BUF both are computed and one is
        // selected, so that no branch separates the loads below from the kernel's start (the
        // singular row kernel measured faster with the branch).
        int s, list;
        const int lr = __builtin_ctz((unsigned)run);
        const int e = 2 * lane + i;
        const int r = e >> lr, q = e & (run - 1);
        if (BUF) {
            const int list_r = wave * (SS_K >> lr) + r;
            const int s_r = (list_r << lr) + ((r & 1) ? run - 1 - q : q);
            const int s_a = 2 * (int)threadIdx.x + i;
            s = run > 1 ? s_r : s_a;
            list = run > 1 ? list_r : slot_list(smp, s_a);
        } else if (run > 1) {
            list = wave * (SS_K >> lr) + r;
            s = (list << lr) + ((r & 1) ? run - 1 - q : q);
        } else {
            s = 2 * (int)threadIdx.x + i;
            list = slot_list(smp, s);
        }
        smp.slot[i] = s;
        smp.base[i] = lm.base(list);
        smp.raw[i] = at(s < ns, list * SS_K + (s - list * kp));
    }
    const int t = (int)threadIdx.x;
    smp.next = at(t < 64 && t < tiles && kp < SS_K, t * SS_K + kp);
    // read before the row's indicator is known, so that a greedy row's merge waits for no
    // further load
    smp.greedy = at(t < 64 && t < tiles, lm.greedy_entry(t));
}

// Lists that merge_refill merges whole; a row with more lists beating its sampled top-128 takes
// the radix merge.
constexpr int SS_REFILL_LISTS = 16;

// Completes an inexact sampled merge (wave 0; `f0`/`f1` hold the sorted top-128 of the samples as
// slot composites). They are rewritten as entry composites (key << 16) | (0xffff - g) with
// g = list * 128 + position (< 2^16 for tiles <= 512), whose order is again (value desc, column
// asc). Then, list by list in tile order, a list whose first unmerged entry beats the current
// 128th element has its remaining 128 - kp entries merged in: the elementwise maximum of the
// sorted top-128 and the list's entries in reverse order is bitonic and holds the top-128 of
// both. The 128th element only rises, so a list that does not beat it when visited never does
// later, and every list that did is merged whole: the result is the row's exact top-128.
__device__ __forceinline__ void merge_refill(const uint32_t *scr, const RowSamples &smp, int tiles,
                                             const ListMap &lm, int V, uint32_t f0, uint32_t f1,
                                             float &v0, float &v1, int &i0, int &i1) {
    const int lane = lane_id();
    const int kp = smp.kp;
    auto to_entry = [&](uint32_t f) -> uint32_t {
        if (!f) return 0u;
        const int s = (int)(0xffffu - (f & 0xffffu));
        const int l = slot_list(smp, s);
        return (f & 0xffff0000u) | (0xffffu - (uint32_t)(l * SS_K + s - l * kp));
    };
    f0 = to_entry(f0);
    f1 = to_entry(f1);
    for (int t0 = 0; t0 < tiles; t0 += 64) {
        const int t = t0 + lane;
        const uint32_t nx = t >= tiles ? 0u : t < 64 ? smp.next : scr[t * SS_K + kp];
        const uint32_t cn = nx ? (nx & 0xffff0000u) | (0xffffu - (uint32_t)(t * SS_K + kp)) : 0u;
        uint64_t m = __ballot(cn > lane_u32(f1, 63));
        while (m) {
            const int l = t0 + (int)__builtin_ctzll(m);
            uint32_t r[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                // element e pairs with entry kp + 127 - e of list l (entries kp .. 127 exist)
                const int e = 2 * lane + i;
                const int g = l * SS_K + kp + 127 - e;
                const uint32_t raw = e >= kp ? scr[g] : 0u;
                r[i] = raw ? (raw & 0xffff0000u) | (0xffffu - (uint32_t)g) : 0u;
            }
            f0 = max(f0, r[0]);
            f1 = max(f1, r[1]);
            wave_bitonic128_desc<128>(f0, f1);
            m &= m - 1;
            m &= __ballot(cn > lane_u32(f1, 63));
        }
    }
    auto column = [&](uint32_t f) -> int {
        if (!f) return V - 1;
        const int g = (int)(0xffffu - (f & 0xffffu));
        const int idx = lm.base(g >> 7) + (int)(0xffffu - (scr[g] & 0xffffu));
        return idx < V ? idx : V - 1;
    };
    v0 = bf2f(unkey16(f0 >> 16));
    v1 = bf2f(unkey16(f1 >> 16));
    i0 = column(f0);
    i1 = column(f1);
}

// Row merge over the tiles' sorted candidate lists, from the samples of load_samples. All threads
// call; on return wave 0 holds the row's top-128 sorted by (value desc, column asc), element
// e = 2 * lane + i as (v_i, idx_i), and sm.tok[e] holds idx_e, visible to every wave (the return
// follows a barrier).
//
// Only the first kp = min(128, 512 / tiles) entries of every list are merged: 512 sample slots,
// slot s = list * kp + position, as composites (key << 16) | (0xffff - s), whose order is the
// (value desc, column asc) order because lists are in tile order and equal keys of one list are
// in column order. Each wave sorts 128 slots (from merge size 2 kp when whole lists fill its
// elements, see merge_run), and two rounds of bitonic merges keep the top-128 of the four runs.
// The result is exact unless some list holds more than kp of the row's top-128, i.e. unless a
// list's first unmerged entry beats the 128th merged one. Up to SS_REFILL_LISTS such lists are
// merged whole by merge_refill; more (or tiles > 512) fall back to the radix merge over every
// candidate.
__device__ __forceinline__ void merge_row(SampleSmem &sm, const uint32_t *scr,
                                          const RowSamples &smp, int tiles, const ListMap &lm, int V,
                                          float &v0, float &v1, int &i0, int &i1) {
    const int lane = lane_id();
    const int wave = (int)threadIdx.x >> 6;
    const int kp = smp.kp;
    uint32_t c[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int s = smp.slot[i];
        uint32_t comp = 0;
        const uint32_t raw = smp.raw[i];
        if (raw) {
            const int idx = smp.base[i] + (int)(0xffffu - (raw & 0xffffu));
            sm.col[s] = idx < V ? idx : V - 1;
            comp = (raw & 0xffff0000u) | (0xffffu - (uint32_t)s);
        }
        c[i] = comp;
    }
    // sorted lists in alternating directions are already the runs of a bitonic network of size
    // 2 * run; equal composites cannot occur (the slot is part of them)
    switch (merge_run(kp)) {
        case 8: wave_bitonic128_desc<16>(c[0], c[1]); break;
        case 16: wave_bitonic128_desc<32>(c[0], c[1]); break;
        case 32: wave_bitonic128_desc<64>(c[0], c[1]); break;
        case 64: wave_bitonic128_desc<128>(c[0], c[1]); break;
        default: wave_bitonic128_desc<2>(c[0], c[1]); break;
    }
    sm.runs[wave][2 * lane] = c[0];
    sm.runs[wave][2 * lane + 1] = c[1];
    __syncthreads();
    if (wave < 2) {
        // top-128 of runs (2w, 2w+1): the elementwise maximum against the reversed second run is
        // a bitonic sequence holding them
        const uint32_t *a = sm.runs[2 * wave], *b = sm.runs[2 * wave + 1];
        uint32_t x0 = max(a[2 * lane], b[127 - 2 * lane]);
        uint32_t x1 = max(a[2 * lane + 1], b[126 - 2 * lane]);
        wave_bitonic128_desc<128>(x0, x1);
        sm.runs[2 * wave][2 * lane] = x0;
        sm.runs[2 * wave][2 * lane + 1] = x1;
    }
    __syncthreads();
    uint32_t f0 = 0, f1 = 0;
    int beats = 0;
    if (wave == 0) {
        f0 = max(sm.runs[0][2 * lane], sm.runs[2][127 - 2 * lane]);
        f1 = max(sm.runs[0][2 * lane + 1], sm.runs[2][126 - 2 * lane]);
        wave_bitonic128_desc<128>(f0, f1);
        // exactness check: no list's first unmerged entry may beat the 128th merged element.
        // At equal keys the entry of list t comes first iff t is below the list of that element:
        // tiles are in column order and a list's unmerged entries follow its merged ones.
        const uint32_t last = lane_u32(f1, 63);
        const uint32_t klast = last >> 16;
        const int llast = last ? slot_list(smp, (int)(0xffffu - (last & 0xffffu))) : tiles;
        if (kp < SS_K) {
            for (int t0 = 0; t0 < tiles; t0 += 64) {
                const int t = t0 + lane;
                const uint32_t nx = t >= tiles ? 0u : t < 64 ? smp.next : scr[t * SS_K + kp];
                const uint32_t kn = nx >> 16;
                beats += __popcll(__ballot(nx != 0u && (kn > klast || (kn == klast && t < llast))));
            }
        }
        // exact (refilled when few lists are short), or the radix merge by every wave after the
        // barrier; one barrier publishes both the decision and the exact result's columns
        const bool radix = beats > SS_REFILL_LISTS || (beats > 0 && kp == 0);
        if (lane == 0) sm.flag = radix ? 1 : 0;
        if (!radix) {
            if (beats > 0) {
                merge_refill(scr, smp, tiles, lm, V, f0, f1, v0, v1, i0, i1);
            } else {
                v0 = bf2f(unkey16(f0 >> 16));
                v1 = bf2f(unkey16(f1 >> 16));
                i0 = f0 ? sm.col[0xffffu - (f0 & 0xffffu)] : V - 1;
                i1 = f1 ? sm.col[0xffffu - (f1 & 0xffffu)] : V - 1;
            }
            sm.tok[2 * lane] = i0;
            sm.tok[2 * lane + 1] = i1;
        }
    }
    __syncthreads();
    if (sm.flag) {
        merge_row_radix(sm, scr, tiles, lm, V, v0, v1, i0, i1);
        if (wave == 0) {
            sm.tok[2 * lane] = i0;
            sm.tok[2 * lane + 1] = i1;
        }
        __syncthreads();
    }
}

// exp(v - m) of the lane's two elements of the sorted top-128 (wave 0), m = v[0] (the maximum),
// kept across the truncation stages and the log-softmax that follows them. A stage that removes
// an element (v = -inf) sets its part to exp(-inf - m), the value recomputing it would give, so
// every later sum reads exactly the parts it would recompute; they are recomputed when v[0] is no
// longer m (position 0 removed by an out-of-range parameter, or NaN).
struct SoftmaxParts {
    float m = 0.0f, x0 = 0.0f, x1 = 0.0f;
    bool valid = false;
};

// Sum of exp(v - v[0]) over the wave's 128 elements, with `sp` holding m = v[0] and the parts.
__device__ __forceinline__ float softmax_sum(SoftmaxParts &sp, float v0, float v1) {
    const float m = lane_f32(v0, 0);
    if (!sp.valid || !(m == sp.m)) {
        sp.m = m;
        sp.x0 = expf(v0 - m);
        sp.x1 = expf(v1 - m);
        sp.valid = true;
    }
    return wave_sum_f32(sp.x0 + sp.x1);
}

// Removes the lane's elements whose flag is set: v = -inf, part exp(-inf - m).
__device__ __forceinline__ void softmax_remove(SoftmaxParts &sp, bool r0, bool r1, float &v0, float &v1) {
    if (r0) v0 = -INFINITY;
    if (r1) v1 = -INFINITY;
    if (sp.valid) {
        const float z = expf(-INFINITY - sp.m);
        if (r0) sp.x0 = z;
        if (r1) sp.x1 = z;
    }
}

// top-k -> top-p -> min-p on the sorted top-128 (wave 0), each on the values left by the
// previous one, as in reference core/naive.py:270-328 (applied in that order by
// `thread_first(values, self.top_k, self.top_p, self.min_p)`, core/naive.py:338). `sp` leaves
// with the softmax parts of the last stage that took them.
__device__ __forceinline__ void truncate(uint32_t ind, int32_t topk, float topp, float minp,
                                         float &v0, float &v1, SoftmaxParts &sp) {
    const int e0 = 2 * lane_id(), e1 = e0 + 1;
    if (ind & IND_TOPK) softmax_remove(sp, e0 >= topk, e1 >= topk, v0, v1);
    if (ind & IND_TOPP) {
        // softmax in fp32 (x * (1 / sum)), cumulative sum accumulated in fp64 and compared in
        // fp32 against p; position 0 is always kept.
        const float s = softmax_sum(sp, v0, v1);
        const float inv = 1.0f / s;
        const float p0 = sp.x0 * inv, p1 = sp.x1 * inv;
        const double inc = wave_inclusive_sum_f64((double)p0 + (double)p1);
        const double exc = shift_up1_f64(inc);  // 0 in lane 0
        const double c0 = exc + (double)p0, c1 = c0 + (double)p1;
        softmax_remove(sp, e0 > 0 && (float)c0 > topp, (float)c1 > topp, v0, v1);
    }
    if (ind & IND_MINP) {
        // bf16 softmax, masked where the rounded probability is below bf16(min_p * p_max).
        const float s = softmax_sum(sp, v0, v1);
        const float inv = 1.0f / s;
        const float s0 = rbf(sp.x0 * inv), s1 = rbf(sp.x1 * inv);
        const float lower = rbf(minp * lane_f32(s0, 0));
        softmax_remove(sp, s0 < lower, s1 < lower, v0, v1);
    }
}

// wave_argmax_first for bfloat16 values z (the low 16 bits of each float are zero): distinct
// values differ in the upper half of their order keys, so that half and the position make one
// 32-bit word and the reduction runs on single words.
__device__ __forceinline__ int wave_argmax_first_bf16(float z0, float z1) {
    const int e0 = 2 * lane_id();
    const uint32_t a = (key32(__float_as_uint(z0)) & 0xffff0000u) | (uint32_t)(127 - e0);
    const uint32_t b = (key32(__float_as_uint(z1)) & 0xffff0000u) | (uint32_t)(126 - e0);
    return 127 - (int)(wave_max_u32(a > b ? a : b) & 0xffffu);
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
