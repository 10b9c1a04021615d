// Fused single-step sampling (replaces K1 ops/prologue.py:272-472 followed by K4
// ops/singular.py:154-358 of the reference), as two back-to-back launches on the caller's stream.
//
// Tile stage, grid (tiles, rows): every workgroup runs the logit-processor prologue over one
// vocabulary tile of one row and leaves either the tile argmax (greedy rows) or its exact top-128
// in the row's scratch. Row stage, grid rows: one workgroup per row merges the candidates and
// performs the selection: truncation, d2t remap, Gumbel-max over bf16(v - w), decode-count update,
// logprobs, top-Z logprobs and the draft-probability scatter. The launch boundary orders the two
// stages across all XCDs without per-workgroup cache maintenance. Semantics follow the
// reference's PyTorch path (core/naive.py:377-495 `selection`, :648-692 `preamble` / `singular`).
#include <atomic>
#include <mutex>

#include "ss_launch.h"
#include "ss_sampling.h"
#include "../../include/sonic_sampler.h"

// Candidate lists of ss_fused_singular_noalloc. Host code never names this array in a launch or a
// copy: its device address comes from hipGetSymbolAddress, once per device (static_scratch).
static __device__ __align__(256) uint32_t scratch[SS_STATIC_SCRATCH_BYTES / 4];

namespace ss {

__device__ __forceinline__ RowState singular_row_state(const ss_singular_args &a, int row,
                                                       int slot, uint32_t ind) {
    RowState rs;
    rs.ind = ind;
    rs.logits = a.logits + (int64_t)row * a.stride_logits;
    rs.d2t = a.d2t;
    rs.grammar = a.grammar ? a.grammar + (int64_t)slot * a.stride_grammar : nullptr;
    rs.ctx = a.context_counts ? a.context_counts + (int64_t)slot * a.stride_context : nullptr;
    rs.dec = a.decode_counts ? a.decode_counts + (int64_t)slot * a.stride_decode : nullptr;
    rs.bias = a.logit_bias ? a.logit_bias + (int64_t)slot * a.stride_bias : nullptr;
    const float rep = param_bf16(a.repetition, a.indicators, slot, 1.0f);
    const float freq = param_bf16(a.frequency, a.indicators, slot, 0.0f);
    const float pres = param_bf16(a.presence, a.indicators, slot, 0.0f);
    const float temp = param_bf16(a.temperature, a.indicators, slot, 1.0f);
    rs.rep = (ind & IND_MULT) ? rep : 1.0f;
    rs.freq = (ind & IND_FREQ) ? freq : 0.0f;
    rs.pres = (ind & IND_PRES) ? pres : 0.0f;
    rs.temp = (ind & IND_TEMP) ? temp : 1.0f;
    if (!a.temperature) rs.ind &= ~IND_TEMP;
    rs.vt = a.target_vocab > 0 ? a.target_vocab : a.vocab_size;
    rs.nhist = 0;
    rs.glds = nullptr;
    rs.shard = a.world_size > 1 ? a.local_rank * a.shard_size : 0;
    return rs;
}

// Tile stage: grid (tiles, rows). With d2t and a grammar mask, `stage_words` > 0 stages the
// row's grammar words in workgroup memory (dynamic shared memory) before the prologue, so that the
// per-element lookups through d2t read LDS: as scattered global gathers (one cache line per
// element) they are bounded by the vector cache's line rate, not by HBM. Such launches number
// their workgroups XCD by XCD (xcd_grouped), so that a row's tiles share one L2.
template <int E, int MODE>
__global__ __launch_bounds__(SS_BLOCK) void singular_tiles_kernel(const uint16_t *p_logits, int64_t p_stride,
                                                                  int p_block_n, int p_vocab, int tiles,
                                                                  int stage_words, const int32_t *p_slots,
                                                                  const uint16_t *p_ind, ss_singular_args a) {
    // the tile stage's memory and, overlaying its runs and keys, a staged grammar row (dynamic
    // shared memory of tile_smem_bytes)
    extern __shared__ __align__(16) uint32_t tile_smem[];
    TileSmem<E> &sm = *reinterpret_cast<TileSmem<E> *>(tile_smem);
    uint32_t *grammar_words = tile_smem + TILE_OVERLAY / 4;
    int row = blockIdx.y, tile = blockIdx.x;
    if (MODE != MODE_DIRECT && stage_words > 0) {
        // the tiles of a row stage the same grammar row: run them on one XCD, whose L2 then
        // fetches it once
        const int v = xcd_grouped((int)(blockIdx.y * gridDim.x + blockIdx.x), (int)(gridDim.x * gridDim.y));
        row = v / tiles;
        tile = v - row * tiles;
    }
    u32x2 lw[E / 4];
    if (MODE != MODE_SCALAR) load_logits_vec<E>(p_logits + (int64_t)row * p_stride, tile * p_block_n, p_vocab, lw);
    // the row's slot and indicator decide which planes the tile reads: through preloaded pointers
    const int slot = p_slots ? uniform_i32(p_slots, row) : row;
    const uint32_t ind = uniform_u16(p_ind, slot);
    RowState rs = singular_row_state(a, row, slot, ind);
    bool sync = false;
    const Uses u = row_uses(rs);
    if (MODE != MODE_DIRECT && stage_words > 0 && u.g && u.remap) {
        stage_grammar(rs.grammar, rs.vt, grammar_words);
        rs.glds = grammar_words;
        sync = true;
    }
    // the d2t targets of the tile's columns, requested while the grammar row is staged: the
    // workgroup barrier below then waits for both rounds of loads at once
    constexpr bool PRE = MODE == MODE_GATHER_VEC && E <= 32;
    int32_t pre[PRE ? E : 1];
    if constexpr (PRE) {
        if (u.remap) load_d2t<E>(rs, tile * a.block_n, a.vocab_size, pre);
    }
    if (a.drafted_tokens && a.timestep > 0 && (ind & (IND_MULT | IND_FREQ | IND_PRES))) {
        rs.nhist = a.timestep;
        if ((int)threadIdx.x < rs.nhist)
            sm.hist[threadIdx.x] = a.drafted_tokens[(int64_t)row * a.stride_drafted + threadIdx.x];
        sync = true;
    }
    if (rs.glds) stage_grammar_finish(rs.vt, grammar_words);
    if (sync) __syncthreads();
    Keys<E> keys;
    prologue_keys<E, MODE, PRE>(rs, tile * a.block_n, a.vocab_size, sm.hist, lw, keys, pre);
    // this shard's slice of the row's [world_size, tiles, 128] lists
    uint32_t *scr = a.scratch + (int64_t)row * a.stride_scratch + (a.world_size > 1 ? a.local_rank * tiles * SS_K : 0);
    tile_stage<E>(sm, (ind & IND_GREEDY) != 0, keys, scr, tile, min(a.block_n, a.vocab_size - tile * a.block_n));
}

// Greedy row (wave 0): the argmax over the tiles' maxima, d2t remap, count update, outputs.
// `first` is scr[lane], read ahead by load_samples.
__device__ __forceinline__ void singular_greedy(const ss_singular_args &a, const uint32_t *scr,
                                                int lists, const ListMap &lm, int V, int row, int slot,
                                                uint32_t first) {
    if (threadIdx.x >= 64) return;
    int token = greedy_merge(scr, lists, lm, V, first);
    if (a.d2t) token = a.d2t[token];
    if (threadIdx.x == 0) {
        if (a.update_counts && a.decode_counts) {
            int32_t *d = a.decode_counts + (int64_t)slot * a.stride_decode + token;
            if (a.is_prefill) atomicExch(d, 1); else atomicAdd(d, 1);
        }
        if (a.return_logprobs && a.logprobs) a.logprobs[(int64_t)row * a.stride_logprobs] = 0;
        a.tokens[(int64_t)row * a.stride_tokens] = token;
    }
}

// Selection of a non-greedy row from its sorted top-128 (wave 0 holds element e = 2 * lane + i
// as (v_i, idx_i), sm.tok[e] = idx_e as merge_row leaves them): truncation, d2t remap, Gumbel-max
// over bf16(v - w), count update, logprobs, top-Z logprobs and the probability scatter. All
// threads call.
__device__ __forceinline__ void singular_select(const ss_singular_args &a, SampleSmem &sm, int row,
                                                int slot, uint32_t prm, float v0, float v1, int i0,
                                                int i1) {
    const uint32_t ind = lane_u32(prm, RP_IND);
    // Waves 1 and 2 remap the 128 candidates' columns and draw their noise (one candidate per
    // lane) while wave 0 applies the truncation and the log-softmax.
    const int wave = (int)threadIdx.x >> 6;
    const int lane = lane_id();
    const int e0 = 2 * lane, e1 = e0 + 1;
    if (wave == 1 || wave == 2) {
        const int e = (wave - 1) * 64 + lane;
        int t = sm.tok[e];
        if (a.d2t) t = a.d2t[t];
        sm.noise[e] = a.philox.enabled
                          ? philox_gumbel(a.philox.seed, a.philox.offset, slot, a.philox_step, t)
                          : bf2f(a.gumbel[(int64_t)slot * a.stride_gumbel + t]);
        sm.tok[e] = t;
    }
    // wave 0: the truncation, then the log-softmax of the truncated values (independent of the
    // noise, so it runs before the barrier, while waves 1 and 2 draw the noise)
    const bool want_lp = a.return_logprobs && a.logprobs;
    const bool want_probs = a.return_probabilities && a.probabilities;
    float o0 = 0.0f, o1 = 0.0f;  // the logprob of each element as the reference computes it
    if (wave == 0) {
        SoftmaxParts sp;
        truncate(ind, (int32_t)lane_u32(prm, RP_TOPK), __uint_as_float(lane_u32(prm, RP_TOPP)),
                 __uint_as_float(lane_u32(prm, RP_MINP)), v0, v1, sp);
        if (want_lp || want_probs) {
            const float logs = logf(softmax_sum(sp, v0, v1));
            if (want_probs) {
                // log_softmax in fp32: (v - max) - log(sum)
                o0 = (v0 - sp.m) - logs;
                o1 = (v1 - sp.m) - logs;
            } else {
                // v - logsumexp(v), logsumexp = max + log(sum(exp(v - max)))
                const float lse = sp.m + logs;
                o0 = v0 - lse;
                o1 = v1 - lse;
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;
    i0 = sm.tok[e0];
    i1 = sm.tok[e1];
    const float w0 = sm.noise[e0], w1 = sm.noise[e1];
    const int sel = wave_argmax_first_bf16(rbf(v0 - w0), rbf(v1 - w1));
    const int token = lane_i32((sel & 1) ? i1 : i0, sel >> 1);

    if (lane == 0 && a.update_counts && a.decode_counts) {
        int32_t *d = a.decode_counts + (int64_t)slot * a.stride_decode + token;
        if (a.is_prefill) atomicExch(d, 1); else atomicAdd(d, 1);
    }
    if (want_probs) {
        uint16_t *p = a.probabilities + (int64_t)slot * a.stride_probabilities;
        p[i0] = (uint16_t)f2bf(expf(o0));
        p[i1] = (uint16_t)f2bf(expf(o1));
    }
    if (want_lp) {
        const float osel = lane_f32((sel & 1) ? o1 : o0, sel >> 1);
        if (lane == 0) a.logprobs[(int64_t)row * a.stride_logprobs] = (uint16_t)f2bf(osel);
        if ((ind & IND_TOPLOGPROBS) && a.top_values && a.max_top_logprobs > 0) {
            const int top_lim = (int)lane_u32(prm, RP_TOPZ);
            const int lim = top_lim < a.max_top_logprobs ? top_lim : a.max_top_logprobs;
            const int64_t o = (int64_t)row * a.stride_top;
            if (e0 < lim) {
                a.top_values[o + e0] = (uint16_t)f2bf(o0);
                a.top_tokens[o + e0] = i0;
            }
            if (e1 < lim) {
                a.top_values[o + e1] = (uint16_t)f2bf(o1);
                a.top_tokens[o + e1] = i1;
            }
        }
    }
    if (lane == 0) a.tokens[(int64_t)row * a.stride_tokens] = token;
}

// Row stage of one row: merge of the row's `lists` candidate lists (`scr`, global scratch or
// workgroup memory; list l starts at column lm.base(l) of a V-column vocabulary) and the
// selection. All threads call.
__device__ __forceinline__ void singular_row(const ss_singular_args &a, SampleSmem &sm, int row,
                                             int lists, const ListMap &lm, int V, const uint32_t *scr) {
    RowSamples smp;
    load_samples(scr, lists, lm, smp);  // depends on the row only: issued first
    const int slot = a.slot_mapping ? uniform_i32(a.slot_mapping, row) : row;
    const uint32_t prm = row_params(a.indicators, a.top_k, a.top_p, a.min_p, a.top_logprobs, slot,
                                    a.max_top_logprobs);
    if (lane_u32(prm, RP_IND) & IND_GREEDY) {
        singular_greedy(a, scr, lists, lm, V, row, slot, smp.greedy);
        return;
    }
    float v0 = 0.f, v1 = 0.f;
    int i0 = 0, i1 = 0;
    merge_row(sm, scr, smp, lists, lm, V, v0, v1, i0, i1);
    singular_select(a, sm, row, slot, prm, v0, v1, i0, i1);
}

// Row stage: grid rows; `lists` = world_size * tiles candidate lists per row, `V` the width of
// the column space they index (all shards).
__global__ __launch_bounds__(SS_BLOCK) void singular_rows_kernel(const uint32_t *p_scratch, int64_t p_stride,
                                                                int lists, uint32_t lm_magic, int lm_per,
                                                                int lm_shard, int lm_block_n, int V,
                                                                ss_singular_args a) {
    __shared__ SampleSmem sm;
    touch_kernargs<sizeof(ss_singular_args)>();
    const int row = blockIdx.x;
    ListMap lm;
    lm.magic = lm_magic; lm.per = lm_per; lm.shard = lm_shard; lm.block_n = lm_block_n;
    singular_row(a, sm, row, lists, lm, V, p_scratch + (int64_t)row * p_stride);
}

// Workgroup memory of the one-launch form. The tile stage's and the row stage's memory share
// space (a barrier separates the phases); the tiles' candidate lists stay resident throughout.
constexpr int ROWWISE_MAX_TILES = 16;

template <int E>
struct RowwiseSmem {
    union {
        TileSmem<E> tile;
        SampleSmem sample;
    };
    alignas(16) uint32_t lists[ROWWISE_MAX_TILES * SS_K];
};

// One-launch form, grid rows: one workgroup per row streams the row tile by tile (the next tile's
// logits are in flight while the current tile is selected), keeps every tile's sorted top-128 in
// workgroup memory, merges them and performs the selection -- no scratch round trip through
// global memory and no second launch. With d2t and a grammar mask, `stage_words` > 0 asks for the
// row's grammar words to be staged in workgroup memory first (dynamic shared memory), so that the
// per-element lookups through d2t read LDS instead of scattered global words.
template <int E, int MODE>
__global__ __launch_bounds__(SS_BLOCK) void singular_rowwise_kernel(ss_singular_args a, int tiles,
                                                                    int stage_words) {
    __shared__ RowwiseSmem<E> sm;
    extern __shared__ __align__(16) uint32_t grammar_words[];
    const int row = blockIdx.x;
    const uint16_t *lrow = a.logits + (int64_t)row * a.stride_logits;
    u32x2 lw[E / 4];
    if (MODE != MODE_SCALAR) load_logits_vec<E>(lrow, 0, a.vocab_size, lw);
    const int slot = a.slot_mapping ? uniform_i32(a.slot_mapping, row) : row;
    const uint32_t ind = uniform_u16(a.indicators, slot);
    RowState rs = singular_row_state(a, row, slot, ind);
    const Uses u = row_uses(rs);
    if (stage_words > 0 && u.g && u.remap) {
        stage_grammar(rs.grammar, rs.vt, grammar_words);
        rs.glds = grammar_words;
    }
    if (a.drafted_tokens && a.timestep > 0 && (ind & (IND_MULT | IND_FREQ | IND_PRES))) {
        rs.nhist = a.timestep;
        if ((int)threadIdx.x < rs.nhist)
            sm.tile.hist[threadIdx.x] = a.drafted_tokens[(int64_t)row * a.stride_drafted + threadIdx.x];
    }
    if (rs.glds) stage_grammar_finish(rs.vt, grammar_words);
    __syncthreads();
    const bool greedy = (ind & IND_GREEDY) != 0;
#pragma unroll 1
    for (int t = 0; t < tiles; ++t) {
        u32x2 nx[E / 4];
        if (MODE != MODE_SCALAR && t + 1 < tiles)
            load_logits_vec<E>(lrow, (t + 1) * a.block_n, a.vocab_size, nx);
        Keys<E> keys;
        prologue_keys<E, MODE>(rs, t * a.block_n, a.vocab_size, sm.tile.hist, lw, keys);
        tile_stage<E>(sm.tile, greedy, keys, sm.lists, t, min(a.block_n, a.vocab_size - t * a.block_n));
        // the next tile reuses the tile stage's memory, and the lists feed the row stage
        __syncthreads();
        if (MODE != MODE_SCALAR) {
#pragma unroll
            for (int c = 0; c < E / 4; ++c) lw[c] = nx[c];
        }
    }
    const uint32_t *scr = sm.lists;
    const ListMap lm = make_list_map(tiles, 0, a.block_n);
    RowSamples smp;
    load_samples(scr, tiles, lm, smp);
    const uint32_t prm = row_params(a.indicators, a.top_k, a.top_p, a.min_p, a.top_logprobs, slot,
                                    a.max_top_logprobs);
    if (greedy) {
        singular_greedy(a, scr, tiles, lm, a.vocab_size, row, slot, smp.greedy);
        return;
    }
    float v0 = 0.f, v1 = 0.f;
    int i0 = 0, i1 = 0;
    merge_row(sm.sample, scr, smp, tiles, lm, a.vocab_size, v0, v1, i0, i1);
    singular_select(a, sm.sample, row, slot, prm, v0, v1, i0, i1);
}

// Grammar words to stage per workgroup: with d2t and a grammar mask whose row fits, else 0.
static int staged_grammar_words(const ss_singular_args *a) {
    const int words = ((a->target_vocab > 0 ? a->target_vocab : a->vocab_size) + 31) >> 5;
    return (a->d2t && a->grammar && words <= SS_STAGE_MAX_WORDS) ? words : 0;
}

// Workgroup memory of a staged grammar row (stage_grammar): whole 64-quad blocks, at least one
// quad of zeros after the row.
static size_t staged_grammar_bytes(const ss_singular_args *a) {
    const int vt = a->target_vocab > 0 ? a->target_vocab : a->vocab_size;
    return staged_grammar_words(a) ? (size_t)stage_region_quads(vt) * 16 : 0;
}

// Dynamic shared memory of singular_tiles_kernel<E>: its TileSmem, or a staged grammar row from
// TILE_OVERLAY on where that is larger.
template <int E>
static size_t tile_smem_bytes(const ss_singular_args *a) {
    const size_t g = staged_grammar_bytes(a);
    const size_t t = sizeof(TileSmem<E>);
    return g && TILE_OVERLAY + g > t ? TILE_OVERLAY + g : t;
}

template <int MODE>
static int launch_rowwise(const ss_singular_args *a, int tiles) {
    const int stage = staged_grammar_words(a);
    const size_t dyn = staged_grammar_bytes(a);
    dim3 grid((unsigned)a->rows), block(SS_BLOCK);
    hipStream_t s = (hipStream_t)a->stream;
    switch (a->block_n) {
        case 1024: hipLaunchKernelGGL((singular_rowwise_kernel<4, MODE>), grid, block, dyn, s, *a, tiles, stage); break;
        case 2048: hipLaunchKernelGGL((singular_rowwise_kernel<8, MODE>), grid, block, dyn, s, *a, tiles, stage); break;
        case 4096: hipLaunchKernelGGL((singular_rowwise_kernel<16, MODE>), grid, block, dyn, s, *a, tiles, stage); break;
        case 8192: hipLaunchKernelGGL((singular_rowwise_kernel<32, MODE>), grid, block, dyn, s, *a, tiles, stage); break;
        default: return SS_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}

template <int MODE>
static int launch_singular(const ss_singular_args *a, int tiles) {
    // x: the tiles of a row, y: rows; the linear dispatch order is row-major as (row, tile)
    dim3 grid((unsigned)tiles, (unsigned)a->rows), block(SS_BLOCK);
    hipStream_t s = (hipStream_t)a->stream;
    const int stage = staged_grammar_words(a);
    const int stages = a->stages ? a->stages : (SS_STAGE_TILES | SS_STAGE_ROWS);
    if (stages & SS_STAGE_TILES) {
        switch (a->block_n) {
            case 1024: launch_timed((singular_tiles_kernel<4, MODE>), grid, block, tile_smem_bytes<4>(a), s, a->tile_start, a->tile_end, (const uint16_t *)a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, stage, a->slot_mapping, a->indicators, *a); break;
            case 2048: launch_timed((singular_tiles_kernel<8, MODE>), grid, block, tile_smem_bytes<8>(a), s, a->tile_start, a->tile_end, (const uint16_t *)a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, stage, a->slot_mapping, a->indicators, *a); break;
            case 4096: launch_timed((singular_tiles_kernel<16, MODE>), grid, block, tile_smem_bytes<16>(a), s, a->tile_start, a->tile_end, (const uint16_t *)a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, stage, a->slot_mapping, a->indicators, *a); break;
            case 8192: launch_timed((singular_tiles_kernel<32, MODE>), grid, block, tile_smem_bytes<32>(a), s, a->tile_start, a->tile_end, (const uint16_t *)a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, stage, a->slot_mapping, a->indicators, *a); break;
            case 16384: launch_timed((singular_tiles_kernel<64, MODE>), grid, block, tile_smem_bytes<64>(a), s, a->tile_start, a->tile_end, (const uint16_t *)a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, stage, a->slot_mapping, a->indicators, *a); break;
            default: return SS_ERR_UNSUPPORTED;
        }
        if (hipGetLastError() != hipSuccess) return SS_ERR_LAUNCH;
    }
    if (stages & SS_STAGE_ROWS) {
        const int world = a->world_size > 1 ? a->world_size : 1;
        const int shard = world > 1 ? a->shard_size : 0;
        const ListMap lm = make_list_map(tiles, shard, a->block_n);
        const int V = world > 1 ? world * a->shard_size : a->vocab_size;
        hipLaunchKernelGGL(singular_rows_kernel, dim3((unsigned)a->rows), block, 0, s, (const uint32_t *)a->scratch, a->stride_scratch, world * tiles, lm.magic, lm.per, lm.shard, lm.block_n, V, *a);
        if (hipGetLastError() != hipSuccess) return SS_ERR_LAUNCH;
    }
    return SS_OK;
}

static bool aligned(const void *p, int64_t stride, int bytes_per_vec) {
    if (!p) return true;
    return ((uintptr_t)p % bytes_per_vec) == 0 && (stride % 4) == 0;
}

}  // namespace ss

extern "C" int ss_fused_singular(const ss_singular_args *a) {
    using namespace ss;
    if (!a || !a->logits || !a->indicators || !a->tokens || !a->scratch)
        return SS_ERR_INVALID_ARGUMENT;
    if (a->rows < 0 || a->vocab_size <= 0 || a->stride_logits < a->vocab_size)
        return SS_ERR_INVALID_ARGUMENT;
    if (a->block_n != 1024 && a->block_n != 2048 && a->block_n != 4096 && a->block_n != 8192 && a->block_n != 16384)
        return SS_ERR_UNSUPPORTED;
    if (a->rows > 65535) return SS_ERR_UNSUPPORTED;  // rows are the tile grid's y dimension
    const int tiles = (a->vocab_size + a->block_n - 1) / a->block_n;
    const int world = a->world_size > 1 ? a->world_size : 1;
    if (a->world_size < 0 || a->local_rank < 0 || a->local_rank >= world) return SS_ERR_INVALID_ARGUMENT;
    if (world > 1 && a->shard_size < a->vocab_size) return SS_ERR_INVALID_ARGUMENT;
    if (world > 1 && (int64_t)world * a->shard_size > 0x7fffffff) return SS_ERR_INVALID_ARGUMENT;
    if (a->stages < 0 || a->stages > (SS_STAGE_TILES | SS_STAGE_ROWS)) return SS_ERR_INVALID_ARGUMENT;
    if (tiles < 2 || (int64_t)world * tiles * SS_K > a->stride_scratch || (int64_t)world * tiles > 0xffff)
        return SS_ERR_INVALID_ARGUMENT;
    // candidate lists move as 16-byte vectors
    if ((uintptr_t)a->scratch % 16 != 0 || a->stride_scratch % 4 != 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->timestep < 0 || a->timestep > 64) return SS_ERR_INVALID_ARGUMENT;
    if (a->max_top_logprobs < 0 || a->max_top_logprobs > SS_MAX_K) return SS_ERR_INVALID_ARGUMENT;
    if (!a->philox.enabled && !a->gumbel) return SS_ERR_INVALID_ARGUMENT;
    if (a->return_logprobs && a->max_top_logprobs > 0 && a->top_values && !a->top_tokens)
        return SS_ERR_INVALID_ARGUMENT;
    if (a->rows == 0) return SS_OK;
    // a shard whose offset is not a multiple of 32 columns cannot read grammar words and counts as
    // aligned vectors: it takes the per-element gather layout
    const bool direct = a->d2t == nullptr && (world == 1 || (a->local_rank * a->shard_size) % 32 == 0);
    const bool vec = (a->vocab_size % 4) == 0 && aligned(a->logits, a->stride_logits, 8) &&
                     (!direct || (aligned(a->decode_counts, a->stride_decode, 16) &&
                                  aligned(a->context_counts, a->stride_context, 16) &&
                                  aligned(a->logit_bias, a->stride_bias, 8)));
    if (a->strategy < SS_STRATEGY_AUTO || a->strategy > SS_STRATEGY_ROWWISE) return SS_ERR_INVALID_ARGUMENT;
    if (a->strategy == SS_STRATEGY_ROWWISE && (tiles > ROWWISE_MAX_TILES || world > 1 || a->stages))
        return SS_ERR_UNSUPPORTED;
    // AUTO takes the tile grid: one workgroup per row leaves a CU with a single workgroup (one
    // wave per SIMD) working through its tiles one after another, which measured slower on every
    // shape tried (config 4: 36 us for the row kernel against 23 + 7 us for the two launches).
    const bool rowwise = a->strategy == SS_STRATEGY_ROWWISE;
    if (rowwise) {
        if (!vec) return launch_rowwise<MODE_SCALAR>(a, tiles);
        return direct ? launch_rowwise<MODE_DIRECT>(a, tiles) : launch_rowwise<MODE_GATHER_VEC>(a, tiles);
    }
    if (!vec) return launch_singular<MODE_SCALAR>(a, tiles);
    return direct ? launch_singular<MODE_DIRECT>(a, tiles) : launch_singular<MODE_GATHER_VEC>(a, tiles);
}

namespace ss {

constexpr int MAX_DEVICES = 64;
static std::atomic<uint32_t *> g_static_scratch[MAX_DEVICES];
static std::mutex g_static_scratch_lock;

// The copy of `scratch` on the device that runs `stream` (the current device for the null
// stream), looked up on the first call on that device: hipGetSymbolAddress resolves the symbol for
// the current device, so that device is made current for the lookup and the caller's device is
// restored. The lookup may load the code object on the device, which is not a stream operation a
// graph can record: a first call on a device while `stream` is capturing is refused
// (SS_ERR_UNSUPPORTED), so the first call must be made eagerly, before any capture.
static int static_scratch(hipStream_t stream, uint32_t **out) {
    int dev = -1;
    if (stream) {
        if (hipStreamGetDevice(stream, &dev) != hipSuccess) return SS_ERR_LAUNCH;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return SS_ERR_LAUNCH;
    }
    if (dev < 0 || dev >= MAX_DEVICES) return SS_ERR_UNSUPPORTED;
    uint32_t *p = g_static_scratch[dev].load(std::memory_order_acquire);
    if (p) {
        *out = p;
        return SS_OK;
    }
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess) return SS_ERR_LAUNCH;
    if (capture != hipStreamCaptureStatusNone) return SS_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_static_scratch_lock);
    p = g_static_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
        int current = -1;
        if (hipGetDevice(&current) != hipSuccess) return SS_ERR_LAUNCH;
        if (current != dev && hipSetDevice(dev) != hipSuccess) return SS_ERR_LAUNCH;
        void *addr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
        if (current != dev && hipSetDevice(current) != hipSuccess) return SS_ERR_LAUNCH;
        if (e != hipSuccess || !addr) return SS_ERR_LAUNCH;
        p = static_cast<uint32_t *>(addr);
        g_static_scratch[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return SS_OK;
}

}  // namespace ss

extern "C" int ss_fused_singular_noalloc(const ss_singular_args *a) {
    using namespace ss;
    if (!a || a->vocab_size <= 0 || a->rows < 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->block_n != 1024 && a->block_n != 2048 && a->block_n != 4096 && a->block_n != 8192 && a->block_n != 16384)
        return SS_ERR_UNSUPPORTED;
    const int64_t tiles = ((int64_t)a->vocab_size + a->block_n - 1) / a->block_n;
    const int64_t world = a->world_size > 1 ? a->world_size : 1;
    if ((int64_t)a->rows * world * tiles * SS_K * (int64_t)sizeof(uint32_t) > (int64_t)SS_STATIC_SCRATCH_BYTES)
        return SS_ERR_SCRATCH_LIMIT;
    uint32_t *ptr = nullptr;
    const int st = static_scratch((hipStream_t)a->stream, &ptr);
    if (st != SS_OK) return st;
    // Every list entry the row stage uses is written by the tile stage of the same call, or, with
    // the stages split, by the tile-stage calls of every shard made just before it on the device
    // (a greedy row's merge samples are read but ignored), so the array needs no clearing between
    // calls.
    ss_singular_args b = *a;
    b.scratch = ptr;
    b.stride_scratch = world * tiles * SS_K;
    return ss_fused_singular(&b);
}
