// Fused chain speculative verification (replaces K1 ops/prologue.py:272-472, K5
// ops/multistep.py:76-226 and K6 ops/verify.py:244-434 of the reference), as three back-to-back
// launches on the caller's stream; rows = B * (gamma + 1) or cu_seqlens[B] (variable lookahead).
//   tile stage    grid (tiles, rows): prologue over one tile of one row -> tile argmax / top-128;
//   row stage     grid rows: merge -> truncation -> fp32 log_softmax, written to values /
//                 indices [row, 128] (greedy rows: the argmax in indices[row, 0]);
//   request stage grid B (one wavefront each): greedy chain verification, or the stochastic
//                 chain from the rows' verification records (acceptance, residual / bonus
//                 samples, computed by the row stage); logprobs, top-Z, decode-count update.
// Semantics follow the reference's PyTorch path (core/naive.py:497-646 `verification`,
// :694-708 `multistep`), applied per request so that slots and variable lookahead compose.
#include "ss_launch.h"
#include "ss_sampling.h"
#include "../../include/sonic_sampler.h"

namespace ss {

struct Request {
    int b, margin, n;
};

// The lane's pivot of the first round of resolve_request's search, cu_seqlens[lane * step] with
// step = ceil(batch / 64) (INT_MAX past the end; 0 without cu_seqlens). Kernels issue it ahead of
// their bulk loads: vector loads return in order, so behind a tile of logits it would wait for the
// whole tile, and the request's reads that depend on it would start only then.
__device__ __forceinline__ int request_pivot(const int32_t *cu_seqlens, int batch) {
    if (!cu_seqlens) return 0;
    const int p = lane_id() * ((batch + 63) >> 6);
    return p < batch ? cu_seqlens[p] : INT_MAX;
}

__device__ __forceinline__ int request_pivot(const ss_multistep_args &a) {
    return request_pivot(a.cu_seqlens, a.batch);
}

__device__ __forceinline__ Request resolve_request(const ss_multistep_args &a, int row, int pivot) {
    Request r;
    if (a.cu_seqlens) {
        // Every wave searches on its own: each round tests 64 evenly spaced pivots of (lo, hi), so
        // one round of loads resolves up to 64 requests and two up to 4096 (cu_seqlens is
        // non-decreasing, so the pivots at or below `row` are a prefix of the lanes). The first
        // round's pivots (lo = 0, hi = batch) come from request_pivot.
        const int lane = lane_id();
        int lo = 0, hi = a.batch;  // invariant: cu[lo] <= row < cu[hi]
        bool first = true;
        while (hi - lo > 1) {
            const int step = (hi - lo + 63) >> 6;
            const int p = lo + lane * step;
            const bool le = p < hi && (first ? pivot : a.cu_seqlens[p]) <= row;
            first = false;
            const uint64_t m = __ballot(le);  // lane 0 (pivot lo) is set unless cu[0] > row
            if (!m) break;
            const int k = 63 - __clzll((long long)m);
            lo += k * step;
            hi = min(lo + step, hi);
        }
        r.b = lo;
        r.margin = uniform_i32(a.cu_seqlens, lo);
        r.n = uniform_i32(a.cu_seqlens, lo + 1) - r.margin;
    } else {
        r.n = a.lookahead + 1;
        r.b = row / r.n;
        r.margin = r.b * r.n;
    }
    return r;
}

__device__ __forceinline__ RowState multistep_row_state(const ss_multistep_args &a, int row,
                                                        int step, int slot, uint32_t ind) {
    RowState rs;
    rs.ind = ind;
    rs.logits = a.logits + (int64_t)row * a.stride_logits;
    rs.d2t = nullptr;
    rs.grammar = a.grammar ? a.grammar + (int64_t)slot * a.grammar_stride_slot +
                                 (int64_t)step * a.grammar_stride_step
                           : nullptr;
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
    rs.vt = a.vocab_size;
    rs.nhist = 0;
    rs.glds = nullptr;
    rs.shard = 0;
    return rs;
}

// Rows outside every request, or requests longer than lookahead + 1, break the layout contract;
// they are skipped (their outputs stay unwritten) rather than read out of bounds.
__device__ __forceinline__ bool row_in_contract(const ss_multistep_args &a, const Request &rq,
                                                int step) {
    return step >= 0 && step < rq.n && rq.n <= a.lookahead + 1;
}

// Tile stage: grid (tiles, rows).
template <int E, int MODE>
__global__ __launch_bounds__(SS_BLOCK) void multistep_tiles_kernel(const uint16_t *p_logits, int64_t p_stride,
                                                                   int p_block_n, int p_vocab, int tiles,
                                                                   const int32_t *p_cu, int p_batch,
                                                                   const int32_t *p_slots, const uint16_t *p_ind,
                                                                   ss_multistep_args a) {
    __shared__ TileSmem<E> sm;
    const int row = blockIdx.y;
    const int tile = blockIdx.x;
    // the request search, the slot and the indicator start from preloaded pointers
    const int pivot = request_pivot(p_cu, p_batch);
    u32x2 lw[E / 4];
    if (MODE != MODE_SCALAR) load_logits_vec<E>(p_logits + (int64_t)row * p_stride, tile * p_block_n, p_vocab, lw);
    const Request rq = resolve_request(a, row, pivot);
    const int step = row - rq.margin;
    if (!row_in_contract(a, rq, step)) return;
    const int slot = p_slots ? uniform_i32(p_slots, rq.b) : rq.b;
    const uint32_t ind = uniform_u16(p_ind, slot);
    RowState rs = multistep_row_state(a, row, step, slot, ind);
    if (step > 0 && (ind & (IND_MULT | IND_FREQ | IND_PRES))) {
        // Step s of a request sees the drafts of steps < s as extra decode history
        // (core/naive.py:179-198, the `tril` history with timestep None).
        rs.nhist = step;
        if ((int)threadIdx.x < step) sm.hist[threadIdx.x] = a.drafted_tokens[rq.margin + threadIdx.x];
        __syncthreads();
    }
    Keys<E> keys;
    prologue_keys<E, MODE>(rs, tile * a.block_n, a.vocab_size, sm.hist, lw, keys);
    tile_stage<E>(sm, (ind & IND_GREEDY) != 0, keys, a.scratch + (int64_t)row * a.stride_scratch, tile,
                  min(a.block_n, a.vocab_size - tile * a.block_n));
}

// Row stage: grid rows; merge -> truncation -> fp32 log_softmax into values / indices [row, 128]
// (greedy rows: the argmax in indices[row, 0]). A stochastic row also does its own part of the
// chain verification (core/naive.py:580-620), which depends on no other row: whether its drafted
// token is accepted, that token's logprob, and the token it emits if the chain stops here (the
// residual sample at a rejection, the bonus sample on the last row) with its logprob. It writes
// them as one 16-byte record at the start of its scratch row, whose candidates it has consumed:
// {accepted, stop token, logprob if accepted (fp32 bits), stop token's logprob (fp32 bits)}.
__global__ __launch_bounds__(SS_BLOCK) void multistep_rows_kernel(uint32_t *p_scratch, int64_t p_stride,
                                                                  int p_block_n, int tiles,
                                                                  ss_multistep_args a) {
    __shared__ SampleSmem sm;
    const int row = blockIdx.x;
    uint32_t *scr = p_scratch + (int64_t)row * p_stride;
    const ListMap lm = make_list_map(tiles, 0, p_block_n);
    // the merge samples depend on the row and the preloaded arguments only: issued first, ahead
    // of the argument lines the rest of the row stage reads
    RowSamples smp;
    load_samples<true>(scr, tiles, lm, smp);
    touch_kernargs<sizeof(ss_multistep_args)>();
    const int pivot = request_pivot(a);
    const Request rq = resolve_request(a, row, pivot);
    const int step = row - rq.margin;
    if (!row_in_contract(a, rq, step)) return;
    const int slot = a.slot_mapping ? uniform_i32(a.slot_mapping, rq.b) : rq.b;
    const uint32_t prm = row_params(a.indicators, a.top_k, a.top_p, a.min_p, nullptr, slot, 0);
    const uint32_t ind = lane_u32(prm, RP_IND);
    float *vrow = a.values + (int64_t)row * SS_K;
    int32_t *irow = a.indices + (int64_t)row * SS_K;
    if (ind & IND_GREEDY) {
        if (threadIdx.x < 64) {
            const int token = greedy_merge(scr, tiles, lm, a.vocab_size, smp.greedy);
            if (threadIdx.x == 0) {
                irow[0] = token;
                vrow[0] = 0.0f;
            }
        }
        return;
    }
    // The drafted token of this step and its uniform, read while the candidates merge, as vector
    // loads: a scalar load shares its wait counter with workgroup memory, so the merge's first
    // wait for its own LDS traffic would also wait for these.
    const bool last = step == rq.n - 1;
    int d = 0;
    float ud = 0.0f;
    if (!last) {
        const __amdgpu_buffer_rsrc_t dr = row_buffer(a.drafted_tokens + row, 4);
        const __amdgpu_buffer_rsrc_t ur = row_buffer(a.uniform + (int64_t)slot * a.stride_uniform + step, 2);
        d = (int)__builtin_amdgcn_raw_buffer_load_b32(dr, 0, 0, 0);
        ud = bf2f((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(ur, 0, 0, 0));
    }
    float v0 = 0.f, v1 = 0.f;
    int i0 = 0, i1 = 0;
    merge_row(sm, scr, smp, tiles, lm, a.vocab_size, v0, v1, i0, i1);
    // Waves 1 and 2 draw the 128 candidates' noise and gather their draft probabilities (one
    // candidate per lane) while wave 0 truncates and tests the drafted token.
    const int wave = (int)threadIdx.x >> 6;
    const int lane = lane_id();
    const int e0 = 2 * lane;
    const bool svgd = (ind & IND_SVGD) || !a.draft_probabilities;
    const uint16_t *qrow = svgd ? nullptr
                                : a.draft_probabilities + (int64_t)slot * a.probs_stride_slot +
                                      (int64_t)step * a.probs_stride_step;
    if (wave == 1 || wave == 2) {
        const int e = (wave - 1) * 64 + lane;
        const int t = sm.tok[e];
        sm.noise[e] = a.philox.enabled
                          ? philox_gumbel(a.philox.seed, a.philox.offset, slot, step, t)
                          : bf2f(a.gumbel[(int64_t)slot * a.gumbel_stride_slot + (int64_t)step * a.gumbel_stride_step + t]);
        sm.qcand[e] = qrow && !last ? bf2f(qrow[t]) : 0.0f;
    }
    int accepted = 1;
    float l0 = 0.f, l1 = 0.f, lacc = 0.0f;
    if (wave == 0) {
        const bool in_vocab = d >= 0 && d < a.vocab_size;
        const uint16_t qd16 = qrow && !last ? qrow[in_vocab ? d : 0] : (uint16_t)0;
        SoftmaxParts sp;
        truncate(ind, (int32_t)lane_u32(prm, RP_TOPK), __uint_as_float(lane_u32(prm, RP_TOPP)),
                 __uint_as_float(lane_u32(prm, RP_MINP)), v0, v1, sp);
        const float logs = logf(softmax_sum(sp, v0, v1));
        l0 = (v0 - sp.m) - logs;  // log_softmax in fp32, as the reference's softmax()
        l1 = (v1 - sp.m) - logs;
        vrow[e0] = l0;
        vrow[e0 + 1] = l1;
        irow[e0] = i0;
        irow[e0 + 1] = i1;
        // acceptance of the drafted token: p at its first sorted position (0 when absent; its
        // logprob then is the value at position 0, the argmax of an all-false match row),
        // bf16(u * q) <= p (core/naive.py:580-599)
        if (!last) {
            const uint64_t m0 = __ballot(i0 == d), m1 = __ballot(i1 == d);
            const int p0 = m0 ? 2 * (__ffsll((unsigned long long)m0) - 1) : 1 << 20;
            const int p1 = m1 ? 2 * (__ffsll((unsigned long long)m1) - 1) + 1 : 1 << 20;
            const int pos = min(p0, p1) < SS_K ? min(p0, p1) : -1;
            const int at = pos >= 0 ? pos : 0;
            lacc = lane_f32((at & 1) ? l1 : l0, at >> 1);
            const float pk = pos >= 0 ? expf(lacc) : 0.0f;
            const float qd = svgd ? 1.0f : in_vocab ? bf2f(qd16) : 0.0f;
            accepted = rbf(ud * qd) <= pk ? 1 : 0;
        }
    }
    __syncthreads();
    if (wave != 0) return;
    if (accepted && !last) {
        // an accepted draft never ends the chain: no stop token
        if (lane == 0) *(int4 *)scr = make_int4(1, 0, __float_as_int(lacc), 0);
        return;
    }
    // the token emitted if the chain stops at this row: the residual max(p - q, 0) at a rejection
    // (q a point mass on the draft under 0x800), p itself on the last row
    const float pe0 = expf(l0), pe1 = expf(l1);
    float r0, r1;
    if (last) {
        r0 = pe0;
        r1 = pe1;
    } else if (svgd) {
        r0 = i0 == d ? 0.0f : pe0;
        r1 = i1 == d ? 0.0f : pe1;
    } else {
        r0 = fmaxf(pe0 - sm.qcand[e0], 0.0f);
        r1 = fmaxf(pe1 - sm.qcand[e0 + 1], 0.0f);
    }
    const float w0 = sm.noise[e0], w1 = sm.noise[e0 + 1];
    const int sel = wave_argmax_first(logf(r0) - w0, logf(r1) - w1);
    const int token = lane_i32((sel & 1) ? i1 : i0, sel >> 1);
    const float lsel = lane_f32((sel & 1) ? l1 : l0, sel >> 1);
    if (lane == 0) *(int4 *)scr = make_int4(accepted, token, __float_as_int(lacc), __float_as_int(lsel));
}

// Request stage: grid B, one wavefront per request.
__global__ __launch_bounds__(64) void multistep_verify_kernel(const int32_t *p_cu, const int32_t *p_slots,
                                                             const uint16_t *p_ind, int p_lookahead,
                                                             int p_rows, ss_multistep_args a) {
    const int b = blockIdx.x;
    Request rq;
    if (p_cu) {
        rq.b = b;
        rq.margin = p_cu[b];
        rq.n = p_cu[b + 1] - rq.margin;
    } else {
        rq.b = b;
        rq.n = p_lookahead + 1;
        rq.margin = b * rq.n;
    }
    if (rq.n < 1 || rq.n > p_lookahead + 1 || rq.margin < 0 || rq.margin + rq.n > p_rows) return;
    const int slot = p_slots ? p_slots[rq.b] : rq.b;
    const uint32_t ind = p_ind[slot];
    const bool greedy = (ind & IND_GREEDY) != 0;
    const int top_lim = a.top_logprobs ? a.top_logprobs[slot] : a.max_top_logprobs;

    // ---- request stage (wave 0) -------------------------------------------------------------------
    const int lane = threadIdx.x;
    const int e0 = 2 * lane, e1 = e0 + 1;
    const int n = rq.n;
    const int32_t *drafted = a.drafted_tokens + rq.margin;
    const float *vals = a.values + (int64_t)rq.margin * SS_K;
    const int32_t *idxs = a.indices + (int64_t)rq.margin * SS_K;

    const bool want_lp = a.return_logprobs && a.logprobs;
    if (p_cu) {
        // rows outside every request's span (cu_seqlens starting above 0 or ending before the last
        // row) keep their drafts, as in a copy of the drafts: the first request copies the rows
        // before it, the last the rows after it (bounds clamped to the rows)
        if (b == 0) {
            const int hi = min(max(p_cu[0], 0), p_rows);
            for (int r = lane; r < hi; r += 64) a.out_tokens[r] = a.drafted_tokens[r];
        }
        if (b == (int)gridDim.x - 1) {
            for (int r = min(max(p_cu[gridDim.x], 0), p_rows) + lane; r < p_rows; r += 64)
                a.out_tokens[r] = a.drafted_tokens[r];
        }
    }
    if (a.all_greedy && !greedy) {
        // The caller's all_greedy hint is wrong for this request: no row launch left its records.
        // It is not served, and says so: offsets -1 (outside 0..gamma), its tokens the drafts,
        // nothing else written.
        if (lane < n) a.out_tokens[rq.margin + lane] = drafted[lane];
        if (lane == 0) a.offsets[rq.b] = -1;
        return;
    }
    int j = n - 1;
    int token;
    if (greedy && a.all_greedy) {
        // No row launch ran: row i's argmax comes from its tiles' maxima here (lane i holds it),
        // and it is written where the row stage would have left it (indices[row, 0], values 0).
        const int tiles = (a.vocab_size + a.block_n - 1) / a.block_n;
        const ListMap lm = make_list_map(tiles, 0, a.block_n);
        int argmax = 0;
        if (n * tiles <= 64) {
            // every (row, tile) maximum in one round of loads, lane r * tiles + t
            const int r = lane / tiles, t = lane - r * tiles;
            const uint32_t c = r < n ? a.scratch[(int64_t)(rq.margin + r) * a.stride_scratch + lm.greedy_entry(t)] : 0u;
            const uint64_t c64 = ((uint64_t)(c >> 16) << 32) | ((uint64_t)(0xffffu - (uint32_t)t) << 16) |
                                 (uint64_t)(c & 0xffffu);
            for (int i = 0; i < n; ++i) {
                const uint64_t best = wave_max_u64(r == i ? c64 : 0ull);
                const int tile = (int)(0xffffu - (uint32_t)((best >> 16) & 0xffffu));
                const int idx = lm.base(tile) + (int)(0xffffu - (uint32_t)(best & 0xffffu));
                if (lane == i) argmax = idx < a.vocab_size ? idx : a.vocab_size - 1;
            }
        } else {
            for (int i = 0; i < n; ++i) {
                const uint32_t *srow = a.scratch + (int64_t)(rq.margin + i) * a.stride_scratch;
                const uint32_t first = lane < tiles ? srow[lm.greedy_entry(lane)] : 0u;
                const int idx = greedy_merge(srow, tiles, lm, a.vocab_size, first);
                if (lane == i) argmax = idx;
            }
        }
        if (lane < n) {
            a.indices[(int64_t)(rq.margin + lane) * SS_K] = argmax;
            a.values[(int64_t)(rq.margin + lane) * SS_K] = 0.0f;
        }
        const uint64_t m = __ballot(lane < n - 1 && argmax != drafted[lane < n - 1 ? lane : 0]);
        j = m ? __ffsll((unsigned long long)m) - 1 : n - 1;
        token = lane_i32(argmax, j);
    } else if (greedy) {
        // lane i compares row i's argmax with drafted token i; all of them in one round of loads
        for (int base = 0; base < n - 1; base += 64) {
            const int i = base + lane;
            const bool mismatch = i < n - 1 && idxs[(int64_t)i * SS_K] != drafted[i];
            const uint64_t m = __ballot(mismatch);
            if (m) {
                j = base + __ffsll((unsigned long long)m) - 1;
                break;
            }
        }
        token = idxs[(int64_t)j * SS_K];
    } else {
        // The rows' records (multistep_rows_kernel), one lane per row, in one round with the top
        // logprobs of the first VCH rows; the chain stops at the first rejected draft, else at
        // the bonus row n - 1 (core/naive.py:600-620).
        constexpr int VCH = 8;
        const bool want_top = want_lp && (ind & IND_TOPLOGPROBS) && a.top_values && a.max_top_logprobs > 0;
        const int lim = top_lim < a.max_top_logprobs ? top_lim : a.max_top_logprobs;
        int4 rec = make_int4(1, 0, 0, 0);
        if (lane < n) rec = *(const int4 *)(a.scratch + (int64_t)(rq.margin + lane) * a.stride_scratch);
        int2 w[VCH];
        float2 vv[VCH];
        if (want_top) {
#pragma unroll
            for (int k = 0; k < VCH; ++k) {
                const int r = min(k, n - 1);
                w[k] = *(const int2 *)(idxs + (int64_t)r * SS_K + e0);
                vv[k] = *(const float2 *)(vals + (int64_t)r * SS_K + e0);
            }
        }
        const uint64_t rej = __ballot(lane < n - 1 && rec.x == 0);
        j = rej ? __ffsll((unsigned long long)rej) - 1 : n - 1;
        token = lane_i32(rec.y, j);
        if (want_lp && lane <= j)
            a.logprobs[rq.margin + lane] = (uint16_t)f2bf(__int_as_float(lane < j ? rec.z : rec.w));
        if (want_top) {
            // top logprobs of the rows up to j, from their candidate pairs
            auto write_top = [&](int r, int2 tok, float2 val) {
                const int64_t o = (int64_t)(rq.margin + r) * a.stride_top;
                if (e0 < lim) {
                    a.top_values[o + e0] = (uint16_t)f2bf(val.x);
                    a.top_tokens[o + e0] = tok.x;
                }
                if (e1 < lim) {
                    a.top_values[o + e1] = (uint16_t)f2bf(val.y);
                    a.top_tokens[o + e1] = tok.y;
                }
            };
#pragma unroll
            for (int k = 0; k < VCH; ++k)
                if (k <= j) write_top(k, w[k], vv[k]);
            for (int r = VCH; r <= j; ++r)
                write_top(r, *(const int2 *)(idxs + (int64_t)r * SS_K + e0), *(const float2 *)(vals + (int64_t)r * SS_K + e0));
        }
    }
    if (greedy && a.return_logprobs && a.logprobs) {
        if (lane <= j) a.logprobs[rq.margin + lane] = 0;
    }
    if (a.update_counts && a.decode_counts && lane <= j) {
        const int tok = lane < j ? drafted[lane] : token;
        if (tok >= 0 && tok < a.vocab_size)
            atomicAdd(a.decode_counts + (int64_t)slot * a.stride_decode + tok, 1);
    }
    // the request's tokens: its drafts, the emitted token at j (the buffer needs no pre-fill and
    // may be the drafts' own; each lane stores one position)
    if (lane < n) a.out_tokens[rq.margin + lane] = lane == j ? token : drafted[lane];
    if (lane == 0) a.offsets[rq.b] = j;
}

template <int MODE>
static int launch_multistep(const ss_multistep_args *a, int tiles) {
    // x: the tiles of a row, y: rows; the linear dispatch order is row-major as (row, tile)
    dim3 grid((unsigned)tiles, (unsigned)a->rows), block(SS_BLOCK);
    hipStream_t s = (hipStream_t)a->stream;
    switch (a->block_n) {
        case 1024: launch_timed((multistep_tiles_kernel<4, MODE>), grid, block, 0, s, a->tile_start, a->tile_end, a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, a->cu_seqlens, a->batch, a->slot_mapping, a->indicators, *a); break;
        case 2048: launch_timed((multistep_tiles_kernel<8, MODE>), grid, block, 0, s, a->tile_start, a->tile_end, a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, a->cu_seqlens, a->batch, a->slot_mapping, a->indicators, *a); break;
        case 4096: launch_timed((multistep_tiles_kernel<16, MODE>), grid, block, 0, s, a->tile_start, a->tile_end, a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, a->cu_seqlens, a->batch, a->slot_mapping, a->indicators, *a); break;
        case 8192: launch_timed((multistep_tiles_kernel<32, MODE>), grid, block, 0, s, a->tile_start, a->tile_end, a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, a->cu_seqlens, a->batch, a->slot_mapping, a->indicators, *a); break;
        case 16384: launch_timed((multistep_tiles_kernel<64, MODE>), grid, block, 0, s, a->tile_start, a->tile_end, a->logits, a->stride_logits, a->block_n, a->vocab_size, tiles, a->cu_seqlens, a->batch, a->slot_mapping, a->indicators, *a); break;
        default: return SS_ERR_UNSUPPORTED;
    }
    if (hipGetLastError() != hipSuccess) return SS_ERR_LAUNCH;
    if (!a->all_greedy) {
        hipLaunchKernelGGL(multistep_rows_kernel, dim3((unsigned)a->rows), block, 0, s, a->scratch, a->stride_scratch, a->block_n, tiles, *a);
        if (hipGetLastError() != hipSuccess) return SS_ERR_LAUNCH;
    }
    hipLaunchKernelGGL(multistep_verify_kernel, dim3((unsigned)a->batch), dim3(64), 0, s, a->cu_seqlens,
                       a->slot_mapping, a->indicators, a->lookahead, a->rows, *a);
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}

static bool aligned_ms(const void *p, int64_t stride, int bytes) {
    if (!p) return true;
    return ((uintptr_t)p % bytes) == 0 && (stride % 4) == 0;
}

}  // namespace ss

extern "C" int ss_fused_multistep(const ss_multistep_args *a) {
    using namespace ss;
    if (!a || !a->logits || !a->indicators || !a->drafted_tokens || !a->out_tokens || !a->offsets ||
        !a->values || !a->indices || !a->scratch || !a->uniform)
        return SS_ERR_INVALID_ARGUMENT;
    if (a->rows < 0 || a->batch < 0 || a->vocab_size <= 0 || a->stride_logits < a->vocab_size)
        return SS_ERR_INVALID_ARGUMENT;
    if (a->lookahead < 0 || a->lookahead > 63) return SS_ERR_INVALID_ARGUMENT;
    if (!a->cu_seqlens && a->rows != a->batch * (a->lookahead + 1)) return SS_ERR_INVALID_ARGUMENT;
    if (a->block_n != 1024 && a->block_n != 2048 && a->block_n != 4096 && a->block_n != 8192 && a->block_n != 16384)
        return SS_ERR_UNSUPPORTED;
    if (a->rows > 65535) return SS_ERR_UNSUPPORTED;  // rows are the tile grid's y dimension
    const int tiles = (a->vocab_size + a->block_n - 1) / a->block_n;
    if (tiles < 2 || (int64_t)tiles * SS_K > a->stride_scratch || tiles > 0xffff)
        return SS_ERR_INVALID_ARGUMENT;
    // candidate lists move as 16-byte vectors
    if ((uintptr_t)a->scratch % 16 != 0 || a->stride_scratch % 4 != 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->max_top_logprobs < 0 || a->max_top_logprobs > SS_MAX_K) return SS_ERR_INVALID_ARGUMENT;
    if (!a->philox.enabled && !a->gumbel) return SS_ERR_INVALID_ARGUMENT;
    if (a->rows == 0 || a->batch == 0) return SS_OK;
    const bool vec = (a->vocab_size % 4) == 0 && aligned_ms(a->logits, a->stride_logits, 8) &&
                     aligned_ms(a->decode_counts, a->stride_decode, 16) &&
                     aligned_ms(a->context_counts, a->stride_context, 16) &&
                     aligned_ms(a->logit_bias, a->stride_bias, 8);
    if (!vec) return launch_multistep<MODE_SCALAR>(a, tiles);
    return launch_multistep<MODE_DIRECT>(a, tiles);
}
