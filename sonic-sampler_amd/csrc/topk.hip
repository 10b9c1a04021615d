// Bounded top-k over [rows, vocab] logits (replaces K2 ops/topk/bitpack.py:99-158 followed by K3
// ops/topk/unpack.py:312-377 of the reference), as two back-to-back launches.
//
// Tile stage, grid rows * tiles: each workgroup turns block_n logits into order-preserving keys
// and writes its exact top-k (ties to the lowest column) to the scratch row in column order.
// Merge stage, grid rows: selects the row's top-k among the tiles * k candidates, sorts them by
// (value desc, column asc) with a wave64 bitonic network and writes values / indices densely as
// [rows, k].
#include "ss_select.h"
#include "../../include/sonic_sampler.h"

namespace ss {

struct TopkSmem {
    SelectSmem sel;
    uint64_t cand[SS_K];
    int32_t idx[SS_K];
    uint64_t runs[SS_WAVES][SS_K];  // merge of up to 512 candidates: the waves' sorted runs
};

template <bool F32>
struct TopkTraits;

template <>
struct TopkTraits<false> {
    using Cand = uint32_t;
    static constexpr int KEYBITS = 16;
    __device__ static uint32_t key_of(const void *p, int64_t off) {
        return key16(((const uint16_t *)p)[off]);
    }
    __device__ static Cand pack(uint32_t key, int li) { return (key << 16) | (uint32_t)li; }
    __device__ static uint32_t cand_key(Cand c) { return c >> 16; }
    __device__ static int cand_li(Cand c) { return (int)(c & 0xffffu); }
};

template <>
struct TopkTraits<true> {
    using Cand = uint64_t;
    static constexpr int KEYBITS = 32;
    __device__ static uint32_t key_of(const void *p, int64_t off) {
        return key32(__float_as_uint(((const float *)p)[off]));
    }
    __device__ static Cand pack(uint32_t key, int li) { return ((uint64_t)key << 32) | (uint32_t)li; }
    __device__ static uint32_t cand_key(Cand c) { return (uint32_t)(c >> 32); }
    __device__ static int cand_li(Cand c) { return (int)(c & 0xffffffffu); }
};

// Tile stage: grid rows * tiles.
template <bool F32, int E>
__global__ __launch_bounds__(SS_BLOCK) void topk_tiles_kernel(ss_topk_args a, int tiles) {
    using Tr = TopkTraits<F32>;
    using Cand = typename Tr::Cand;
    constexpr int CH = 4;
    __shared__ TopkSmem sm;

    const int row = blockIdx.x / tiles;
    const int tile = blockIdx.x - row * tiles;
    const int V = a.vocab_size;
    const int k = a.k;
    const int64_t base = (int64_t)row * a.stride_logits;
    const int col0 = tile * a.block_n;

    // ---- tile stage ---------------------------------------------------------------------------
    uint32_t keys[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int li = order_pos<E, CH>(0, j);
        const int col = col0 + li;
        keys[j] = col < V ? Tr::key_of(a.logits, base + col) : 0u;
    }
    auto tile_load = [&](int, uint32_t(&out)[E]) {
#pragma unroll
        for (int j = 0; j < E; ++j) out[j] = keys[j];
    };
    uint32_t thi, margin;
    int level;
    radix_threshold<E, Tr::KEYBITS>(sm.sel, 1, tile_load, (uint32_t)k, thi, level, margin);
    Cand *scr = (Cand *)a.scratch + (int64_t)row * a.stride_scratch;
    compact<E, CH>(sm.sel, 1, tile_load, thi, level, margin, [&](uint32_t pos, int, int j) {
        if (pos < (uint32_t)k) scr[tile * k + (int)pos] = Tr::pack(keys[j], order_pos<E, CH>(0, j));
    });

}

// Merge stage: grid rows.
template <bool F32>
__global__ __launch_bounds__(SS_BLOCK) void topk_merge_kernel(ss_topk_args a, int tiles) {
    touch_kernargs<sizeof(ss_topk_args)>();
    using Tr = TopkTraits<F32>;
    using Cand = typename Tr::Cand;
    constexpr int CH = 4;
    __shared__ TopkSmem sm;
    const int row = blockIdx.x;
    const int V = a.vocab_size;
    const int k = a.k;
    const Cand *scr = (const Cand *)a.scratch + (int64_t)row * a.stride_scratch;
    const int ncand = tiles * k;
    if (ncand <= 2 * SS_BLOCK) {
        // Up to 512 candidates, two per thread, as composites (key << 32) | (~column): their
        // descending order is (value desc, column asc). Every wave sorts its 128, and two rounds
        // of bitonic merges keep the top-128 of the four runs (the elementwise maximum of a run
        // and its reversed partner is a bitonic sequence holding the top-128 of both).
        const int lane = lane_id(), wave = (int)threadIdx.x >> 6;
        const int lk = __builtin_ctz((unsigned)k);  // k is a power of two
        uint64_t c[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int p = 2 * (int)threadIdx.x + i;
            uint64_t v = 0;
            if (p < ncand) {
                const Cand cd = scr[p];
                const uint32_t col = (uint32_t)((p >> lk) * a.block_n + Tr::cand_li(cd));
                v = ((uint64_t)Tr::cand_key(cd) << 32) | (uint64_t)(0xffffffffu - col);
            }
            c[i] = v;
        }
        wave_sort128_desc(c[0], c[1]);
        sm.runs[wave][2 * lane] = c[0];
        sm.runs[wave][2 * lane + 1] = c[1];
        __syncthreads();
        if (wave < 2) {
            const uint64_t *A = sm.runs[2 * wave], *B = sm.runs[2 * wave + 1];
            uint64_t x0 = max_u64(A[2 * lane], B[127 - 2 * lane]);
            uint64_t x1 = max_u64(A[2 * lane + 1], B[126 - 2 * lane]);
            wave_bitonic128_desc<128>(x0, x1);
            sm.runs[2 * wave][2 * lane] = x0;
            sm.runs[2 * wave][2 * lane + 1] = x1;
        }
        __syncthreads();
        if (wave == 0) {
            uint64_t f[2];
            f[0] = max_u64(sm.runs[0][2 * lane], sm.runs[2][127 - 2 * lane]);
            f[1] = max_u64(sm.runs[0][2 * lane + 1], sm.runs[2][126 - 2 * lane]);
            wave_bitonic128_desc<128>(f[0], f[1]);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int e = 2 * lane + i;
                if (e < k) {
                    const uint32_t key = (uint32_t)(f[i] >> 32);
                    const int col = (int)(0xffffffffu - (uint32_t)f[i]);
                    const int64_t o = (int64_t)row * k + e;
                    if (F32) {
                        ((float *)a.values)[o] = __uint_as_float(unkey32(key));
                    } else {
                        ((uint16_t *)a.values)[o] = (uint16_t)unkey16(key);
                    }
                    a.indices[o] = col < V ? col : V - 1;
                }
            }
        }
        return;
    }
    uint32_t thi, margin;
    int level;
    constexpr int EM = 16;
    const int nsc = (ncand + SS_BLOCK * EM - 1) / (SS_BLOCK * EM);
    auto cand_load = [&](int sc, uint32_t(&out)[EM]) {
#pragma unroll
        for (int j = 0; j < EM; ++j) {
            const int p = order_pos<EM, CH>(sc, j);
            out[j] = p < ncand ? Tr::cand_key(scr[p]) : 0u;
        }
    };
    radix_threshold<EM, Tr::KEYBITS>(sm.sel, nsc, cand_load, (uint32_t)k, thi, level, margin);
    compact<EM, CH>(sm.sel, nsc, cand_load, thi, level, margin, [&](uint32_t pos, int sc, int j) {
        if (pos >= (uint32_t)k) return;
        const int p = order_pos<EM, CH>(sc, j);
        const Cand c = scr[p];
        const int idx = (p / k) * a.block_n + Tr::cand_li(c);
        sm.cand[pos] = ((uint64_t)Tr::cand_key(c) << 8) | (uint64_t)(127u - pos);
        sm.idx[pos] = idx < V ? idx : V - 1;
    });
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        uint64_t c0 = (2 * lane < k) ? sm.cand[2 * lane] : 0ull;
        uint64_t c1 = (2 * lane + 1 < k) ? sm.cand[2 * lane + 1] : 0ull;
        wave_sort128_desc(c0, c1);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = 2 * lane + i;
            const uint64_t c = i ? c1 : c0;
            if (e < k) {
                const uint32_t key = (uint32_t)(c >> 8);
                const int pos = 127 - (int)(c & 0x7fu);
                const int64_t o = (int64_t)row * k + e;
                if (F32) {
                    ((float *)a.values)[o] = __uint_as_float(unkey32(key));
                } else {
                    ((uint16_t *)a.values)[o] = (uint16_t)unkey16(key);
                }
                a.indices[o] = sm.idx[pos];
            }
        }
    }
}

template <bool F32>
static int launch_topk(const ss_topk_args *a, int tiles) {
    dim3 grid((unsigned)(a->rows * tiles)), block(SS_BLOCK);
    hipStream_t s = (hipStream_t)a->stream;
    switch (a->block_n) {
        case 1024: hipLaunchKernelGGL((topk_tiles_kernel<F32, 4>), grid, block, 0, s, *a, tiles); break;
        case 2048: hipLaunchKernelGGL((topk_tiles_kernel<F32, 8>), grid, block, 0, s, *a, tiles); break;
        case 4096: hipLaunchKernelGGL((topk_tiles_kernel<F32, 16>), grid, block, 0, s, *a, tiles); break;
        case 8192: hipLaunchKernelGGL((topk_tiles_kernel<F32, 32>), grid, block, 0, s, *a, tiles); break;
        default: return SS_ERR_UNSUPPORTED;
    }
    if (hipGetLastError() != hipSuccess) return SS_ERR_LAUNCH;
    hipLaunchKernelGGL((topk_merge_kernel<F32>), dim3((unsigned)a->rows), block, 0, s, *a, tiles);
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}

}  // namespace ss

extern "C" int ss_topk(const ss_topk_args *a) {
    if (!a || !a->logits || !a->scratch || !a->values || !a->indices)
        return SS_ERR_INVALID_ARGUMENT;
    if (a->rows < 0 || a->vocab_size <= 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->k < 1 || a->k > SS_MAX_K || (a->k & (a->k - 1)) != 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->block_n != 1024 && a->block_n != 2048 && a->block_n != 4096 && a->block_n != 8192)
        return SS_ERR_UNSUPPORTED;
    if (a->dtype != SS_DTYPE_BF16 && a->dtype != SS_DTYPE_F32) return SS_ERR_UNSUPPORTED;
    const int tiles = (a->vocab_size + a->block_n - 1) / a->block_n;
    if (tiles < 2) return SS_ERR_INVALID_ARGUMENT;
    if ((int64_t)tiles * a->k > a->stride_scratch) return SS_ERR_INVALID_ARGUMENT;
    if (a->stride_logits < a->vocab_size) return SS_ERR_INVALID_ARGUMENT;
    if (a->rows == 0) return SS_OK;
    return a->dtype == SS_DTYPE_F32 ? ss::launch_topk<true>(a, tiles)
                                    : ss::launch_topk<false>(a, tiles);
}
