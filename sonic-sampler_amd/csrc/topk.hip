// Bounded top-k over [rows, vocab] logits (replaces K2 ops/topk/bitpack.py:99-158 followed by K3
// ops/topk/unpack.py:312-377 of the reference), as two back-to-back launches, or one launch of a
// 1024-thread workgroup per row (topk_wide_kernel) for many rows of at most 32768 columns.
//
// Tile stage, grid rows * tiles: each workgroup turns block_n logits into order-preserving keys
// and writes its exact top-k (ties to the lowest column) to the scratch row in column order.
// Merge stage, grid rows: selects the row's top-k among the tiles * k candidates from a sample of
// at most 512 (the first entries of every sorted list), completed list by list where the sample
// was not exact and by a radix selection over every candidate where many lists were cut short;
// sorts them by (value desc, column asc) with wave64 bitonic networks and writes values / indices
// densely as [rows, k].
#include "ss_sampling.h"
#include "../../include/sonic_sampler.h"

namespace ss {

struct TopkSmem {
    SelectSmem sel;
    uint64_t cand[SS_K];
    int32_t idx[SS_K];
    uint64_t runs[SS_WAVES][SS_K];  // merge of up to 512 candidates: the waves' sorted runs
    int32_t flag;                   // the sampled merge was not exact: take the radix merge
};

// Lists that the merge stage merges whole after its sampled merge before it takes the radix merge.
constexpr int TOPK_REFILL_LISTS = 16;

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

// Merge stage: grid rows.
template <bool F32>
__global__ __launch_bounds__(SS_BLOCK) void topk_merge_kernel(void *p_scratch, int64_t p_stride, int p_vocab,
                                                              int p_k, int p_block_n, int tiles,
                                                              ss_topk_args a) {
    using Tr = TopkTraits<F32>;
    using Cand = typename Tr::Cand;
    constexpr int CH = 4;
    __shared__ TopkSmem sm;
    const int row = blockIdx.x;
    const int V = p_vocab;
    const int k = p_k;
    const Cand *scr = (const Cand *)p_scratch + (int64_t)row * p_stride;
    const int ncand = tiles * k;
    // Samples: the first kp entries of every sorted list, kp = k when all tiles * k candidates
    // fit in 512 slots, else the largest power of two <= 512 / tiles (0 above 512 tiles).
    const int kp = ncand <= 2 * SS_BLOCK ? k
                   : tiles <= 2 * SS_BLOCK ? 1 << (31 - __builtin_clz((unsigned)(2 * SS_BLOCK / tiles))) : 0;
    // k <= 64: 256 samples, one per thread, and the network one element per lane (the same
    // exactness check and list refill as below against the k-th of the top-64)
    const int kp64 = ncand <= SS_BLOCK ? k
                     : tiles <= SS_BLOCK ? 1 << (31 - __builtin_clz((unsigned)(SS_BLOCK / tiles))) : 0;
    if (k <= 64 && kp64 > 0) {
        const int lane = lane_id(), wave = (int)threadIdx.x >> 6;
        const int lk = __builtin_ctz((unsigned)k), lkp = __builtin_ctz((unsigned)kp64);
        auto composite = [&](int p) {
            const Cand cd = scr[p];
            const uint32_t col = (uint32_t)((p >> lk) * p_block_n + Tr::cand_li(cd));
            return ((uint64_t)Tr::cand_key(cd) << 32) | (uint64_t)(0xffffffffu - col);
        };
        const int s = (int)threadIdx.x;
        const int list = s >> lkp;
        uint64_t c = list < tiles ? composite(list * k + (s & (kp64 - 1))) : 0ull;
        // wave 0: the first unsampled entry of list t = lane, read with the samples so that the
        // exactness check below waits for no further load
        const uint64_t head = threadIdx.x < 64 && kp64 < k && lane < tiles ? composite(lane * k + kp64) : 0ull;
        // the samples depend on the row and the preloaded arguments only: in flight before the
        // argument lines the rest of the merge reads
        touch_kernargs<sizeof(ss_topk_args)>();
        wave_sort64_desc(c);
        sm.runs[wave][lane] = c;
        __syncthreads();
        if (wave < 2) {
            uint64_t x = max_u64(sm.runs[2 * wave][lane], sm.runs[2 * wave + 1][63 - lane]);
            wave_bitonic64_desc(x);
            sm.runs[2 * wave][lane] = x;
        }
        __syncthreads();
        if (wave == 0) {
            uint64_t f = max_u64(sm.runs[0][lane], sm.runs[2][63 - lane]);
            wave_bitonic64_desc(f);
            auto kth = [&]() {
                return ((uint64_t)__builtin_amdgcn_readlane((int)(f >> 32), k - 1) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)f, k - 1);
            };
            int beats = 0;
            if (kp64 < k) {
                const uint64_t last = kth();
                for (int t0 = 0; t0 < tiles; t0 += 64) {
                    const int t = t0 + lane;
                    beats += __popcll(__ballot(t < tiles && (t0 ? composite(t * k + kp64) : head) > last));
                }
            }
            if (beats > TOPK_REFILL_LISTS) {
                if (lane == 0) sm.flag = 1;
            } else {
                for (int t0 = 0; beats > 0 && t0 < tiles; t0 += 64) {
                    const int t = t0 + lane;
                    const uint64_t nx = t < tiles ? (t0 ? composite(t * k + kp64) : head) : 0ull;
                    uint64_t m = __ballot(nx > kth());
                    while (m) {
                        const int l = t0 + (int)__builtin_ctzll(m);
                        // lane pairs with entry kp + 63 - lane of list l (kp .. k - 1 exist)
                        const uint64_t r = lane >= 64 - k + kp64 ? composite(l * k + kp64 + 63 - lane) : 0ull;
                        f = max_u64(f, r);
                        wave_bitonic64_desc(f);
                        m &= m - 1;
                        m &= __ballot(nx > kth());
                    }
                }
                if (lane < k) {
                    const uint32_t key = (uint32_t)(f >> 32);
                    const int col = (int)(0xffffffffu - (uint32_t)f);
                    const int64_t o = (int64_t)row * k + lane;
                    if (F32) {
                        ((float *)a.values)[o] = __uint_as_float(unkey32(key));
                    } else {
                        ((uint16_t *)a.values)[o] = (uint16_t)unkey16(key);
                    }
                    a.indices[o] = col < V ? col : V - 1;
                }
                if (lane == 0) sm.flag = 0;
            }
        }
        __syncthreads();
        if (!sm.flag) return;
    } else if (kp > 0) {
        // Up to 512 samples, two per thread, as composites (key << 32) | (~column): their
        // descending order is (value desc, column asc). Every wave sorts its 128, and two rounds
        // of bitonic merges keep the top-128 of the four runs (the elementwise maximum of a run
        // and its reversed partner is a bitonic sequence holding the top-128 of both).
        const int lane = lane_id(), wave = (int)threadIdx.x >> 6;
        const int lk = __builtin_ctz((unsigned)k), lkp = __builtin_ctz((unsigned)kp);  // powers of two
        auto composite = [&](int p) {
            const Cand cd = scr[p];
            const uint32_t col = (uint32_t)((p >> lk) * p_block_n + Tr::cand_li(cd));
            return ((uint64_t)Tr::cand_key(cd) << 32) | (uint64_t)(0xffffffffu - col);
        };
        uint64_t c[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int s = 2 * (int)threadIdx.x + i;
            const int list = s >> lkp;
            c[i] = list < tiles ? composite(list * k + (s & (kp - 1))) : 0ull;
        }
        // wave 0: the first unsampled entry of list t = lane, read with the samples
        const uint64_t head = threadIdx.x < 64 && kp < k && lane < tiles ? composite(lane * k + kp) : 0ull;
        touch_kernargs<sizeof(ss_topk_args)>();
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
            // the k-th merged composite (element k - 1)
            auto kth = [&]() {
                const uint64_t x = ((k - 1) & 1) ? f[1] : f[0];
                const int src = (k - 1) >> 1;
                return ((uint64_t)__builtin_amdgcn_readlane((int)(x >> 32), src) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, src);
            };
            // Exactness: no list's first unsampled entry may beat the k-th merged composite. Up
            // to TOPK_REFILL_LISTS lists that do are merged whole, in list order, each against
            // the current k-th (which only rises, so a list passed over never beats it later):
            // the elementwise maximum of the sorted top-128 and the list's remaining k - kp
            // entries in reverse order is bitonic and holds the top-128 of both.
            int beats = 0;
            if (kp < k) {
                const uint64_t last = kth();
                for (int t0 = 0; t0 < tiles; t0 += 64) {
                    const int t = t0 + lane;
                    beats += __popcll(__ballot(t < tiles && (t0 ? composite(t * k + kp) : head) > last));
                }
            }
            if (beats > TOPK_REFILL_LISTS) {
                if (lane == 0) sm.flag = 1;
            } else {
                for (int t0 = 0; beats > 0 && t0 < tiles; t0 += 64) {
                    const int t = t0 + lane;
                    const uint64_t nx = t < tiles ? (t0 ? composite(t * k + kp) : head) : 0ull;
                    uint64_t m = __ballot(nx > kth());
                    while (m) {
                        const int l = t0 + (int)__builtin_ctzll(m);
#pragma unroll
                        for (int i = 0; i < 2; ++i) {
                            // element e pairs with entry kp + 127 - e of list l (kp .. k - 1 exist)
                            const int e = 2 * lane + i;
                            const uint64_t r = e >= SS_K - k + kp ? composite(l * k + kp + 127 - e) : 0ull;
                            f[i] = max_u64(f[i], r);
                        }
                        wave_bitonic128_desc<128>(f[0], f[1]);
                        m &= m - 1;
                        m &= __ballot(nx > kth());
                    }
                }
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
                if (lane == 0) sm.flag = 0;
            }
        }
        __syncthreads();
        if (!sm.flag) return;
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
        const int idx = (p / k) * p_block_n + Tr::cand_li(c);
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

// ---------------------------------------------------------------------------------------------
// Block selection: one workgroup holds a block of SS_BLOCK * E columns (E values per thread,
// element j of thread t at column (j / 4) * 1024 + 4 t + j % 4 of the block, loaded as 16-byte fp32
// / 8-byte bf16 chunks) and selects its top-k: the block is tile blockIdx.x % tiles of row
// blockIdx.x / tiles and its top-k goes to the scratch row as packed candidates for the merge
// kernel.
//
// Lower bound: every wave sorts its 64 lane maxima; at least need_w of its lanes hold a value >= the
// need_w-th largest of them, with need_w the wave's share of k (k / 4 in a full block, in
// proportion to its valid columns in a partial one, summing to at least k), so with lo the
// smallest of the waves' bounds the block holds at least k values >= lo. The survivors (values >= lo: a few dozen on unstructured rows) are
// collected per wave by a ballot at each element position, skipped uniformly where no lane of the
// wave survives, as composites (key32 << 32) | ~column. Every wave sorts its survivors, two rounds
// of bitonic merges keep the top-128 of the four runs, and the first k are written. A wave with more
// than 128 survivors (long runs of equal values) sends the row to the exact radix selection.
// ---------------------------------------------------------------------------------------------
struct TopkRowSmem {
    SelectSmem sel;                 // exact fallback
    uint64_t runs[SS_WAVES][SS_K];  // each wave's survivors, then its sorted run
    uint64_t cand[SS_K];            // exact fallback: the selected composites
    uint32_t red[SS_WAVES];
};

// Order-preserving 32-bit key of a float (-0 and +0 share the key of +0).
__device__ __forceinline__ uint32_t float_key(float v) {
    const uint32_t u = __float_as_uint(v + 0.0f);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}

template <bool F32, bool VEC, int E>
__global__ __launch_bounds__(SS_BLOCK) void topk_block_kernel(const void *p_logits, int64_t p_stride,
                                                              int p_block_n, int p_vocab, int p_k, int tiles,
                                                              ss_topk_args a) {
    __shared__ TopkRowSmem sm;
    const int row = (int)blockIdx.x / tiles;
    const int tile = (int)blockIdx.x - row * tiles;
    const int col0 = tile * p_block_n;  // first column of the block
    const int V = min(p_block_n, p_vocab - col0);  // columns of the block
    const int k = p_k;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane4 = 4 * (int)threadIdx.x;
    const int64_t bytes = (int64_t)V * (F32 ? 4 : 2);
    const char *base = (const char *)p_logits + ((int64_t)row * p_stride + col0) * (F32 ? 4 : 2);
    const __amdgpu_buffer_rsrc_t rb = row_buffer(base, bytes);
    // the block's top-k: packed candidates of the merge kernel
    auto emit = [&](int e, uint32_t key, int col) {
        using Tr = TopkTraits<F32>;
        typename Tr::Cand *scr = (typename Tr::Cand *)a.scratch + (int64_t)row * a.stride_scratch;
        // absent elements (key 0) keep key 0 in the 16-bit packing too
        const uint32_t pk = F32 ? key : key ? key16(__float_as_uint(__uint_as_float(unkey32(key))) >> 16) : 0u;
        scr[tile * k + e] = Tr::pack(pk, col);
    };

    // ---- the row, every load issued before any is used; columns past V read -inf -----------------
    float v[E];
#pragma unroll
    for (int c = 0; c < E / 4; ++c) {
        const int col = c * (SS_BLOCK * 4) + lane4;
        uint32_t w[4];
        if (VEC) {
            if (F32) {
                const i32x4 q = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, col * 4, 0, NT));
                w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
            } else {
                const u32x2 q = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rb, col * 2, 0, NT));
                w[0] = q.x << 16; w[1] = q.x & 0xffff0000u; w[2] = q.y << 16; w[3] = q.y & 0xffff0000u;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[i] = F32 ? __builtin_amdgcn_raw_buffer_load_b32(rb, (col + i) * 4, 0, NT)
                           : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb, (col + i) * 2, 0, NT) << 16;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 * c + i] = col + i < V ? __uint_as_float(w[i]) : -INFINITY;
    }
    auto col_of = [&](int j) { return (j >> 2) * (SS_BLOCK * 4) + lane4 + (j & 3); };
    auto composite = [&](int j) {
        return ((uint64_t)float_key(v[j]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)col_of(j));
    };

    // ---- lower bound from the waves' sorted lane maxima ------------------------------------------
    float m = v[0];
#pragma unroll
    for (int j = 1; j < E; ++j) m = fmaxf(m, v[j]);
    uint32_t mk = float_key(m);
    wave_sort64_desc(mk);
    // The wave's share of k is proportional to the valid columns it holds (chunk c gives it
    // columns c * 1024 + 256 * wave .. + 255), so a partial last tile, whose columns sit in its
    // first waves, still gets a bound; a wave without columns takes no part in the minimum, and
    // a share above its 64 lanes leaves the bound to the exact selection.
    int nw = 0;
#pragma unroll
    for (int c = 0; c < E / 4; ++c) nw += min(max(V - (c * (SS_BLOCK * 4) + 256 * wave), 0), 256);
    const int need = nw ? (k * nw + V - 1) / V : 0;
    if (need == 0 && lane == 0) sm.red[wave] = 0xffffffffu;
    if (need > 64 && lane == 0) sm.red[wave] = 0u;
    if (need > 0 && need <= 64 && lane == need - 1) sm.red[wave] = mk;
    __syncthreads();
    const uint32_t lo = min(min(sm.red[0], sm.red[1]), min(sm.red[2], sm.red[3]));
    const bool no_bound = lo == 0u;
    // the float whose key is lo (lo is the key of a lane maximum, so it is a value of the row)
    const float lo_f = __uint_as_float((lo & 0x80000000u) ? (lo & 0x7fffffffu) : ~lo);
    __syncthreads();

    // ---- survivors per wave ----------------------------------------------------------------------
    uint64_t *run = sm.runs[wave];
    uint32_t cnt = 0;  // wave-uniform
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const bool p = v[j] >= lo_f;
        const uint64_t msk = __ballot(p);
        if (msk) {
            const uint32_t pos = cnt + mbcnt64(msk);
            if (p && pos < (uint32_t)SS_K) run[pos] = composite(j);
            cnt += (uint32_t)__popcll(msk);
        }
    }
    if (lane == 0) sm.red[wave] = cnt;
    __syncthreads();
    const uint32_t most = max(max(sm.red[0], sm.red[1]), max(sm.red[2], sm.red[3]));
    const bool overflow = most > (uint32_t)SS_K || V < k || no_bound;
    if (!overflow && k <= 64 && most <= 64) {
        // k <= 64 and at most 64 survivors per wave: the same network one element per lane
        uint64_t c = lane < (int)cnt ? run[lane] : 0ull;
        wave_sort64_desc(c);
        run[lane] = c;
        __syncthreads();
        if (wave < 2) {
            // top-64 of runs 2w and 2w+1 (the second reversed: a bitonic sequence)
            uint64_t x = max_u64(sm.runs[2 * wave][lane], sm.runs[2 * wave + 1][63 - lane]);
            wave_bitonic64_desc(x);
            sm.runs[2 * wave][lane] = x;
        }
        __syncthreads();
        if (wave == 0) {
            uint64_t f = max_u64(sm.runs[0][lane], sm.runs[2][63 - lane]);
            wave_bitonic64_desc(f);
            if (lane < k) emit(lane, (uint32_t)(f >> 32), (int)(0xffffffffu - (uint32_t)f));
        }
        return;
    }
    if (!overflow) {
        uint64_t c0 = 2 * lane < (int)cnt ? run[2 * lane] : 0ull;
        uint64_t c1 = 2 * lane + 1 < (int)cnt ? run[2 * lane + 1] : 0ull;
        wave_sort128_desc(c0, c1);
        run[2 * lane] = c0;
        run[2 * lane + 1] = c1;
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
                if (e < k) emit(e, (uint32_t)(f[i] >> 32), (int)(0xffffffffu - (uint32_t)f[i]));
            }
        }
        return;
    }

    // ---- exact selection over the whole block (ties at the k-th value kept in column order) -------
    auto keys_of = [&](int, uint32_t(&out)[E]) {
#pragma unroll
        for (int j = 0; j < E; ++j) out[j] = col_of(j) < V ? float_key(v[j]) : 0u;
    };
    uint32_t thi, margin;
    int level;
    radix_threshold<E, 32>(sm.sel, 1, keys_of, (uint32_t)k, thi, level, margin);
    compact<E, 4>(sm.sel, 1, keys_of, thi, level, margin, [&](uint32_t pos, int, int j) {
        if (pos < (uint32_t)k) sm.cand[pos] = col_of(j) < V ? composite(j) : (uint64_t)(0xffffffffu - (uint32_t)col_of(j));
    });
    __syncthreads();
    if (wave == 0) {
        uint64_t c0 = 2 * lane < k ? sm.cand[2 * lane] : 0ull;
        uint64_t c1 = 2 * lane + 1 < k ? sm.cand[2 * lane + 1] : 0ull;
        wave_sort128_desc(c0, c1);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int e = 2 * lane + i;
            const uint64_t c = i ? c1 : c0;
            if (e < k) emit(e, (uint32_t)(c >> 32), (int)(0xffffffffu - (uint32_t)c));
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Whole rows of at most 32768 columns in one workgroup of 1024 threads: one launch and no scratch
// round trip. 32 values per thread, element j of thread t at column (j / 4) * 4096 + 4 t + j % 4,
// loaded as 16-byte fp32 / 8-byte bf16 chunks. The lower bound of topk_block_kernel over 16 waves
// (each wave's share of k from its sorted lane maxima, the smallest of the 16 bounds), the
// survivors of every wave gathered into one list and sorted by wave 0 (waves 0 and 1 for more than
// 128). Rows whose survivors overflow the list (long runs of equal values) take an exact selection
// over the registers: the k-th largest key by bisection on workgroup counts, the ties at it kept
// in column order by workgroup scans, chunk by chunk.
// ---------------------------------------------------------------------------------------------
constexpr int TOPK_WIDE_THREADS = 1024;
constexpr int TOPK_WIDE_WAVES = TOPK_WIDE_THREADS / 64;
constexpr int TOPK_WIDE_E = 32;                          // 32768 columns
constexpr int TOPK_WIDE_CHUNK = 4 * TOPK_WIDE_THREADS;   // columns of one 4-element chunk
constexpr int TOPK_WIDE_LIST = 2 * SS_K;

struct TopkWideSmem {
    uint64_t runs[TOPK_WIDE_WAVES][SS_K];  // each wave's survivors
    uint64_t list[TOPK_WIDE_LIST];         // the row's survivors, or its exact selection
    uint32_t red[TOPK_WIDE_WAVES];
};

// Workgroup sum of one count per thread (all threads call).
__device__ __forceinline__ uint32_t wide_sum(uint32_t n, uint32_t *red) {
    n = wave_sum(n);
    if (lane_id() == 0) red[threadIdx.x >> 6] = n;
    __syncthreads();
    uint32_t s = 0;
#pragma unroll
    for (int w = 0; w < TOPK_WIDE_WAVES; ++w) s += red[w];
    __syncthreads();
    return s;
}

// Exclusive scan of one count per thread in thread order, and the total (all threads call).
__device__ __forceinline__ uint32_t wide_exclusive_scan(uint32_t n, uint32_t *red, uint32_t &total) {
    const int wave = (int)threadIdx.x >> 6;
    const uint32_t inc = wave_inclusive_sum(n);
    if (lane_id() == 63) red[wave] = inc;
    __syncthreads();
    uint32_t before = 0, t = 0;
#pragma unroll
    for (int w = 0; w < TOPK_WIDE_WAVES; ++w) {
        const uint32_t r = red[w];
        before += w < wave ? r : 0u;
        t += r;
    }
    __syncthreads();
    total = t;
    return before + inc - n;
}

template <bool F32, bool VEC>
__global__ __launch_bounds__(TOPK_WIDE_THREADS) void topk_wide_kernel(const void *p_logits, int64_t p_stride, int p_vocab,
                                                                     int p_k, ss_topk_args a) {
    __shared__ TopkWideSmem sm;
    constexpr int E = TOPK_WIDE_E;
    const int row = (int)blockIdx.x;
    const int V = p_vocab;
    const int k = p_k;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane4 = 4 * (int)threadIdx.x;
    const char *base = (const char *)p_logits + (int64_t)row * p_stride * (F32 ? 4 : 2);
    const __amdgpu_buffer_rsrc_t rb = row_buffer(base, (int64_t)V * (F32 ? 4 : 2));
    auto emit = [&](int e, uint64_t c) {
        const float val = __uint_as_float(unkey32((uint32_t)(c >> 32)));
        const int col = (int)(0xffffffffu - (uint32_t)c);
        const int64_t o = (int64_t)row * k + e;
        if (F32) ((float *)a.values)[o] = val;
        else ((uint16_t *)a.values)[o] = (uint16_t)(__float_as_uint(val) >> 16);
        a.indices[o] = col < V ? col : V - 1;
    };

    float v[E];
#pragma unroll
    for (int c = 0; c < E / 4; ++c) {
        const int col = c * TOPK_WIDE_CHUNK + lane4;
        uint32_t w[4];
        if (VEC) {
            if (F32) {
                const i32x4 q = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, col * 4, 0, NT));
                w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
            } else {
                const u32x2 q = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rb, col * 2, 0, NT));
                w[0] = q.x << 16; w[1] = q.x & 0xffff0000u; w[2] = q.y << 16; w[3] = q.y & 0xffff0000u;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w[i] = F32 ? __builtin_amdgcn_raw_buffer_load_b32(rb, (col + i) * 4, 0, NT)
                           : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb, (col + i) * 2, 0, NT) << 16;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) v[4 * c + i] = col + i < V ? __uint_as_float(w[i]) : -INFINITY;
    }
    auto col_of = [&](int j) { return (j >> 2) * TOPK_WIDE_CHUNK + lane4 + (j & 3); };
    auto composite = [&](int j) {
        return ((uint64_t)float_key(v[j]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)col_of(j));
    };

    // ---- lower bound: the wave's share of k from its sorted lane maxima -------------------------
    float m = v[0];
#pragma unroll
    for (int j = 1; j < E; ++j) m = fmaxf(m, v[j]);
    uint32_t mk = float_key(m);
    wave_sort64_desc(mk);
    int nw = 0;  // columns of the row this wave holds (256 of every chunk)
#pragma unroll
    for (int c = 0; c < E / 4; ++c) nw += min(max(V - (c * TOPK_WIDE_CHUNK + 256 * wave), 0), 256);
    const int need = nw ? (k * nw + V - 1) / V : 0;
    if (need == 0 && lane == 0) sm.red[wave] = 0xffffffffu;
    if (need > 64 && lane == 0) sm.red[wave] = 0u;
    if (need > 0 && need <= 64 && lane == need - 1) sm.red[wave] = mk;
    __syncthreads();
    uint32_t lo = 0xffffffffu;
#pragma unroll
    for (int w = 0; w < TOPK_WIDE_WAVES; ++w) lo = min(lo, sm.red[w]);
    const bool no_bound = lo == 0u;
    const float lo_f = __uint_as_float((lo & 0x80000000u) ? (lo & 0x7fffffffu) : ~lo);
    __syncthreads();

    // ---- survivors per wave, then one list -----------------------------------------------------
    uint64_t *run = sm.runs[wave];
    uint32_t cnt = 0;  // wave-uniform
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const bool p = v[j] >= lo_f;
        const uint64_t msk = __ballot(p);
        if (msk) {
            const uint32_t pos = cnt + mbcnt64(msk);
            if (p && pos < (uint32_t)SS_K) run[pos] = composite(j);
            cnt += (uint32_t)__popcll(msk);
        }
    }
    if (lane == 0) sm.red[wave] = cnt;
    __syncthreads();
    uint32_t off = 0, total = 0, most = 0;
#pragma unroll
    for (int w = 0; w < TOPK_WIDE_WAVES; ++w) {
        const uint32_t c = sm.red[w];
        off += w < wave ? c : 0u;
        total += c;
        most = max(most, c);
    }
    const bool overflow = most > (uint32_t)SS_K || total > (uint32_t)TOPK_WIDE_LIST || no_bound;
    if (!overflow) {
        for (uint32_t i = (uint32_t)lane; i < cnt; i += 64) sm.list[off + i] = run[i];
        __syncthreads();
        if (total <= 64) {
            if (wave == 0) {
                uint64_t c = lane < (int)total ? sm.list[lane] : 0ull;
                wave_sort64_desc(c);
                if (lane < k) emit(lane, c);
            }
            return;
        }
        // up to 256: waves 0 and 1 sort 128 each, wave 0 keeps the top-128 of the two runs
        if (wave < 2) {
            const int b0 = SS_K * wave;
            uint64_t c0 = b0 + 2 * lane < (int)total ? sm.list[b0 + 2 * lane] : 0ull;
            uint64_t c1 = b0 + 2 * lane + 1 < (int)total ? sm.list[b0 + 2 * lane + 1] : 0ull;
            wave_sort128_desc(c0, c1);
            sm.runs[wave][2 * lane] = c0;
            sm.runs[wave][2 * lane + 1] = c1;
        }
        __syncthreads();
        if (wave == 0) {
            uint64_t f0 = max_u64(sm.runs[0][2 * lane], sm.runs[1][127 - 2 * lane]);
            uint64_t f1 = max_u64(sm.runs[0][2 * lane + 1], sm.runs[1][126 - 2 * lane]);
            wave_bitonic128_desc<128>(f0, f1);
            if (2 * lane < k) emit(2 * lane, f0);
            if (2 * lane + 1 < k) emit(2 * lane + 1, f1);
        }
        return;
    }

    // ---- exact selection: the k-th largest key T, then every key > T and the first ties --------
    // Every wave has read the survivor counts in sm.red before any wave passes this barrier, so
    // the first wide_sum below cannot overwrite a count a slower wave still has to read (which
    // could send that wave down the other branch).
    __syncthreads();
    uint32_t key[E];
#pragma unroll
    for (int j = 0; j < E; ++j) key[j] = col_of(j) < V ? float_key(v[j]) : 0u;
    uint32_t T = 0;  // the largest t with at least k keys >= t
#pragma unroll 1
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = T | (1u << b);
        uint32_t n = 0;
#pragma unroll
        for (int j = 0; j < E; ++j) n += key[j] >= c ? 1u : 0u;
        if (wide_sum(n, sm.red) >= (uint32_t)k) T = c;
    }
    uint32_t n_above = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) n_above += key[j] > T ? 1u : 0u;
    const uint32_t margin = (uint32_t)k - wide_sum(n_above, sm.red);  // ties kept
    uint32_t base_g = 0, base_q = 0;
#pragma unroll
    for (int c = 0; c < E / 4; ++c) {
        uint32_t g = 0, q = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g += key[4 * c + i] > T ? 1u : 0u;
            q += key[4 * c + i] == T ? 1u : 0u;
        }
        uint32_t tot;
        const uint32_t ex = wide_exclusive_scan(g | (q << 16), sm.red, tot);
        g = base_g + (ex & 0xffffu);
        q = base_q + (ex >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * c + i;
            if (key[j] > T) {
                sm.list[g + (q < margin ? q : margin)] = composite(j);
                ++g;
            } else if (key[j] == T) {
                if (q < margin) sm.list[g + q] = composite(j);
                ++q;
            }
        }
        base_g += tot & 0xffffu;
        base_q += tot >> 16;
    }
    __syncthreads();
    if (wave == 0) {
        uint64_t c0 = 2 * lane < k ? sm.list[2 * lane] : 0ull;
        uint64_t c1 = 2 * lane + 1 < k ? sm.list[2 * lane + 1] : 0ull;
        wave_sort128_desc(c0, c1);
        if (2 * lane < k) emit(2 * lane, c0);
        if (2 * lane + 1 < k) emit(2 * lane + 1, c1);
    }
}

template <bool F32>
static bool topk_vec(const ss_topk_args *a) {
    const int esz = F32 ? 4 : 2;
    return (a->vocab_size % 4) == 0 && (a->stride_logits % 4) == 0 && ((uintptr_t)a->logits % (4 * esz)) == 0;
}

template <bool F32>
static int launch_topk_rows(const ss_topk_args *a) {
    dim3 grid((unsigned)a->rows), block(TOPK_WIDE_THREADS);
    hipStream_t s = (hipStream_t)a->stream;
    if (topk_vec<F32>(a)) hipLaunchKernelGGL((topk_wide_kernel<F32, true>), grid, block, 0, s, a->logits, a->stride_logits, a->vocab_size, a->k, *a);
    else hipLaunchKernelGGL((topk_wide_kernel<F32, false>), grid, block, 0, s, a->logits, a->stride_logits, a->vocab_size, a->k, *a);
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}

template <bool F32, bool VEC>
static int launch_topk_tiles(const ss_topk_args *a, int tiles, dim3 grid, dim3 block, hipStream_t s) {
    switch (a->block_n) {
        case 1024: hipLaunchKernelGGL((topk_block_kernel<F32, VEC, 4>), grid, block, 0, s, a->logits, a->stride_logits, a->block_n, a->vocab_size, a->k, tiles, *a); break;
        case 2048: hipLaunchKernelGGL((topk_block_kernel<F32, VEC, 8>), grid, block, 0, s, a->logits, a->stride_logits, a->block_n, a->vocab_size, a->k, tiles, *a); break;
        case 4096: hipLaunchKernelGGL((topk_block_kernel<F32, VEC, 16>), grid, block, 0, s, a->logits, a->stride_logits, a->block_n, a->vocab_size, a->k, tiles, *a); break;
        case 8192: hipLaunchKernelGGL((topk_block_kernel<F32, VEC, 32>), grid, block, 0, s, a->logits, a->stride_logits, a->block_n, a->vocab_size, a->k, tiles, *a); break;
        case 16384: hipLaunchKernelGGL((topk_block_kernel<F32, VEC, 64>), grid, block, 0, s, a->logits, a->stride_logits, a->block_n, a->vocab_size, a->k, tiles, *a); break;
        default: return SS_ERR_UNSUPPORTED;
    }
    return SS_OK;
}

template <bool F32>
static int launch_topk(const ss_topk_args *a, int tiles) {
    dim3 grid((unsigned)(a->rows * tiles)), block(SS_BLOCK);
    hipStream_t s = (hipStream_t)a->stream;
    // tiles start at multiples of block_n, so the 16 / 8-byte chunks of every tile stay aligned
    const int st = topk_vec<F32>(a) ? launch_topk_tiles<F32, true>(a, tiles, grid, block, s)
                                    : launch_topk_tiles<F32, false>(a, tiles, grid, block, s);
    if (st != SS_OK) return st;
    if (hipGetLastError() != hipSuccess) return SS_ERR_LAUNCH;
    hipLaunchKernelGGL((topk_merge_kernel<F32>), dim3((unsigned)a->rows), block, 0, s, a->scratch, a->stride_scratch, a->vocab_size, a->k,
                       a->block_n, tiles, *a);
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}

}  // namespace ss

extern "C" int ss_topk(const ss_topk_args *a) {
    if (!a || !a->logits || !a->scratch || !a->values || !a->indices)
        return SS_ERR_INVALID_ARGUMENT;
    if (a->rows < 0 || a->vocab_size <= 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->k < 1 || a->k > SS_MAX_K || (a->k & (a->k - 1)) != 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->block_n != 1024 && a->block_n != 2048 && a->block_n != 4096 && a->block_n != 8192 && a->block_n != 16384)
        return SS_ERR_UNSUPPORTED;
    if (a->dtype != SS_DTYPE_BF16 && a->dtype != SS_DTYPE_F32) return SS_ERR_UNSUPPORTED;
    const int tiles = (a->vocab_size + a->block_n - 1) / a->block_n;
    if (tiles < 2) return SS_ERR_INVALID_ARGUMENT;
    if ((int64_t)tiles * a->k > a->stride_scratch) return SS_ERR_INVALID_ARGUMENT;
    if (a->stride_logits < a->vocab_size) return SS_ERR_INVALID_ARGUMENT;
    if (a->rows == 0) return SS_OK;
    if (a->strategy < SS_STRATEGY_AUTO || a->strategy > SS_STRATEGY_ROWWISE) return SS_ERR_INVALID_ARGUMENT;
    // One 1024-thread workgroup per row (one launch) serves rows of at most 32768 columns on
    // request. AUTO takes it where it measured faster than the tile grid at the tuned widths: at
    // least 48 rows of more than 16384 columns and k <= 32 (rows of 32000 columns at k = 32, back
    // to back: fp32 48 rows 9.3 us against 9.6, 128 rows 9.7 against 11.3, 256 rows 12.1 against
    // 17.0; bf16 64 rows 8.8 against 9.5). Fewer rows leave CUs idle while one CU streams each
    // row (fp32 32 rows: 9.2 against 8.6 us), narrower rows leave most of a thread's 32 elements
    // empty, and a larger k overflows the survivor list into the exact selection.
    if (a->strategy == SS_STRATEGY_ROWWISE && a->vocab_size > ss::TOPK_WIDE_THREADS * ss::TOPK_WIDE_E) return SS_ERR_UNSUPPORTED;
    const bool wide = a->strategy == SS_STRATEGY_ROWWISE ||
                      (a->strategy == SS_STRATEGY_AUTO && a->rows >= 48 && a->k <= 32 && a->vocab_size > 16384 &&
                       a->vocab_size <= ss::TOPK_WIDE_THREADS * ss::TOPK_WIDE_E);
    if (wide)
        return a->dtype == SS_DTYPE_F32 ? ss::launch_topk_rows<true>(a) : ss::launch_topk_rows<false>(a);
    return a->dtype == SS_DTYPE_F32 ? ss::launch_topk<true>(a, tiles)
                                    : ss::launch_topk<false>(a, tiles);
}
