// Exact, stable bounded top-k selection for one workgroup (SS_BLOCK threads).
//
// Elements are unsigned keys (see key16 / key32); a larger key is a better element and key 0 is
// the "absent" sentinel. Each thread owns E keys laid out in "chunks" of CH consecutive elements:
// element j of thread t has order position
//     (j / CH) * (SS_BLOCK * CH) + t * CH + (j % CH)
// which is the order of 16-byte (or 8-byte) coalesced loads, so the order position equals the
// column offset inside a vocabulary tile. Selection returns exactly `need` elements: every key
// above a threshold plus the first `margin` keys equal to it in order position, i.e. ties go to
// the lowest position, the rule torch's stable descending sort applies (reference semantics:
// ops/encoding.py:63-91 packs the inverted index below the key for the same effect).
//
// The threshold is found MSB-first with LDS histograms: a 12-bit first digit (4096 bins) keeps
// same-address LDS atomics rare on low-entropy logits, whose keys share sign and exponent bits,
// then the remaining 4 (16-bit keys) or 12 + 8 (32-bit keys) bits.
#pragma once

#include "ss_device.h"

namespace ss {

struct SelectSmem {
    uint32_t hist[4096];
    uint32_t scan[SS_WAVES * 8];
    uint32_t result[4];
    int32_t flag;
};

// Finds the largest bin b of hist[0, nbins) with (count of bins >= b) >= need. Returns the bin,
// the count strictly above it and the bin's own count. All threads must call.
__device__ __forceinline__ void find_bin(SelectSmem &sm, int nbins, uint32_t need, uint32_t &bin,
                                         uint32_t &above, uint32_t &count) {
    const int tid = threadIdx.x;
    const int per = nbins >= SS_BLOCK ? nbins / SS_BLOCK : 1;
    const int owners = nbins >= SS_BLOCK ? SS_BLOCK : nbins;
    if (tid == 0) {
        sm.result[0] = 0;
        sm.result[1] = 0;
        sm.result[2] = 0;
    }
    uint32_t s = 0;
    if (tid < owners) {
        for (int i = 0; i < per; ++i) s += sm.hist[tid * per + i];
    }
    uint32_t v[1] = {s}, tot[1];
    block_exclusive_scan<1>(v, tot, sm.scan);
    // v[0] = sum of bins below this thread's range.
    const uint32_t above_me = tot[0] - v[0] - s;
    if (tid < owners && above_me < need && need <= above_me + s) {
        uint32_t run = above_me;
        for (int b = tid * per + per - 1; b >= tid * per; --b) {
            uint32_t h = sm.hist[b];
            if (run + h >= need) {
                sm.result[0] = (uint32_t)b;
                sm.result[1] = run;
                sm.result[2] = h;
                break;
            }
            run += h;
        }
    }
    __syncthreads();
    bin = sm.result[0];
    above = sm.result[1];
    count = sm.result[2];
    __syncthreads();
}

// Threshold over keys supplied super-chunk by super-chunk: `load(sc, keys)` fills this thread's
// E keys of super-chunk sc (absent elements as 0). On return the selection rule is
//     select  <=>  (key >> level) > thi  ||  ((key >> level) == thi && rank_among_equal < margin)
template <int E, int KEYBITS, class Loader>
__device__ __forceinline__ void radix_threshold(SelectSmem &sm, int nsc, Loader load, uint32_t need, uint32_t &thi,
                                int &level, uint32_t &margin) {
    constexpr int ND = KEYBITS == 16 ? 2 : 3;
    const int shifts[3] = {KEYBITS - 12, KEYBITS == 16 ? 0 : 8, 0};
    const int widths[3] = {12, KEYBITS == 16 ? 4 : 12, 8};
    uint32_t prefix = 0, pmask = 0, remaining = need;
    int lvl = KEYBITS;
    for (int d = 0; d < ND; ++d) {
        const int sh = shifts[d];
        const int nb = 1 << widths[d];
        const uint32_t dm = (uint32_t)nb - 1u;
        for (int i = threadIdx.x; i < nb; i += SS_BLOCK) sm.hist[i] = 0;
        __syncthreads();
        for (int sc = 0; sc < nsc; ++sc) {
            uint32_t keys[E];
            load(sc, keys);
#pragma unroll
            for (int j = 0; j < E; ++j) {
                if ((keys[j] & pmask) == prefix) atomicAdd(&sm.hist[(keys[j] >> sh) & dm], 1u);
            }
        }
        __syncthreads();
        uint32_t b, above, cnt;
        find_bin(sm, nb, remaining, b, above, cnt);
        remaining -= above;
        prefix |= b << sh;
        pmask |= dm << sh;
        lvl = sh;
        if (remaining == cnt) break;  // the whole bin is taken: no finer digit needed
    }
    level = lvl;
    thi = prefix >> lvl;
    margin = remaining;
}

// Emits the selected elements in order position. `emit(pos, sc, j)` is called for element j of
// super-chunk sc with its output position pos in [0, need). Positions are dense and increasing in
// order position. Elements of one thread are visited in increasing order position.
template <int E, int CH, class Loader, class Emit>
__device__ __forceinline__ void compact(SelectSmem &sm, int nsc, Loader load, uint32_t thi, int level,
                        uint32_t margin, Emit emit) {
    constexpr int NCH = E / CH;
    uint32_t base_gt = 0, base_eq = 0;
    for (int sc = 0; sc < nsc; ++sc) {
        uint32_t keys[E];
        load(sc, keys);
        uint32_t cnt[NCH], tot[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            uint32_t g = 0, q = 0;
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const uint32_t kh = keys[c * CH + i] >> level;
                g += kh > thi;
                q += kh == thi;
            }
            cnt[c] = g | (q << 16);
        }
        block_exclusive_scan<NCH>(cnt, tot, sm.scan);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            uint32_t g = base_gt + (cnt[c] & 0xffffu);
            uint32_t q = base_eq + (cnt[c] >> 16);
#pragma unroll
            for (int i = 0; i < CH; ++i) {
                const int j = c * CH + i;
                const uint32_t kh = keys[j] >> level;
                if (kh > thi) {
                    emit(g + (q < margin ? q : margin), sc, j);
                    ++g;
                } else if (kh == thi) {
                    if (q < margin) emit(g + q, sc, j);
                    ++q;
                }
            }
            base_gt += tot[c] & 0xffffu;
            base_eq += tot[c] >> 16;
        }
    }
}

// Order position of element j of this thread inside super-chunk sc.
template <int E, int CH>
__device__ __forceinline__ int order_pos(int sc, int j) {
    return sc * (SS_BLOCK * E) + (j / CH) * (SS_BLOCK * CH) + (int)threadIdx.x * CH + (j % CH);
}

// Lane mask of one compare-exchange step at lane distance LD: bit l is set when lane l keeps the
// larger value of its pair, i.e. when it is the pair's lower lane (bit LD clear) in a descending
// run or its upper lane in an ascending one. The run of lane l descends when bit DB of l is clear
// (DB = 64: every run descends).
constexpr uint64_t keep_hi_mask(int LD, int DB) {
    uint64_t m = 0;
    for (int l = 0; l < 64; ++l)
        if (((l & LD) == 0) == ((l & DB) == 0)) m |= 1ull << l;
    return m;
}

// Lanes whose run descends (bit DB clear).
constexpr uint64_t desc_mask(int DB) { return keep_hi_mask(0, DB); }

// Larger and smaller of a and the value of lane (lane ^ LD).
template <int LD>
__device__ __forceinline__ void pair_max_min(uint32_t a, uint32_t &hi, uint32_t &lo) {
    static_assert(LD == 1 || LD == 2 || LD == 4 || LD == 8 || LD == 16 || LD == 32, "lane distance");
    if constexpr (LD == 1 || LD == 2 || LD == 8) {
        // quad_perm [1,0,3,2] / [2,3,0,1] and row_ror:8 are exact xor permutations; a DPP move
        // that writes every lane and has no old value folds into the max and the min as their DPP
        // operand
        constexpr int CTRL = LD == 1 ? 0xB1 : LD == 2 ? 0x4E : 0x128;
        const uint32_t p = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a, CTRL, 0xf, 0xf, true);
        hi = max(a, p);
        lo = min(a, p);
    } else if constexpr (LD == 4) {
        // lane - 4 (row_shr:4), then lane + 4 (row_shl:4) written only to the 4-lane banks 0 and
        // 2 of every row, whose bit 2 is clear
        uint32_t p = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a, 0x114, 0xf, 0xf, false);
        p = (uint32_t)__builtin_amdgcn_update_dpp((int)p, (int)a, 0x104, 0xf, 0x5, false);
        hi = max(a, p);
        lo = min(a, p);
    } else {
        // the gfx950 row swaps leave every lane's own value in one output and its partner's in
        // the other
        const auto q = LD == 16 ? __builtin_amdgcn_permlane16_swap(a, a, false, false)
                                : __builtin_amdgcn_permlane32_swap(a, a, false, false);
        hi = max(q[0], q[1]);
        lo = min(q[0], q[1]);
    }
}

__device__ __forceinline__ uint64_t lane_select(uint64_t m, uint64_t a, uint64_t b) {
    return ((uint64_t)lane_select(m, (uint32_t)(a >> 32), (uint32_t)(b >> 32)) << 32) |
           lane_select(m, (uint32_t)a, (uint32_t)b);
}

// One compare-exchange step at lane distance LD of a bitonic network whose runs descend where
// bit DB of the lane is clear; every element of the lane pairs with the same element of lane
// (lane ^ LD).
template <int LD, int DB, int N>
__device__ __forceinline__ void bitonic_lane_step(uint32_t (&a)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        uint32_t hi, lo;
        pair_max_min<LD>(a[i], hi, lo);
        a[i] = lane_select(keep_hi_mask(LD, DB), lo, hi);
    }
}

template <int LD, int DB, int N>
__device__ __forceinline__ void bitonic_lane_step(uint64_t (&a)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const uint64_t p = xor_lanes<LD>(a[i]);
        const uint64_t hi = a[i] > p ? a[i] : p, lo = a[i] > p ? p : a[i];
        a[i] = lane_select(keep_hi_mask(LD, DB), lo, hi);
    }
}

// The lane-distance steps LD, LD / 2, ..., 1 of one merge size.
template <int LD, int DB, int N, typename T>
__device__ __forceinline__ void bitonic_lane_steps(T (&a)[N]) {
    if constexpr (LD >= 1) {
        bitonic_lane_step<LD, DB>(a);
        bitonic_lane_steps<LD / 2, DB>(a);
    }
}

// One merge size of a bitonic network over 128 values held by one wave, two per lane (element
// 2 * lane + i in a_i), ordering each run of SIZE elements descending or ascending by the run's
// parity, as the descending network needs: the runs of lane l descend where bit SIZE / 2 of l is
// clear.
template <int SIZE, typename T>
__device__ __forceinline__ void bitonic128_size(T &a0, T &a1) {
    constexpr int DB = SIZE / 2;
    T a[2] = {a0, a1};
    bitonic_lane_steps<SIZE / 4, DB>(a);
    // partner inside the lane: elements 2 * lane and 2 * lane + 1
    const T lo = a[0] < a[1] ? a[0] : a[1], hi = a[0] < a[1] ? a[1] : a[0];
    if constexpr (DB >= 64) {
        a0 = hi;
        a1 = lo;
    } else {
        a0 = lane_select(desc_mask(DB), lo, hi);
        a1 = lane_select(desc_mask(DB), hi, lo);
    }
}

// Bitonic network sorting 128 values held by one wave (two per lane) in descending order, from
// merge size FIRST: 2 sorts arbitrary input; 128 only runs the final merge, which sorts any
// bitonic sequence. Values must be distinct for a deterministic order.
template <int FIRST = 2, typename T>
__device__ __forceinline__ void wave_bitonic128_desc(T &a0, T &a1) {
    if constexpr (FIRST <= 128) {
        bitonic128_size<FIRST>(a0, a1);
        wave_bitonic128_desc<FIRST * 2>(a0, a1);
    }
}

// Sorts 128 64-bit composites held by one wave (element 2 * lane + i) in descending order.
__device__ __forceinline__ void wave_sort128_desc(uint64_t &a0, uint64_t &a1) {
    wave_bitonic128_desc<2>(a0, a1);
}

// Sorts 64 values held by one wave (one per lane, element = lane) in descending order.
__device__ __forceinline__ void wave_sort64_desc(uint32_t &v) {
    uint32_t a[1] = {v};
    bitonic_lane_steps<1, 2>(a);
    bitonic_lane_steps<2, 4>(a);
    bitonic_lane_steps<4, 8>(a);
    bitonic_lane_steps<8, 16>(a);
    bitonic_lane_steps<16, 32>(a);
    bitonic_lane_steps<32, 64>(a);
    v = a[0];
}

// Sorts 64 64-bit composites held by one wave (one per lane, element = lane) in descending order.
__device__ __forceinline__ void wave_sort64_desc(uint64_t &v) {
    uint64_t a[1] = {v};
    bitonic_lane_steps<1, 2>(a);
    bitonic_lane_steps<2, 4>(a);
    bitonic_lane_steps<4, 8>(a);
    bitonic_lane_steps<8, 16>(a);
    bitonic_lane_steps<16, 32>(a);
    bitonic_lane_steps<32, 64>(a);
    v = a[0];
}

// Sorts a bitonic sequence of 64 composites held by one wave (one per lane) in descending order:
// the final merge of the network.
__device__ __forceinline__ void wave_bitonic64_desc(uint64_t &v) {
    uint64_t a[1] = {v};
    bitonic_lane_steps<32, 64>(a);
    v = a[0];
}

}  // namespace ss
