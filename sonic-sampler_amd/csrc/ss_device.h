// Device helpers shared by every kernel of the library: bf16 rounding, order-preserving keys,
// wave64 / workgroup scans and reductions.
//
// All kernels run with SS_BLOCK = 256 threads (four wave64 wavefronts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SS_BLOCK 256
#define SS_WAVES (SS_BLOCK / 64)
#define SS_K 128

namespace ss {

// ---------------------------------------------------------------------------------------------
// bf16 <-> fp32. Rounding is round-to-nearest-even, which is what torch applies when it stores a
// float32 intermediate into a bfloat16 tensor on the CPU, so every rounding point of the
// reference's PyTorch path can be reproduced exactly.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;  // quiet NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// ---------------------------------------------------------------------------------------------
// Order-preserving unsigned keys. A larger key means a larger value, and -0 and +0 share a key,
// so that equal values compare equal, as they do in torch's sort. 16-bit keys: a non-negative
// bf16 h maps to h | 0x8000, a negative one to its 16-bit two's complement negation (-0 = 0x8000
// lands on 0x8000 itself, the key of +0). Key 0 is never produced and serves as the "absent
// element" sentinel.
__device__ __forceinline__ uint32_t key16(uint32_t h) {
    h &= 0xffffu;
    return (h & 0x8000u) ? ((0x10000u - h) & 0xffffu) : (h | 0x8000u);
}

__device__ __forceinline__ uint32_t unkey16(uint32_t k) {
    k &= 0xffffu;
    return (k & 0x8000u) ? (k & 0x7fffu) : ((0x10000u - k) & 0xffffu);
}

__device__ __forceinline__ uint32_t key32(uint32_t u) {
    if ((u & 0x7fffffffu) == 0) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint32_t unkey32(uint32_t k) {
    return (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
}

// ---------------------------------------------------------------------------------------------
// Wave64 primitives.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

// The value of lane (lane ^ LD) for LD in {1, 2, 4, 8, 16, 32}: DPP lane permutations within a
// 16-lane row (quad_perm for 1 and 2, row shifts for 4, row rotation by 8 for 8) and the gfx950
// row swaps for 16 and 32. Register-to-register, no LDS round trip.
template <int LD>
__device__ __forceinline__ uint32_t xor_lanes(uint32_t v) {
    static_assert(LD == 1 || LD == 2 || LD == 4 || LD == 8 || LD == 16 || LD == 32, "lane distance");
    const int x = (int)v;
    if constexpr (LD == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    } else if constexpr (LD == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    } else if constexpr (LD == 4) {
        const int up = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xf, 0xf, false);    // row_shl:4, lane + 4
        const int down = __builtin_amdgcn_update_dpp(x, x, 0x114, 0xf, 0xf, false);  // row_shr:4, lane - 4
        return (uint32_t)((__lane_id() & 4) ? down : up);
    } else if constexpr (LD == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(x, x, 0x128, 0xf, 0xf, false);  // row_ror:8
    } else if constexpr (LD == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (__lane_id() & 16) ? p[0] : p[1];
    } else {
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (__lane_id() & 32) ? p[0] : p[1];
    }
}

template <int LD>
__device__ __forceinline__ uint64_t xor_lanes(uint64_t v) {
    return ((uint64_t)xor_lanes<LD>((uint32_t)(v >> 32)) << 32) | xor_lanes<LD>((uint32_t)v);
}

__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
    const int lane = lane_id();
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t n = __shfl_up(v, off, 64);
        if (lane >= off) v += n;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        uint64_t o = __shfl_xor(v, off, 64);
        v = v > o ? v : o;
    }
    return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ double wave_inclusive_sum_f64(double v) {
    const int lane = lane_id();
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        double n = __shfl_up(v, off, 64);
        if (lane >= off) v += n;
    }
    return v;
}

// ---------------------------------------------------------------------------------------------
// Workgroup-wide exclusive prefix sum of NV independent 32-bit lanes of data per thread, in
// thread order. `totals` receives the workgroup totals. `tmp` must hold SS_WAVES * NV words.
// ---------------------------------------------------------------------------------------------
template <int NV>
__device__ __forceinline__ void block_exclusive_scan(uint32_t (&v)[NV], uint32_t (&totals)[NV],
                                                     uint32_t *tmp) {
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    uint32_t inc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) inc[i] = wave_inclusive_sum(v[i]);
    if (lane == 63) {
#pragma unroll
        for (int i = 0; i < NV; ++i) tmp[wave * NV + i] = inc[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        uint32_t before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < SS_WAVES; ++w) {
            uint32_t t = tmp[w * NV + i];
            before += (w < wave) ? t : 0u;
            total += t;
        }
        v[i] = before + inc[i] - v[i];
        totals[i] = total;
    }
    __syncthreads();
}

}  // namespace ss
