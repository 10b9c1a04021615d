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

// DPP move with a compile-time control word; lanes whose source is outside the pattern (or whose
// row is masked off) read 0.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = dpp_u32<CTRL, ROW_MASK>((uint32_t)u);
    const uint64_t hi = dpp_u32<CTRL, ROW_MASK>((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, (hi << 32) | lo);
}

// DPP controls: row_shr:n shifts within each 16-lane row; row_bcast:15 / row_bcast:31 carry lane
// 15 of each row into the next row, and lane 31 into rows 2 and 3; wave_shr:1 shifts by one lane
// across the whole wave.
constexpr int DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114,
              DPP_ROW_SHR8 = 0x118, DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143,
              DPP_WAVE_SHR1 = 0x138;

// Inclusive prefix sum over the wave's lanes: four in-row shift-and-add steps, then the row
// carries. Register-to-register, no LDS.
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
    v += dpp_u32<DPP_ROW_SHR1>(v);
    v += dpp_u32<DPP_ROW_SHR2>(v);
    v += dpp_u32<DPP_ROW_SHR4>(v);
    v += dpp_u32<DPP_ROW_SHR8>(v);
    v += dpp_u32<DPP_ROW_BCAST15, 0xa>(v);
    v += dpp_u32<DPP_ROW_BCAST31, 0xc>(v);
    return v;
}

__device__ __forceinline__ double wave_inclusive_sum_f64(double v) {
    v += dpp_f64<DPP_ROW_SHR1>(v);
    v += dpp_f64<DPP_ROW_SHR2>(v);
    v += dpp_f64<DPP_ROW_SHR4>(v);
    v += dpp_f64<DPP_ROW_SHR8>(v);
    v += dpp_f64<DPP_ROW_BCAST15, 0xa>(v);
    v += dpp_f64<DPP_ROW_BCAST31, 0xc>(v);
    return v;
}

// The value of lane - 1 (0 in lane 0).
__device__ __forceinline__ double shift_up1_f64(double v) { return dpp_f64<DPP_WAVE_SHR1>(v); }

// Reductions by xor butterfly (distances 32, 16, ..., 1); every lane ends with the result.
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
    v += xor_lanes<32>(v);
    v += xor_lanes<16>(v);
    v += xor_lanes<8>(v);
    v += xor_lanes<4>(v);
    v += xor_lanes<2>(v);
    v += xor_lanes<1>(v);
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, xor_lanes<32>(v));
    v = max(v, xor_lanes<16>(v));
    v = max(v, xor_lanes<8>(v));
    v = max(v, xor_lanes<4>(v));
    v = max(v, xor_lanes<2>(v));
    v = max(v, xor_lanes<1>(v));
    return v;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max_u64(v, xor_lanes<32>(v));
    v = max_u64(v, xor_lanes<16>(v));
    v = max_u64(v, xor_lanes<8>(v));
    v = max_u64(v, xor_lanes<4>(v));
    v = max_u64(v, xor_lanes<2>(v));
    v = max_u64(v, xor_lanes<1>(v));
    return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, __uint_as_float(xor_lanes<32>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xor_lanes<16>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xor_lanes<8>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xor_lanes<4>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xor_lanes<2>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(xor_lanes<1>(__float_as_uint(v))));
    return v;
}

// Sum by the butterfly of a __shfl_xor loop over distances 32, 16, ..., 1, so every lane adds
// in the same order as that loop would.
__device__ __forceinline__ float wave_sum_f32(float v) {
    v += __uint_as_float(xor_lanes<32>(__float_as_uint(v)));
    v += __uint_as_float(xor_lanes<16>(__float_as_uint(v)));
    v += __uint_as_float(xor_lanes<8>(__float_as_uint(v)));
    v += __uint_as_float(xor_lanes<4>(__float_as_uint(v)));
    v += __uint_as_float(xor_lanes<2>(__float_as_uint(v)));
    v += __uint_as_float(xor_lanes<1>(__float_as_uint(v)));
    return v;
}

// b in the lanes whose bit of the wave-uniform mask m is set, a in the others: one v_cndmask with
// the mask as its lane-select operand.
__device__ __forceinline__ uint32_t lane_select(uint64_t m, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(m));
    return r;
}

// Reads one dword of every 64-byte line of the kernel's first BYTES argument bytes, all issued
// before one wait: the argument reads spread over the kernel then find their lines in the scalar
// cache instead of each waiting for a memory round trip of its own. Worth it in the row stages,
// which read arguments from most lines at different points of one dependent chain; a kernel
// whose first reads need only a few lines (the verify stage) loses more by waiting for all of
// them first than it saves later.
template <int BYTES>
__device__ __forceinline__ void touch_kernargs() {
    typedef const __attribute__((address_space(4))) uint32_t kword;
    kword *p = (kword *)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t acc = 0;
#pragma unroll
    for (int o = 0; o < BYTES / 4; o += 16) acc ^= p[o];
    asm volatile("" ::"s"(acc));
}

// Value of lane `src` (uniform) in every lane, through the scalar unit.
__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int src) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, __builtin_amdgcn_readfirstlane(src));
}

__device__ __forceinline__ float lane_f32(float v, int src) {
    return __uint_as_float(lane_u32(__float_as_uint(v), src));
}

__device__ __forceinline__ int lane_i32(int v, int src) { return (int)lane_u32((uint32_t)v, src); }

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
