// Counter-based Gumbel noise: Philox4x32-10 (Salmon et al., "Parallel random numbers: as easy as
// 1, 2, 3", SC'11) keyed by a 64-bit seed, one counter per (token, slot, timestep, offset).
//
// The reference stores w = log(Exp(1)) noise in [B, gamma+1, V] bf16 planes drawn by torch
// (reference core/buffer.py:95-120, `exponential_(1.0).log_()`) and samples argmax(v - w). The
// same transform is applied here to a uniform u in (0, 1) derived from the first output word:
//     u = (2 * (x >> 9) + 1) * 2^-24          (exact in fp32, never 0 or 1)
//     w = bf16(log(bf16(-log(u))))            (Exp(1) rounded to bf16 first, as torch does)
#pragma once

#include "ss_device.h"

namespace ss {

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
        const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
        c = make_uint4(hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0);
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c;
}

__device__ __forceinline__ uint32_t philox_word(uint64_t seed, uint32_t offset, uint32_t slot,
                                                uint32_t step, uint32_t token) {
    const uint4 r = philox4x32_10(make_uint4(token, slot, step, offset), (uint32_t)seed,
                                  (uint32_t)(seed >> 32));
    return r.x;
}

__device__ __forceinline__ float gumbel_from_word(uint32_t x) {
    const float u = (float)(2u * (x >> 9) + 1u) * 5.9604644775390625e-08f;  // * 2^-24
    const float e = rbf(-logf(u));
    return rbf(logf(e));
}

__device__ __forceinline__ float philox_gumbel(uint64_t seed, uint32_t offset, uint32_t slot,
                                               uint32_t step, uint32_t token) {
    return gumbel_from_word(philox_word(seed, offset, slot, step, token));
}

}  // namespace ss
