// Indexed copy of noise rows (replaces the reference's indexed_copy, ops/copy.py:21-127, used by
// GumbelNoise.stage_weights, core/buffer.py:151-159): for every listed slot whose indicator is
// stochastic (bit 0x40 clear), copy the slot's source row into its target row. Grid (count, blocks):
// each workgroup copies 16 KB of one row with 16-byte non-temporal loads and stores, or element by
// element when the rows are not 16-byte aligned.
#include "ss_device.h"
#include "../../include/sonic_sampler.h"

namespace ss {

// Elements one workgroup copies: four 16-byte (8-element) accesses per thread, 16 KB of uint16.
constexpr int COPY_CHUNK = SS_BLOCK * 4 * 8;

typedef int32_t i32x4c __attribute__((ext_vector_type(4)));

template <bool VEC>
__global__ __launch_bounds__(SS_BLOCK) void indexed_copy_kernel(ss_indexed_copy_args a) {
    const int64_t slot = a.indices[blockIdx.x];
    if (slot < 0 || slot >= a.slots) return;
    if (a.indicators && (a.indicators[slot] & 0x40u)) return;  // greedy: nothing to stage
    const uint16_t *src = a.source + slot * a.stride_source;
    uint16_t *dst = a.target + slot * a.stride_target;
    const int64_t begin = (int64_t)blockIdx.y * COPY_CHUNK;
    const int64_t end = min(begin + (int64_t)COPY_CHUNK, a.cols);
    if (VEC) {
        // 8 elements (16 bytes) per access; cols is a multiple of 8
        i32x4c q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t e = begin + 8 * ((int64_t)threadIdx.x + i * SS_BLOCK);
            q[i] = e < end ? __builtin_nontemporal_load((const i32x4c *)(src + e)) : (i32x4c){0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t e = begin + 8 * ((int64_t)threadIdx.x + i * SS_BLOCK);
            if (e < end) __builtin_nontemporal_store(q[i], (i32x4c *)(dst + e));
        }
    } else {
        for (int64_t e = begin + threadIdx.x; e < end; e += SS_BLOCK) dst[e] = src[e];
    }
}

}  // namespace ss

extern "C" int ss_indexed_copy(const ss_indexed_copy_args *a) {
    using namespace ss;
    if (!a || !a->source || !a->target || !a->indices) return SS_ERR_INVALID_ARGUMENT;
    if (a->count < 0 || a->slots < 0 || a->cols < 0) return SS_ERR_INVALID_ARGUMENT;
    if (a->stride_source < a->cols || a->stride_target < a->cols) return SS_ERR_INVALID_ARGUMENT;
    if (a->count == 0 || a->cols == 0) return SS_OK;
    const int64_t blocks = (a->cols + COPY_CHUNK - 1) / COPY_CHUNK;
    if (a->count > 0x7fffffff || blocks > 65535) return SS_ERR_UNSUPPORTED;
    const bool vec = ((uintptr_t)a->source % 16) == 0 && ((uintptr_t)a->target % 16) == 0 &&
                     a->stride_source % 8 == 0 && a->stride_target % 8 == 0 && a->cols % 8 == 0;
    dim3 grid((unsigned)a->count, (unsigned)blocks), block(SS_BLOCK);
    hipStream_t s = (hipStream_t)a->stream;
    if (vec) hipLaunchKernelGGL(indexed_copy_kernel<true>, grid, block, 0, s, *a);
    else hipLaunchKernelGGL(indexed_copy_kernel<false>, grid, block, 0, s, *a);
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}
