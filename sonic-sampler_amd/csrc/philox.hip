// Writes the counter-based noise that the fused kernels generate in registers when Philox mode is
// enabled, so that callers can inspect it and tests can hand the identical noise to a CPU checker.
#include "ss_philox.h"
#include "../../include/sonic_sampler.h"

namespace ss {

__global__ __launch_bounds__(SS_BLOCK) void gumbel_materialize_kernel(
    uint64_t seed, uint32_t offset, int slots, int steps, int vocab, uint16_t *out,
    int64_t stride_slot, int64_t stride_step) {
    const int64_t total = (int64_t)slots * steps * vocab;
    for (int64_t i = (int64_t)blockIdx.x * SS_BLOCK + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * SS_BLOCK) {
        const int v = (int)(i % vocab);
        const int64_t st = i / vocab;
        const int t = (int)(st % steps);
        const int s = (int)(st / steps);
        out[s * stride_slot + t * stride_step + v] = (uint16_t)f2bf(philox_gumbel(seed, offset, s, t, v));
    }
}

__global__ __launch_bounds__(SS_BLOCK) void philox_raw_kernel(uint64_t seed, uint32_t offset,
                                                              int slots, int steps, int vocab,
                                                              uint32_t *out) {
    const int64_t total = (int64_t)slots * steps * vocab;
    for (int64_t i = (int64_t)blockIdx.x * SS_BLOCK + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * SS_BLOCK) {
        const int v = (int)(i % vocab);
        const int64_t st = i / vocab;
        const int t = (int)(st % steps);
        const int s = (int)(st / steps);
        out[i] = philox_word(seed, offset, s, t, v);
    }
}

static unsigned grid_for(int64_t total) {
    int64_t g = (total + SS_BLOCK - 1) / SS_BLOCK;
    if (g > 65536) g = 65536;
    return (unsigned)(g > 0 ? g : 1);
}

}  // namespace ss

extern "C" int ss_gumbel_materialize(uint64_t seed, uint32_t offset, int32_t slots,
                                     int32_t timesteps, int32_t vocab, uint16_t *out,
                                     int64_t stride_slot, int64_t stride_step, void *stream) {
    if (!out || slots < 0 || timesteps < 0 || vocab < 0) return SS_ERR_INVALID_ARGUMENT;
    if (stride_step < vocab || (slots > 1 && stride_slot < (int64_t)timesteps * stride_step))
        return SS_ERR_INVALID_ARGUMENT;
    const int64_t total = (int64_t)slots * timesteps * vocab;
    if (total == 0) return SS_OK;
    hipLaunchKernelGGL(ss::gumbel_materialize_kernel, dim3(ss::grid_for(total)), dim3(SS_BLOCK), 0,
                       (hipStream_t)stream, seed, offset, slots, timesteps, vocab, out, stride_slot,
                       stride_step);
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}

extern "C" int ss_philox_raw(uint64_t seed, uint32_t offset, int32_t slots, int32_t timesteps,
                             int32_t vocab, uint32_t *out, void *stream) {
    if (!out || slots < 0 || timesteps < 0 || vocab < 0) return SS_ERR_INVALID_ARGUMENT;
    const int64_t total = (int64_t)slots * timesteps * vocab;
    if (total == 0) return SS_OK;
    hipLaunchKernelGGL(ss::philox_raw_kernel, dim3(ss::grid_for(total)), dim3(SS_BLOCK), 0,
                       (hipStream_t)stream, seed, offset, slots, timesteps, vocab, out);
    return hipGetLastError() == hipSuccess ? SS_OK : SS_ERR_LAUNCH;
}
