// Version, status strings and struct sizes of the C-ABI (no device code).
#include "../../include/sonic_sampler.h"

extern "C" int ss_abi_version(void) { return SS_ABI_VERSION; }

extern "C" const char *ss_status_string(int status) {
    switch (status) {
        case SS_OK: return "ok";
        case SS_ERR_INVALID_ARGUMENT: return "invalid argument";
        case SS_ERR_UNSUPPORTED: return "unsupported configuration";
        case SS_ERR_LAUNCH: return "kernel launch failed";
        case SS_ERR_SCRATCH_LIMIT:
            return "the call needs more candidate storage than the static scratch holds "
                   "(rows * tiles * 128 * 4 > SS_STATIC_SCRATCH_BYTES)";
        default: return "unknown status";
    }
}

extern "C" int64_t ss_args_size(int which) {
    switch (which) {
        case 0: return (int64_t)sizeof(ss_topk_args);
        case 1: return (int64_t)sizeof(ss_singular_args);
        case 2: return (int64_t)sizeof(ss_multistep_args);
        case 3: return (int64_t)sizeof(ss_indexed_copy_args);
        default: return -1;
    }
}
