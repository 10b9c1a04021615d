/*
 * sonic_sampler.h -- C-ABI of the MI355X (gfx950) fused sampling / verification library.
 *
 * Every entry point takes a pointer to a plain argument struct (raw device pointers, element
 * strides, sizes, flags and a hipStream_t passed as void*), enqueues its kernel launches (two or
 * three, back to back) on that stream and returns an ss_status code. No entry point allocates
 * device memory, synchronises the host or throws, so all of them may be recorded into a hipGraph.
 *
 * Conventions shared by all structs:
 *   - strides are in ELEMENTS of the pointed-to type, never bytes;
 *   - the vocabulary axis is unit-stride (contiguous);
 *   - a NULL pointer means "stage / buffer absent" exactly like a `None` tensor in the reference's
 *     functional API (src/sonic_sampler/interface/functional/singular.py:75-121).
 *
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   ss_topk             <- UnshardedBoundedTopK.__call__, src/sonic_sampler/interface/topk.py:98-161
 *                          (launches K2 ops/topk/bitpack.py:99-158 + K3 ops/topk/unpack.py:312-377)
 *   ss_fused_singular   <- fused_singular, src/sonic_sampler/interface/functional/singular.py:75-322
 *                          (launches K1 ops/prologue.py:272-472 + K4 ops/singular.py:154-358)
 *   ss_fused_multistep  <- fused_multistep, src/sonic_sampler/interface/functional/multistep.py:175-461
 *                          (launches K1 + K5 ops/multistep.py:76-226 + K6 ops/verify.py:244-434)
 *   ss_indexed_copy     <- indexed_copy, src/sonic_sampler/ops/copy.py:21-127 (noise staging)
 *   ss_gumbel_materialize / ss_philox_raw  <- no kernel counterpart: the reference draws its noise
 *                          with torch (`exponential_().log_()`, src/sonic_sampler/core/buffer.py:118);
 *                          these write the counter-based Philox noise the fused kernels can generate
 *                          in-register, so callers and tests can see the exact noise used.
 */
#ifndef SONIC_SAMPLER_H
#define SONIC_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SS_ABI_VERSION 3

/* Upper bound on top-k and the width of every candidate block (reference ops/base.py:24). */
#define SS_MAX_K 128

typedef enum ss_status {
    SS_OK = 0,
    SS_ERR_INVALID_ARGUMENT = 1, /* a size, stride, pointer or alignment the kernels cannot honour */
    SS_ERR_UNSUPPORTED = 2,      /* a configuration outside what was compiled (e.g. block_n)      */
    SS_ERR_LAUNCH = 3,           /* the HIP runtime rejected the launch (hipGetLastError)         */
    SS_ERR_SCRATCH_LIMIT = 4     /* ss_fused_singular_noalloc: the call needs more candidate      */
                                 /* storage than SS_STATIC_SCRATCH_BYTES                         */
} ss_status;

typedef enum ss_dtype {
    SS_DTYPE_BF16 = 0,
    SS_DTYPE_F32 = 1
} ss_dtype;

/* Indicator bits (reference core/flags.py:58-95). */
#define SS_GRAMMAR 0x001
#define SS_MULTIPLICATIVE 0x002
#define SS_FREQUENCY 0x004
#define SS_PRESENCE 0x008
#define SS_BIAS 0x010
#define SS_TEMPERATURE 0x020
#define SS_GREEDY 0x040
#define SS_TOP_K 0x080
#define SS_TOP_P 0x100
#define SS_MIN_P 0x200
#define SS_TOP_K_LOGPROBS 0x400
#define SS_STOCHASTIC_VERIFY_GREEDY_DRAFT 0x800

/* Counter-based noise source. When `enabled` is non-zero the kernels ignore the Gumbel noise
 * pointer and derive log(Exp(1)) noise for (slot, timestep, token) from Philox4x32-10 keyed by
 * `seed`, at counter (token, slot, timestep, offset); see ss_gumbel_materialize. */
typedef struct ss_philox {
    uint64_t seed;
    uint32_t offset;
    int32_t enabled;
} ss_philox;

/* Kernel layout of ss_fused_singular and ss_topk. TILES: a tile grid (rows x tiles) writes every tile's
 * top-128 to the scratchpad, then one workgroup per row merges and selects (two launches).
 * ROWWISE: one workgroup per row streams the row tile by tile and selects in the same launch
 * (rows of at most 16 tiles; the scratchpad is not touched). AUTO: ss_fused_singular always takes
 * TILES; ss_topk takes ROWWISE for at least 48 rows of 16385-32768 columns at k <= 32 and TILES
 * otherwise. */
typedef enum ss_strategy {
    SS_STRATEGY_AUTO = 0,
    SS_STRATEGY_TILES = 1,
    SS_STRATEGY_ROWWISE = 2
} ss_strategy;

/* ---------------------------------------------------------------------------------------------
 * Bounded top-k over [rows, vocab] logits, ties broken to the lowest index.
 * Replaces UnshardedBoundedTopK.__call__ (reference interface/topk.py:98-161).
 * values/indices are written densely as [rows, k] (row stride k); values in the logits dtype.
 * scratch holds rows x (tiles * k) candidates: uint32 for bf16 logits, uint64 for fp32 logits.
 * ------------------------------------------------------------------------------------------- */
typedef struct ss_topk_args {
    const void *logits;
    int64_t stride_logits;
    int32_t dtype;       /* ss_dtype */
    int32_t rows;
    int32_t vocab_size;
    int32_t k;           /* power of two, 1 <= k <= 128 */
    int32_t block_n;     /* tile width: 1024, 2048, 4096, 8192 or 16384 */
    int32_t strategy;    /* ss_strategy: 0 automatic (tile grid; one workgroup per row for >= 48 rows
                            of 16385-32768 columns at k <= 32), 2 one workgroup per row (V <= 32768) */
    void *scratch;       /* rows * stride_scratch elements (uint32 or uint64) */
    int64_t stride_scratch;
    void *values;        /* [rows, k] bf16 or fp32 */
    int32_t *indices;    /* [rows, k] */
    void *stream;        /* hipStream_t */
} ss_topk_args;

int ss_topk(const ss_topk_args *args);

/* ---------------------------------------------------------------------------------------------
 * Fused single-step sampling: logit processors -> bounded top-128 -> truncation -> Gumbel-max,
 * with optional logprobs, top-Z logprobs, draft-probability scatter and decode-count update.
 * Replaces fused_singular (reference interface/functional/singular.py:75-322).
 * Row r reads its request state at slot = slot_mapping ? slot_mapping[r] : r.
 * Caller contract, not checked on the device (as in the reference): slot_mapping values lie in
 * [0, slots) of every slot-indexed buffer, d2t values in [0, target_vocab), and `probabilities`
 * has a row for every slot a row may map to (the Python driver checks the last against the
 * buffer's storage before the call).
 * ------------------------------------------------------------------------------------------- */
typedef struct ss_singular_args {
    /* logits [rows, vocab] bf16 */
    const uint16_t *logits;
    int64_t stride_logits;
    int32_t rows;
    int32_t vocab_size;          /* draft vocabulary when d2t is given */
    int32_t target_vocab;        /* width of counts/bias/noise/probabilities rows */
    int32_t block_n;
    int32_t lookahead;           /* gamma: columns of drafted_tokens that may be read */
    int32_t timestep;            /* t: drafted_tokens[:, :t] feed the penalty history */
    int32_t max_top_logprobs;    /* Z */
    int32_t is_prefill;
    int32_t update_counts;
    int32_t return_logprobs;
    int32_t return_probabilities;
    int32_t strategy;            /* ss_strategy: kernel layout (0 = chosen by the library) */
    const uint16_t *indicators;  /* [slots] */
    const int32_t *slot_mapping; /* [rows] or NULL */
    const int32_t *d2t;          /* [vocab_size] or NULL */
    const uint32_t *grammar;     /* row slot at grammar + slot * stride_grammar, or NULL */
    int64_t stride_grammar;
    const int32_t *context_counts; int64_t stride_context;
    int32_t *decode_counts; int64_t stride_decode;
    const int32_t *drafted_tokens; int64_t stride_drafted; /* [rows, >= timestep] or NULL */
    const uint16_t *repetition;  /* [slots] bf16 */
    const uint16_t *frequency;
    const uint16_t *presence;
    const uint16_t *logit_bias; int64_t stride_bias;
    const uint16_t *temperature;
    const int32_t *top_k;
    const uint16_t *top_p;
    const uint16_t *min_p;
    const int32_t *top_logprobs;
    const uint16_t *gumbel; int64_t stride_gumbel;  /* [slots, target_vocab] bf16 */
    ss_philox philox;            /* used instead of gumbel when enabled */
    int32_t philox_step;         /* timestep index used in the Philox counter */
    int32_t stages;              /* SS_STAGE_* bits to launch; 0 = both */
    /* outputs */
    int32_t *tokens; int64_t stride_tokens;
    uint16_t *logprobs; int64_t stride_logprobs;           /* [rows, 1] bf16 or NULL */
    uint16_t *top_values; int32_t *top_tokens; int64_t stride_top; /* [rows, Z] or NULL */
    uint16_t *probabilities; int64_t stride_probabilities; /* [slots, target_vocab] bf16 or NULL */
    /* in-flight */
    uint32_t *scratch; int64_t stride_scratch;             /* [rows, tiles * 128] */
    void *stream;
    /* timing: hipEvent_t pair recorded by the tile kernel's own dispatch (start, end), or NULL */
    void *tile_start;
    void *tile_end;
    /* Sharded vocabulary (reference interface/functional/singular.py:80-83,129-133): `logits` holds
     * columns [local_rank * shard_size, + vocab_size) of a vocabulary split over world_size shards.
     * The tile stage writes this shard's candidate lists to slice local_rank of every scratch row
     * ([world_size, tiles, 128], tiles = ceil(vocab_size / block_n), the same on every shard); the
     * row stage merges all world_size slices, so an engine runs SS_STAGE_TILES, exchanges the
     * slices (all-gather) and then runs SS_STAGE_ROWS. world_size = 1 (or 0): unsharded. */
    int32_t world_size;
    int32_t local_rank;
    int32_t shard_size;
    int32_t reserved;
} ss_singular_args;

/* ss_singular_args.stages */
#define SS_STAGE_TILES 1
#define SS_STAGE_ROWS 2

int ss_fused_singular(const ss_singular_args *args);

/* ---------------------------------------------------------------------------------------------
 * ss_fused_singular without a caller-provided scratchpad. No counterpart in the reference: it is
 * for callers that cannot allocate device memory at all (code under hipGraph capture, serving
 * loops or harnesses that forbid hipMalloc), which then need not size or own the in-flight
 * candidate lists either. `scratch` / `stride_scratch` of `args` are ignored; the tiles' candidate
 * lists (rows * ceil(vocab_size / block_n) * 128 * 4 bytes) go to a static device array of
 * SS_STATIC_SCRATCH_BYTES that every device the library runs on holds until the process ends.
 * A larger call fails with SS_ERR_SCRATCH_LIMIT. The call allocates nothing; the first call on a
 * device (the device of args->stream) only looks up that device's copy of the array. That lookup
 * is not a stream operation, so the first call on a device must be made outside graph capture: a
 * first call while args->stream is capturing fails with SS_ERR_UNSUPPORTED, and every later call
 * on that device may be captured. All calls on one device share the array:
 * calls that overlap on one device (two streams, or two threads) race, so they must be ordered.
 * With the stages split (SS_STAGE_TILES per shard, then SS_STAGE_ROWS), the row-stage call reads
 * the lists the tile-stage calls left in the array: no other call on the device may come between
 * them, and the row count, world_size and tile count must match (the array's row stride is
 * world_size * tiles * 128 words); the array then holds rows * world_size * tiles lists.
 * Every other argument, output and error is that of ss_fused_singular.
 * ------------------------------------------------------------------------------------------- */
#define SS_STATIC_SCRATCH_BYTES (8u << 20)

int ss_fused_singular_noalloc(const ss_singular_args *args);

/* ---------------------------------------------------------------------------------------------
 * Fused chain speculative verification over rows = B*(gamma+1) (fixed) or cu_seqlens[B] (varlen)
 * logit rows: logit processors -> bounded top-128 -> truncation -> softmax -> greedy or
 * stochastic acceptance with residual resampling.
 * Replaces fused_multistep (reference interface/functional/multistep.py:175-461).
 * Caller contract, not checked on the device: slot_mapping values lie in [0, slots), and
 * draft_probabilities has a [gamma, vocab] block for every slot a request may map to (the Python
 * driver checks the last before the call). A drafted token outside [0, vocab_size) reads no
 * memory out of bounds, but its acceptance is not defined (the reference indexes with it).
 * ------------------------------------------------------------------------------------------- */
typedef struct ss_multistep_args {
    const uint16_t *logits;      /* [rows, vocab] bf16 */
    int64_t stride_logits;
    int32_t rows;
    int32_t batch;               /* requests B */
    int32_t vocab_size;
    int32_t block_n;
    int32_t lookahead;           /* gamma (maximum gamma when varlen) */
    int32_t max_top_logprobs;    /* Z */
    int32_t update_counts;
    int32_t return_logprobs;
    const int32_t *cu_seqlens;   /* [B + 1] or NULL (fixed gamma) */
    const uint16_t *indicators;
    const int32_t *slot_mapping;
    const int32_t *drafted_tokens; /* flat [rows]: request b owns [margin_b, margin_b + n_b) */
    const uint32_t *grammar; int64_t grammar_stride_slot; int64_t grammar_stride_step;
    const int32_t *context_counts; int64_t stride_context;
    int32_t *decode_counts; int64_t stride_decode;
    const uint16_t *repetition;
    const uint16_t *frequency;
    const uint16_t *presence;
    const uint16_t *logit_bias; int64_t stride_bias;
    const uint16_t *temperature;
    const int32_t *top_k;
    const uint16_t *top_p;
    const uint16_t *min_p;
    const int32_t *top_logprobs;
    const uint16_t *draft_probabilities; int64_t probs_stride_slot; int64_t probs_stride_step;
    const uint16_t *uniform; int64_t stride_uniform;
    const uint16_t *gumbel; int64_t gumbel_stride_slot; int64_t gumbel_stride_step;
    ss_philox philox;
    /* outputs */
    int32_t *out_tokens;         /* flat [rows]: every row's draft, each request's emitted token at
                                    its offset; written whole by the call (no pre-fill needed), and
                                    it may be drafted_tokens itself */
    int32_t *offsets;            /* [B] */
    uint16_t *logprobs;          /* flat [rows] bf16 or NULL */
    uint16_t *top_values; int32_t *top_tokens; int64_t stride_top; /* [rows, Z] or NULL */
    /* in-flight */
    float *values;               /* [rows, 128] fp32 truncated log-probabilities */
    int32_t *indices;            /* [rows, 128] */
    uint32_t *scratch; int64_t stride_scratch;
    void *stream;
    /* timing: hipEvent_t pair recorded by the tile kernel's own dispatch (start, end), or NULL */
    void *tile_start;
    void *tile_end;
    /* 1: the caller knows that every row's indicator has SS_GREEDY (for example from its host
       copy of the indicators): the request stage takes each row's argmax from the tiles' maxima
       itself and the row launch is skipped, one launch fewer. A request whose indicator lacks
       SS_GREEDY is then not served: its offsets entry is set to -1 (outside 0..gamma) and no
       other output of it is written. 0: any mix of rows. */
    int32_t all_greedy;
} ss_multistep_args;

int ss_fused_multistep(const ss_multistep_args *args);

/* ---------------------------------------------------------------------------------------------
 * Indexed copy of noise rows: for i < count, slot = indices[i]; when indicators is NULL or
 * (indicators[slot] & SS_GREEDY) == 0, copy source[slot * stride_source + c] into
 * target[slot * stride_target + c] for c < cols (bf16 elements; a slot outside [0, slots) is
 * skipped). Replaces indexed_copy (reference ops/copy.py:21-127), which stages the drafter's
 * Gumbel noise into the verifier's (GumbelNoise.stage_weights, core/buffer.py:151-159).
 * ------------------------------------------------------------------------------------------- */
typedef struct ss_indexed_copy_args {
    const uint16_t *source; int64_t stride_source;  /* [slots, >= cols] */
    uint16_t *target; int64_t stride_target;        /* [slots, >= cols] */
    const int64_t *indices;                          /* [count] slots to copy */
    const uint16_t *indicators;                      /* [slots] or NULL */
    int64_t cols;
    int32_t count;
    int32_t slots;
    void *stream;
} ss_indexed_copy_args;

int ss_indexed_copy(const ss_indexed_copy_args *args);

/* ---------------------------------------------------------------------------------------------
 * Philox noise, written out so that the in-register noise of the fused kernels is observable.
 * out[s * stride_slot + t * stride_step + v] = bf16(log(bf16(-log(u)))),  u in (0, 1),
 * for s < slots, t < timesteps, v < vocab, u drawn at counter (v, s, t, offset).
 * ------------------------------------------------------------------------------------------- */
int ss_gumbel_materialize(uint64_t seed, uint32_t offset, int32_t slots, int32_t timesteps,
                          int32_t vocab, uint16_t *out, int64_t stride_slot,
                          int64_t stride_step, void *stream);

/* The raw first Philox4x32-10 output word for the same counters (for known-answer checks). */
int ss_philox_raw(uint64_t seed, uint32_t offset, int32_t slots, int32_t timesteps,
                  int32_t vocab, uint32_t *out, void *stream);

/* Introspection. */
int ss_abi_version(void);
const char *ss_status_string(int status);
/* sizeof of each argument struct, by index 0=topk, 1=singular, 2=multistep, 3=indexed copy
 * (ABI self-check). */
int64_t ss_args_size(int which);

#ifdef __cplusplus
}
#endif

#endif /* SONIC_SAMPLER_H */
