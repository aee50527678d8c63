/*
 * pvlc_hip — MI355X (gfx950) backend for the PaddleOCR-VL decoder KV-cache hot
 * path: KV append with rotary, GQA decode attention and causal prefill.
 *
 * C ABI.  Plain pointers and sizes; no C++ or framework types.  Every entry
 * point below names the reference interface it replaces
 * (glebkudr/paddleocr-vl-webgpu; paths relative to the repository root).
 *
 * Pinned topology (runtime-core lib.rs:1123-1131): 16 query heads, 2 key/value
 * heads (contiguous groups of 8 query heads), head_dim 128.
 *
 * Status codes: 0 is success.  A failure packs the reference's
 * RuntimeErrorCode (crates/pvlc-runtime-native/src/lib.rs:273-283) in bits
 * 8..15 and, for plan failures, the InvocationErrorCode
 * (crates/pvlc-runtime-core/src/lib.rs:5335-5351) in bits 0..7.  The message of
 * the last failure on the calling thread is pvlc_hip_last_error_message().
 *
 * Two families of entry points:
 *  - the reference surface (host f32 buffers, copied in and out, plan
 *    validation before any GPU effect, persistent sessions that poison on a
 *    failure after submission);
 *  - the device-resident hot path (fp16 device buffers, caller stream, blocked
 *    paged KV layout below), used for batched decode, the 18-layer decode step
 *    and prefill.  These never synchronise and never allocate.
 */
#ifndef PVLC_HIP_H
#define PVLC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t pvlc_hip_status;

/* RuntimeErrorCode, native lib.rs:273-283 (bits 8..15 of a status). */
enum {
    PVLC_HIP_OK = 0,
    PVLC_HIP_ADAPTER_UNAVAILABLE = 1,
    PVLC_HIP_DEVICE_REQUEST = 2,
    PVLC_HIP_INVALID_INVOCATION = 3,
    PVLC_HIP_VALIDATION = 4,
    PVLC_HIP_OUT_OF_MEMORY = 5,
    PVLC_HIP_INTERNAL = 6,
    PVLC_HIP_OPERATION = 7,
    PVLC_HIP_MAPPING = 8,
    PVLC_HIP_CAPTURE = 9
};

/* InvocationErrorCode, runtime-core lib.rs:5335-5351 (bits 0..7 of a status). */
enum {
    PVLC_HIP_INV_NONE = 0,
    PVLC_HIP_INV_ZERO_DIMENSION = 1,
    PVLC_HIP_INV_LENGTH_MISMATCH = 2,
    PVLC_HIP_INV_ARITHMETIC_OVERFLOW = 3,
    PVLC_HIP_INV_INVALID_EPSILON = 4,
    PVLC_HIP_INV_INVALID_ROTARY_DIMENSION = 5,
    PVLC_HIP_INV_INVALID_ROPE_BASE = 6,
    PVLC_HIP_INV_UNSUPPORTED_HEAD_DIMENSION = 7,
    PVLC_HIP_INV_INVALID_DECODER_GEOMETRY = 8,
    PVLC_HIP_INV_INVALID_VISION_GEOMETRY = 9,
    PVLC_HIP_INV_INVALID_PROJECTOR_GEOMETRY = 10,
    PVLC_HIP_INV_INVALID_SEQUENCE_BOUNDARIES = 11,
    PVLC_HIP_INV_INVALID_CHECKPOINT_SELECTION = 12,
    PVLC_HIP_INV_INVALID_ACTIVATION_LAYOUT = 13,
    PVLC_HIP_INV_INVALID_FUSION_TARGET = 14,
    PVLC_HIP_INV_NON_FINITE_INPUT = 15
};

#define PVLC_HIP_QUERY_HEADS 16u
#define PVLC_HIP_KV_HEADS 2u
#define PVLC_HIP_HEAD_DIM 128u
/* Tokens per KV block of the device layout. */
#define PVLC_HIP_BLOCK_TOKENS 16u
/* runtime-core PINNED_DECODER_GQA_SPLIT_CHUNK_SIZE / _PARTIAL_STRIDE_F32, lib.rs:2884-2887 */
#define PVLC_HIP_REFERENCE_SPLIT_CHUNK 32u
#define PVLC_HIP_REFERENCE_PARTIAL_STRIDE_F32 192u

/* Message of the last failure on this thread ("" after a success). */
const char *pvlc_hip_last_error_message(void);

/* ---------------------------------------------------------------------------
 * Plans (host only, no GPU): the runtime-core plan authority.
 * ------------------------------------------------------------------------- */

/* DecoderKvSessionDescriptor, runtime-core lib.rs:833-843.  The caches are the
 * compact physical planes [cache_capacity, 2, 128]; only the first
 * prefix_tokens rows are semantic (rows after them may hold poison). */
typedef struct pvlc_hip_kv_session_descriptor {
    uint32_t query_heads;
    uint32_t key_value_heads;
    uint32_t head_dim;
    uint32_t prefix_tokens;
    uint32_t cache_capacity;
    const float *key_cache;
    size_t key_cache_len;
    const float *value_cache;
    size_t value_cache_len;
} pvlc_hip_kv_session_descriptor;

/* DecoderKvSessionPlan, runtime-core lib.rs:853-870. */
typedef struct pvlc_hip_kv_session_plan {
    uint32_t initial_cache_tokens;
    uint32_t cache_capacity;
    uint32_t query_heads;
    uint32_t key_value_heads;
    uint32_t head_dim;
    uint64_t query_elements;
    uint64_t key_value_width;
    uint64_t cache_elements;
    uint64_t cache_bytes;
    uint64_t attention_bytes;
    uint64_t split_partials_bytes;
} pvlc_hip_kv_session_plan;

/* DecoderKvSessionStep, runtime-core lib.rs:845-851. */
typedef struct pvlc_hip_kv_step_operands {
    const float *query;
    size_t query_len;
    const float *appended_key;
    size_t appended_key_len;
    const float *appended_value;
    size_t appended_value_len;
} pvlc_hip_kv_step_operands;

/* DecoderGqaSplitPlan, runtime-core lib.rs:2871-2881 (the reference split-K
 * geometry; this backend's kernels use their own partition size, but the plan
 * is kept so callers see the same admission rules). */
typedef struct pvlc_hip_gqa_split_plan {
    uint32_t chunk_size;
    uint32_t chunk_count;
    uint64_t partials_elements;
    uint64_t partials_bytes;
    uint32_t partial_stride_f32;
    uint32_t partial_workgroups;
    uint32_t merge_workgroups;
    uint32_t uniform_words[4];
} pvlc_hip_gqa_split_plan;

/* DecoderKvSessionStepPlan, runtime-core lib.rs:872-881. */
typedef struct pvlc_hip_kv_step_plan {
    uint32_t cache_tokens_before;
    uint32_t cache_tokens_after;
    uint64_t valid_cache_elements;
    uint32_t append_uniform_words[4];
    uint32_t attention_uniform_words[4];
    pvlc_hip_gqa_split_plan split_gqa;
} pvlc_hip_kv_step_plan;

/* DecoderKvSessionDescriptor::plan, runtime-core lib.rs:952-968. */
pvlc_hip_status pvlc_hip_kv_session_plan_create(const pvlc_hip_kv_session_descriptor *descriptor,
                                                pvlc_hip_kv_session_plan *plan_out);

/* DecoderKvSessionPlan::plan_cache_transition / plan_step, runtime-core
 * lib.rs:976-1054.  step may be NULL (transition only). */
pvlc_hip_status pvlc_hip_kv_session_plan_step(const pvlc_hip_kv_session_plan *plan, uint32_t cache_tokens,
                                              const pvlc_hip_kv_step_operands *step,
                                              pvlc_hip_kv_step_plan *step_plan_out);

/* DecoderGqaSplitDescriptor::plan, runtime-core lib.rs:2889-2978. */
pvlc_hip_status pvlc_hip_gqa_split_plan_create(uint32_t cache_tokens, uint32_t query_heads,
                                               uint32_t key_value_heads, uint32_t head_dim,
                                               pvlc_hip_gqa_split_plan *plan_out);

/* require_decoder_prefill_tokens, runtime-core lib.rs:2491-2498 (the token
 * bound of DecoderStackGeometryDescriptor::plan_prefill, :2293-2297). */
pvlc_hip_status pvlc_hip_prefill_plan_check(uint32_t tokens, uint32_t cache_capacity);

/* ---------------------------------------------------------------------------
 * Runtime and persistent KV sessions (pvlc-runtime-native surface).
 * ------------------------------------------------------------------------- */

typedef struct pvlc_hip_runtime pvlc_hip_runtime;
typedef struct pvlc_hip_kv_session pvlc_hip_kv_session;

/* NativeOptions, native lib.rs:268-271 (the observer is replaced by counters).
 * Every wait for submitted GPU work (session creation, step, finish, and the
 * one-shot call) is bounded by gpu_wait_timeout_ns (0: 30 s, GPU_WAIT_TIMEOUT
 * of native lib.rs:56).  A wait that expires fails with PVLC_HIP_OPERATION,
 * and a session step that fails so leaves the session terminally poisoned
 * (decoder_kv_session.rs:729-735, :513-528).  A session whose GPU work never
 * completes keeps its device buffers allocated when it is destroyed, rather
 * than freeing memory a kernel may still access. */
typedef struct pvlc_hip_runtime_options {
    int32_t device;               /* HIP device ordinal */
    uint64_t gpu_wait_timeout_ns; /* 0 = 30 s */
} pvlc_hip_runtime_options;

/* Per-runtime counters (RuntimeCounters, native lib.rs:134-145). */
typedef struct pvlc_hip_runtime_counters {
    uint64_t kernel_launches;
    uint64_t host_to_device_copies;
    uint64_t device_to_host_copies;
    uint64_t synchronizations;
    uint64_t sessions_created;
} pvlc_hip_runtime_counters;

/* NativeRuntime::new, native lib.rs:912-1018.  Fails with
 * PVLC_HIP_ADAPTER_UNAVAILABLE when no gfx950 device is visible. */
pvlc_hip_status pvlc_hip_runtime_create(const pvlc_hip_runtime_options *options, pvlc_hip_runtime **runtime_out);
/* Sessions borrow their runtime, as NativeDecoderKvSession<'runtime> borrows
 * NativeRuntime (decoder_kv_session.rs:23-30): destroying a runtime whose
 * sessions are still live defers its release to the last of them (finish or
 * destroy); those sessions keep working until then.  No other call may use
 * the runtime after this one. */
void pvlc_hip_runtime_destroy(pvlc_hip_runtime *runtime);
pvlc_hip_status pvlc_hip_runtime_counters_get(const pvlc_hip_runtime *runtime, pvlc_hip_runtime_counters *out);

/* DecoderCachedGqaInvocation, runtime-core lib.rs:883-900. */
typedef struct pvlc_hip_cached_gqa_invocation {
    uint32_t query_heads;
    uint32_t key_value_heads;
    uint32_t head_dim;
    uint32_t prefix_tokens;
    uint32_t cache_capacity;
    const float *query;
    size_t query_len;
    const float *appended_key;
    size_t appended_key_len;
    const float *appended_value;
    size_t appended_value_len;
    const float *key_cache;
    size_t key_cache_len;
    const float *value_cache;
    size_t value_cache_len;
} pvlc_hip_cached_gqa_invocation;

/* DecoderCachedGqaExecution, native lib.rs:519-526: caller-owned outputs. */
typedef struct pvlc_hip_cached_gqa_execution {
    float *attention; /* query_heads*head_dim */
    size_t attention_len;
    float *key_cache; /* cache_capacity*2*128: the physical planes after the append */
    size_t key_cache_len;
    float *value_cache;
    size_t value_cache_len;
    uint32_t cache_tokens;   /* out */
    uint32_t cache_capacity; /* out */
    uint64_t queue_wall_time_ns;
} pvlc_hip_cached_gqa_execution;

/* NativeRuntime::run_decoder_cached_gqa, native lib.rs:1259-1264 (one-shot:
 * upload the cache, append, attend, read everything back). */
pvlc_hip_status pvlc_hip_run_decoder_cached_gqa(pvlc_hip_runtime *runtime,
                                                const pvlc_hip_cached_gqa_invocation *invocation,
                                                pvlc_hip_cached_gqa_execution *execution);

/* NativeRuntime::begin_decoder_kv_session, native lib.rs:1266-1271 and
 * decoder_kv_session.rs:62-82.  Validation precedes every GPU effect. */
pvlc_hip_status pvlc_hip_begin_decoder_kv_session(pvlc_hip_runtime *runtime,
                                                  const pvlc_hip_kv_session_descriptor *descriptor,
                                                  pvlc_hip_kv_session **session_out);

/* NativeDecoderKvSession::cache_tokens / cache_capacity, decoder_kv_session.rs:486-496. */
uint32_t pvlc_hip_kv_session_cache_tokens(const pvlc_hip_kv_session *session);
uint32_t pvlc_hip_kv_session_cache_capacity(const pvlc_hip_kv_session *session);
/* 1 while the session is terminally poisoned (decoder_kv_session.rs:18-21). */
int32_t pvlc_hip_kv_session_is_poisoned(const pvlc_hip_kv_session *session);

/* DecoderKvSessionStepExecution diagnostics, native lib.rs:566-594. */
typedef struct pvlc_hip_kv_step_execution {
    uint32_t cache_tokens_before;
    uint32_t cache_tokens_after;
    uint64_t queue_wall_time_ns;
    uint32_t dispatch_count;
} pvlc_hip_kv_step_execution;

/* NativeDecoderKvSession::step, decoder_kv_session.rs:499-529: append the
 * (already rotated) key/value row at cache_tokens, attend over cache_tokens+1
 * rows, write query_heads*head_dim f32 to attention.  The GPU rounds the
 * query, key and value to fp16 once (RNE) and attends over the fp16 cache; the
 * session keeps the f32 row as given for finish.  An invalid step has no
 * effect; a failure after submission poisons the session terminally. */
pvlc_hip_status pvlc_hip_kv_session_step(pvlc_hip_kv_session *session, const pvlc_hip_kv_step_operands *step,
                                         float *attention, size_t attention_len,
                                         pvlc_hip_kv_step_execution *execution_out);

/* NativeDecoderKvSession::finish, decoder_kv_session.rs:531-545, :812-925:
 * read the full physical planes back and return the capacity rows as given
 * (the descriptor's, then each committed step's), bit for bit, once each is
 * checked to match its fp16 row on the GPU (PVLC_HIP_OPERATION otherwise).
 * Consumes the session: it is freed whether or not the call succeeds, like
 * Rust's `finish(self)`. */
pvlc_hip_status pvlc_hip_kv_session_finish(pvlc_hip_kv_session *session, float *key_cache, size_t key_cache_len,
                                           float *value_cache, size_t value_cache_len, uint32_t *cache_tokens_out,
                                           uint32_t *cache_capacity_out);

/* Drop without finishing (Rust's Drop of NativeDecoderKvSession). */
void pvlc_hip_kv_session_destroy(pvlc_hip_kv_session *session);

/* Fault injection for tests, standing in for the reference's panicking
 * observer (decoder_kv_session_native_contract.rs:848-909): the next step
 * fails after its GPU work is submitted, which poisons the session. */
void pvlc_hip_kv_session_fail_next_step_after_submit(pvlc_hip_kv_session *session);

/* Fault injection for tests, standing in for a GPU that does not finish
 * within the wait bound: the next bounded wait of this session (its next step
 * or its finish) reports the deadline as passed whatever the GPU's state, so
 * the call fails with PVLC_HIP_OPERATION and a step leaves the session
 * poisoned, as the reference's poll timeout does (decoder_kv_session.rs:729-735).
 * The submitted work itself runs to completion. */
void pvlc_hip_kv_session_expire_next_wait(pvlc_hip_kv_session *session);

/* ---------------------------------------------------------------------------
 * Device-resident hot path (fp16, caller stream, no allocation, no sync).
 *
 * Blocked KV layout in HBM.  A cache is two planes of 16-token blocks:
 *   key plane   [num_blocks][2 kv heads][16 dim-chunks][16 token slots][8 dims]
 *   value plane [num_blocks][2 kv heads][128 dims][16 tokens]
 * so key element (block b, head h, token t, dim d) is at
 *   ((b*2 + h)*16 + d/8)*128 + slot(t)*8 + d%8,  slot(t) = t with bits 2 and 3 swapped
 * and value element at ((b*2 + h)*128 + d)*16 + t (fp16 elements).  (The
 * slot order lets the decode and prefill kernels read values with 16-byte
 * loads into 16x16x32 MFMAs.)  Each
 * (block, head) is 4 KiB per plane.  The compact reference planes
 * [tokens][2][128] convert to and from this layout bit-exactly with
 * pvlc_hip_kv_pack_f16 / pvlc_hip_kv_unpack_f16.
 *
 * A "sequence" owns a row of a block table; contiguous caches (block_tables
 * NULL) give sequence s the blocks s*max_blocks_per_seq + j, which is how the
 * 18-layer decode step addresses one cache per layer.
 * ------------------------------------------------------------------------- */

/* cos/sin tables [rows][rotary_dim/2] f32 with angle(pos, i) =
 * pos * base^(-(2i/rotary_dim)), computed exactly as apply_rope_neox
 * (cpu-ref lib.rs:459-461) with the host libm.  Host only. */
pvlc_hip_status pvlc_hip_rope_table_f32(float base, uint32_t rotary_dim, uint32_t rows, float *cos_out,
                                        float *sin_out);

/* Multimodal RoPE tables: the section selection of decoder_mrope_f32 and
 * decoder_prefill_mrope_f32 (pvlc-wgsl lib.rs:1185-1234, :1334-1380;
 * apply_multimodal_rope_f32, cpu-ref lib.rs:562-672) applied to raw cos/sin
 * tables [3][capacity][128] (temporal, height, width) with sections
 * (section_t, section_h, section_w) of the 64 frequency pairs (16, 24, 24 in
 * the shaders), giving the [capacity][64] tables the decode and prefill
 * entry points read; slot p of the tables is selected by the token's position
 * p.  Raw rows must repeat their first half (the device rotation reads one
 * cos/sin per pair); rows that do not are rejected (InvalidRotaryDimension),
 * as are non-finite values (NonFiniteInput).  Host only. */
pvlc_hip_status pvlc_hip_mrope_table_f32(const float *raw_cos, const float *raw_sin, uint32_t capacity,
                                         uint32_t section_t, uint32_t section_h, uint32_t section_w, float *cos_out,
                                         float *sin_out);

/* IEEE binary16 round-to-nearest-even conversion on the host (the rounding the
 * kernels apply to every value they store). */
void pvlc_hip_f32_to_f16_host(const float *in, uint16_t *out, size_t n);
void pvlc_hip_f16_to_f32_host(const uint16_t *in, float *out, size_t n);

typedef struct pvlc_hip_paged_decode_args {
    uint32_t num_seqs;           /* sequences (or layers of one step) in this launch */
    uint32_t num_blocks;         /* blocks in each plane (bounds every block id) */
    uint32_t max_blocks_per_seq; /* row stride of block_tables */
    const int32_t *block_tables; /* [num_seqs][max_blocks_per_seq] or NULL (contiguous) */
    const int32_t *cache_lens;   /* [num_seqs] rows already cached = append position, or NULL */
    uint32_t uniform_cache_len;  /* used for every sequence when cache_lens is NULL */
    uint32_t max_context;        /* >= cache_len+1 of every sequence (sizes the grid) */
    uint16_t *key_cache;
    uint16_t *value_cache;
    const uint16_t *query;     /* [num_seqs][16][128] fp16 */
    const uint16_t *new_key;   /* [num_seqs][2][128] fp16, rotated in-kernel when rope tables given */
    const uint16_t *new_value; /* [num_seqs][2][128] fp16 */
    uint16_t *out;             /* [num_seqs][16][128] fp16 */
    const float *rope_cos;     /* [rope_rows][64] or NULL: no rotary */
    const float *rope_sin;
    uint32_t rope_rows;
    const int32_t *positions; /* [num_seqs] rotary position of the new token, or NULL = cache_len */
    uint32_t rotate_query;    /* also rotate the query at that position */
    uint32_t partition_tokens; /* split-K partition (16..4096, multiple of 16); 0 = automatic */
    void *workspace;           /* from pvlc_hip_paged_decode_workspace_bytes, initialised once */
    size_t workspace_bytes;
} pvlc_hip_paged_decode_args;

/* Partition size the automatic choice (partition_tokens = 0) plans with.  A
 * streaming launch (ragged cache_lens, or contexts beyond one round of
 * single-shot workgroups) may lengthen it on the device, to at most twice this
 * and at most 4096 tokens, so the items spread evenly over the compute units;
 * it records the partition it used in the workspace word after the error word
 * (pvlc_hip_paged_decode_streaming_partition gives the same choice on the
 * host).  Ragged batches of more than 2048 sequences (more than the streaming
 * kernel numbers) run one workgroup per (partition, kv head, sequence) at
 * this partition instead, with the in-kernel merge. */
uint32_t pvlc_hip_paged_decode_partition(uint32_t num_seqs, uint32_t max_context);
/* The partition an automatic launch over these ragged cache lengths (rows
 * cached before the append; host memory, num_seqs entries) settles on, on a
 * device of compute_units compute units: the planned partition P0 above, or
 * the candidate P0 + c*max(16, P0/4 rounded down to 16), c = 1..4, with the
 * least ceil(items / compute_units) * P, items counting (sequence, partition,
 * kv head) triples -- never longer than the 4096 tokens one streaming
 * workgroup covers.  The streaming kernel makes this choice on the device by
 * the same rule and records it in the workspace word after the error word.
 * Lengths outside 0..max_context-1 are not counted; 0 for NULL or empty
 * input.  Host only.  (No reference counterpart: the reference plans fixed
 * 32-key chunks, runtime-core lib.rs:2889-2978.) */
uint32_t pvlc_hip_paged_decode_streaming_partition(const int32_t *cache_lens, uint32_t num_seqs, uint32_t max_context,
                                                   uint32_t compute_units);
/* Workspace for split-K partials, merge counters and the device error word. */
size_t pvlc_hip_paged_decode_workspace_bytes(uint32_t num_seqs, uint32_t max_context, uint32_t partition_tokens);
/* Zero a workspace on `stream` (a fill kernel; safe under graph capture). */
pvlc_hip_status pvlc_hip_workspace_init(void *workspace, size_t workspace_bytes, void *stream);
/* Device error word of a workspace (0 = none); synchronises.  Bits: 1 = a
 * cache length with no room for the append (sequence skipped), 2 = a block id
 * outside the planes (block 0 read, the appended row not written), 4 = a
 * rotary position outside the tables (no rotation). */
pvlc_hip_status pvlc_hip_workspace_error(const void *workspace, size_t workspace_bytes, void *stream,
                                         uint32_t *error_out);

/* One decode step for every sequence: rotate the new key (and optionally the
 * query), append the new K/V row at cache_len, then GQA attention over
 * cache_len+1 rows with split-K partitions merged in-kernel by the last
 * partition to finish (LSE merge).  Replaces the per-layer chain
 * decoder_mrope_f32 -> decoder_kv_append_f32 -> decoder_gqa_split_partial_f32 ->
 * decoder_gqa_split_merge_f32 (pvlc-wgsl lib.rs:927-952, 1024-1234; issued by
 * pvlc-runtime-web decoder_stack_session.rs:4698-4729) with one launch. */
pvlc_hip_status pvlc_hip_paged_decode_f16(const pvlc_hip_paged_decode_args *args, void *stream);
/* The same step with the per-token operands in f32, as the reference's chain
 * passes them between its dispatches (decoder_mrope_f32 reads the f32 q/k/v
 * its projections wrote, decoder_gqa_split_merge_f32 writes the f32 attention
 * output the o projection reads; pvlc-wgsl lib.rs:1024-1234, web
 * decoder_stack_session.rs:4698-4729): query [num_seqs][16][128], new_key and
 * new_value [num_seqs][2][128], out [num_seqs][16][128], all f32 device
 * pointers.  The query and the new key are rotated from their f32 values and
 * rounded to fp16 once (RNE); the new value is rounded to fp16; the cache
 * stays fp16.  The softmax weights enter P.V as exact pairs of fp16 values
 * (hi = fp16(p), lo = fp16(p - hi): ~22 bits), so the f32 output meets the
 * reference's native comparison policy (decoder_cached_gqa_native_contract.rs:
 * 147-158) where the fp16 entry point's fp16 weights and output do not.
 * args->query, new_key, new_value and out must be NULL; everything else as
 * pvlc_hip_paged_decode_f16. */
pvlc_hip_status pvlc_hip_paged_decode_f32io(const pvlc_hip_paged_decode_args *args, const float *query,
                                            const float *new_key, const float *new_value, float *out, void *stream);

/* pvlc_hip_paged_decode_f16 without allocation: the same validation, kernels
 * and results (bit-identical outputs and caches), with the split-K state kept
 * in a file-scope device array of the library (16 MiB per device, held until
 * the process ends) instead of a caller workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  args->workspace must be NULL and args->workspace_bytes 0.
 * error_word (device, caller-zeroed) receives the device error bits of
 * pvlc_hip_workspace_error.  At most 4096 sequences; a launch whose split-K
 * state exceeds 16 MiB is rejected (InvalidDecoderGeometry) -- configs with
 * up to 64 sequences of 8192 rows fit.  The first call on a device looks up
 * the array's address there (hipGetSymbolAddress); no call launches anything
 * but the decode kernels or synchronises, so any call, the first included,
 * may be captured into a HIP graph.  Every call on one device shares that
 * device's array and leaves it ready for the next call (the merge counters
 * start at zero and count whole generations per launch): calls that overlap
 * on one device (two streams, two threads, a graph replay beside a direct
 * call) race and garble their outputs; later calls are unaffected. */
pvlc_hip_status pvlc_hip_paged_decode_f16_no_alloc(const pvlc_hip_paged_decode_args *args, uint32_t *error_word,
                                                   void *stream);

typedef struct pvlc_hip_paged_prefill_args {
    uint32_t tokens;            /* N */
    uint32_t num_blocks;
    const int32_t *block_table; /* [ceil(N/16)] or NULL = blocks 0.. */
    uint16_t *key_cache;
    uint16_t *value_cache;
    const uint16_t *query; /* [N][16][128] fp16 */
    const uint16_t *key;   /* [N][2][128] */
    const uint16_t *value; /* [N][2][128] */
    uint16_t *out;         /* [N][16][128] */
    const float *rope_cos; /* [rope_rows][64] or NULL */
    const float *rope_sin;
    uint32_t rope_rows;
    const int32_t *positions; /* [N] or NULL = 0..N-1 */
    uint16_t *query_scratch;  /* optional [N][16][128] fp16: receives the rotated query (NULL: not written) */
    uint32_t *error_word;     /* optional: bit 1 = block id out of range (row skipped), bit 2 = position outside the rope table */
    void *workspace;          /* optional, 256-byte aligned, zeroed once (pvlc_hip_workspace_init): split-K schedule
                                 (long query blocks split over several workgroups and merged); NULL: one workgroup
                                 per query block.  Launches that share one workspace must be stream-ordered. */
    uint64_t workspace_bytes; /* at least pvlc_hip_paged_prefill_workspace_bytes(tokens) when workspace is given */
} pvlc_hip_paged_prefill_args;

/* Bytes of the split-K prefill workspace for N tokens (0: nothing splits). */
size_t pvlc_hip_paged_prefill_workspace_bytes(uint32_t tokens);

/* Causal prefill: rotary on Q and K, write all N K/V rows into the blocked
 * cache, then MFMA causal GQA attention (fp16 in, f32 accumulate, fp16 out).
 * Query, key, value, output, caches and query scratch are 16-byte aligned
 * (rejected otherwise).
 * Replaces decoder_prefill_mrope_f32 -> decoder_kv_append_range_f32 ->
 * decoder_prefill_gqa_f32 (pvlc-wgsl lib.rs:1262-1416; issued by
 * decoder_stack_session.rs:5044-5064). */
pvlc_hip_status pvlc_hip_paged_prefill_f16(const pvlc_hip_paged_prefill_args *args, void *stream);
/* The same prefill with the per-token operands in f32, as the reference's
 * prefill chain passes them (decoder_prefill_mrope_f32 reads the projections'
 * f32 q/k/v, decoder_prefill_gqa_f32 writes the f32 output the o projection
 * reads; pvlc-wgsl lib.rs:1262-1416, web decoder_stack_session.rs:5044-5064):
 * query [tokens][16][128], key and value [tokens][2][128], out
 * [tokens][16][128], all f32 device pointers.  The query and the keys are
 * rotated from their f32 values and rounded to fp16 once (RNE), the values
 * rounded to fp16; the cache (and the optional query scratch) stays fp16; the
 * softmax weights enter P.V as exact hi + lo pairs of fp16 values (~22 bits),
 * and the output is the normalised f32 product o * (1/l).  args->query, key,
 * value and out must be NULL; everything else as pvlc_hip_paged_prefill_f16. */
pvlc_hip_status pvlc_hip_paged_prefill_f32io(const pvlc_hip_paged_prefill_args *args, const float *query,
                                             const float *key, const float *value, float *out, void *stream);

/* Compact [tokens][2][128] fp16 rows <-> blocked planes (bit-exact), rows
 * 0..tokens-1 of one sequence through its block table (NULL = blocks 0..). */
pvlc_hip_status pvlc_hip_kv_pack_f16(const uint16_t *key_rows, const uint16_t *value_rows, uint32_t tokens,
                                     const int32_t *block_table, uint32_t num_blocks, uint16_t *key_cache,
                                     uint16_t *value_cache, void *stream);
pvlc_hip_status pvlc_hip_kv_unpack_f16(const uint16_t *key_cache, const uint16_t *value_cache, uint32_t tokens,
                                       const int32_t *block_table, uint32_t num_blocks, uint16_t *key_rows,
                                       uint16_t *value_rows, void *stream);

/* ---------------------------------------------------------------------------
 * Decoder GEMV with fp16 weights (the next path widened from this backend).
 * ------------------------------------------------------------------------- */

/* GemvTiledPlan, runtime-core lib.rs:729-745 (the reference's tiled GEMV
 * lattice: 8 rows x 32 lanes per 256-thread workgroup, vec4 columns). */
typedef struct pvlc_hip_gemv_tiled_plan {
    uint32_t tile_rows;
    uint32_t threads_per_row;
    uint32_t vector_width;
    uint32_t shared_capacity;
    uint32_t workgroup_storage_bytes;
    uint32_t dispatch[3];
    uint32_t workgroup_size[3];
    uint32_t uniform_words[4];
    uint64_t output_elements;
    uint64_t output_bytes;
} pvlc_hip_gemv_tiled_plan;

/* GemvTiledDescriptor::plan, runtime-core lib.rs:753-785: nonzero rows, the
 * decoder input widths 1024/2048/3072, at most 8 x 65535 rows. */
pvlc_hip_status pvlc_hip_gemv_tiled_plan_create(uint32_t rows, uint32_t columns, pvlc_hip_gemv_tiled_plan *plan_out);

/* out[r] = sum_c weights[r][c] * vector[c] for r < rows: fp16 weights,
 * output-major [rows][columns]; f32 vector and output; f32 accumulation.
 * Device pointers, caller stream, no allocation, no synchronisation; the
 * geometry is admitted exactly as the plan above.  Replaces
 * gemv_tiled_f16_weights (pvlc-wgsl lib.rs:1770-1835) in the seven per-layer
 * projections and the LM head (decoder_stack_session.rs; web module contract
 * decoder_stack_tiled_gemv_web_module_contract.rs). */
pvlc_hip_status pvlc_hip_gemv_f16(const uint16_t *weights, const float *vector, float *out, uint32_t rows,
                                  uint32_t columns, void *stream);

/* Up to 4 GEMVs of one width that read the same vector, in one launch: member
 * i writes members[i].out[r] = sum_c members[i].weights[r][c] * vector[c] for
 * r < members[i].rows, with pvlc_hip_gemv_f16's arithmetic (results
 * bit-identical to separate calls); the members' total rows are admitted as
 * one pvlc_hip_gemv_f16.  For the projections that read the same normalised
 * hidden state (q, k and v of a layer; gate and up), which the reference
 * dispatches as separate gemv_tiled_f16_weights passes (pvlc-wgsl
 * lib.rs:1770-1835, decoder_stack_session.rs): one launch instead of three or
 * two, weights left in their own tensors.  No single reference entry point
 * corresponds to it. */
typedef struct pvlc_hip_gemv_member {
    const uint16_t *weights; /* [rows][columns] fp16, output-major */
    float *out;              /* [rows] f32 */
    uint32_t rows;
} pvlc_hip_gemv_member;
pvlc_hip_status pvlc_hip_gemv_group_f16(const pvlc_hip_gemv_member *members, uint32_t count, const float *vector,
                                        uint32_t columns, void *stream);

/* ---------------------------------------------------------------------------
 * LM head and greedy top-1 on the device.
 * ------------------------------------------------------------------------- */

/* Bytes of the top-1 workspace (64 candidate slots, one per 256-byte line:
 * 16384 bytes).  Zero it once (pvlc_hip_workspace_init); every call leaves it
 * zeroed, so calls ordered on one stream reuse it; calls that overlap on one
 * workspace race.  The pointer must be 256-byte aligned.  Each top-1 call is
 * two launches on the caller's stream: the scan (or the LM-head GEMV), whose
 * workgroups fold their best into the slots, and a one-wave finish that reads
 * and clears them. */
size_t pvlc_hip_top1_workspace_bytes(void);

/* decoder_logits_top1_f32 (pvlc-runtime-web decoder_stack_session.rs:308-366,
 * dispatched by top1_decoder_stack_session, web.rs:2628): result[0] = index of
 * the largest of `vocab` f32 logits under the total order key
 * bits ^ ((u32)(bits >> 31) >> 1) (-NaN < -inf < -0 < +0 < +inf < +NaN), equal
 * keys to the lowest index; result[1] = that logit's f32 bits.  Device
 * pointers, caller stream; 1 <= vocab <= 2^31. */
pvlc_hip_status pvlc_hip_logits_top1_f32(const float *logits, uint32_t vocab, uint32_t *result, void *workspace,
                                         size_t workspace_bytes, void *stream);

/* The LM-head GEMV (pvlc_hip_gemv_f16 semantics and admission: the logits
 * pass of decoder_stack_session.rs, gemv_tiled_f16_weights at 103424 x 1024)
 * and the top-1 above over its output, selected while the GEMV streams (no
 * second pass over the logits).  logits may be NULL
 * (not written); result as pvlc_hip_logits_top1_f32 over the same logits. */
pvlc_hip_status pvlc_hip_lm_head_top1_f16(const uint16_t *weights, const float *hidden, float *logits, uint32_t rows,
                                          uint32_t columns, uint32_t *result, void *workspace, size_t workspace_bytes,
                                          void *stream);

/* ---------------------------------------------------------------------------
 * Prefill projections with fp16 weights (multi-token linear layers).
 * ------------------------------------------------------------------------- */

/* VisionPatchProjectionBytesErrorCode, runtime-core lib.rs:1751-1759. */
typedef enum pvlc_hip_projection_error {
    PVLC_HIP_PROJ_OK = 0,
    PVLC_HIP_PROJ_INVALID_GEOMETRY = 1,
    PVLC_HIP_PROJ_OVERFLOW = 2,
    PVLC_HIP_PROJ_LENGTH_MISMATCH = 3,
    PVLC_HIP_PROJ_NON_FINITE = 4,
    PVLC_HIP_PROJ_MISSING_SHADER_F16 = 5,
    PVLC_HIP_PROJ_DISPATCH_LIMIT_EXCEEDED = 6
} pvlc_hip_projection_error;

/* VisionPatchProjectionBytesPlan, runtime-core lib.rs:1741-1749. */
typedef struct pvlc_hip_projection_plan {
    uint32_t kernel;         /* 0 = vision_patch_projection_f32, 1 = linear_projection_f16_weights */
    uint32_t weight_storage; /* 0 = f32 weights, 1 = f16 weights */
    uint64_t input_bytes;
    uint64_t weight_bytes;
    uint64_t bias_bytes;
    uint64_t output_bytes;
    uint32_t dispatch[3];
} pvlc_hip_projection_plan;

/* VisionPatchProjectionBytesDescriptor::plan (runtime-core lib.rs:1768-1840):
 * positive geometry, widths a multiple of 4 for f16 weights, checked sizes,
 * dispatch [ceil(out / 32), ceil(rows / 32), 1].  Returns the error code. */
int32_t pvlc_hip_projection_plan_create(uint32_t patch_count, uint32_t input_width, uint32_t output_width,
                                        uint32_t weight_storage, pvlc_hip_projection_plan *plan_out);
/* VisionPatchProjectionBytesPlan::validate_capabilities (:1863-1885). */
int32_t pvlc_hip_projection_validate_capabilities(const pvlc_hip_projection_plan *plan, int32_t shader_f16_available,
                                                  uint32_t max_workgroups_per_dimension);
/* VisionPatchProjectionBytesPlan::validate_operands (:1887-1905): exact byte
 * lengths, then finite values (host memory, little-endian f32 / f16). */
int32_t pvlc_hip_projection_validate_operands(const pvlc_hip_projection_plan *plan, const void *input,
                                              size_t input_bytes, const void *weight, size_t weight_bytes,
                                              const void *bias, size_t bias_bytes);

/* Bytes of the workspace of pvlc_hip_linear_projection_f16 for rows x input_width. */
size_t pvlc_hip_linear_projection_workspace_bytes(uint32_t rows, uint32_t input_width);
/* out[r][n] = sum_k input[r][k] * weight[n][k] + bias[n]: f32 activations
 * [rows][input_width], fp16 weights output-major [output_width][input_width],
 * f32 bias and output [rows][output_width] -- linear_projection_f16_weights
 * (pvlc-wgsl lib.rs:1836-1964, the prefill projection stages of runtime-core
 * :2545-2560) with f32-grade products on MFMA (each activation row scaled by a
 * power of two and split exactly into two fp16 halves).  Device pointers
 * (16-byte aligned), caller stream, caller workspace (256-byte aligned),
 * nothing allocated.  Admitted as the f16 plan above, plus input_width a
 * multiple of 32 (the MFMA depth step); input-major weights are not taken. */
pvlc_hip_status pvlc_hip_linear_projection_f16(const float *input, const uint16_t *weight, const float *bias,
                                               float *output, uint32_t rows, uint32_t input_width,
                                               uint32_t output_width, void *workspace, size_t workspace_bytes,
                                               void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PVLC_HIP_H */
