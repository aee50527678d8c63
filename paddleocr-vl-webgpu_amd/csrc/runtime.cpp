// Host runtime: the NativeRuntime / NativeDecoderKvSession surface of
// crates/pvlc-runtime-native (glebkudr/paddleocr-vl-webgpu) on HIP, plus host
// validation of the device-resident entry points.
//
// Contract kept from the reference:
//  - every plan check runs before any GPU effect (decoder_kv_session.rs:62-82,
//    :499-512), so an invalid step changes nothing;
//  - a step marks the session Poisoned before submitting and restores Healthy
//    only on success (:513-528); a poisoned session refuses step and finish;
//  - one execution lock per runtime serialises GPU work (lib.rs:739);
//  - cache planes cross the boundary in the compact [capacity][2][128] layout.
// Storage is fp16: f32 operands are rounded to nearest even on the way in and
// widened exactly on the way out; a finite f32 whose fp16 rounding overflows is
// rejected as NonFiniteInput before any GPU effect.

#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "pvlc_internal.hpp"

using namespace pvlc;

struct pvlc_hip_runtime {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t done = nullptr;     // recorded behind submitted work, polled by bounded waits
    uint64_t wait_timeout_ns = 0;  // bound of every wait for submitted work
    std::mutex execution_lock;
    pvlc_hip_runtime_counters counters{};
    // Sessions borrow their runtime (NativeDecoderKvSession<'runtime> in the
    // reference): a runtime destroyed while sessions live is released by the
    // last of them.
    std::mutex life_lock;
    uint32_t live_sessions = 0;
    bool destroy_requested = false;
};

struct pvlc_hip_kv_session {
    pvlc_hip_runtime *runtime = nullptr;
    pvlc_hip_kv_session_plan plan{};
    uint32_t cache_tokens = 0;
    bool poisoned = false;
    bool fail_next_after_submit = false;
    bool expire_next_wait = false;
    uint32_t num_blocks = 0;
    uint16_t *key_cache = nullptr;    // blocked planes
    uint16_t *value_cache = nullptr;
    float *step_operands = nullptr;  // device: query | key | value (f32, rounded to fp16 by the kernel)
    // device: 16*128 f32, then the decode workspace in the same allocation,
    // so one readback of attention + 4 bytes returns the workspace's error
    // word with the attention
    float *attention = nullptr;
    void *workspace = nullptr;
    float *host_staging = nullptr;  // pinned: operands in, attention and error word out
    size_t workspace_bytes = 0;
    // Host: the rows exactly as given, compact [capacity][2][128] f32 (the
    // descriptor's planes, then each committed step's appended row).  The
    // device planes hold these rounded to fp16; finish returns these.
    std::vector<float> key_rows, value_rows;
};

namespace {

constexpr size_t kQueryElems = kQueryHeads * kHeadDim;
constexpr size_t kStepElems = kQueryElems + 2 * kRowElems;

pvlc_hip_status hip_fail(hipError_t e, const char *what) {
    const int code = e == hipErrorOutOfMemory ? PVLC_HIP_OUT_OF_MEMORY : PVLC_HIP_OPERATION;
    return fail(code, PVLC_HIP_INV_NONE, std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                            \
    do {                                               \
        hipError_t e_ = (expr);                        \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

uint64_t now_ns() {
    return static_cast<uint64_t>(
        std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch())
            .count());
}

// GPU_WAIT_TIMEOUT (native lib.rs:56): every wait for submitted work is
// bounded, 30 s unless the runtime options give another bound.
constexpr uint64_t kDefaultWaitTimeoutNs = 30ull * 1000 * 1000 * 1000;

// Wait for everything queued on the runtime's stream so far, at most the
// runtime's timeout: an event recorded behind the work is polled, first
// spinning, then sleeping 20 us between polls.  Returns hipSuccess, the HIP
// error of the queue, or hipErrorNotReady when the deadline passed with the
// work still pending.  `expire` reports the deadline as passed at the first
// poll whatever the GPU's state (the tests' stand-in for a GPU that does not
// finish, so that no GPU is made to hang).
hipError_t wait_bounded(pvlc_hip_runtime *rt, bool expire) {
    if (hipError_t e = hipEventRecord(rt->done, rt->stream)) return e;
    const uint64_t deadline = now_ns() + rt->wait_timeout_ns;
    for (uint32_t polls = 0;; ++polls) {
        const hipError_t e = expire ? hipErrorNotReady : hipEventQuery(rt->done);
        if (e != hipErrorNotReady) return e;
        if (expire || now_ns() >= deadline) return hipErrorNotReady;
        if (polls >= 64) std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

// wait_bounded as a status: a wait that expires is an Operation failure, as
// the reference's poll timeout is (decoder_kv_session.rs:729-735, :890-896).
pvlc_hip_status wait_or_fail(pvlc_hip_runtime *rt, bool expire, const char *what) {
    const hipError_t e = wait_bounded(rt, expire);
    if (e == hipErrorNotReady)
        return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE,
                    std::string(what) + ": GPU work did not complete within " +
                        std::to_string(rt->wait_timeout_ns / 1000000) + " ms");
    if (e != hipSuccess) return hip_fail(e, what);
    rt->counters.synchronizations += 1;
    return PVLC_HIP_OK;
}

// Frees the session's buffers once the GPU work queued on the runtime has
// completed (a bounded wait).  A session whose work does not complete within
// the bound keeps its device buffers allocated (leaked) rather than freeing
// memory a kernel may still access.
void free_session_buffers(pvlc_hip_kv_session *s) {
    if (!s) return;
    if (s->runtime) {
        (void)hipSetDevice(s->runtime->device);
        if (wait_bounded(s->runtime, false) == hipErrorNotReady) return;  // pinned staging may still be written
    }
    (void)hipFree(s->key_cache);
    (void)hipFree(s->value_cache);
    (void)hipFree(s->step_operands);
    (void)hipFree(s->attention);  // also holds the workspace
    (void)hipHostFree(s->host_staging);
    s->key_cache = s->value_cache = nullptr;
    s->step_operands = s->attention = nullptr;
    s->workspace = nullptr;
    s->host_staging = nullptr;
}

void destroy_runtime_now(pvlc_hip_runtime *rt) {
    (void)hipSetDevice(rt->device);
    if (rt->done) (void)hipEventDestroy(rt->done);
    if (rt->stream) (void)hipStreamDestroy(rt->stream);
    delete rt;
}

// Releases a session: its buffers (after a bounded wait for the runtime's
// queued work), the session, and its hold on the runtime, which the last
// session of a destroyed runtime releases.  `lock_held`: the caller holds the
// runtime's execution lock.
void release_session(pvlc_hip_kv_session *s, bool lock_held) {
    if (!s) return;
    pvlc_hip_runtime *rt = s->runtime;
    {
        std::unique_lock<std::mutex> guard(rt->execution_lock, std::defer_lock);
        if (!lock_held) guard.lock();
        free_session_buffers(s);
    }
    delete s;
    bool last = false;
    {
        std::lock_guard<std::mutex> life(rt->life_lock);
        last = --rt->live_sessions == 0 && rt->destroy_requested;
    }
    if (last) destroy_runtime_now(rt);
}

}  // namespace

namespace pvlc {

// Device-resident argument validation, the workspace aside, shared by the
// public entry points and the session path: the partition and the
// partitions per (sequence, kv head) the launch runs.  Returns a status
// (0 = ok) without touching the GPU.
pvlc_hip_status validate_decode_geometry(const pvlc_hip_paged_decode_args *a, uint32_t *partition_out,
                                         uint32_t *max_parts_out, const DecodeOperands32 *f32) {
    if (!a) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "paged decode args are NULL");
    if (a->num_seqs == 0 || a->num_blocks == 0 || a->max_blocks_per_seq == 0 || a->max_context == 0)
        return invalid(PVLC_HIP_INV_ZERO_DIMENSION, "all paged decode dimensions must be nonzero");
    if (f32) {
        if (a->query || a->new_key || a->new_value || a->out)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH,
                           "pvlc_hip_paged_decode_f32io takes its query, new key, new value and output as f32 "
                           "arguments; the fp16 ones in the args must be NULL");
        if (!f32->query || !f32->new_key || !f32->new_value || !f32->out)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "paged decode f32 operand pointer is NULL");
    } else if (!a->query || !a->new_key || !a->new_value || !a->out) {
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "paged decode buffer pointer is NULL");
    }
    if (!a->key_cache || !a->value_cache)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "paged decode buffer pointer is NULL");
    if ((a->rope_cos == nullptr) != (a->rope_sin == nullptr) || (a->rope_cos && a->rope_rows == 0))
        return invalid(PVLC_HIP_INV_INVALID_ROTARY_DIMENSION, "rotary tables must be given together with rows");
    if (!a->block_tables &&
        static_cast<uint64_t>(a->num_seqs) * a->max_blocks_per_seq > static_cast<uint64_t>(a->num_blocks))
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "contiguous caches need num_seqs * max_blocks_per_seq blocks");
    if (static_cast<uint64_t>(a->max_context) > static_cast<uint64_t>(a->max_blocks_per_seq) * kBlockTokens)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "max_context exceeds the block table span");
    if (!a->cache_lens && a->uniform_cache_len + 1ull > a->max_context)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "uniform cache length leaves no append row");
    if (a->num_seqs > 65535u) return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "num_seqs exceeds 65535");
    uint32_t partition = a->partition_tokens;
    if (partition != 0) {
        if (partition < kBlockTokens || partition > 4096 || partition % kBlockTokens != 0)
            return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                           "partition_tokens must be a multiple of 16 in 16..4096");
        if ((a->max_context + partition - 1) / partition > kMaxMergeParts)
            return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                           "max_context / partition_tokens exceeds the 64 partitions one merge combines");
    } else {
        partition = auto_partition(a->num_seqs, a->max_context);
        // A uniform cache length is known here: balance the partitions for
        // the rows actually attended when they fit one round.
        if (!a->cache_lens) {
            if (const uint32_t p = single_shot_partition(a->num_seqs, a->uniform_cache_len + 1)) partition = p;
        }
    }
    // Grid partitions: the attended rows bound them when they are uniform.
    const uint32_t rows = a->cache_lens ? a->max_context : a->uniform_cache_len + 1;
    const uint32_t max_parts = (rows + partition - 1) / partition;
    if (max_parts > kMaxMergeParts)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "the context needs more than the 64 partitions one merge combines");
    {
        // The kernels read the query and the cache planes as 16-byte vectors
        // and the split-K state with 16-byte buffer accesses; every operand
        // is held to the same rule, in both operand widths.
        const void *rows[] = {a->query,  a->new_key, a->new_value, a->out, a->key_cache, a->value_cache,
                              a->workspace, f32 ? f32->query : nullptr, f32 ? f32->new_key : nullptr,
                              f32 ? f32->new_value : nullptr, f32 ? f32->out : nullptr};
        for (const void *r : rows)
            if (reinterpret_cast<uintptr_t>(r) % 16 != 0)
                return invalid(PVLC_HIP_INV_LENGTH_MISMATCH,
                               "paged decode query, new key, new value, output, cache planes and workspace must be "
                               "16-byte aligned");
    }
    if (partition_out) *partition_out = partition;
    if (max_parts_out) *max_parts_out = max_parts;
    return PVLC_HIP_OK;
}

pvlc_hip_status launch_decode_state(const pvlc_hip_paged_decode_args *a, uint32_t partition, uint32_t max_parts,
                                    const DecodeState &state, void *stream, uint32_t *launches_out,
                                    const DecodeOperands32 *f32) {
    // Streaming regime: ragged lengths, or partitions longer than one chunk
    // of the largest single-shot workgroup.
    const uint32_t part_tiles = (partition + kBlockTokens - 1) / kBlockTokens;
    const bool streaming = (a->cache_lens != nullptr || part_tiles > kSingleShotTiles) && a->num_seqs <= kMaxRaggedSeqs;
    const DecodeShape shape = decode_shape(partition, streaming);
    DecodeLaunch launch{a,
                        partition,
                        shape.waves,
                        shape.pairs,
                        streaming,
                        max_parts,
                        state.part_stride,
                        state.part_o,
                        state.part_ml,
                        state.counters,
                        state.error_word,
                        nullptr,
                        f32};
    // An automatic streaming launch records the partition it settled on and
    // the compute units it assumed in the two status words.
    if (streaming && a->partition_tokens == 0) launch.partition_word = state.status_words;
    const int e = launch_paged_decode(launch, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "paged decode launch");
    if (launches_out) *launches_out = streaming ? 2u : 1u;  // persistent kernel + merge kernel, or one kernel
    return PVLC_HIP_OK;
}

}  // namespace pvlc

namespace {

// The caller's workspace checked and laid out (decode_workspace_layout): the
// error word first, the two status words after it in the same 256-byte slot.
pvlc_hip_status launch_decode_checked(const pvlc_hip_paged_decode_args *a, void *stream,
                                      uint32_t *launches_out = nullptr, const DecodeOperands32 *f32 = nullptr) {
    uint32_t partition = 0, max_parts = 0;
    if (pvlc_hip_status st = validate_decode_geometry(a, &partition, &max_parts, f32)) return st;
    if (!a->workspace) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "paged decode workspace is NULL");
    const DecodeWorkspace layout = decode_workspace_layout(a->num_seqs, max_parts);
    if (a->workspace_bytes < layout.total)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "workspace holds " + std::to_string(a->workspace_bytes) +
                                                         " bytes but the launch needs " + std::to_string(layout.total));
    char *ws = static_cast<char *>(a->workspace);
    const DecodeState state{reinterpret_cast<float *>(ws + layout.part_o_offset),
                            reinterpret_cast<float *>(ws + layout.part_ml_offset),
                            reinterpret_cast<uint32_t *>(ws + layout.counters_offset),
                            reinterpret_cast<uint32_t *>(ws + layout.error_offset),
                            reinterpret_cast<uint32_t *>(ws + layout.error_offset) + 1,
                            layout.part_stride};
    return launch_decode_state(a, partition, max_parts, state, stream, launches_out, f32);
}

// Session creation shared by begin_decoder_kv_session and the one-shot path.
// The plan is already validated.
pvlc_hip_status create_session(pvlc_hip_runtime *rt, const pvlc_hip_kv_session_plan &plan, const float *key_cache,
                               const float *value_cache, pvlc_hip_kv_session **out) {
    auto *s = new (std::nothrow) pvlc_hip_kv_session();
    if (!s) return fail(PVLC_HIP_OUT_OF_MEMORY, PVLC_HIP_INV_NONE, "session allocation failed");
    s->runtime = rt;
    {
        std::lock_guard<std::mutex> life(rt->life_lock);
        rt->live_sessions += 1;
    }
    s->plan = plan;
    s->cache_tokens = plan.initial_cache_tokens;
    s->num_blocks = (plan.cache_capacity + kBlockTokens - 1) / kBlockTokens;
    // Steps use the automatic (per-length balanced) partition; the workspace
    // holds the most partitions any automatic launch up to capacity uses.
    s->workspace_bytes = decode_workspace_layout(1, auto_workspace_parts(1, plan.cache_capacity)).total;
    const size_t plane_elems = static_cast<size_t>(s->num_blocks) * kBlockTokens * kRowElems;

    auto cleanup = [&](pvlc_hip_status st) {
        release_session(s, true);  // the caller holds the execution lock
        return st;
    };
    hipError_t e;
    if ((e = hipSetDevice(rt->device)) != hipSuccess) return cleanup(hip_fail(e, "hipSetDevice"));
    if ((e = hipMalloc(&s->key_cache, plane_elems * 2)) != hipSuccess) return cleanup(hip_fail(e, "key cache"));
    if ((e = hipMalloc(&s->value_cache, plane_elems * 2)) != hipSuccess) return cleanup(hip_fail(e, "value cache"));
    if ((e = hipMalloc(&s->step_operands, kStepElems * 4)) != hipSuccess) return cleanup(hip_fail(e, "operands"));
    if ((e = hipMalloc(&s->attention, kQueryElems * 4 + s->workspace_bytes)) != hipSuccess)
        return cleanup(hip_fail(e, "attention and workspace"));
    s->workspace = s->attention + kQueryElems;  // 8 KiB in: 256-byte aligned
    if ((e = hipHostMalloc(reinterpret_cast<void **>(&s->host_staging), (kStepElems + kQueryElems + 1) * 4,
                           hipHostMallocDefault)) != hipSuccess)
        return cleanup(hip_fail(e, "pinned staging"));

    // Initial planes: keep the f32 rows, round to fp16 and scatter into the
    // blocked layout on the host (rows past the capacity stay zero), then one
    // copy per plane.
    std::vector<uint16_t> kb, vb;
    try {
        const size_t rows_elems = static_cast<size_t>(plan.cache_capacity) * kRowElems;
        s->key_rows.assign(key_cache, key_cache + rows_elems);
        s->value_rows.assign(value_cache, value_cache + rows_elems);
        kb.assign(plane_elems, 0);
        vb.assign(plane_elems, 0);
    } catch (const std::bad_alloc &) {
        return cleanup(fail(PVLC_HIP_OUT_OF_MEMORY, PVLC_HIP_INV_NONE, "host copy of the cache rows"));
    }
    for (uint32_t t = 0; t < plan.cache_capacity; ++t) {
        for (uint32_t h = 0; h < kKvHeads; ++h) {
            for (uint32_t d = 0; d < kHeadDim; ++d) {
                const size_t src = (static_cast<size_t>(t) * kKvHeads + h) * kHeadDim + d;
                kb[key_blocked_index(t, h, d)] = f32_to_f16_rne(key_cache[src]);
                vb[value_blocked_index(t, h, d)] = f32_to_f16_rne(value_cache[src]);
            }
        }
    }
    hipStream_t st = rt->stream;
    if ((e = hipMemcpyAsync(s->key_cache, kb.data(), plane_elems * 2, hipMemcpyHostToDevice, st)) != hipSuccess)
        return cleanup(hip_fail(e, "key cache upload"));
    if ((e = hipMemcpyAsync(s->value_cache, vb.data(), plane_elems * 2, hipMemcpyHostToDevice, st)) != hipSuccess)
        return cleanup(hip_fail(e, "value cache upload"));
    const int fe = launch_fill_u32(static_cast<uint32_t *>(s->workspace), s->workspace_bytes / 4, 0u, st);
    if (fe != 0) return cleanup(hip_fail(static_cast<hipError_t>(fe), "workspace init"));
    rt->counters.host_to_device_copies += 2;
    rt->counters.kernel_launches += 1;
    if (pvlc_hip_status ws = wait_or_fail(rt, false, "session creation")) return cleanup(ws);
    rt->counters.sessions_created += 1;
    *out = s;
    return PVLC_HIP_OK;
}

// One append + attention on the session's device state.  Caller holds the
// execution lock and has validated the step.
pvlc_hip_status execute_step(pvlc_hip_kv_session *s, const pvlc_hip_kv_step_operands *step, float *attention,
                             pvlc_hip_kv_step_execution *exec) {
    pvlc_hip_runtime *rt = s->runtime;
    const uint64_t started = now_ns();
    // The operands travel as f32; the kernel rounds the query, key and value
    // to fp16 (RNE) and writes the attention as f32.
    float *stage = s->host_staging;
    std::memcpy(stage, step->query, kQueryElems * 4);
    std::memcpy(stage + kQueryElems, step->appended_key, kRowElems * 4);
    std::memcpy(stage + kQueryElems + kRowElems, step->appended_value, kRowElems * 4);
    HIP_TRY(hipSetDevice(rt->device), "hipSetDevice");
    HIP_TRY(hipMemcpyAsync(s->step_operands, stage, kStepElems * 4, hipMemcpyHostToDevice, rt->stream),
            "step operand upload");
    rt->counters.host_to_device_copies += 1;

    pvlc_hip_paged_decode_args a{};
    a.num_seqs = 1;
    a.num_blocks = s->num_blocks;
    a.max_blocks_per_seq = s->num_blocks;
    a.block_tables = nullptr;
    a.cache_lens = nullptr;
    a.uniform_cache_len = s->cache_tokens;
    a.max_context = s->plan.cache_capacity;
    a.key_cache = s->key_cache;
    a.value_cache = s->value_cache;
    a.partition_tokens = 0;
    a.workspace = s->workspace;
    a.workspace_bytes = s->workspace_bytes;
    const DecodeOperands32 f32{s->step_operands, s->step_operands + kQueryElems,
                               s->step_operands + kQueryElems + kRowElems, s->attention};
    uint32_t launches = 0;
    if (pvlc_hip_status st = launch_decode_checked(&a, rt->stream, &launches, &f32)) return st;
    rt->counters.kernel_launches += launches;

    float *result = stage + kStepElems;
    // The attention and, right after it, the workspace's device error word.
    HIP_TRY(hipMemcpyAsync(result, s->attention, (kQueryElems + 1) * 4, hipMemcpyDeviceToHost, rt->stream),
            "attention readback");
    rt->counters.device_to_host_copies += 1;
    const bool expire = s->expire_next_wait;
    s->expire_next_wait = false;
    if (pvlc_hip_status st = wait_or_fail(rt, expire, "decoder KV session step")) return st;
    if (s->fail_next_after_submit) {
        s->fail_next_after_submit = false;
        return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE, "decoder KV session step: injected failure after submission");
    }
    uint32_t device_error = 0;
    std::memcpy(&device_error, result + kQueryElems, 4);
    if (device_error != 0)
        return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE,
                    "decoder KV session step: the decode kernel reported device error bits " +
                        std::to_string(device_error));
    std::memcpy(attention, result, kQueryElems * 4);
    const size_t row = static_cast<size_t>(s->cache_tokens) * kRowElems;
    std::memcpy(s->key_rows.data() + row, step->appended_key, kRowElems * 4);
    std::memcpy(s->value_rows.data() + row, step->appended_value, kRowElems * 4);
    if (exec) {
        exec->cache_tokens_before = s->cache_tokens;
        exec->cache_tokens_after = s->cache_tokens + 1;
        exec->queue_wall_time_ns = now_ns() - started;
        exec->dispatch_count = launches;
    }
    return PVLC_HIP_OK;
}

// Read the planes back and return the session's f32 rows (rows
// 0..capacity-1, compact layout) once every device row is checked to hold
// its f32 row rounded to fp16.  Rows the steps appended are finite and
// rounded by the kernel; every other row (NaN tails included) was rounded by
// f32_to_f16_rne at creation, so the comparison is bit for bit.
pvlc_hip_status read_planes(pvlc_hip_kv_session *s, float *key_out, float *value_out) {
    pvlc_hip_runtime *rt = s->runtime;
    const size_t plane_elems = static_cast<size_t>(s->num_blocks) * kBlockTokens * kRowElems;
    HIP_TRY(hipSetDevice(rt->device), "hipSetDevice");
    // Pinned staging keeps both copies asynchronous, so the one wait below
    // (bounded) covers them.
    uint16_t *staged = nullptr;
    HIP_TRY(hipHostMalloc(reinterpret_cast<void **>(&staged), plane_elems * 4, hipHostMallocDefault),
            "finish staging");
    struct Release {
        uint16_t *p;
        bool keep = false;  // the copies may still write into it
        ~Release() {
            if (!keep) (void)hipHostFree(p);
        }
    } release{staged};
    uint16_t *kb = staged, *vb = staged + plane_elems;
    HIP_TRY(hipMemcpyAsync(kb, s->key_cache, plane_elems * 2, hipMemcpyDeviceToHost, rt->stream),
            "key cache readback");
    HIP_TRY(hipMemcpyAsync(vb, s->value_cache, plane_elems * 2, hipMemcpyDeviceToHost, rt->stream),
            "value cache readback");
    rt->counters.device_to_host_copies += 2;
    const bool expire = s->expire_next_wait;
    s->expire_next_wait = false;
    if (pvlc_hip_status st = wait_or_fail(rt, expire, "decoder KV session finish")) {
        // After a real time-out (or a failed queue) the copies may still write
        // into the staging: it is kept (leaked) without waiting a second bound.
        // After the tests' injected expiry one query of the event decides.
        // The session's release makes the one remaining bounded wait.
        release.keep = !expire || hipEventQuery(rt->done) != hipSuccess;
        return st;
    }
    auto same = [](uint16_t device, float row) { return device == f32_to_f16_rne(row); };
    for (uint32_t t = 0; t < s->plan.cache_capacity; ++t) {
        for (uint32_t h = 0; h < kKvHeads; ++h) {
            for (uint32_t d = 0; d < kHeadDim; ++d) {
                const size_t src = (static_cast<size_t>(t) * kKvHeads + h) * kHeadDim + d;
                if (!same(kb[key_blocked_index(t, h, d)], s->key_rows[src]) ||
                    !same(vb[value_blocked_index(t, h, d)], s->value_rows[src]))
                    return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE,
                                "decoder KV session finish: the device cache differs from the session's rows at row " +
                                    std::to_string(t));
            }
        }
    }
    const size_t rows_elems = static_cast<size_t>(s->plan.cache_capacity) * kRowElems;
    std::memcpy(key_out, s->key_rows.data(), rows_elems * 4);
    std::memcpy(value_out, s->value_rows.data(), rows_elems * 4);
    return PVLC_HIP_OK;
}

pvlc_hip_status check_fp16_range(const float *v, size_t n, const char *what) {
    if (!fp16_representable(v, n))
        return invalid(PVLC_HIP_INV_NON_FINITE_INPUT, std::string(what) + " holds a value outside the fp16 range");
    return PVLC_HIP_OK;
}

}  // namespace

extern "C" {

pvlc_hip_status pvlc_hip_runtime_create(const pvlc_hip_runtime_options *options, pvlc_hip_runtime **runtime_out) {
    if (!runtime_out) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "runtime_out is NULL");
    *runtime_out = nullptr;
    const int device = options ? options->device : 0;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(PVLC_HIP_ADAPTER_UNAVAILABLE, PVLC_HIP_INV_NONE, "no HIP device is visible");
    if (device < 0 || device >= count)
        return fail(PVLC_HIP_ADAPTER_UNAVAILABLE, PVLC_HIP_INV_NONE, "device ordinal out of range");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail(PVLC_HIP_DEVICE_REQUEST, PVLC_HIP_INV_NONE, "device properties unavailable");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(PVLC_HIP_ADAPTER_UNAVAILABLE, PVLC_HIP_INV_NONE,
                    std::string("pvlc_hip requires gfx950, found ") + prop.gcnArchName);
    auto *rt = new (std::nothrow) pvlc_hip_runtime();
    if (!rt) return fail(PVLC_HIP_OUT_OF_MEMORY, PVLC_HIP_INV_NONE, "runtime allocation failed");
    rt->device = device;
    rt->wait_timeout_ns = options && options->gpu_wait_timeout_ns ? options->gpu_wait_timeout_ns : kDefaultWaitTimeoutNs;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&rt->done, hipEventDisableTiming);
    if (e != hipSuccess) {
        if (rt->stream) (void)hipStreamDestroy(rt->stream);
        delete rt;
        return fail(PVLC_HIP_DEVICE_REQUEST, PVLC_HIP_INV_NONE,
                    std::string("stream and event creation: ") + hipGetErrorString(e));
    }
    *runtime_out = rt;
    return ok();
}

void pvlc_hip_runtime_destroy(pvlc_hip_runtime *runtime) {
    if (!runtime) return;
    bool now = false;
    {
        std::lock_guard<std::mutex> life(runtime->life_lock);
        runtime->destroy_requested = true;
        now = runtime->live_sessions == 0;
    }
    if (now) destroy_runtime_now(runtime);
}

pvlc_hip_status pvlc_hip_runtime_counters_get(const pvlc_hip_runtime *runtime, pvlc_hip_runtime_counters *out) {
    if (!runtime || !out) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "NULL argument");
    *out = runtime->counters;
    return ok();
}

pvlc_hip_status pvlc_hip_begin_decoder_kv_session(pvlc_hip_runtime *runtime,
                                                  const pvlc_hip_kv_session_descriptor *descriptor,
                                                  pvlc_hip_kv_session **session_out) {
    if (!runtime || !descriptor || !session_out) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "NULL argument");
    *session_out = nullptr;
    pvlc_hip_kv_session_plan plan{};
    if (PlanError e = plan_descriptor(descriptor, &plan)) return invalid(e.code, e.message);
    const size_t semantic = static_cast<size_t>(plan.initial_cache_tokens) * kRowElems;
    if (pvlc_hip_status st = check_fp16_range(descriptor->key_cache, semantic, "key cache")) return st;
    if (pvlc_hip_status st = check_fp16_range(descriptor->value_cache, semantic, "value cache")) return st;
    std::lock_guard<std::mutex> guard(runtime->execution_lock);
    pvlc_hip_status st = create_session(runtime, plan, descriptor->key_cache, descriptor->value_cache, session_out);
    if (st != PVLC_HIP_OK) return fail(st >> 8, st & 0xff, std::string("decoder KV session creation: ") +
                                                            pvlc_hip_last_error_message());
    return ok();
}

uint32_t pvlc_hip_kv_session_cache_tokens(const pvlc_hip_kv_session *session) {
    return session ? session->cache_tokens : 0;
}

uint32_t pvlc_hip_kv_session_cache_capacity(const pvlc_hip_kv_session *session) {
    return session ? session->plan.cache_capacity : 0;
}

int32_t pvlc_hip_kv_session_is_poisoned(const pvlc_hip_kv_session *session) {
    return session && session->poisoned ? 1 : 0;
}

void pvlc_hip_kv_session_fail_next_step_after_submit(pvlc_hip_kv_session *session) {
    if (session) session->fail_next_after_submit = true;
}

void pvlc_hip_kv_session_expire_next_wait(pvlc_hip_kv_session *session) {
    if (session) session->expire_next_wait = true;
}

pvlc_hip_status pvlc_hip_kv_session_step(pvlc_hip_kv_session *session, const pvlc_hip_kv_step_operands *step,
                                         float *attention, size_t attention_len,
                                         pvlc_hip_kv_step_execution *execution_out) {
    if (!session || !step) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "NULL argument");
    if (session->poisoned)
        return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE, "decoder KV session is terminally poisoned");
    pvlc_hip_kv_step_plan sp{};
    if (PlanError e = plan_step(&session->plan, session->cache_tokens, step, &sp)) return invalid(e.code, e.message);
    if (!attention || attention_len != kQueryElems)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "attention output must hold 2048 floats");
    if (pvlc_hip_status st = check_fp16_range(step->query, step->query_len, "query")) return st;
    if (pvlc_hip_status st = check_fp16_range(step->appended_key, step->appended_key_len, "appended key")) return st;
    if (pvlc_hip_status st = check_fp16_range(step->appended_value, step->appended_value_len, "appended value"))
        return st;
    std::lock_guard<std::mutex> guard(session->runtime->execution_lock);
    session->poisoned = true;
    pvlc_hip_status st = execute_step(session, step, attention, execution_out);
    if (st != PVLC_HIP_OK) return st;
    session->cache_tokens = sp.cache_tokens_after;
    session->poisoned = false;
    return ok();
}

pvlc_hip_status pvlc_hip_kv_session_finish(pvlc_hip_kv_session *session, float *key_cache, size_t key_cache_len,
                                           float *value_cache, size_t value_cache_len, uint32_t *cache_tokens_out,
                                           uint32_t *cache_capacity_out) {
    if (!session) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "session is NULL");
    struct Consume {
        pvlc_hip_kv_session *s;
        ~Consume() { release_session(s, false); }  // after the execution lock below is released
    } consume{session};
    if (session->poisoned)
        return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE, "decoder KV session is terminally poisoned");
    if (!key_cache || !value_cache || key_cache_len != session->plan.cache_elements ||
        value_cache_len != session->plan.cache_elements)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "finish outputs must hold cache_capacity*256 floats each");
    std::lock_guard<std::mutex> guard(session->runtime->execution_lock);
    if (pvlc_hip_status st = read_planes(session, key_cache, value_cache)) return st;
    if (cache_tokens_out) *cache_tokens_out = session->cache_tokens;
    if (cache_capacity_out) *cache_capacity_out = session->plan.cache_capacity;
    return ok();
}

void pvlc_hip_kv_session_destroy(pvlc_hip_kv_session *session) { release_session(session, false); }

pvlc_hip_status pvlc_hip_run_decoder_cached_gqa(pvlc_hip_runtime *runtime,
                                                const pvlc_hip_cached_gqa_invocation *invocation,
                                                pvlc_hip_cached_gqa_execution *execution) {
    if (!runtime || !invocation || !execution) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "NULL argument");
    pvlc_hip_kv_session_plan plan{};
    pvlc_hip_kv_step_plan sp{};
    if (PlanError e = plan_cached_gqa(invocation, &plan, &sp)) return invalid(e.code, e.message);
    const size_t semantic = static_cast<size_t>(invocation->prefix_tokens) * kRowElems;
    if (pvlc_hip_status st = check_fp16_range(invocation->key_cache, semantic, "key cache")) return st;
    if (pvlc_hip_status st = check_fp16_range(invocation->value_cache, semantic, "value cache")) return st;
    if (pvlc_hip_status st = check_fp16_range(invocation->query, invocation->query_len, "query")) return st;
    if (pvlc_hip_status st = check_fp16_range(invocation->appended_key, kRowElems, "appended key")) return st;
    if (pvlc_hip_status st = check_fp16_range(invocation->appended_value, kRowElems, "appended value")) return st;
    if (!execution->attention || execution->attention_len != kQueryElems || !execution->key_cache ||
        !execution->value_cache || execution->key_cache_len != plan.cache_elements ||
        execution->value_cache_len != plan.cache_elements)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "execution outputs have the wrong lengths");
    const uint64_t started = now_ns();
    std::lock_guard<std::mutex> guard(runtime->execution_lock);
    pvlc_hip_kv_session *s = nullptr;
    if (pvlc_hip_status st = create_session(runtime, plan, invocation->key_cache, invocation->value_cache, &s))
        return st;
    pvlc_hip_kv_step_operands step{invocation->query, invocation->query_len, invocation->appended_key,
                                  invocation->appended_key_len, invocation->appended_value,
                                  invocation->appended_value_len};
    pvlc_hip_status st = execute_step(s, &step, execution->attention, nullptr);
    if (st == PVLC_HIP_OK) st = read_planes(s, execution->key_cache, execution->value_cache);
    release_session(s, true);
    if (st != PVLC_HIP_OK) return st;
    execution->cache_tokens = sp.cache_tokens_after;
    execution->cache_capacity = plan.cache_capacity;
    execution->queue_wall_time_ns = now_ns() - started;
    return ok();
}

uint32_t pvlc_hip_paged_decode_partition(uint32_t num_seqs, uint32_t max_context) {
    return auto_partition(num_seqs, max_context);
}

uint32_t pvlc_hip_paged_decode_streaming_partition(const int32_t *cache_lens, uint32_t num_seqs, uint32_t max_context,
                                                   uint32_t compute_units) {
    if (!cache_lens || num_seqs == 0 || max_context == 0) return 0;
    const uint32_t p0 = auto_partition(num_seqs, max_context);
    // Launches with more ragged sequences than the persistent kernel numbers
    // run one workgroup per (partition, head, sequence) at the planned partition.
    if (num_seqs > kMaxRaggedSeqs) return p0;
    const uint32_t span = streaming_span(decode_shape(p0, true).waves);
    uint32_t items[kPartitionChoices] = {};
    for (uint32_t i = 0; i < num_seqs; ++i) {
        const int64_t len = cache_lens[i];
        if (len < 0 || len + 1 > static_cast<int64_t>(max_context)) continue;  // not attended by the launch
        for (int c = 0; c < kPartitionChoices; ++c) {
            const uint32_t pc = streaming_partition_candidate(p0, c, span);
            if (pc != 0) items[c] += static_cast<uint32_t>((len + pc) / pc) * kKvHeads;
        }
    }
    return choose_streaming_partition(items, p0, compute_units, span);
}

pvlc_hip_status pvlc_hip_gemv_f16(const uint16_t *weights, const float *vector, float *out, uint32_t rows,
                                  uint32_t columns, void *stream) {
    if (!weights || !vector || !out) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "GEMV buffer pointer is NULL");
    if (pvlc_hip_status st = plan_gemv_tiled(rows, columns, nullptr)) return st;
    const int e = launch_gemv_f16(weights, vector, out, rows, columns, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "GEMV launch");
    return ok();
}

pvlc_hip_status pvlc_hip_gemv_group_f16(const pvlc_hip_gemv_member *members, uint32_t count, const float *vector,
                                        uint32_t columns, void *stream) {
    if (!members || !vector) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "GEMV group members or vector pointer is NULL");
    if (count == 0 || count > kGemvGroupMax)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "a GEMV group holds 1 to 4 members, not " + std::to_string(count));
    GemvGroup g{};
    for (uint32_t i = 0; i + 1 < kGemvGroupMax; ++i) g.end[i] = 0xFFFFFFFFu;
    uint64_t total = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (!members[i].weights || !members[i].out)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "GEMV group member " + std::to_string(i) + " has a NULL pointer");
        if (members[i].rows == 0)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "GEMV group member " + std::to_string(i) + " has no rows");
        total += members[i].rows;
        if (total > 0xFFFFFFFFull) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "GEMV group rows overflow");
        g.weights[i] = members[i].weights;
        g.out[i] = members[i].out;
        if (i + 1 < count) g.end[i] = static_cast<uint32_t>(total);
    }
    g.total = static_cast<uint32_t>(total);
    // The launch is one GEMV of the members' total rows: admitted as such.
    if (pvlc_hip_status st = plan_gemv_tiled(static_cast<uint32_t>(total), columns, nullptr)) return st;
    const int e = launch_gemv_group_f16(g, vector, columns, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "grouped GEMV launch");
    return ok();
}

size_t pvlc_hip_top1_workspace_bytes(void) { return kTop1WorkspaceBytes; }

namespace {
pvlc_hip_status top1_workspace(void *workspace, size_t workspace_bytes, uint32_t *result, Top1Slot **slots) {
    if (!workspace || !result) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "top-1 workspace or result pointer is NULL");
    if (workspace_bytes < kTop1WorkspaceBytes)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "top-1 workspace holds " + std::to_string(workspace_bytes) +
                                                         " bytes but needs " + std::to_string(kTop1WorkspaceBytes));
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "top-1 workspace must be 256-byte aligned");
    *slots = static_cast<Top1Slot *>(workspace);
    return PVLC_HIP_OK;
}
}  // namespace

pvlc_hip_status pvlc_hip_logits_top1_f32(const float *logits, uint32_t vocab, uint32_t *result, void *workspace,
                                         size_t workspace_bytes, void *stream) {
    if (!logits) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "logits pointer is NULL");
    if (vocab == 0 || vocab > 0x80000000u)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "top-1 needs 1 <= vocab <= 2^31 logits");
    if (reinterpret_cast<uintptr_t>(logits) % 4 != 0)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "logits must be 4-byte aligned f32");
    Top1Slot *slots = nullptr;
    if (pvlc_hip_status st = top1_workspace(workspace, workspace_bytes, result, &slots)) return st;
    const int e = launch_logits_top1_f32(logits, vocab, slots, result, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "top-1 launch");
    return ok();
}

pvlc_hip_status pvlc_hip_lm_head_top1_f16(const uint16_t *weights, const float *hidden, float *logits, uint32_t rows,
                                          uint32_t columns, uint32_t *result, void *workspace, size_t workspace_bytes,
                                          void *stream) {
    if (!weights || !hidden) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "LM-head buffer pointer is NULL");
    if (pvlc_hip_status st = plan_gemv_tiled(rows, columns, nullptr)) return st;
    Top1Slot *slots = nullptr;
    if (pvlc_hip_status st = top1_workspace(workspace, workspace_bytes, result, &slots)) return st;
    const int e = launch_gemv_top1_f16(weights, hidden, logits, rows, columns, slots, result, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "LM-head top-1 launch");
    return ok();
}

size_t pvlc_hip_linear_projection_workspace_bytes(uint32_t rows, uint32_t input_width) {
    if (rows == 0 || input_width == 0) return 0;
    return projection_workspace_layout(rows, input_width).total;
}

pvlc_hip_status pvlc_hip_linear_projection_f16(const float *input, const uint16_t *weight, const float *bias,
                                               float *output, uint32_t rows, uint32_t input_width,
                                               uint32_t output_width, void *workspace, size_t workspace_bytes,
                                               void *stream) {
    if (!input || !weight || !bias || !output || !workspace)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "projection buffer pointer is NULL");
    const int32_t pe = plan_projection(rows, input_width, output_width, 1, nullptr);
    if (pe == PVLC_HIP_PROJ_OVERFLOW)
        return invalid(PVLC_HIP_INV_ARITHMETIC_OVERFLOW, "projection byte geometry overflowed");
    if (pe != PVLC_HIP_PROJ_OK)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "projection geometry must be positive with widths a multiple of 4");
    if (input_width % 32 != 0)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "device projection needs input_width a multiple of 32");
    // One workgroup of 256 threads per 128 x 128 output tile: the grid holds fewer than 2^32 threads.
    const uint64_t out_tiles = (static_cast<uint64_t>(rows) + 127) / 128 * ((static_cast<uint64_t>(output_width) + 127) / 128);
    if (rows > 65535u * 128u || out_tiles >= (1u << 24))
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "projection rows or output tiles exceed the grid");
    for (const void *ptr : {static_cast<const void *>(input), static_cast<const void *>(weight),
                            static_cast<const void *>(output)})
        if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "projection input, weight and output must be 16-byte aligned");
    const ProjectionWorkspaceLayout layout = projection_workspace_layout(rows, input_width);
    if (workspace_bytes < layout.total)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "projection workspace holds " + std::to_string(workspace_bytes) +
                                                         " bytes but needs " + std::to_string(layout.total));
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "projection workspace must be 256-byte aligned");
    auto *base = static_cast<unsigned char *>(workspace);
    const ProjectionWorkspace ws{reinterpret_cast<uint16_t *>(base),
                                 reinterpret_cast<int32_t *>(base + layout.exponents_offset)};
    const int e = launch_linear_projection_f16(input, weight, bias, output, rows, input_width, output_width, ws, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "projection launch");
    return ok();
}

size_t pvlc_hip_paged_decode_workspace_bytes(uint32_t num_seqs, uint32_t max_context, uint32_t partition_tokens) {
    if (num_seqs == 0 || max_context == 0) return 0;
    if (partition_tokens == 0) return decode_workspace_layout(num_seqs, auto_workspace_parts(num_seqs, max_context)).total;
    if (partition_tokens % kBlockTokens != 0) return 0;
    return decode_workspace_layout(num_seqs, (max_context + partition_tokens - 1) / partition_tokens).total;
}

pvlc_hip_status pvlc_hip_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
    if (!workspace || workspace_bytes % 4 != 0)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "workspace must be non-NULL and a multiple of 4 bytes");
    const int e = launch_fill_u32(static_cast<uint32_t *>(workspace), workspace_bytes / 4, 0u, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "workspace init");
    return ok();
}

pvlc_hip_status pvlc_hip_workspace_error(const void *workspace, size_t workspace_bytes, void *stream,
                                         uint32_t *error_out) {
    if (!workspace || !error_out || workspace_bytes < 256)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "workspace too small");
    // The error word is the first word of every decode workspace.
    hipStream_t st = static_cast<hipStream_t>(stream);
    HIP_TRY(hipMemcpyAsync(error_out, workspace, sizeof(uint32_t), hipMemcpyDeviceToHost, st), "error word readback");
    HIP_TRY(hipStreamSynchronize(st), "error word readback");
    return ok();
}

pvlc_hip_status pvlc_hip_paged_decode_f16(const pvlc_hip_paged_decode_args *args, void *stream) {
    if (pvlc_hip_status st = launch_decode_checked(args, stream)) return st;
    return ok();
}

pvlc_hip_status pvlc_hip_paged_decode_f32io(const pvlc_hip_paged_decode_args *args, const float *query,
                                            const float *new_key, const float *new_value, float *out, void *stream) {
    const DecodeOperands32 f32{query, new_key, new_value, out};
    if (pvlc_hip_status st = launch_decode_checked(args, stream, nullptr, &f32)) return st;
    return ok();
}

pvlc_hip_status pvlc_hip_kv_pack_f16(const uint16_t *key_rows, const uint16_t *value_rows, uint32_t tokens,
                                     const int32_t *block_table, uint32_t num_blocks, uint16_t *key_cache,
                                     uint16_t *value_cache, void *stream) {
    if (!key_rows || !value_rows || !key_cache || !value_cache)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "NULL buffer");
    if (tokens == 0 || num_blocks == 0) return invalid(PVLC_HIP_INV_ZERO_DIMENSION, "tokens and blocks must be nonzero");
    if (!block_table && (tokens + kBlockTokens - 1) / kBlockTokens > num_blocks)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "tokens exceed the contiguous blocks");
    const int e = launch_kv_pack(key_rows, value_rows, tokens, block_table, num_blocks, key_cache, value_cache,
                                 nullptr, stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "kv pack launch");
    return ok();
}

pvlc_hip_status pvlc_hip_kv_unpack_f16(const uint16_t *key_cache, const uint16_t *value_cache, uint32_t tokens,
                                       const int32_t *block_table, uint32_t num_blocks, uint16_t *key_rows,
                                       uint16_t *value_rows, void *stream) {
    if (!key_rows || !value_rows || !key_cache || !value_cache)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "NULL buffer");
    if (tokens == 0 || num_blocks == 0) return invalid(PVLC_HIP_INV_ZERO_DIMENSION, "tokens and blocks must be nonzero");
    if (!block_table && (tokens + kBlockTokens - 1) / kBlockTokens > num_blocks)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "tokens exceed the contiguous blocks");
    const int e = launch_kv_unpack(key_cache, value_cache, tokens, block_table, num_blocks, key_rows, value_rows,
                                   stream);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "kv unpack launch");
    return ok();
}

size_t pvlc_hip_paged_prefill_workspace_bytes(uint32_t tokens) { return prefill_workspace_layout(tokens).total; }

namespace {

// Checks and launch shared by the fp16 and f32-operand prefill entry points.
pvlc_hip_status prefill_checked(const pvlc_hip_paged_prefill_args *args, void *stream, const PrefillOperands32 *f32) {
    if (!args) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "prefill args are NULL");
    if (args->tokens == 0 || args->num_blocks == 0)
        return invalid(PVLC_HIP_INV_ZERO_DIMENSION, "tokens and blocks must be nonzero");
    if (f32) {
        if (args->query || args->key || args->value || args->out)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH,
                           "pvlc_hip_paged_prefill_f32io takes its query, key, value and output as f32 arguments; "
                           "the fp16 ones in the args must be NULL");
        if (!f32->query || !f32->key || !f32->value || !f32->out)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "prefill f32 operand pointer is NULL");
    } else if (!args->query || !args->key || !args->value || !args->out) {
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "prefill buffer pointer is NULL");
    }
    if (!args->key_cache || !args->value_cache)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "prefill buffer pointer is NULL");
    {
        // The kernels move query, key, value, output and cache rows as 16-byte vectors.
        const void *rows[] = {args->query, args->key, args->value, args->out, args->key_cache, args->value_cache,
                              args->query_scratch, f32 ? f32->query : nullptr, f32 ? f32->key : nullptr,
                              f32 ? f32->value : nullptr, f32 ? f32->out : nullptr};
        for (const void *r : rows)
            if (reinterpret_cast<uintptr_t>(r) % 16 != 0)
                return invalid(PVLC_HIP_INV_LENGTH_MISMATCH,
                               "prefill query, key, value, output, cache and scratch must be 16-byte aligned");
    }
    if ((args->rope_cos == nullptr) != (args->rope_sin == nullptr) || (args->rope_cos && args->rope_rows == 0))
        return invalid(PVLC_HIP_INV_INVALID_ROTARY_DIMENSION, "rotary tables must be given together with rows");
    if (!args->positions && args->rope_cos && args->tokens > args->rope_rows)
        return invalid(PVLC_HIP_INV_INVALID_ROTARY_DIMENSION, "rotary table shorter than the prefill");
    if (!args->block_table && (args->tokens + kBlockTokens - 1) / kBlockTokens > args->num_blocks)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, "tokens exceed the contiguous blocks");
    if (args->workspace) {
        const PrefillWorkspace ws = prefill_workspace_layout(args->tokens);
        if (args->workspace_bytes < ws.total)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "prefill workspace holds " +
                                                             std::to_string(args->workspace_bytes) +
                                                             " bytes but the split schedule needs " +
                                                             std::to_string(ws.total));
        if (reinterpret_cast<uintptr_t>(args->workspace) % 256 != 0)
            return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "prefill workspace must be 256-byte aligned");
    }
    const int e = launch_prefill(args, stream, f32);
    if (e != 0) return hip_fail(static_cast<hipError_t>(e), "prefill launch");
    return ok();
}

}  // namespace

pvlc_hip_status pvlc_hip_paged_prefill_f16(const pvlc_hip_paged_prefill_args *args, void *stream) {
    return prefill_checked(args, stream, nullptr);
}

pvlc_hip_status pvlc_hip_paged_prefill_f32io(const pvlc_hip_paged_prefill_args *args, const float *query,
                                             const float *key, const float *value, float *out, void *stream) {
    const PrefillOperands32 f32{query, key, value, out};
    return prefill_checked(args, stream, &f32);
}

}  // extern "C"
