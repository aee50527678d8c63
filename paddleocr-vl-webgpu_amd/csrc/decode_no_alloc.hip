// Paged decode without allocation: pvlc_hip_paged_decode_f16 with its split-K
// state (partials, merge counters, status words) in a file-scope device array
// instead of a caller workspace.  For callers that cannot allocate device
// memory: code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc.  The reference has no counterpart (its sessions allocate
// their split-K scratch at creation, decoder_kv_session.rs:169-173).
//
// Each GPU holds its own copy of `scratch` until the process ends.  In host
// code the array's name is only a stand-in for the symbol, never a device
// address: the address on a device comes from hipGetSymbolAddress with that
// device current, once per device, and only that address reaches kernels and
// fill launches.

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "pvlc_internal.hpp"

namespace {

using namespace pvlc;

// Bytes of split-K state per device: configs 1-3 of the benchmark plan (up to
// 64 sequences of 8192 rows, 8.6 MiB) and single sequences to the longest
// context fit; larger launches are rejected and use a workspace.
constexpr size_t kScratchBytes = size_t{16} << 20;
// Sequences (or layers) one call admits.  The merge counters sit at a fixed
// place for every call.  They start at zero (the array is static storage,
// zero when the code object is loaded) and count arrivals in generations
// (kArrivalSpan): every completed launch leaves each counter a multiple of
// the span, which is all the next launch needs, so nothing is cleared here.
// Calls that overlap on one device garble their own outputs, but once both
// have completed the counters are consistent again.
constexpr uint32_t kMaxSeqs = 4096;
constexpr size_t kStatusOffset = 0;  // [unused error word][automatic partition][compute units], 256-byte slot
// (the two status words are written by the streaming kernel before its merge
// kernel reads them, so they need no initial value)
constexpr size_t kCountersOffset = 256;
constexpr size_t kPartialsOffset = kCountersOffset + size_t{kMaxSeqs} * kKvHeads * sizeof(uint32_t);
static_assert(kPartialsOffset % 256 == 0, "partials start on a 256-byte line");

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// The device address of `scratch` per device ordinal, set up once per device.
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_scratch[kMaxDevices] = {};

// Set-up on the current device (first call there): the array's address on
// this device.  Nothing is launched or waited for, so a first call made
// while the caller's stream is being captured into a graph is captured like
// any other.
pvlc_hip_status device_scratch(char **out) {
    int device = 0;
    if (hipError_t e = hipGetDevice(&device))
        return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE, std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (device < 0 || device >= kMaxDevices)
        return fail(PVLC_HIP_DEVICE_REQUEST, PVLC_HIP_INV_NONE, "device ordinal beyond the 64 the scratch table holds");
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[device]) {
        void *ptr = nullptr;
        if (hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)))
            return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE,
                        std::string("decode scratch address: ") + hipGetErrorString(e));
        if (!ptr) return fail(PVLC_HIP_OPERATION, PVLC_HIP_INV_NONE, "decode scratch address is NULL");
        g_scratch[device] = ptr;
    }
    *out = static_cast<char *>(g_scratch[device]);
    return PVLC_HIP_OK;
}

}  // namespace

extern "C" pvlc_hip_status pvlc_hip_paged_decode_f16_no_alloc(const pvlc_hip_paged_decode_args *args,
                                                              uint32_t *error_word, void *stream) {
    uint32_t partition = 0, max_parts = 0;
    if (pvlc_hip_status st = validate_decode_geometry(args, &partition, &max_parts)) return st;
    if (args->workspace || args->workspace_bytes)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH,
                       "pvlc_hip_paged_decode_f16_no_alloc takes no workspace (workspace must be NULL and "
                       "workspace_bytes 0): its split-K state lives in the library's per-device scratch");
    if (!error_word) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "error_word is NULL");
    if (args->num_seqs > kMaxSeqs)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "pvlc_hip_paged_decode_f16_no_alloc admits at most 4096 sequences, not " +
                           std::to_string(args->num_seqs));
    const uint32_t stride = max_parts | 1u;  // odd partial slots, as the workspace layout
    const size_t units = static_cast<size_t>(args->num_seqs) * kKvHeads * stride;
    const size_t ml_offset = kPartialsOffset;
    const size_t o_offset = (ml_offset + units * 2 * kGroup * sizeof(float) + 255) & ~size_t{255};
    const size_t total = o_offset + units * kGroup * kHeadDim * sizeof(float);
    if (total > kScratchBytes)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "this decode needs " + std::to_string(total) + " bytes of split-K state, more than the " +
                           std::to_string(kScratchBytes) +
                           " bytes of scratch pvlc_hip_paged_decode_f16_no_alloc holds per device; use "
                           "pvlc_hip_paged_decode_f16 with a workspace");
    char *base = nullptr;
    if (pvlc_hip_status st = device_scratch(&base)) return st;
    const DecodeState state{reinterpret_cast<float *>(base + o_offset),
                            reinterpret_cast<float *>(base + ml_offset),
                            reinterpret_cast<uint32_t *>(base + kCountersOffset),
                            error_word,
                            reinterpret_cast<uint32_t *>(base + kStatusOffset) + 1,
                            stride};
    if (pvlc_hip_status st = launch_decode_state(args, partition, max_parts, state, stream, nullptr)) return st;
    return ok();
}
