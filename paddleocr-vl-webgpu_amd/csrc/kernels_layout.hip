// Bit-exact moves between the compact reference rows [tokens][2][128] (the
// cache planes of DecoderKvSessionDescriptor, runtime-core lib.rs:833-843) and
// the blocked device layout (see pvlc_hip.h), through a block table.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));

// One thread per (token, head, 8-dim chunk).
__global__ void kv_pack_kernel(const uint16_t *__restrict__ key_rows, const uint16_t *__restrict__ value_rows,
                               uint32_t tokens, const int32_t *__restrict__ table, uint32_t num_blocks,
                               uint16_t *__restrict__ key_cache, uint16_t *__restrict__ value_cache,
                               uint32_t *__restrict__ error_word) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * kKvHeads * (kHeadDim / 8)) return;
    const uint32_t chunk = i % (kHeadDim / 8);
    const uint32_t h = (i / (kHeadDim / 8)) % kKvHeads;
    const uint32_t t = i / (kHeadDim / 8 * kKvHeads);
    const int32_t b = table ? table[t / kBlockTokens] : static_cast<int32_t>(t / kBlockTokens);
    if (b < 0 || static_cast<uint32_t>(b) >= num_blocks) {
        if (error_word) atomicOr(error_word, 2u);
        return;
    }
    const size_t slab = (static_cast<size_t>(b) * kKvHeads + h) * kBlockHeadElems;
    const uint32_t tt = t % kBlockTokens;
    const size_t src = (static_cast<size_t>(t) * kKvHeads + h) * kHeadDim + chunk * 8;
    const u16x8_t k = *reinterpret_cast<const u16x8_t *>(key_rows + src);
    *reinterpret_cast<u16x8_t *>(key_cache + slab + chunk * 128 + key_slot(tt) * 8) = k;
    const u16x8_t v = *reinterpret_cast<const u16x8_t *>(value_rows + src);
#pragma unroll
    for (int j = 0; j < 8; ++j) value_cache[slab + (chunk * 8 + j) * kBlockTokens + tt] = v[j];
}

__global__ void kv_unpack_kernel(const uint16_t *__restrict__ key_cache, const uint16_t *__restrict__ value_cache,
                                 uint32_t tokens, const int32_t *__restrict__ table, uint32_t num_blocks,
                                 uint16_t *__restrict__ key_rows, uint16_t *__restrict__ value_rows) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * kKvHeads * (kHeadDim / 8)) return;
    const uint32_t chunk = i % (kHeadDim / 8);
    const uint32_t h = (i / (kHeadDim / 8)) % kKvHeads;
    const uint32_t t = i / (kHeadDim / 8 * kKvHeads);
    const int32_t b = table ? table[t / kBlockTokens] : static_cast<int32_t>(t / kBlockTokens);
    const size_t dst = (static_cast<size_t>(t) * kKvHeads + h) * kHeadDim + chunk * 8;
    if (b < 0 || static_cast<uint32_t>(b) >= num_blocks) {
        *reinterpret_cast<u16x8_t *>(key_rows + dst) = u16x8_t{};
        *reinterpret_cast<u16x8_t *>(value_rows + dst) = u16x8_t{};
        return;
    }
    const size_t slab = (static_cast<size_t>(b) * kKvHeads + h) * kBlockHeadElems;
    const uint32_t tt = t % kBlockTokens;
    *reinterpret_cast<u16x8_t *>(key_rows + dst) =
        *reinterpret_cast<const u16x8_t *>(key_cache + slab + chunk * 128 + key_slot(tt) * 8);
    u16x8_t v;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = value_cache[slab + (chunk * 8 + j) * kBlockTokens + tt];
    *reinterpret_cast<u16x8_t *>(value_rows + dst) = v;
}

}  // namespace

int launch_kv_pack(const uint16_t *key_rows, const uint16_t *value_rows, uint32_t tokens, const int32_t *table,
                   uint32_t num_blocks, uint16_t *key_cache, uint16_t *value_cache, uint32_t *error_word,
                   void *stream) {
    const uint32_t work = tokens * kKvHeads * (kHeadDim / 8);
    if (work == 0) return 0;
    hipLaunchKernelGGL(kv_pack_kernel, dim3((work + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                       key_rows, value_rows, tokens, table, num_blocks, key_cache, value_cache, error_word);
    return static_cast<int>(hipGetLastError());
}

int launch_kv_unpack(const uint16_t *key_cache, const uint16_t *value_cache, uint32_t tokens, const int32_t *table,
                     uint32_t num_blocks, uint16_t *key_rows, uint16_t *value_rows, void *stream) {
    const uint32_t work = tokens * kKvHeads * (kHeadDim / 8);
    if (work == 0) return 0;
    hipLaunchKernelGGL(kv_unpack_kernel, dim3((work + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                       key_cache, value_cache, tokens, table, num_blocks, key_rows, value_rows);
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
