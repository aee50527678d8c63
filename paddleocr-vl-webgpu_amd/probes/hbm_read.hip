// HBM read probe: how long one launch takes to stream a given number of
// bytes with a given grid, the floor against which the decode step (which
// reads the same bytes and also computes and merges) is judged.  Not part of
// the backend's C ABI: built into libpvlc_probes.so and loaded only by the
// benchmark's --read-floor leg.
//
// Launch: `workgroups` workgroups of WAVES waves; wave w of workgroup g reads
// the contiguous run of LOADS x 1 KiB starting at (g*WAVES + w) * LOADS KiB,
// every lane 16 bytes per load, all loads issued before the first use (the
// decode kernel's pattern: 16 loads of 1 KiB per wave in flight), with the
// same non-temporal hint.  The loaded words are folded with XOR and stored
// only if the fold equals a value the caller passes and the data never holds
// (so no load is dead), one word per wave.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int WAVES, int LOADS>
__global__ __launch_bounds__(WAVES * 64) void hbm_read_kernel(const u32x4 *src, uint32_t *sink, uint32_t never) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const size_t run = (static_cast<size_t>(blockIdx.x) * WAVES + wave) * LOADS * 64;  // in 16-byte units
    u32x4 v[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) v[i] = __builtin_nontemporal_load(src + run + i * 64 + lane);
    u32x4 x = v[0];
#pragma unroll
    for (int i = 1; i < LOADS; ++i) x ^= v[i];
    const uint32_t f = x.x ^ x.y ^ x.z ^ x.w;
    if (f == never) sink[blockIdx.x * WAVES + wave] = f;
}

}  // namespace

// Bytes one launch reads: workgroups * waves * loads KiB.  waves in {4, 8, 12,
// 16} with loads in {8, 16, 32}, or 10 waves of 16; returns 0, the launch's
// hipError_t, or -1 for another shape.
extern "C" int pvlc_probe_hbm_read(const void *src, uint32_t *sink, uint32_t workgroups, uint32_t waves,
                                   uint32_t loads, uint32_t never, void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const u32x4 *s = static_cast<const u32x4 *>(src);
    (void)hipGetLastError();  // report this launch's status only
#define PVLC_PROBE(W, L)                                                                                 \
    if (waves == (W) && loads == (L)) {                                                                  \
        hipLaunchKernelGGL((hbm_read_kernel<W, L>), dim3(workgroups), dim3((W) * 64), 0, st, s, sink, never); \
        return static_cast<int>(hipGetLastError());                                                      \
    }
    PVLC_PROBE(4, 8)
    PVLC_PROBE(4, 16)
    PVLC_PROBE(4, 32)
    PVLC_PROBE(8, 8)
    PVLC_PROBE(8, 16)
    PVLC_PROBE(8, 32)
    PVLC_PROBE(10, 16)
    PVLC_PROBE(12, 8)
    PVLC_PROBE(12, 16)
    PVLC_PROBE(12, 32)
    PVLC_PROBE(16, 8)
    PVLC_PROBE(16, 16)
#undef PVLC_PROBE
    return -1;
}
