// Measurement probes (not on the op's path).
//
// HBM read-rate probe: reads `bytes`
// once with 16-byte loads spread over every CU and writes one word per
// workgroup, so that bench.py can time a plain stream of a decode step's weight
// bytes next to the decode kernel that streams them.
//
// Workgroup b of G reads the contiguous chunk [b * bytes / G, (b+1) * bytes / G)
// with `lookahead` 16-byte loads per thread in flight (non-temporal, as the
// decode kernel's weight loads), xors what it read and stores the word, so
// nothing can be skipped.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

constexpr int kProbeThreads = 512;
constexpr int kProbeUnroll = 8;

__global__ void __launch_bounds__(kProbeThreads) read_probe_kernel(const u32x4_t* __restrict__ src, int64_t n16,
                                                                   uint32_t* __restrict__ out) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = int64_t(blockIdx.x) * per;
  const int64_t b1 = b0 + per < n16 ? b0 + per : n16;
  uint32_t acc = 0;
  for (int64_t i0 = b0 + threadIdx.x; i0 < b1; i0 += int64_t(kProbeThreads) * kProbeUnroll) {
    u32x4_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const int64_t i = i0 + int64_t(u) * kProbeThreads;
      v[u] = i < b1 ? __builtin_nontemporal_load(src + i) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  __shared__ uint32_t red[kProbeThreads / 64];
  for (int m = 32; m >= 1; m >>= 1) acc ^= uint32_t(__shfl_xor(int(acc), m));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int w = 0; w < kProbeThreads / 64; ++w) r ^= red[w];
    out[blockIdx.x] = r;
  }
}

// Shader clock probe: one lane runs a dependent FMA chain of `spins` steps and
// reads the shader clock counter (s_memtime) and the constant 100 MHz counter
// (s_memrealtime) around it, so the host gets the clock the GPU ran at right then:
// out[0] = shader clocks, out[1] = 100 MHz ticks, out[2] = the chain's result.
__global__ void clock_probe_kernel(uint64_t* __restrict__ out, int spins) {
  if (threadIdx.x != 0) return;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  float v = float(spins);
  for (int i = 0; i < spins; ++i) v = __builtin_fmaf(v, 0.999f, 1.0f);
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  out[0] = t1 - t0;
  out[1] = r1 - r0;
  out[2] = uint64_t(__float_as_uint(v));
}

}  // namespace

hipError_t launch_clock_probe(uint64_t* out, int spins, hipStream_t stream) {
  if (!out || spins < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, stream, out, spins);
  return hipGetLastError();
}

hipError_t launch_read_probe(const void* src, size_t bytes, int blocks, uint32_t* out, hipStream_t stream) {
  if (!src || !out || bytes % 16 != 0 || blocks < 1 || (reinterpret_cast<uintptr_t>(src) & 15u) != 0)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(kProbeThreads), 0, stream,
                     static_cast<const u32x4_t*>(src), int64_t(bytes / 16), out);
  return hipGetLastError();
}

}  // namespace mqk
