// Pre-pass of the fused input RMSNorm: the per-token scale
// rsqrt(mean(x^2) + eps) of the decoder's input_layernorm
// (mini_qwen/model/layers/rms_norm.py:15-17), written to the workspace.  The
// projection kernels then apply bf16(gamma * bf16(x * scale)) to their
// activation tiles as they stage them (input_norm8), so the normalised
// activations are never written to HBM.
//
// One wave per token row: 16-byte loads, all of a row's loads in flight at
// once (hidden <= 8192: 8 per lane), fp32 sum of squares, 64-lane butterfly.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

constexpr int kRowsPerBlock = 4;

__global__ void __launch_bounds__(kRowsPerBlock * 64)
row_scale_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K, float eps, float* __restrict__ scale) {
  const int64_t row = int64_t(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= M) return;
  const int lane = threadIdx.x & 63;
  const u32x4_t* src = reinterpret_cast<const u32x4_t*>(x + row * K);
  const int64_t chunks = K / 8;
  float ss = 0.f;
  for (int64_t c0 = 0; c0 < chunks; c0 += 64 * 8) {
    u32x4_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t c = c0 + i * 64 + lane;
      v[i] = c < chunks ? src[c] : u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = bf16_to_f32(v[i][j] & 0xFFFFu), b = bf16_to_f32(v[i][j] >> 16);
        ss += a * a + b * b;
      }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  if (lane == 0) scale[row] = rsqrtf(ss / float(K) + eps);
}

}  // namespace

hipError_t launch_row_scale(const uint16_t* x, int64_t M, int64_t K, float eps, float* scale,
                            hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  const dim3 grid(unsigned((M + kRowsPerBlock - 1) / kRowsPerBlock));
  hipLaunchKernelGGL(row_scale_kernel, grid, dim3(kRowsPerBlock * 64), 0, stream, x, M, K, eps, scale);
  return hipGetLastError();
}

}  // namespace mqk
