// Standalone QK-Norm + RoPE on already-projected q/k (bf16 in, bf16 out): the
// functional twin of the reference's _qk_norm_rope_kernel
// (mini_qwen/kernels/fused_qkv_rope.py:46-127).  One wave per (token, 128-column
// block): with head_dim 128 lane l owns the RoPE pair (l, l+64), with head_dim 64
// lanes 32h + j own the pair (j, j+32) of the block's head h, so the rotation is
// lane-local and the sum of squares is one 64- or 32-lane butterfly.  Used by the
// unfused paths (already-projected activations); the fused kernels carry their
// own register epilogue.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

constexpr int kNrWaves = 4;

__global__ void __launch_bounds__(kNrWaves * 64)
norm_rope_kernel(const uint16_t* __restrict__ q_raw, const uint16_t* __restrict__ k_raw,
                 EpilogueArgs e, int64_t T) {
  const int lane = threadIdx.x & 63;
  const int heads = e.Hq + e.Hkv;  // 128-column blocks
  const int64_t item = int64_t(blockIdx.x) * kNrWaves + (threadIdx.x >> 6);
  if (item >= T * heads) return;
  const int64_t t = item / heads;
  const int h = int(item - t * heads);
  const bool is_q = h < e.Hq;
  const int hh = is_q ? h : h - e.Hq;
  const int H = is_q ? e.Hq : e.Hkv;
  const uint16_t* src = (is_q ? q_raw : k_raw) + (t * H + hh) * kHeadDim;
  uint16_t* dst = (is_q ? e.q : e.k) + (t * H + hh) * kHeadDim;
  const uint16_t* gamma = is_q ? e.q_gamma : e.k_gamma;
  // head_dim 128: lane l owns the pair (l, l+64) of the block's head; head_dim 64:
  // lanes 32h .. 32h+31 own the pairs (j, j+32) of head h of the block (j = l % 32)
  const int hd = e.head_dim, hd2 = hd / 2;
  const int d = hd == 64 ? (lane & 31) : lane;
  const int col = hd == 64 ? (lane >> 5) * 64 + d : d;

  const float x1 = bf16_to_f32(src[col]);
  const float x2 = bf16_to_f32(src[col + hd2]);
  float ss = x1 * x1 + x2 * x2;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1)
    if (m < hd2 || hd != 64) ss += __shfl_xor(ss, m);
  const float rms = rsqrtf(ss * (hd == 64 ? 1.0f / 64.0f : 1.0f / float(kHeadDim)) + e.eps);
  const float x1n = x1 * rms * bf16_to_f32(gamma[d]);
  const float x2n = x2 * rms * bf16_to_f32(gamma[d + hd2]);
  const int64_t prow = rope_row(e, t) * hd;
  const float c1 = bf16_to_f32(e.cos[prow + d]);
  const float c2 = bf16_to_f32(e.cos[prow + d + hd2]);
  const float s1 = bf16_to_f32(e.sin[prow + d]);
  const float s2 = bf16_to_f32(e.sin[prow + d + hd2]);
  // in-place safe: every lane has read its inputs before the butterfly completes
  dst[col] = f32_to_bf16(x1n * c1 - x2n * s1);
  dst[col + hd2] = f32_to_bf16(x2n * c2 + x1n * s2);
}

// Any head_dim D that is a multiple of 8 up to kAnyMaxD (the op's generic path for
// head sizes its fused kernels do not tile: the projections run as plain GEMMs
// into q / k / v, then this kernel normalises and rotates q and k in place and,
// with a paged cache, writes the k and v rows into it).  One wave per (token,
// head) over the Hq + 2 * Hkv heads: lane l owns the RoPE pairs (d, d + D/2) for
// d = l + 64 i, so the rotation is lane-local and the sum of squares is one
// 64-lane butterfly.  V heads only copy their row into the cache.
constexpr int kAnyMaxD = 512;

__global__ void __launch_bounds__(kNrWaves * 64)
norm_rope_any_kernel(EpilogueArgs e, int64_t T) {
  const int lane = threadIdx.x & 63;
  const int heads = e.Hq + 2 * e.Hkv;
  const int64_t item = int64_t(blockIdx.x) * kNrWaves + (threadIdx.x >> 6);
  if (item >= T * heads) return;
  const int64_t t = item / heads;
  const int h = int(item - t * heads);
  const int proj = h < e.Hq ? 0 : (h < e.Hq + e.Hkv ? 1 : 2);
  const int hh = proj == 0 ? h : (proj == 1 ? h - e.Hq : h - e.Hq - e.Hkv);
  const int H = proj == 0 ? e.Hq : e.Hkv;
  const int hd = e.head_dim, hd2 = hd / 2;
  const int64_t slot = proj != 0 ? paged_slot(e, t) : -1;
  uint16_t* crow = nullptr;  // this head's row in the paged cache (k or v), if any
  // (arithmetic selects of argument fields: a select of their addresses would copy
  // the argument struct to scratch memory)
  if (slot >= 0) crow = pick3<uint16_t>(proj, nullptr, e.k_cache, e.v_cache) + (slot * e.Hkv + hh) * hd;
  uint16_t* row = pick3<uint16_t>(proj, e.q, e.k, e.v) + (t * H + hh) * hd;
  if (proj == 2) {  // V: the projection as it is, into the cache
    if (crow)
      for (int d = lane; d < hd; d += 64) crow[d] = row[d];
    return;
  }
  const uint16_t* gamma = pick3<const uint16_t>(proj, e.q_gamma, e.k_gamma, e.k_gamma);
  constexpr int kPer = kAnyMaxD / 128;  // pairs per lane at most
  float x1[kPer], x2[kPer];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = lane + 64 * i;
    x1[i] = d < hd2 ? bf16_to_f32(row[d]) : 0.f;
    x2[i] = d < hd2 ? bf16_to_f32(row[d + hd2]) : 0.f;
    ss += x1[i] * x1[i] + x2[i] * x2[i];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
  const float rms = rsqrtf(ss / float(hd) + e.eps);
  const int64_t prow = rope_row(e, t) * hd;
  // in place: every lane has read its inputs before the butterfly completes
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = lane + 64 * i;
    if (d < hd2) {
      const float x1n = x1[i] * rms * bf16_to_f32(gamma[d]);
      const float x2n = x2[i] * rms * bf16_to_f32(gamma[d + hd2]);
      const float c1 = bf16_to_f32(e.cos[prow + d]), c2 = bf16_to_f32(e.cos[prow + d + hd2]);
      const float s1 = bf16_to_f32(e.sin[prow + d]), s2 = bf16_to_f32(e.sin[prow + d + hd2]);
      const uint16_t o1 = f32_to_bf16(x1n * c1 - x2n * s1), o2 = f32_to_bf16(x2n * c2 + x1n * s2);
      row[d] = o1;
      row[d + hd2] = o2;
      if (crow) {
        crow[d] = o1;
        crow[d + hd2] = o2;
      }
    }
  }
}

}  // namespace

hipError_t launch_norm_rope_any(const EpilogueArgs& e, int64_t T, hipStream_t stream) {
  if (e.head_dim <= 0 || e.head_dim % 8 != 0 || e.head_dim > kAnyMaxD) return hipErrorInvalidValue;
  const int64_t items = T * (e.Hq + 2 * e.Hkv);
  const int64_t blocks = (items + kNrWaves - 1) / kNrWaves;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL(norm_rope_any_kernel, dim3(unsigned(blocks)), dim3(kNrWaves * 64), 0, stream, e, T);
  return hipGetLastError();
}

hipError_t launch_norm_rope(const uint16_t* q_raw, const uint16_t* k_raw, const EpilogueArgs& e,
                            int64_t T, hipStream_t stream) {
  const int64_t items = T * (e.Hq + e.Hkv);
  const int64_t blocks = (items + kNrWaves - 1) / kNrWaves;
  hipLaunchKernelGGL(norm_rope_kernel, dim3(unsigned(blocks)), dim3(kNrWaves * 64), 0, stream,
                     q_raw, k_raw, e, T);
  return hipGetLastError();
}

}  // namespace mqk
