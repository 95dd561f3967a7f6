// The fused front for fp32 (and fp16) callers: x, weights, norm weights and
// RoPE tables in that type, q / k / v out in it.  The reference op accepts such
// tensors too (mini_qwen/kernels/fused_qkv_rope.py:130-195; the fp32 layer of the
// reference's CPU-runnable configuration), but its Triton kernel rounds every Q /
// K output to bf16 before storing it into the fp32 / fp16 buffer (:117-120), and
// with fp16 tensors its GEMM output is rounded to fp16 before the norm.  This
// kernel keeps the fp32 projection, norm and RoPE and rounds once, to the output
// type: it computes the op's fp32 composition (the unfused reference path,
// attention.py:102-109) to fp32 / fp16 precision, not the fused reference's bits.
//
// One workgroup of four waves computes 32 (or 16) token rows x one head (128
// columns): each wave owns 32 columns and runs the fp32 matrix core (products
// and sums in fp32) over k tiles of 32 staged in LDS, the next tile's loads in
// registers under the current tile's MFMAs.
// The accumulators then go through LDS so that eight threads hold a row's
// 128 dims (each the RoPE pairs d, d+64 for eight d), apply RMSNorm and RoPE
// in fp32, and store.  fp16 tiles stay fp16 in LDS and run on the fp16 matrix
// cores (exact products, fp32 sums).
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

constexpr int kKT = kF32BK;
constexpr int kPitch = kKT + 1;          // LDS row pitch of the staged tiles (odd: no bank conflicts)
constexpr int kEpiPitch = kHeadDim + 4;  // LDS row pitch of the accumulator tile
constexpr int kHPitch = kKT + 4;         // LDS row pitch (halves) of the fp16 staged tiles
constexpr int kThreads = 256;
static_assert(kHeadDim * kPitch >= 32 * kEpiPitch, "the accumulator tile reuses the weight tile's LDS");

// ROWS = 32: each wave runs v_mfma_f32_32x32x2_f32 on its 32 x 32 block.
// ROWS = 16 (launches whose 32-row tiles would leave CUs idle): each wave runs
// v_mfma_f32_16x16x4_f32 on two 16 x 16 blocks.
// Element type T: float, or _Float16 (the norm weights and RoPE tables are
// read as fp32; fp16 tiles go to the fp16 matrix cores, see the kernel).
template <class T>
__device__ __forceinline__ float elem(const void* p, int64_t i) {
  return float(static_cast<const T*>(p)[i]);
}
// 4 consecutive elements as fp32 (16-byte or 8-byte loads)
template <class T>
__device__ __forceinline__ f32x4_t load4(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const f32x4_t*>(p);
  } else {
    typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
    const h4_t h = *reinterpret_cast<const h4_t*>(p);
    return f32x4_t{float(h.x), float(h.y), float(h.z), float(h.w)};
  }
}
// 8 values stored as 8 consecutive elements
template <class T>
__device__ __forceinline__ void store8(void* dst, const float (&v)[8], int i0) {
  if constexpr (sizeof(T) == 4) {
    float* d = static_cast<float*>(dst);
    *reinterpret_cast<f32x4_t*>(d) = f32x4_t{v[i0], v[i0 + 1], v[i0 + 2], v[i0 + 3]};
    *reinterpret_cast<f32x4_t*>(d + 4) = f32x4_t{v[i0 + 4], v[i0 + 5], v[i0 + 6], v[i0 + 7]};
  } else {
    typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
    h8_t h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = _Float16(v[i0 + i]);
    *static_cast<h8_t*>(dst) = h;
  }
}

template <int ROWS, class T>
__global__ void __launch_bounds__(kThreads) f32_qkv_kernel(F32Args a, int xcds) {
  static_assert(ROWS == 16 || ROWS == 32, "row tile");
  __shared__ float xs[ROWS * kPitch];
  __shared__ float ws[kHeadDim * kPitch];
  const int n_rt = int((a.M + ROWS - 1) / ROWS);
  const int tile = xcd_tile_id(int(blockIdx.x), int(gridDim.x), xcds);
  const int rt = tile % n_rt;
  const int h = tile / n_rt;
  int proj, hh;
  split_head(h, a.Hq, a.Hkv, proj, hh);
  const T* W = static_cast<const T*>(a.w[proj]) + int64_t(hh) * kHeadDim * a.K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = int64_t(rt) * ROWS;

  // staging: thread tid loads 4 consecutive k of x row (tid / 8) (threads of
  // rows < ROWS) and of weight rows (tid / 8) + 32 j, j = 0..3
  const int sr = tid >> 3, sk = (tid & 7) * 4;
  const bool x_row = sr < ROWS;
  const bool x_in = x_row && row0 + sr < a.M;
  const T* xp = static_cast<const T*>(a.x) + (x_in ? (row0 + sr) * a.K : 0) + sk;
  const T* wp = W + int64_t(sr) * a.K + sk;
  f32x4_t xr, wr[4];
  auto load = [&](int64_t k0) {
    xr = x_in ? load4<T>(xp + k0) : f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) wr[j] = load4<T>(wp + int64_t(32 * j) * a.K + k0);
  };
  auto stage = [&]() {
    if (x_row) {
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[sr * kPitch + sk + i] = xr[i];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) ws[(sr + 32 * j) * kPitch + sk + i] = wr[j][i];
  };

  float* ep = ws;  // (after the k loop) the accumulator tile [ROWS][kEpiPitch]
  if constexpr (sizeof(T) == 2) {
    // fp16: the tiles stay fp16 in LDS (row pitch kHPitch halves: 8-byte reads
    // free of bank conflicts) and run on the fp16 matrix cores, whose products
    // are exact and sums fp32
    typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
    _Float16* xh = reinterpret_cast<_Float16*>(xs);
    _Float16* wh = reinterpret_cast<_Float16*>(ws);
    h4_t xr4, wr4[4];
    auto hload = [&](int64_t k0) {
      xr4 = x_in ? *reinterpret_cast<const h4_t*>(xp + k0) : h4_t{};
#pragma unroll
      for (int j = 0; j < 4; ++j) wr4[j] = *reinterpret_cast<const h4_t*>(wp + int64_t(32 * j) * a.K + k0);
    };
    auto hstage = [&]() {
      if (x_row) *reinterpret_cast<h4_t*>(xh + sr * kHPitch + sk) = xr4;
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<h4_t*>(wh + (sr + 32 * j) * kHPitch + sk) = wr4[j];
    };
    if constexpr (ROWS == 32) {
      f32x16_t acc;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.f;
      // lane l: x row (l & 31), weight row 32 * wave + (l & 31), k 4 (l >> 5) .. +4 of each 8
      const _Float16* xa = xh + (lane & 31) * kHPitch + 4 * (lane >> 5);
      const _Float16* wb = wh + (32 * wave + (lane & 31)) * kHPitch + 4 * (lane >> 5);
      hload(0);
      for (int64_t k0 = 0; k0 < a.K; k0 += kKT) {
        hstage();
        __syncthreads();
        if (k0 + kKT < a.K) hload(k0 + kKT);
#pragma unroll
        for (int kk = 0; kk < kKT / 8; ++kk)
          acc = __builtin_amdgcn_mfma_f32_32x32x8f16(*reinterpret_cast<const h4_t*>(xa + 8 * kk),
                                                      *reinterpret_cast<const h4_t*>(wb + 8 * kk), acc, 0, 0, 0);
        __syncthreads();
      }
#pragma unroll
      for (int i = 0; i < 16; ++i)
        ep[(8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) * kEpiPitch + 32 * wave + (lane & 31)] = acc[i];
    } else {
      f32x4_t acc[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      // lane l: x row (l & 15), weight rows 32 * wave + 16 b + (l & 15), k 4 (l >> 4) .. +4 of each 16
      const _Float16* xa = xh + (lane & 15) * kHPitch + 4 * (lane >> 4);
      const _Float16* wb = wh + (32 * wave + (lane & 15)) * kHPitch + 4 * (lane >> 4);
      hload(0);
      for (int64_t k0 = 0; k0 < a.K; k0 += kKT) {
        hstage();
        __syncthreads();
        if (k0 + kKT < a.K) hload(k0 + kKT);
#pragma unroll
        for (int kk = 0; kk < kKT / 16; ++kk)
#pragma unroll
          for (int b = 0; b < 2; ++b)
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(
                *reinterpret_cast<const h4_t*>(xa + 16 * kk),
                *reinterpret_cast<const h4_t*>(wb + 16 * b * kHPitch + 16 * kk), acc[b], 0, 0, 0);
        __syncthreads();
      }
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          ep[(4 * (lane >> 4) + j) * kEpiPitch + 32 * wave + 16 * b + (lane & 15)] = acc[b][j];
    }
  } else if constexpr (ROWS == 32) {
    f32x16_t acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    // lane l multiplies x row (l & 31) with weight row 32 * wave + (l & 31), at k
    // slot (l >> 5) of each pair of k
    const float* xa = xs + (lane & 31) * kPitch + (lane >> 5);
    const float* wb = ws + (32 * wave + (lane & 31)) * kPitch + (lane >> 5);
    load(0);
    for (int64_t k0 = 0; k0 < a.K; k0 += kKT) {
      stage();
      __syncthreads();
      if (k0 + kKT < a.K) load(k0 + kKT);
#pragma unroll
      for (int kk = 0; kk < kKT / 2; ++kk)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(xa[2 * kk], wb[2 * kk], acc, 0, 0, 0);
      __syncthreads();
    }
    // accumulators -> LDS: acc[i] = C[8 * (i / 4) + 4 * (l >> 5) + i % 4][l & 31]
#pragma unroll
    for (int i = 0; i < 16; ++i)
      ep[(8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) * kEpiPitch + 32 * wave + (lane & 31)] = acc[i];
  } else {
    f32x4_t acc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // lane l multiplies x row (l & 15) with weight rows 32 * wave + 16 b + (l & 15),
    // at k slot (l >> 4) of each group of four k
    const float* xa = xs + (lane & 15) * kPitch + (lane >> 4);
    const float* wb = ws + (32 * wave + (lane & 15)) * kPitch + (lane >> 4);
    load(0);
    for (int64_t k0 = 0; k0 < a.K; k0 += kKT) {
      stage();
      __syncthreads();
      if (k0 + kKT < a.K) load(k0 + kKT);
#pragma unroll
      for (int kk = 0; kk < kKT / 4; ++kk)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[4 * kk], wb[16 * b * kPitch + 4 * kk], acc[b], 0, 0, 0);
      __syncthreads();
    }
    // accumulators -> LDS: acc[b][j] = C[4 * (l >> 4) + j][16 b + (l & 15)]
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ep[(4 * (lane >> 4) + j) * kEpiPitch + 32 * wave + 16 * b + (lane & 15)] = acc[b][j];
  }
  __syncthreads();

  // thread tid: row r = tid / 8, dims d = 8c .. 8c+7 and 64 + 8c .. (c = tid % 8);
  // with 16-row tiles only the first two waves hold rows
  const int r = tid >> 3, c = tid & 7;
  if (r >= ROWS) return;
  const int64_t t = row0 + r;
  const int hd = a.head_dim;
  const PairRuns pr = pair_runs(c, hd);  // (head_dim 64: two heads per block)
  float lo[8], hi[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    lo[i] = ep[r * kEpiPitch + pr.col_lo + i];
    hi[i] = ep[r * kEpiPitch + pr.col_hi + i];
  }
  if (proj < 2) {
    // (every lane of the row's lane group takes part in the sum; rows past M hold zeros)
    const float ss = head_sum(run_sumsq(lo, hi), hd);
    const float rms = head_rms(ss, a.eps, hd);
    if (t < a.M) {
      const void* g = proj == 0 ? a.q_gamma : a.k_gamma;
      const int64_t prow = rope_row(a, t) * hd;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma clang fp contract(off)
        const int d = pr.dim_lo + i, d2 = pr.dim_hi + i;
        const float x1n = lo[i] * rms * elem<T>(g, d);
        const float x2n = hi[i] * rms * elem<T>(g, d2);
        lo[i] = __builtin_fmaf(x1n, elem<T>(a.cos, prow + d), -(x2n * elem<T>(a.sin, prow + d)));
        hi[i] = __builtin_fmaf(x2n, elem<T>(a.cos, prow + d2), x1n * elem<T>(a.sin, prow + d2));
      }
    }
  }
  if (t < a.M) {
    const int H = proj == 0 ? a.Hq : a.Hkv;
    T* dst = static_cast<T*>(pick3(proj, a.q, a.k, a.v)) + (t * H + hh) * kHeadDim;
    store8<T>(dst + pr.col_lo, lo, 0);
    store8<T>(dst + pr.col_hi, hi, 0);
  }
}

}  // namespace

hipError_t launch_f32_qkv(const F32Args& a, int rows, bool half, int xcds, hipStream_t stream) {
  if (rows != 16 && rows != 32) return hipErrorInvalidValue;
  const int64_t n_rt = (a.M + rows - 1) / rows;
  const int64_t blocks = n_rt * (a.Hq + 2 * a.Hkv);
  if (a.K % kKT != 0 || blocks <= 0 || blocks > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;
  using Kernel = void (*)(F32Args, int);
  const Kernel k = rows == 16 ? (half ? f32_qkv_kernel<16, _Float16> : f32_qkv_kernel<16, float>)
                              : (half ? f32_qkv_kernel<32, _Float16> : f32_qkv_kernel<32, float>);
  hipLaunchKernelGGL(k, dim3(unsigned(blocks)), dim3(kThreads), 0, stream, a, xcds);
  return hipGetLastError();
}

}  // namespace mqk
