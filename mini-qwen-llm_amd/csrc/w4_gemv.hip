// W4A16 GEMM for small M (the decode regime: M <= 16 rows of x), column-parallel
// with no partial exchange between workgroups.
//
//   out[M, N] = x[M, K] @ W,  W[k, n] = (q[k, n] - z[k / group, n]) * s[k / group, n]
//
// with the reference's packed layout (mini_qwen/kernels/w4a16_gemm.py:8-15):
// qweight [K/8, N] int32 (nibble e of word [j, n] is q[8j + e, n]), scales
// [K/group, N] (bf16 or fp16), qzeros [K/group, N/8] int32 (nibble e of word
// [g, i] is z[g, 8i + e]).  The reference's M = 1 GEMV (w4a16_gemm.py:110-189)
// and its tiled kernel both dequantise in fp32 and accumulate in fp32; so does
// this kernel: the weight (q - z) * s is exact in fp32 (a 16-bit scale times
// integers of at most 4 bits), every product and sum is an fp32 FMA, and the
// output is rounded once to bf16.
//
// Three kernels, chosen by M and the operands (launch_w4_gemv), every one with
// one 16-column output slab per workgroup (N = 4096: 256 workgroups, one per
// CU), no partial exchange between workgroups and nothing written but the
// output: no workspace, no second kernel.
//   * w4_gemv_kernel (M <= 2): fp32 FMAs on the vector ALUs.  Thread (g, r) takes
//     columns 4g .. 4g+3 over the r-th of 64 contiguous ranges of packed rows.
//   * w4_gemv_lds_kernel (M > 2, aligned operands, N % 16 == 0, LDS permitting):
//     every operand staged in LDS with 16-byte direct loads, then the fp32
//     matrix cores (v_mfma_f32_16x16x4_f32).
//   * w4_gemv_mfma_kernel (M > 2 otherwise): the same multiplies with operands
//     read from global memory in batches of 16 packed rows.
// Partial sums over k ranges are added in a fixed order (butterflies and wave
// order), so results do not depend on scheduling.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

constexpr int kGroups = 4;               // groups of 4 columns per workgroup
constexpr int kCols = 4 * kGroups;      // output columns per workgroup
constexpr int kRanges = 64;             // packed-row ranges per column
constexpr int kThreads = kGroups * kRanges;
constexpr int kWaves = kThreads / 64;
extern __shared__ __attribute__((aligned(16))) unsigned char g_gemv_x[];

// MM: rows of x held per thread (M rounded up to 1 or 2).
template <int MM>
__global__ void __launch_bounds__(kThreads)
w4_gemv_kernel(const uint16_t* __restrict__ x, const int32_t* __restrict__ qw, const uint16_t* __restrict__ sc,
               const int32_t* __restrict__ qz, int M, int64_t K, int64_t N, int group, int scale_fp16,
               uint16_t* __restrict__ out) {
  __shared__ float red[kWaves][MM][kCols];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int grp = tid % kGroups, r = tid / kGroups;
  const int64_t col0 = int64_t(blockIdx.x) * kCols + 4 * grp;  // N % 8 == 0: four columns are all in or all out
  const int64_t cc = col0 < N ? col0 : N - 4;  // (groups past N read the last four columns; never stored)
  const int64_t rows = K / 8;
  const int64_t per = (rows + kRanges - 1) / kRanges;
  const int64_t j0 = int64_t(r) * per;
  const int64_t j1 = j0 + per < rows ? j0 + per : rows;
  const int zshift = int(cc % 8) * 4;  // 0 or 16: the four columns' nibbles of their zero word

  float acc[MM][4];
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[m][c] = 0.f;
  // quantisation group of row j, tracked without a division per row (group % 8 == 0)
  const int64_t rpg = group / 8;
  int64_t g = j0 / rpg, gnext = (g + 1) * rpg;
#pragma unroll 2
  for (int64_t j = j0; j < j1; ++j) {
    if (j == gnext) {
      ++g;
      gnext += rpg;
    }
    const uint32_t zw = uint32_t(qz[g * (N / 8) + cc / 8]) >> zshift;
    float wv[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t word = uint32_t(qw[j * N + cc + c]);
      const uint32_t sraw = sc[g * N + cc + c];
      const float scale = scale_fp16 ? f16_to_f32(sraw) : bf16_to_f32(sraw);
      // (q - z) * s exactly: q * s and z * s have at most 15 significant bits
      const float zs = float((zw >> (4 * c)) & 0xFu) * scale;
#pragma unroll
      for (int e = 0; e < 8; ++e) wv[c][e] = __builtin_fmaf(float((word >> (4 * e)) & 0xFu), scale, -zs);
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      if (m < M) {
        const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(x + int64_t(m) * K + 8 * j);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float xe = bf16_to_f32((xv[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[m][c] = __builtin_fmaf(wv[c][e], xe, acc[m][c]);
        }
      }
    }
  }
  // sum over the wave's 16 ranges (lane bits 2..5), a fixed butterfly, then over
  // the waves in order
#pragma unroll
  for (int m = 0; m < MM; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float v = acc[m][c];
#pragma unroll
      for (int b = 4; b < 64; b <<= 1) v += __shfl_xor(v, b);
      acc[m][c] = v;
    }
  if (lane < kGroups) {
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) red[wave][m][4 * lane + c] = acc[m][c];
  }
  __syncthreads();
  if (tid < MM * kCols) {
    const int m = tid / kCols, c2 = tid % kCols;
    const int64_t col = int64_t(blockIdx.x) * kCols + c2;
    if (m < M && col < N) {
      float v = red[0][m][c2];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) v += red[w][m][c2];
      out[int64_t(m) * N + col] = f32_to_bf16(v);
    }
  }
}

// The same product on the fp32 matrix cores, for 4 < M <= 16 (x rows past M are
// zero).  v_mfma_f32_16x16x4_f32 multiplies x rows 0..15 by 16 columns, 4 k per
// instruction: lane l supplies A[l % 16][kq] = x[l % 16][k] and B[kq][l % 16] =
// W[k][col] with kq = l / 16, and holds D[4 kq + r][l % 16] (r = 0..3).  The k
// slot order inside an instruction is free as long as A and B agree: row j of
// the packed weights is taken as two instructions, lane kq supplying k = 8j + 2kq
// and 8j + 2kq + 1, so each lane reads one dword of x (two bf16) and dequantises
// two nibbles of one packed word per row.  Products of a bf16 x and the exact
// fp32 weight (at most 8 + 15 significant bits) are exact in fp32, and the matrix
// core sums them in fp32, so the numerics are those of the FMA kernel above up
// to summation order.  x is staged in LDS as in the FMA kernel.  Grid: one
// 512-thread workgroup per 16 columns; wave w
// takes the w-th eighth of the packed rows, issuing the loads of 16 rows before
// their multiplies, and the eight partial tiles are added in wave order through
// LDS.
constexpr int kMfmaWaves = 8;    // waves per workgroup of the matrix-core kernel
constexpr int kMfmaBatch = 16;   // packed rows whose loads a wave issues before multiplying

__global__ void __launch_bounds__(kMfmaWaves * 64)
w4_gemv_mfma_kernel(const uint16_t* __restrict__ x, const int32_t* __restrict__ qw, const uint16_t* __restrict__ sc,
                    const int32_t* __restrict__ qz, int M, int64_t K, int64_t N, int group, int scale_fp16,
                    uint16_t* __restrict__ out) {
  __shared__ f32x4_t red[kMfmaWaves][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 15, kq = lane >> 4;
  const int64_t col = int64_t(blockIdx.x) * 16 + n;
  const int64_t cc = col < N ? col : N - 1;  // (columns past N read column N - 1; never stored)
  const int m = lane & 15;
  const bool xrow = m < M;
  const int64_t rows = K / 8;
  const int64_t per = (rows + kMfmaWaves - 1) / kMfmaWaves;
  const int64_t j0 = int64_t(wave) * per;
  const int64_t j1 = j0 + per < rows ? j0 + per : rows;
  const int zshift = int(cc % 8) * 4;
  // quantisation group of each row: a batch of 16 rows spans at most three
  // groups of >= 8 rows (group % 64 == 0), so no division per row
  const int64_t rpg = group / 8;
  const int64_t ngroups = K / group;
  uint32_t wq[kMfmaBatch], sr[3], zq[3];
  int64_t g0 = 0, gb1 = 0, gb2 = 0;
  auto load_batch = [&](int64_t jb) {
    g0 = jb / rpg;
    gb1 = (g0 + 1) * rpg;
    gb2 = gb1 + rpg;
#pragma unroll
    for (int b = 0; b < kMfmaBatch; ++b) {
      const int64_t j = jb + b < j1 ? jb + b : j1 - 1;  // (rows past the range: loaded, not multiplied)
      wq[b] = uint32_t(qw[j * N + cc]);
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {  // the batch's (at most three) groups
      const int64_t g = g0 + i < ngroups ? g0 + i : ngroups - 1;
      sr[i] = sc[g * N + cc];
      zq[i] = uint32_t(qz[g * (N / 8) + cc / 8]);
    }
  };
  if (j0 < j1) load_batch(j0);
  const uint32_t* xr = reinterpret_cast<const uint32_t*>(x + int64_t(xrow ? m : 0) * K) + kq;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t jb = j0; jb < j1; jb += kMfmaBatch) {
    uint32_t xs[kMfmaBatch];
#pragma unroll
    for (int b = 0; b < kMfmaBatch; ++b) {
      const int64_t j = jb + b < j1 ? jb + b : j1 - 1;
      xs[b] = xrow ? xr[4 * j] : 0u;  // x[m][8j + 2kq], x[m][8j + 2kq + 1]
    }
#pragma unroll
    for (int b = 0; b < kMfmaBatch; ++b) {
      if (jb + b < j1) {
        const int64_t j = jb + b;
        const int gi = int(j >= gb1) + int(j >= gb2);
        const uint32_t sraw = gi == 0 ? sr[0] : (gi == 1 ? sr[1] : sr[2]);
        const uint32_t zw = gi == 0 ? zq[0] : (gi == 1 ? zq[1] : zq[2]);
        const float scale = scale_fp16 ? f16_to_f32(sraw) : bf16_to_f32(sraw);
        const float zs = float((zw >> zshift) & 0xFu) * scale;
        const uint32_t word = wq[b] >> (8 * kq);  // nibbles 2kq, 2kq + 1
        const float w0 = __builtin_fmaf(float(word & 0xFu), scale, -zs);
        const float w1 = __builtin_fmaf(float((word >> 4) & 0xFu), scale, -zs);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bf16_to_f32(xs[b] & 0xFFFFu), w0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bf16_to_f32(xs[b] >> 16), w1, acc, 0, 0, 0);
      }
    }
    if (jb + kMfmaBatch < j1) load_batch(jb + kMfmaBatch);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4_t v = red[0][lane];
#pragma unroll
    for (int w = 1; w < kMfmaWaves; ++w) v += red[w][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int mm = 4 * kq + r;
      if (mm < M && col < N) out[int64_t(mm) * N + col] = f32_to_bf16(v[r]);
    }
  }
}

// The matrix-core kernel with every operand staged in LDS first: the workgroup's
// 16-column slab of qweight (K/8 rows of 64 bytes), its scales and zeros, and x,
// all with 16-byte direct loads (global_load_lds_dwordx4), so a wave issues a
// handful of vector-memory instructions instead of one per packed row; then the
// same multiplies as w4_gemv_mfma_kernel read their operands from LDS.  Needs
// 16-byte aligned operands and N % 16 == 0 (whole slabs).  LDS: qweight slab
// [K/8][16] int32, scales [K/group][16], zeros [K/group][2] int32, x [M][K] bf16.
struct GemvLds {
  int64_t qw_off, sc_off, qz_off, x_off, bytes;
};
inline GemvLds gemv_lds_layout(int64_t M, int64_t K, int group) {
  GemvLds l;
  const int64_t groups = K / group;
  l.qw_off = 0;
  l.sc_off = (K / 8) * 64;
  l.qz_off = l.sc_off + (groups * 32 + 15) / 16 * 16;
  l.x_off = l.qz_off + (groups * 8 + 15) / 16 * 16;
  l.bytes = l.x_off + M * K * 2;
  return l;
}
constexpr int64_t kGemvLdsMax = 120 * 1024;

__global__ void __launch_bounds__(kMfmaWaves * 64)
w4_gemv_lds_kernel(const uint16_t* __restrict__ x, const int32_t* __restrict__ qw, const uint16_t* __restrict__ sc,
                   const int32_t* __restrict__ qz, int M, int64_t K, int64_t N, int group, int scale_fp16,
                   uint16_t* __restrict__ out, GemvLds lay) {
  __shared__ f32x4_t red[kMfmaWaves][64];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(g_gemv_x));
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t col0 = int64_t(blockIdx.x) * 16;
  const int64_t rows = K / 8, groups = K / group;
  // ---- stage: 16-byte chunks, chunk c of a wave's instruction lands at LDS base + 16 c
  {
    // qweight slab: chunk i = row i / 4, columns 4 (i % 4) .. +3
    for (int64_t i0 = int64_t(wave) * 64; i0 < rows * 4; i0 += kMfmaWaves * 64) {
      const int64_t i = i0 + lane;  // (lanes past the end are masked off: they write nothing)
      if (i < rows * 4) dma16(qw + (i / 4) * N + col0 + 4 * (i % 4), lds0 + uint32_t(lay.qw_off + i0 * 16));
    }
    // scales: chunk i = group i / 2, columns 8 (i % 2) .. +7; zeros: chunk i = groups 2i, 2i+1 (8 bytes each)
    for (int64_t i0 = int64_t(wave) * 64; i0 < groups * 2; i0 += kMfmaWaves * 64) {
      const int64_t i = i0 + lane;
      if (i < groups * 2) dma16(sc + (i / 2) * N + col0 + 8 * (i % 2), lds0 + uint32_t(lay.sc_off + i0 * 16));
    }
    for (int64_t i0 = int64_t(wave) * 64; i0 < int64_t(M) * K / 8; i0 += kMfmaWaves * 64) {
      const int64_t i = i0 + lane;
      if (i < int64_t(M) * K / 8) dma16(x + i * 8, lds0 + uint32_t(lay.x_off + i0 * 16));
    }
    // zeros: two words (16 columns) per group, one 8-byte piece per lane, through
    // VGPRs (their LDS store waits for the load); issued after every direct load of
    // the workgroup, so that this wave's one round trip overlaps theirs
    if (wave == kMfmaWaves - 1) {
      for (int64_t g = lane; g < groups; g += 64) {
        const u32x2_t zw = *reinterpret_cast<const u32x2_t*>(qz + g * (N / 8) + col0 / 8);
        *reinterpret_cast<u32x2_t*>(g_gemv_x + lay.qz_off + g * 8) = zw;
      }
    }
    wait_vm<0>();
    __syncthreads();
  }
  const int n = lane & 15, kq = lane >> 4;
  const int64_t col = col0 + n;
  const int m = lane & 15;
  const bool xrow = m < M;
  const int64_t per = (rows + kMfmaWaves - 1) / kMfmaWaves;
  const int64_t j0 = int64_t(wave) * per;
  const int64_t j1 = j0 + per < rows ? j0 + per : rows;
  const int64_t rpg = group / 8;
  const int32_t* lq = reinterpret_cast<const int32_t*>(g_gemv_x + lay.qw_off) + n;
  const uint16_t* ls = reinterpret_cast<const uint16_t*>(g_gemv_x + lay.sc_off) + n;
  const uint32_t* lz = reinterpret_cast<const uint32_t*>(g_gemv_x + lay.qz_off) + n / 8;
  const uint32_t* lx = reinterpret_cast<const uint32_t*>(g_gemv_x + lay.x_off) + int64_t(xrow ? m : 0) * (K / 2) + kq;
  const int zshift = (n % 8) * 4;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  int64_t g = j0 / rpg, gnext = (g + 1) * rpg;
  float scale = 0.f, zs = 0.f;
  auto group_of = [&]() {
    const uint32_t sraw = ls[g * 16];
    scale = scale_fp16 ? f16_to_f32(sraw) : bf16_to_f32(sraw);
    zs = float((lz[g * 2] >> zshift) & 0xFu) * scale;
  };
  if (j0 < j1) group_of();
#pragma unroll 4
  for (int64_t j = j0; j < j1; ++j) {
    if (j == gnext) {
      ++g;
      gnext += rpg;
      group_of();
    }
    const uint32_t word = uint32_t(lq[j * 16]) >> (8 * kq);  // nibbles 2kq, 2kq + 1
    const uint32_t xv = xrow ? lx[4 * j] : 0u;                // x[m][8j + 2kq], x[m][8j + 2kq + 1]
    const float w0 = __builtin_fmaf(float(word & 0xFu), scale, -zs);
    const float w1 = __builtin_fmaf(float((word >> 4) & 0xFu), scale, -zs);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bf16_to_f32(xv & 0xFFFFu), w0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(bf16_to_f32(xv >> 16), w1, acc, 0, 0, 0);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f32x4_t v = red[0][lane];
#pragma unroll
    for (int w = 1; w < kMfmaWaves; ++w) v += red[w][lane];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int mm = 4 * kq + r;
      if (mm < M) out[int64_t(mm) * N + col] = f32_to_bf16(v[r]);
    }
  }
}

}  // namespace

hipError_t launch_w4_gemv(const uint16_t* x, const WeightArgs& w, int64_t M, int64_t K, uint16_t* out,
                          hipStream_t stream) {
  const int64_t N = w.n_cols[0];
  if (M < 1 || M > kGemvMaxM || K % 8 != 0 || N % 8 != 0 || w.group <= 0 || w.group % 64 != 0 || K % w.group != 0)
    return hipErrorInvalidValue;
  const int64_t blocks = (N + kCols - 1) / kCols;
  if (blocks > (int64_t(1) << 31) - 1) return hipErrorInvalidValue;
  const int m = int(M);
  const auto* sc = static_cast<const uint16_t*>(w.sc[0]);
  const int f16 = w.scale_fp16 ? 1 : 0;
  const unsigned nb = unsigned(blocks);
  const GemvLds lay = gemv_lds_layout(M, K, w.group);
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool lds_ok = N % 16 == 0 && lay.bytes <= kGemvLdsMax && a16(x) && a16(w.qw[0]) && a16(w.sc[0]) &&
                      (reinterpret_cast<uintptr_t>(w.qz[0]) & 7u) == 0;
  // M <= 2: the FMA kernel; else the matrix-core kernel, with its operands staged
  // in LDS when they fit and are aligned (measured at K = 1024, N = 4096: 5.1 us
  // at M = 1 against 6.0 for the staged matrix-core kernel; 6.3 / 6.4 / 6.9 us at
  // M = 4 / 8 / 16 against 7.2 / 7.9 / 9.2 for the unstaged one)
  if (m == 1)
    hipLaunchKernelGGL(w4_gemv_kernel<1>, dim3(nb), dim3(kThreads), 0, stream, x, w.qw[0], sc, w.qz[0], m, K, N,
                       w.group, f16, out);
  else if (m == 2)
    hipLaunchKernelGGL(w4_gemv_kernel<2>, dim3(nb), dim3(kThreads), 0, stream, x, w.qw[0], sc, w.qz[0], m, K, N,
                       w.group, f16, out);
  else if (lds_ok)
    hipLaunchKernelGGL(w4_gemv_lds_kernel, dim3(nb), dim3(kMfmaWaves * 64), size_t(lay.bytes), stream, x, w.qw[0],
                       sc, w.qz[0], m, K, N, w.group, f16, out, lay);
  else
    hipLaunchKernelGGL(w4_gemv_mfma_kernel, dim3(nb), dim3(kMfmaWaves * 64), 0, stream, x, w.qw[0], sc, w.qz[0], m,
                       K, N, w.group, f16, out);
  return hipGetLastError();
}

}  // namespace mqk
