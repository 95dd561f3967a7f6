// Split-K projection for small token counts (decode steps, T <= 64), with the
// per-head norm + RoPE done by the last workgroup that finishes each head.
//
// At decode the op is weight-read bound: Qwen3-8B's 50 MB of projection
// weights against 64 tokens.  48 heads alone cannot keep 256 CUs streaming, so
// each head is split along K into `splits` workgroups (XCD-aware: all splits of
// one head are dispatched to the same XCD and so share an L2).  Inside a
// workgroup, wave w owns columns [32w, 32w+32) of the head for all 64 token
// rows (v_mfma_f32_16x16x32_bf16, 4 x 2 blocks); its weight rows are streamed
// HBM -> VGPR with a PREFETCH-deep ring of 64-wide k tiles, each lane loading
// 16 contiguous bytes so that one load instruction covers 16 rows x 64 bytes.
// The activation slice x[:, k-range] is staged once in LDS.
//
// Every workgroup writes its fp32 partial tile [64 x 128] to the workspace,
// fences, and bumps the head's arrival counter; the workgroup that arrives last
// sums the partials, applies RMSNorm over the head (fused_qkv_rope.py:98-100)
// and rotate-half RoPE (:102-118), writes bf16 q/k (or v unchanged), and resets
// the counter to zero for the next call.  No workgroup ever waits on another.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

constexpr int kDecRows = 64;          // token rows per call (T <= 64)
constexpr int kDecThreads = 256;      // 4 waves x 32 columns = one head
constexpr int kDecMaxKc = 512;        // largest k-range of one split (LDS: 64 x 512 bf16 = 64 KB)
constexpr int kPrefetch = 4;          // k tiles in flight per wave
constexpr int kCounterBytes = 4096;   // arrival counters at the head of the workspace

__device__ __forceinline__ int dec_lds_off(int row, int chunk) {
  // row stride kDecMaxKc bf16; 16-byte chunk index swizzled in its low 3 bits
  return row * kDecMaxKc + ((chunk ^ (row & 7)) << 3);
}

template <bool INT4>
__global__ void __launch_bounds__(kDecThreads)
decode_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int splits, float* __restrict__ part,
              int* __restrict__ counters) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kDecRows * kDecMaxKc];
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n_tiles = p.n_tiles;

  // ---- which (head, split): all splits of a head on one XCD -----------------
  int head, split;
  const int bid = blockIdx.x;
  if ((n_tiles & 7) == 0) {
    const int xcd = bid & 7, q = bid >> 3;
    split = q % splits;
    head = (q / splits) * 8 + xcd;
  } else {
    head = bid / splits;
    split = bid % splits;
  }
  const int nkt = int(p.K / kBK);
  const int kt0 = int((int64_t(split) * nkt) / splits);
  const int kt1 = int((int64_t(split + 1) * nkt) / splits);
  const int nk = kt1 - kt0;
  const int64_t kbeg = int64_t(kt0) * kBK;
  const int M = int(p.M);

  int proj, hh;
  split_head(head, e.Hq, e.Hkv, proj, hh);

  // ---- weight stream setup ---------------------------------------------------
  // 16x16x32 operand layout: lane (c = lane & 15, g = lane >> 4) holds column c
  // (B) / row c (A) and 8 k values.  Chosen k order inside a 64-wide tile:
  // block kk (0,1) of 32, lane group g -> k = kk*32 + g*8 .. +8, so one load
  // instruction reads 64 contiguous bytes from each of 16 weight rows.
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int64_t col_base = int64_t(hh) * kHeadDim + wave * 32;  // column inside the projection
  const uint16_t* wrow[2];
  const int32_t* qrow[2];
  float wscale[2] = {0.f, 0.f}, wzero[2] = {0.f, 0.f};
  int64_t qstride = 0;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int64_t col = col_base + nb * 16 + c16;
    if constexpr (!INT4) {
      wrow[nb] = w.w[proj] + col * p.K + kbeg + g4 * 8;
    } else {
      qstride = w.n_cols[proj];
      qrow[nb] = w.qw[proj] + (kbeg / 8 + g4) * qstride + col;
    }
  }

  // Stage x[0:M, kbeg : kbeg + nk*64] into LDS (rows >= M are never read back
  // into a stored result: MFMA row r of the output depends only on row r of x).
  {
    const int chunks_per_row = nk * 8;
    const int total = M * chunks_per_row;
    for (int ci = tid; ci < total; ci += kDecThreads) {
      const int row = ci / chunks_per_row, q = ci - row * chunks_per_row;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(p.x + int64_t(row) * p.K + kbeg + q * 8);
      *reinterpret_cast<u32x4_t*>(xs + dec_lds_off(row, q)) = v;
    }
  }

  // Weight ring: for bf16, 4 x 16 B per lane per k tile; for int4, 4 words.
  u32x4_t wb[kPrefetch][4];
  uint32_t wq[kPrefetch][4];
  auto wload = [&](int slot, int kt) {  // kt relative to kt0
    if constexpr (!INT4) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          wb[slot][nb * 2 + kk] =
              *reinterpret_cast<const u32x4_t*>(wrow[nb] + int64_t(kt) * kBK + kk * 32);
    } else {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          wq[slot][nb * 2 + kk] = uint32_t(qrow[nb][(int64_t(kt) * 8 + kk * 4) * qstride]);
    }
  };

#pragma unroll
  for (int s = 0; s < kPrefetch; ++s)
    if (s < nk) wload(s, s);

  __syncthreads();  // x slice visible

  f32x4_t acc[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f32x4_t{};

  int cur_group = -1;
  for (int base = 0; base < nk; base += kPrefetch) {
#pragma unroll
    for (int s = 0; s < kPrefetch; ++s) {
      const int kt = base + s;
      if (kt < nk) {
        u32x4_t bfrag[2][2];
        if constexpr (!INT4) {
#pragma unroll
          for (int i = 0; i < 4; ++i) bfrag[i >> 1][i & 1] = wb[s][i];
        } else {
          const int64_t k_abs = kbeg + int64_t(kt) * kBK;
          const int grp = int(k_abs / w.group);
          if (grp != cur_group) {
            cur_group = grp;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
              const int64_t col = col_base + nb * 16 + c16;
              const uint32_t sraw = static_cast<const uint16_t*>(w.sc[proj])[grp * qstride + col];
              wscale[nb] = w.scale_fp16 ? f16_to_f32(sraw) : bf16_to_f32(sraw);
              const uint32_t zw = uint32_t(w.qz[proj][grp * (qstride / 8) + col / 8]);
              wzero[nb] = float((zw >> ((col % 8) * 4)) & 0xFu);
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
            bfrag[i >> 1][i & 1] = dequant_int4x8(wq[s][i], wzero[i >> 1], wscale[i >> 1]);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int chunk = kt * 8 + kk * 4 + g4;
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) {
            const int row = mb * 16 + c16;
            const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xs + dec_lds_off(row, chunk));
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma_16x16x32(a, bfrag[nb][kk], acc[mb][nb]);
          }
        }
        if (kt + kPrefetch < nk) wload(s, kt + kPrefetch);
      }
    }
  }

  // ---- publish the partial tile ------------------------------------------------
  // part layout: [splits][n_tiles][64 rows][128 cols] fp32
  float* mypart = part + (int64_t(split) * n_tiles + head) * (kDecRows * kHeadDim);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = mb * 16 + g4 * 4 + j;
        if (row < M) mypart[row * kHeadDim + wave * 32 + nb * 16 + c16] = acc[mb][nb][j];
      }
  __threadfence();
  __syncthreads();
  if (tid == 0) last_flag = (atomicAdd(counters + head, 1) == splits - 1);
  __syncthreads();
  if (!last_flag) return;
  __threadfence();

  // ---- last arrival: reduce partials, norm, RoPE, store --------------------------
  // thread -> row r = tid / 4, quarter q = tid % 4 -> columns [16q, 16q+16) and
  // [64+16q, 64+16q+16): every RoPE pair (d, d+64) is thread-local.
  const int r = tid >> 2;
  const int qq = tid & 3;
  float lo[16], hi[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) lo[i] = hi[i] = 0.f;
  if (r < M) {
    for (int s = 0; s < splits; ++s) {
      const float* src = part + (int64_t(s) * n_tiles + head) * (kDecRows * kHeadDim) + r * kHeadDim;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const f32x4_t a = *reinterpret_cast<const f32x4_t*>(src + qq * 16 + v4 * 4);
        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(src + kHalfDim + qq * 16 + v4 * 4);
        lo[v4 * 4 + 0] += a.x; lo[v4 * 4 + 1] += a.y; lo[v4 * 4 + 2] += a.z; lo[v4 * 4 + 3] += a.w;
        hi[v4 * 4 + 0] += b.x; hi[v4 * 4 + 1] += b.y; hi[v4 * 4 + 2] += b.z; hi[v4 * 4 + 3] += b.w;
      }
    }
  }

  if (proj != 2) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) ss += lo[i] * lo[i] + hi[i] * hi[i];
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    const float rms = rsqrtf(ss * (1.0f / float(kHeadDim)) + e.eps);
    if (r < M) {
      const uint16_t* gamma = proj == 0 ? e.q_gamma : e.k_gamma;
      const int64_t prow = rope_row(e.positions, r, e.S, e.cos_rows) * kHeadDim;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = qq * 16 + i;
        const float x1n = lo[i] * rms * bf16_to_f32(gamma[d]);
        const float x2n = hi[i] * rms * bf16_to_f32(gamma[d + kHalfDim]);
        const float c1 = bf16_to_f32(e.cos[prow + d]);
        const float c2 = bf16_to_f32(e.cos[prow + d + kHalfDim]);
        const float s1 = bf16_to_f32(e.sin[prow + d]);
        const float s2 = bf16_to_f32(e.sin[prow + d + kHalfDim]);
        lo[i] = x1n * c1 - x2n * s1;
        hi[i] = x2n * c2 + x1n * s2;
      }
    }
  }
  if (r < M) {
    const int H = proj == 0 ? e.Hq : e.Hkv;
    uint16_t* dst = (proj == 0 ? e.q : (proj == 1 ? e.k : e.v)) + (int64_t(r) * H + hh) * kHeadDim;
    u32x4_t o;
#pragma unroll
    for (int h8 = 0; h8 < 2; ++h8) {
      o.x = pack_bf16x2(lo[h8 * 8 + 0], lo[h8 * 8 + 1]);
      o.y = pack_bf16x2(lo[h8 * 8 + 2], lo[h8 * 8 + 3]);
      o.z = pack_bf16x2(lo[h8 * 8 + 4], lo[h8 * 8 + 5]);
      o.w = pack_bf16x2(lo[h8 * 8 + 6], lo[h8 * 8 + 7]);
      *reinterpret_cast<u32x4_t*>(dst + qq * 16 + h8 * 8) = o;
      o.x = pack_bf16x2(hi[h8 * 8 + 0], hi[h8 * 8 + 1]);
      o.y = pack_bf16x2(hi[h8 * 8 + 2], hi[h8 * 8 + 3]);
      o.z = pack_bf16x2(hi[h8 * 8 + 4], hi[h8 * 8 + 5]);
      o.w = pack_bf16x2(hi[h8 * 8 + 6], hi[h8 * 8 + 7]);
      *reinterpret_cast<u32x4_t*>(dst + kHalfDim + qq * 16 + h8 * 8) = o;
    }
  }
  if (tid == 0) atomicExch(counters + head, 0);
}

}  // namespace

int decode_splits_for(int64_t M, int64_t K, int n_tiles, int requested) {
  const int nkt = int(K / kBK);
  const int min_splits = (int(K) + kDecMaxKc - 1) / kDecMaxKc;  // LDS bound on the k-range
  int s = requested;
  if (s <= 0) {
    // Keep each workgroup's weight slice >= 4x its fp32 partial tile
    // (128*kc*2 bytes vs M*128*4) and aim for ~1.5 workgroups per CU.
    const int64_t kc_min = ((8 * M + kBK - 1) / kBK) * kBK;
    int by_traffic = int(K / (kc_min > 0 ? kc_min : kBK));
    int by_fill = (384 + n_tiles - 1) / n_tiles;
    s = by_fill < by_traffic ? by_fill : by_traffic;
  }
  if (s < min_splits) s = min_splits;
  if (s > nkt) s = nkt;
  if (s < 1) s = 1;
  return s;
}

size_t decode_workspace_bytes(int n_tiles, int splits) {
  return size_t(kCounterBytes) + size_t(splits) * n_tiles * kDecRows * kHeadDim * sizeof(float);
}

hipError_t launch_decode(int int4, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                         int splits, void* workspace, hipStream_t stream) {
  int* counters = static_cast<int*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  const int blocks = p.n_tiles * splits;
  if (int4)
    hipLaunchKernelGGL(decode_kernel<true>, dim3(blocks), dim3(kDecThreads), 0, stream, p, w, e,
                       splits, part, counters);
  else
    hipLaunchKernelGGL(decode_kernel<false>, dim3(blocks), dim3(kDecThreads), 0, stream, p, w, e,
                       splits, part, counters);
  return hipGetLastError();
}

}  // namespace mqk
