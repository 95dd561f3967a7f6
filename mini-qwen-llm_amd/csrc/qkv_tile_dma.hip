// Tiled MFMA projection with a deep direct-to-LDS pipeline and an LDS epilogue
// (bf16 weights; the prefill / large-T path).
//
// A workgroup computes a BM x (NH*128) tile of  x[M,K] @ W^T  (NH whole heads;
// the Q/K/V weight matrices are addressed directly).  K is consumed in 32-wide
// stages held in an NS-deep LDS ring that is filled with global_load_lds_dwordx4
// (L2 -> LDS without VGPRs): while stage k is multiplied, the loads of stages
// k+1 .. k+NS-1 are in flight, which hides the L2 latency that a single
// register-staged prefetch could not.  One barrier per stage: after it, every
// wave's loads for stage k have landed (each wave first waits for its own with
// vmcnt) and every wave has finished stage k-1, whose buffer is refilled next.
//
// The loads and the waits are inline asm: the compiler neither models
// global_load_lds as a write of the LDS array nor lets a __syncthreads() pass
// without draining every outstanding load, which would serialise the ring.
// Ordering is therefore explicit: asm volatile with "memory" clobbers around
// the waits and barriers; LDS reads are ordinary C++ and the compiler inserts
// their lgkmcnt waits.
//
// LDS layout of a stage: A rows [BM] then B rows [NH*128], 64 bytes each
// (32 bf16 = 4 chunks of 16 B); chunk c of row r sits in slot c ^ ((r >> 2) & 3),
// so the 16 rows read by a quarter-wave land in 16 different 16-byte bank
// groups.  One load instruction fills 16 consecutive rows (1 KB).
//
// Waves form a WM x WN grid; wave (wm, wn) owns rows [wm*TM, +TM) and columns
// [wn*TN, +TN) with v_mfma_f32_32x32x16_bf16.  Epilogue, one head at a time:
// the waves covering the head write its fp32 accumulators to LDS, then threads
// take 8-column pairs of a row (columns [8c, 8c+8) and [64+8c, +8)) so the
// RMSNorm sum of squares is an 8-lane butterfly and every RoPE pair is
// thread-local; each output row segment is written with 16-byte stores.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

constexpr int kSBK = 32;                    // K extent of one stage
constexpr int kRowBytes = kSBK * 2;         // 64 B per staged row
constexpr int kEpiPitch = kHeadDim + 4;     // fp32 pitch of the epilogue head tile

template <int BM, int NH, int WM, int WN, int NS>
struct DmaShape {
  static constexpr int kBN = NH * kHeadDim;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kTM = BM / WM;
  static constexpr int kTN = kBN / WN;
  static constexpr int kMB = kTM / 32;
  static constexpr int kNB = kTN / 32;
  static constexpr int kRows = BM + kBN;                // staged rows per stage
  static constexpr int kStageBytes = kRows * kRowBytes;
  static constexpr int kLoadsPerStage = kRows / 16;     // 1 KB load instructions
  static constexpr int kLoadsPerWave = kLoadsPerStage / kWaves;
  static constexpr int kRingBytes = NS * kStageBytes;
  static constexpr int kEpiBytes = BM * kEpiPitch * 4;
  static constexpr int kLdsBytes = kRingBytes > kEpiBytes ? kRingBytes : kEpiBytes;
  static_assert(kTM % 32 == 0 && kTN % 32 == 0, "wave tile");
  static_assert(kLoadsPerStage % kWaves == 0, "loads per wave");
  static_assert(NS >= 2 && NS <= 8, "stages");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

template <int NS, int LPW>
__device__ __forceinline__ void wait_stage(int remaining_after) {
  // remaining_after = stages issued after the one being waited for (0..NS-2)
  switch (remaining_after) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<(1 * LPW < 63 ? 1 * LPW : 63)>(); break;
    case 2: wait_vm<(2 * LPW < 63 ? 2 * LPW : 63)>(); break;
    case 3: wait_vm<(3 * LPW < 63 ? 3 * LPW : 63)>(); break;
    case 4: wait_vm<(4 * LPW < 63 ? 4 * LPW : 63)>(); break;
    case 5: wait_vm<(5 * LPW < 63 ? 5 * LPW : 63)>(); break;
    default: wait_vm<(6 * LPW < 63 ? 6 * LPW : 63)>(); break;
  }
  (void)NS;
}

__device__ __forceinline__ int stage_slot(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

template <int BM, int NH, int WM, int WN, int NS>
__global__ void __launch_bounds__(WM* WN * 64)
tile_dma_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int group_m) {
  using S = DmaShape<BM, NH, WM, WN, NS>;
  constexpr int BN = S::kBN;
  __shared__ __attribute__((aligned(16))) unsigned char smem[S::kLdsBytes];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;

  // ---- tile coordinates: XCD-contiguous ids, grouped along M ------------------
  const int n_mt = int((p.M + BM - 1) / BM);
  const int n_ht = p.n_tiles / NH;
  const int tile = xcd_tile_id(blockIdx.x, gridDim.x);
  const int per_group = group_m * n_ht;
  const int grp = tile / per_group;
  const int first_m = grp * group_m;
  const int gsz = min(group_m, n_mt - first_m);
  const int rr = tile - grp * per_group;
  const int mt = first_m + rr % gsz;
  const int ht = rr / gsz;
  const int64_t m0 = int64_t(mt) * BM;
  const int64_t K = p.K;

  // ---- this lane's sources: load instruction i of a stage fills staged rows
  // [16*(wave + i*W), +16); lane -> row +lane/4, slot lane%4 ----------------------
  const uint16_t* src[S::kLoadsPerWave];
  uint32_t dst_off[S::kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < S::kLoadsPerWave; ++i) {
    const int row0 = 16 * (wave + i * S::kWaves);
    const int row = row0 + (lane >> 2);
    const int chunk = stage_slot(row, lane & 3);  // global chunk stored in slot lane & 3
    if (row < BM) {
      int64_t grow = m0 + row;
      grow = grow < p.M ? grow : p.M - 1;  // rows past M re-read the last row; never stored
      src[i] = p.x + grow * K + chunk * 8;
    } else {
      const int brow = row - BM;
      int proj, hh;
      split_head(ht * NH + brow / kHeadDim, e.Hq, e.Hkv, proj, hh);
      int64_t col = int64_t(hh) * kHeadDim + (brow % kHeadDim);
      col = col < w.n_cols[proj] ? col : w.n_cols[proj] - 1;
      src[i] = w.w[proj] + col * K + chunk * 8;
    }
    dst_off[i] = uint32_t(row0 * kRowBytes);
  }
  auto issue = [&](int kt) {
    const uint32_t base = lds0 + uint32_t((kt % NS) * S::kStageBytes);
#pragma unroll
    for (int i = 0; i < S::kLoadsPerWave; ++i) dma16(src[i] + int64_t(kt) * kSBK, base + dst_off[i]);
  };

  // ---- main loop -------------------------------------------------------------------
  f32x16_t acc[S::kMB][S::kNB];
#pragma unroll
  for (int mb = 0; mb < S::kMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < S::kNB; ++nb) acc[mb][nb] = f32x16_t{};

  const int c32 = lane & 31;
  const int khalf = lane >> 5;
  const int nkt = int(K / kSBK);
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nkt) issue(s);

  for (int kt = 0; kt < nkt; ++kt) {
    const int ahead = min(NS - 2, nkt - 1 - kt);  // stages already issued after kt
    wait_stage<NS, S::kLoadsPerWave>(ahead);
    barrier();
    if (kt + NS - 1 < nkt) issue(kt + NS - 1);
    const unsigned char* st = smem + (kt % NS) * S::kStageBytes;
#pragma unroll
    for (int ks = 0; ks < kSBK / 16; ++ks) {
      const int chunk = 2 * ks + khalf;
      u32x4_t af[S::kMB], bf[S::kNB];
#pragma unroll
      for (int mb = 0; mb < S::kMB; ++mb) {
        const int row = wm * S::kTM + mb * 32 + c32;
        af[mb] = *reinterpret_cast<const u32x4_t*>(st + row * kRowBytes + stage_slot(row, chunk) * 16);
      }
#pragma unroll
      for (int nb = 0; nb < S::kNB; ++nb) {
        const int row = BM + wn * S::kTN + nb * 32 + c32;
        bf[nb] = *reinterpret_cast<const u32x4_t*>(st + row * kRowBytes + stage_slot(row, chunk) * 16);
      }
#pragma unroll
      for (int mb = 0; mb < S::kMB; ++mb)
#pragma unroll
        for (int nb = 0; nb < S::kNB; ++nb) acc[mb][nb] = mfma_32x32x16(af[mb], bf[nb], acc[mb][nb]);
    }
  }
  barrier();  // every wave is done with the ring; the epilogue reuses the LDS

  // ---- epilogue, one head at a time --------------------------------------------------
  float* ep = reinterpret_cast<float*>(smem);
  const int half = lane >> 5;
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    // columns [j*128, j*128+128) of the tile; wave columns [wn*TN, +TN)
#pragma unroll
    for (int nb = 0; nb < S::kNB; ++nb) {
      const int col = wn * S::kTN + nb * 32;  // first column of this 32-wide block
      if (col >= j * kHeadDim && col < (j + 1) * kHeadDim) {
#pragma unroll
        for (int mb = 0; mb < S::kMB; ++mb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int row = wm * S::kTM + mb * 32 + 8 * (i >> 2) + 4 * half + (i & 3);
            ep[row * kEpiPitch + (col - j * kHeadDim) + c32] = acc[mb][nb][i];
          }
      }
    }
    __syncthreads();
    const int head = ht * NH + j;
    int proj, hh;
    split_head(head, e.Hq, e.Hkv, proj, hh);
    const int c8 = tid & 7;
    for (int r0 = tid >> 3; r0 < BM; r0 += S::kThreads / 8) {
      const int64_t t = m0 + r0;
      const float* rowp = ep + r0 * kEpiPitch;
      float lo[8], hi[8];
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const f32x4_t a = *reinterpret_cast<const f32x4_t*>(rowp + 8 * c8 + 4 * v);
        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(rowp + kHalfDim + 8 * c8 + 4 * v);
        lo[4 * v] = a.x; lo[4 * v + 1] = a.y; lo[4 * v + 2] = a.z; lo[4 * v + 3] = a.w;
        hi[4 * v] = b.x; hi[4 * v + 1] = b.y; hi[4 * v + 2] = b.z; hi[4 * v + 3] = b.w;
      }
      if (e.qkv && proj != 2) {
        // RMSNorm over the head (fused_qkv_rope.py:98-100), then rotate-half RoPE (:102-118)
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += lo[i] * lo[i] + hi[i] * hi[i];
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        const float rms = rsqrtf(ss * (1.0f / float(kHeadDim)) + e.eps);
        if (t < p.M) {
          const uint16_t* gamma = proj == 0 ? e.q_gamma : e.k_gamma;
          const int64_t prow = rope_row(e.positions, t, e.S, e.cos_rows) * kHeadDim;
          const u32x4_t g1 = *reinterpret_cast<const u32x4_t*>(gamma + 8 * c8);
          const u32x4_t g2 = *reinterpret_cast<const u32x4_t*>(gamma + kHalfDim + 8 * c8);
          const u32x4_t cs1 = *reinterpret_cast<const u32x4_t*>(e.cos + prow + 8 * c8);
          const u32x4_t cs2 = *reinterpret_cast<const u32x4_t*>(e.cos + prow + kHalfDim + 8 * c8);
          const u32x4_t sn1 = *reinterpret_cast<const u32x4_t*>(e.sin + prow + 8 * c8);
          const u32x4_t sn2 = *reinterpret_cast<const u32x4_t*>(e.sin + prow + kHalfDim + 8 * c8);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int wd = i >> 1, sh = (i & 1) * 16;
            const float x1n = lo[i] * rms * bf16_to_f32((g1[wd] >> sh) & 0xFFFFu);
            const float x2n = hi[i] * rms * bf16_to_f32((g2[wd] >> sh) & 0xFFFFu);
            const float c1 = bf16_to_f32((cs1[wd] >> sh) & 0xFFFFu);
            const float c2 = bf16_to_f32((cs2[wd] >> sh) & 0xFFFFu);
            const float s1 = bf16_to_f32((sn1[wd] >> sh) & 0xFFFFu);
            const float s2 = bf16_to_f32((sn2[wd] >> sh) & 0xFFFFu);
            lo[i] = x1n * c1 - x2n * s1;
            hi[i] = x2n * c2 + x1n * s2;
          }
        }
      }
      if (t < p.M) {
        u32x4_t o1, o2;
        o1.x = pack_bf16x2(lo[0], lo[1]); o1.y = pack_bf16x2(lo[2], lo[3]);
        o1.z = pack_bf16x2(lo[4], lo[5]); o1.w = pack_bf16x2(lo[6], lo[7]);
        o2.x = pack_bf16x2(hi[0], hi[1]); o2.y = pack_bf16x2(hi[2], hi[3]);
        o2.z = pack_bf16x2(hi[4], hi[5]); o2.w = pack_bf16x2(hi[6], hi[7]);
        if (e.qkv) {
          const int H = proj == 0 ? e.Hq : e.Hkv;
          uint16_t* dst = (proj == 0 ? e.q : (proj == 1 ? e.k : e.v)) + (t * H + hh) * kHeadDim;
          *reinterpret_cast<u32x4_t*>(dst + 8 * c8) = o1;
          *reinterpret_cast<u32x4_t*>(dst + kHalfDim + 8 * c8) = o2;
        } else {
          const int64_t col0 = int64_t(head) * kHeadDim;  // plain GEMM output [M, N]
          uint16_t* dst = e.out + t * e.N + col0;
          if (col0 + 8 * c8 + 8 <= e.N) *reinterpret_cast<u32x4_t*>(dst + 8 * c8) = o1;
          if (col0 + kHalfDim + 8 * c8 + 8 <= e.N) *reinterpret_cast<u32x4_t*>(dst + kHalfDim + 8 * c8) = o2;
        }
      }
    }
    __syncthreads();  // the next head reuses ep
  }
}

template <int BM, int NH, int WM, int WN, int NS>
hipError_t launch_dma(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                      hipStream_t stream) {
  using S = DmaShape<BM, NH, WM, WN, NS>;
  const int n_mt = int((p.M + BM - 1) / BM);
  const int blocks = n_mt * (p.n_tiles / NH);
  hipLaunchKernelGGL((tile_dma_kernel<BM, NH, WM, WN, NS>), dim3(blocks), dim3(S::kThreads), 0, stream, p, w, e,
                     group_m < 1 ? 1 : group_m);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_tile_dma(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                           hipStream_t stream) {
  switch (id) {
    case 10: return launch_dma<256, 2, 4, 2, 4>(p, w, e, group_m, stream);   // 256x256, 8 waves, 4 stages
    case 11: return launch_dma<128, 3, 2, 4, 4>(p, w, e, group_m, stream);   // 128x384, 8 waves (64x96)
    case 12: return launch_dma<256, 1, 4, 1, 4>(p, w, e, group_m, stream);   // 256x128, 4 waves
    case 13: return launch_dma<128, 2, 2, 2, 4>(p, w, e, group_m, stream);   // 128x256, 4 waves
    case 14: return launch_dma<256, 2, 2, 4, 4>(p, w, e, group_m, stream);   // 256x256, 8 waves (128x64)
    case 15: return launch_dma<128, 3, 2, 4, 5>(p, w, e, group_m, stream);   // 128x384, 5 stages
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mqk
