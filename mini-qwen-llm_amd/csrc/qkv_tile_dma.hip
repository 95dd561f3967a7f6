// Tiled MFMA projection with a deep direct-to-LDS pipeline and an LDS epilogue
// (bf16 weights; the prefill / large-T path).
//
// A workgroup computes a BM x (NH*128) tile of  x[M,K] @ W^T  (NH whole heads;
// the Q/K/V weight matrices are addressed directly).  K is consumed in SBK-wide
// (32 or 64) stages held in an NS-deep LDS ring that is filled with global_load_lds_dwordx4
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
#include <type_traits>

#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {

namespace {

constexpr int kEpiPitch = kHeadDim + 4;     // fp32 pitch of the epilogue head tile

// RMSNorm (fused_qkv_rope.py:98-100) then rotate-half RoPE (:102-118) of the
// dim pair (d, d+64); gl / gh are the gammas of d / d+64 and element
// (wd, sh) of the cos / sin registers holds the table values of d and d+64.
__device__ __forceinline__ void norm_rope_pair(float& lo, float& hi, float rms, float gl, float gh,
                                               const u32x4_t (&c2)[2], const u32x4_t (&s2)[2], int wd, int sh) {
#pragma clang fp contract(off)
  const float x1n = lo * rms * gl;
  const float x2n = hi * rms * gh;
  const float co1 = bf16_to_f32((c2[0][wd] >> sh) & 0xFFFFu);
  const float co2 = bf16_to_f32((c2[1][wd] >> sh) & 0xFFFFu);
  const float si1 = bf16_to_f32((s2[0][wd] >> sh) & 0xFFFFu);
  const float si2 = bf16_to_f32((s2[1][wd] >> sh) & 0xFFFFu);
  lo = __builtin_fmaf(x1n, co1, -(x2n * si1));
  hi = __builtin_fmaf(x2n, co2, x1n * si2);
}

// SBK = K extent of one stage (32 or 64): staged rows of 64 or 128 bytes.  A
// CU's L2 -> LDS rate depends on the bytes per row: 128-byte rows measured
// ~1.35x the rate of 64-byte rows (fewer, full-line requests in flight).
// XC: extra columns beyond the NH whole heads (64 in a pair tile: half of a head
// shared with the partner tile).
template <int BM, int NH, int WM, int WN, int NS, int SBK, int XC = 0>
struct DmaShape {
  static constexpr int kRowBytes = SBK * 2;
  static constexpr int kChunks = kRowBytes / 16;         // 16-byte chunks per staged row
  static constexpr int kRowsPerLoad = 1024 / kRowBytes;  // rows filled by one 1 KB load instruction
  static constexpr int kBN = NH * kHeadDim + XC;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kTM = BM / WM;
  static constexpr int kTN = kBN / WN;
  static constexpr int kMB = kTM / 32;
  static constexpr int kNB = kTN / 32;
  static constexpr int kRows = BM + kBN;                // staged rows per stage
  static constexpr int kStageBytes = kRows * kRowBytes;
  static constexpr int kLoadsPerStage = kRows / kRowsPerLoad;  // 1 KB load instructions
  static constexpr int kLoadsPerWave = kLoadsPerStage / kWaves;
  static constexpr int kRingBytes = NS * kStageBytes;
  static constexpr int kEpiBytes = BM * kEpiPitch * 4;
  static constexpr int kLdsBytes = kRingBytes > kEpiBytes ? kRingBytes : kEpiBytes;
  static_assert(kTM % 16 == 0 && kTN % 16 == 0, "wave tile (16 x 16 accumulator blocks)");
  static_assert(kLoadsPerStage % kWaves == 0, "loads per wave");
  static constexpr int kALoads = BM / (kRowsPerLoad * kWaves);  // this wave's loads i < kALoads fill x rows
  static_assert(BM % (kRowsPerLoad * kWaves) == 0, "x rows are whole load rounds");
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

// LDS slot of 16-byte chunk `chunk` of staged row `row`: the 16 rows one
// quarter-wave reads (same chunk) land in 16 different bank groups.
template <int SBK>
__device__ __forceinline__ int stage_slot(int row, int chunk) {
  if constexpr (SBK == 32) return chunk ^ ((row >> 2) & 3);  // 64 B rows: rows r, r+4, r+8, r+12 share banks
  else return chunk ^ ((row >> 1) & 7);                       // 128 B rows: even / odd rows use bank halves
}

// Input RMSNorm support (ProblemArgs::in_gamma): the gamma vector is staged once
// in the dynamic LDS that follows the kernel's static LDS, and every wave applies
// input_norm8 in place to the x chunks its own direct loads brought in, after
// waiting for them and before the stage barrier, so the MFMA reads see normalised
// activations without any extra barrier in the main loop.
extern __shared__ __attribute__((aligned(16))) unsigned char g_dyn_lds[];

template <int THREADS>
__device__ __forceinline__ void stage_gamma(const ProblemArgs& p) {
  for (int64_t c = threadIdx.x; c < p.K / 8; c += THREADS)
    *reinterpret_cast<u32x4_t*>(g_dyn_lds + c * 16) = *reinterpret_cast<const u32x4_t*>(p.in_gamma + c * 8);
}

// In place: the 16-byte x chunk at LDS `chunk_ptr` (k = k0 .. k0+7 of a row whose
// scale is `scale`) becomes bf16(gamma * bf16(x * scale)).
__device__ __forceinline__ void norm_chunk(unsigned char* chunk_ptr, int64_t k0, float scale) {
  const u32x4_t g = *reinterpret_cast<const u32x4_t*>(g_dyn_lds + k0 * 2);
  u32x4_t* q = reinterpret_cast<u32x4_t*>(chunk_ptr);
  *q = input_norm8(*q, scale, g);
}

// Accumulator blocks of the two MFMA shapes: the tile kernel uses 16 x 16 blocks
// (v_mfma_f32_16x16x32_bf16: element j of lane l is row 4 * (l >> 4) + j, column
// l & 15), the int4 and split-K kernels 32 x 32 blocks (v_mfma_f32_32x32x16_bf16:
// element i of lane l is row 8 * (i >> 2) + 4 * (l >> 5) + (i & 3), column l & 31).
template <class V> struct AccBlock;
template <> struct AccBlock<f32x16_t> {
  static constexpr int kDim = 32, kElems = 16;
  static __device__ __forceinline__ int row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }
  static __device__ __forceinline__ int col(int lane) { return lane & 31; }
};
template <> struct AccBlock<f32x4_t> {
  static constexpr int kDim = 16, kElems = 4;
  static __device__ __forceinline__ int row(int i, int lane) { return 4 * (lane >> 4) + i; }
  static __device__ __forceinline__ int col(int lane) { return lane & 15; }
};

// Per-head epilogue of a BM x (NH*128) tile held in MFMA accumulator blocks
// (AccBlock): wave (wm, wn) holds rows [wm*TM, +TM) x columns [wn*TN, +TN) as acc[mb][nb].
// One head at a time, the waves covering it write their fp32 block to LDS `ep`,
// then threads take 8-column pairs of a row (columns [8c, 8c+8) and
// [64+8c, +8)), so the RMSNorm sum of squares is an 8-lane butterfly and every
// RoPE pair is thread-local; each output row segment is written with 16-byte
// stores.  prow[q] holds the RoPE table row of this thread's row (tid/8) + q*kRowStep,
// cslot[q] its paged-KV-cache slot (-1: none).
// units: bit u set = rows [32u, 32u+32) of the tile are stored (the split-K
// launch finishes a tile's rows in 32-row units spread over its workgroups).
template <int BM, int NH, int WM, int WN, int THREADS, int MB, int NB, class AV, class RowV, class SlotV>
__device__ __forceinline__ void tile_epilogue(const AV (&acc)[MB][NB], const RowV& prow,
                                              const SlotV& cslot, int head0, int64_t m0, const ProblemArgs& p,
                                              const EpilogueArgs& e, unsigned char* smem,
                                              uint32_t units = 0xFFFFFFFFu) {
  using Blk = AccBlock<AV>;
  constexpr int kTM = BM / WM;
  constexpr int kTN = NB * Blk::kDim;  // (a pair tile's waves also hold the shared half head's columns)
  constexpr int kRowStep = THREADS / 8;
  constexpr int kPasses = BM / kRowStep;
  static_assert(BM % kRowStep == 0, "the epilogue's row passes must cover the tile");
  // gamma / cos / sin depend only on the token: with few rows per thread they are
  // loaded once for all NH heads of the tile (16 VGPRs per row).  Four rows' worth
  // beside the 128 accumulators of an 8-wave 256-row tile (256 VGPRs per lane at
  // two waves per SIMD) spilled; 4-wave tiles (one wave per SIMD) have room.
  constexpr bool kPreload = kPasses <= 2 || (kPasses <= 4 && THREADS <= 256);
  // beside more than 128 accumulators (the 256 x 320 pair tile) the gammas are read
  // per row pass instead of held through the epilogue
  constexpr bool kLateGamma = MB * NB * Blk::kElems > 128;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  // ---- epilogue, one head at a time --------------------------------------------------
  const int c8 = tid & 7;
  const int hd = e.head_dim;
  const PairRuns pr = pair_runs(c8, hd);
  u32x4_t gq[2] = {}, gk[2] = {}, cs[kPreload ? kPasses : 1][2] = {}, sn[kPreload ? kPasses : 1][2] = {};
  auto load_rows = [&](int q, u32x4_t (&c2)[2], u32x4_t (&s2)[2]) {
    const int64_t base = int64_t(prow[q]) * hd;
    c2[0] = *reinterpret_cast<const u32x4_t*>(e.cos + base + pr.dim_lo);
    c2[1] = *reinterpret_cast<const u32x4_t*>(e.cos + base + pr.dim_hi);
    s2[0] = *reinterpret_cast<const u32x4_t*>(e.sin + base + pr.dim_lo);
    s2[1] = *reinterpret_cast<const u32x4_t*>(e.sin + base + pr.dim_hi);
  };
  if (e.qkv) {
    if constexpr (!kLateGamma) {
      gq[0] = *reinterpret_cast<const u32x4_t*>(e.q_gamma + pr.dim_lo);
      gq[1] = *reinterpret_cast<const u32x4_t*>(e.q_gamma + pr.dim_hi);
      gk[0] = *reinterpret_cast<const u32x4_t*>(e.k_gamma + pr.dim_lo);
      gk[1] = *reinterpret_cast<const u32x4_t*>(e.k_gamma + pr.dim_hi);
    }
    if constexpr (kPreload) {
#pragma unroll
      for (int q = 0; q < kPasses; ++q) load_rows(q, cs[q], sn[q]);
    }
  }
  float* ep = reinterpret_cast<float*>(smem);
  const int bcol = Blk::col(lane);
#pragma unroll
  for (int j = 0; j < NH; ++j) {
    // columns [j*128, j*128+128) of the tile; wave columns [wn*TN, +TN)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = wn * kTN + nb * Blk::kDim;  // first column of this block
      if (col >= j * kHeadDim && col < (j + 1) * kHeadDim) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < Blk::kElems; ++i) {
            const int row = wm * kTM + mb * Blk::kDim + Blk::row(i, lane);
            ep[row * kEpiPitch + (col - j * kHeadDim) + bcol] = acc[mb][nb][i];
          }
      }
    }
    __syncthreads();
    const int head = head0 + j;
    int proj, hh;
    split_head(head, e.Hq, e.Hkv, proj, hh);
    // this head's gamma pairs in fp32, converted once for all its row passes
    // (with up to two passes per head; with more, the 16 extra registers spill)
    constexpr bool kHoistGamma = kPasses <= 2;
    float g1[8], g2[8];
    if constexpr (kHoistGamma) {
      const u32x4_t* g = proj == 0 ? gq : gk;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int wd = i >> 1, sh = (i & 1) * 16;
        g1[i] = bf16_to_f32((g[0][wd] >> sh) & 0xFFFFu);
        g2[i] = bf16_to_f32((g[1][wd] >> sh) & 0xFFFFu);
      }
    }
#pragma unroll
    for (int q = 0; q < kPasses; ++q) {
      constexpr uint32_t kPassUnits = (kRowStep / 32) >= 32 ? 0xFFFFFFFFu : ((1u << (kRowStep / 32)) - 1u);
      if (((units >> (q * kRowStep / 32)) & kPassUnits) == 0) continue;  // no stored row in this pass
      const int r0 = (tid >> 3) + q * kRowStep;
      const int64_t t = m0 + r0;
      const float* rowp = ep + r0 * kEpiPitch;
      float lo[8], hi[8];
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const f32x4_t a = *reinterpret_cast<const f32x4_t*>(rowp + pr.col_lo + 4 * v);
        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(rowp + pr.col_hi + 4 * v);
        lo[4 * v] = a.x; lo[4 * v + 1] = a.y; lo[4 * v + 2] = a.z; lo[4 * v + 3] = a.w;
        hi[4 * v] = b.x; hi[4 * v + 1] = b.y; hi[4 * v + 2] = b.z; hi[4 * v + 3] = b.w;
      }
      if (e.qkv == 1 && proj != 2) {  // (qkv 2: q and k stored as projected)
        // RMSNorm over the head (fused_qkv_rope.py:98-100), then rotate-half RoPE (:102-118)
        const float ss = head_sum(run_sumsq(lo, hi), hd);
        const float rms = head_rms(ss, e.eps, hd);
        u32x4_t c2[2], s2[2];
        if constexpr (kPreload) {
          c2[0] = cs[q][0]; c2[1] = cs[q][1]; s2[0] = sn[q][0]; s2[1] = sn[q][1];
        } else {
          load_rows(q, c2, s2);
        }
        u32x4_t glate[2];
        if constexpr (kLateGamma) {
          const uint16_t* gam = pick3<const uint16_t>(proj, e.q_gamma, e.k_gamma, e.k_gamma);
          glate[0] = *reinterpret_cast<const u32x4_t*>(gam + pr.dim_lo);
          glate[1] = *reinterpret_cast<const u32x4_t*>(gam + pr.dim_hi);
        }
        const u32x4_t* g = kLateGamma ? glate : (proj == 0 ? gq : gk);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int wd = i >> 1, sh = (i & 1) * 16;
          const float gl = kHoistGamma ? g1[i] : bf16_to_f32((g[0][wd] >> sh) & 0xFFFFu);
          const float gh = kHoistGamma ? g2[i] : bf16_to_f32((g[1][wd] >> sh) & 0xFFFFu);
          norm_rope_pair(lo[i], hi[i], rms, gl, gh, c2, s2, wd, sh);
        }
      }
      if (t < p.M && ((units >> (r0 >> 5)) & 1u)) {
        u32x4_t o1, o2;
        o1.x = pack_bf16x2(lo[0], lo[1]); o1.y = pack_bf16x2(lo[2], lo[3]);
        o1.z = pack_bf16x2(lo[4], lo[5]); o1.w = pack_bf16x2(lo[6], lo[7]);
        o2.x = pack_bf16x2(hi[0], hi[1]); o2.y = pack_bf16x2(hi[2], hi[3]);
        o2.z = pack_bf16x2(hi[4], hi[5]); o2.w = pack_bf16x2(hi[6], hi[7]);
        if (e.qkv) {
          const int H = proj == 0 ? e.Hq : e.Hkv;
          uint16_t* base = proj == 0 ? e.q : (proj == 1 ? e.k : e.v);  // k / v may be null (cache only)
          // (non-temporal: the tile's rows are written once and read by a later
          // kernel, so they need not stay in this XCD's L2; measured ~2 % faster)
          if (base) {
            uint16_t* dst = base + (t * H + hh) * kHeadDim;
            __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(dst + pr.col_lo));
            __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(dst + pr.col_hi));
          }
          if (proj != 0 && cslot[q] >= 0) {
            uint16_t* crow = paged_row(e, cslot[q], proj, hh);
            __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(crow + pr.col_lo));
            __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(crow + pr.col_hi));
          }
        } else {
          const int64_t col0 = int64_t(head) * kHeadDim;  // plain GEMM output [M, N]
          uint16_t* dst = e.out + t * e.N + col0;
          if (col0 + pr.col_lo + 8 <= e.N) __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(dst + pr.col_lo));
          if (col0 + pr.col_hi + 8 <= e.N) __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(dst + pr.col_hi));
        }
      }
    }
    __syncthreads();  // the next head reuses ep
  }
}

// Norm, RoPE and 16-byte stores of 32 finished rows of a tile (rows t0 .. t0+31
// of the call), held in LDS as fp32 [32][pitch] over the tile's NH heads: thread
// -> (head j, row, c8) takes the column pairs [8c8, +8) / [64+8c8, +8) of one head
// of one row, the same arithmetic as tile_epilogue.
template <int NH, int THREADS>
__device__ __forceinline__ void finish_unit_rows(const float* tile, int pitch, int64_t t0, int ht,
                                                 const ProblemArgs& p, const EpilogueArgs& e) {
  constexpr int kItems = 32 * NH * 8;
  const int tid = threadIdx.x;
#pragma unroll
  for (int it0 = 0; it0 < kItems; it0 += THREADS) {
    const int it = it0 + tid;
    if (kItems % THREADS != 0 && it >= kItems) break;  // (whole groups of 8 lanes leave together)
    const int j = it / 256, rr = (it >> 3) & 31, c8 = it & 7;
    const int hd = e.head_dim;
    const PairRuns pr = pair_runs(c8, hd);
    const int64_t t = t0 + rr;
    const int head = ht * NH + j;
    int proj, hh;
    split_head(head, e.Hq, e.Hkv, proj, hh);
    const float* rowp = tile + rr * pitch + j * kHeadDim;
    float lo[8], hi[8];
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const f32x4_t a = *reinterpret_cast<const f32x4_t*>(rowp + pr.col_lo + 4 * v);
      const f32x4_t b = *reinterpret_cast<const f32x4_t*>(rowp + pr.col_hi + 4 * v);
      lo[4 * v] = a.x; lo[4 * v + 1] = a.y; lo[4 * v + 2] = a.z; lo[4 * v + 3] = a.w;
      hi[4 * v] = b.x; hi[4 * v + 1] = b.y; hi[4 * v + 2] = b.z; hi[4 * v + 3] = b.w;
    }
    const bool valid = t < p.M;
    if (e.qkv == 1 && proj != 2) {
      const float ss = head_sum(run_sumsq(lo, hi), hd);
      const float rms = head_rms(ss, e.eps, hd);
      const int64_t base = (valid ? rope_row(e, t) : 0) * hd;
      u32x4_t c2[2], s2[2];
      c2[0] = *reinterpret_cast<const u32x4_t*>(e.cos + base + pr.dim_lo);
      c2[1] = *reinterpret_cast<const u32x4_t*>(e.cos + base + pr.dim_hi);
      s2[0] = *reinterpret_cast<const u32x4_t*>(e.sin + base + pr.dim_lo);
      s2[1] = *reinterpret_cast<const u32x4_t*>(e.sin + base + pr.dim_hi);
      const uint16_t* gam = proj == 0 ? e.q_gamma : e.k_gamma;
      const u32x4_t g0 = *reinterpret_cast<const u32x4_t*>(gam + pr.dim_lo);
      const u32x4_t g1 = *reinterpret_cast<const u32x4_t*>(gam + pr.dim_hi);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int wd = i >> 1, sh = (i & 1) * 16;
        norm_rope_pair(lo[i], hi[i], rms, bf16_to_f32((g0[wd] >> sh) & 0xFFFFu),
                       bf16_to_f32((g1[wd] >> sh) & 0xFFFFu), c2, s2, wd, sh);
      }
    }
    if (!valid) continue;
    u32x4_t o1, o2;
    o1.x = pack_bf16x2(lo[0], lo[1]); o1.y = pack_bf16x2(lo[2], lo[3]);
    o1.z = pack_bf16x2(lo[4], lo[5]); o1.w = pack_bf16x2(lo[6], lo[7]);
    o2.x = pack_bf16x2(hi[0], hi[1]); o2.y = pack_bf16x2(hi[2], hi[3]);
    o2.z = pack_bf16x2(hi[4], hi[5]); o2.w = pack_bf16x2(hi[6], hi[7]);
    if (e.qkv) {
      const int H = proj == 0 ? e.Hq : e.Hkv;
      uint16_t* obase = proj == 0 ? e.q : (proj == 1 ? e.k : e.v);  // k / v may be null (cache only)
      if (obase) {
        uint16_t* dst = obase + (t * H + hh) * kHeadDim;
        __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(dst + pr.col_lo));
        __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(dst + pr.col_hi));
      }
      const int64_t slot = proj != 0 ? paged_slot(e, t) : -1;
      if (slot >= 0) {
        uint16_t* crow = paged_row(e, slot, proj, hh);
        __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(crow + pr.col_lo));
        __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(crow + pr.col_hi));
      }
    } else {
      const int64_t col0 = int64_t(head) * kHeadDim;  // plain GEMM output [M, N]
      uint16_t* dst = e.out + t * e.N + col0;
      if (col0 + pr.col_lo + 8 <= e.N) __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(dst + pr.col_lo));
      if (col0 + pr.col_hi + 8 <= e.N) __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(dst + pr.col_hi));
    }
  }
}

// Split-K mode (SPLIT): kernel arguments of a launch_tile_dma_split launch.
struct TileSplit {
  int ksplit;          // K ranges per tile
  int ctl;             // bit 0: every split counts as misplaced (recompute path, for tests)
  int max_spins;       // polls of the arrival word before a split hands its rows off
  float* part;         // fp32 partials: [tile][split][chunk 0..MB*NB*4-1][thread] of f32x4
  uint32_t* counters;  // arrival counter per tile; kDecodeRecomputeWord counts recomputed tiles
};

constexpr uint64_t kSplitForced = uint64_t(1) << 24;  // arrival increment of a split forced to recompute

__device__ __forceinline__ int hw_xcc_id() {
  return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));  // hwreg(HW_REG_XCC_ID, 0, 4)
}

// Exchange area of a pair-tile launch (in the workspace, see launch_pair_tile).
struct PairX {
  uint32_t* words;  // pair q's word at words[q * kSplitLineBytes / 4]: bit s = side s has published its
                    // half's row sums of squares, bit 2 + s = side s has handed its half over; zero
                    // between launches (the pair's last reader clears it)
  float* sumsq;     // [pair][side][BM]: each side's half-head sum of squares per row
  float* handoff;   // [pair][BM][64]: fp32 half-head values of a side that handed its half over
  int max_spins;    // polls of the pair word before a side hands its half over
  int hold;         // (tests) side 1 sleeps this many ~4 us intervals before publishing,
                    // so that side 0's bounded wait runs out and it hands its half over
  int cross;        // (tests) the sides of a pair take adjacent workgroup ids, which the
                    // round-robin dispatch places on different XCDs
};

// Epilogue of a pair tile: the NH whole heads as tile_epilogue, then this side's
// half of the shared head h_pair + NH.  The half holds head dims 32*side + [0, 32)
// and 32*side + [64, 96), which are the runs of threads c8 = 4*side + (0..3) of the
// whole-head epilogue, so every RoPE pair is local to the tile.  Its RMSNorm needs
// the other half's sum of squares: each side publishes its rows' sums (the first
// two butterfly levels of head_sum over its four runs; the third level, own + other,
// gives the bits of the whole-head epilogue) and sets its bit in the pair word, runs
// its whole heads, then reads the partner's sums.  A side that polls max_spins
// times without seeing the partner's bit hands its fp32 half over instead (values,
// then bit 2 + side); the partner, arriving later, sees that bit and finishes both
// halves.  Published data uses agent-scope (device-coherent) stores and loads, so
// the two sides may run on any XCDs.  V heads (and plain outputs) need no exchange.
template <int BM, int NH, int WM, int WN, int THREADS, int MB, int NB, class AV, class RowV, class SlotV>
__device__ __forceinline__ void pair_epilogue(const AV (&acc)[MB][NB], RowV prow, SlotV cslot,
                                              int h_pair, int side, int pair, int64_t m0, const ProblemArgs& p,
                                              const EpilogueArgs& e, unsigned char* smem, const PairX& px) {
  using Blk = AccBlock<AV>;
  constexpr int kTM = BM / WM;
  constexpr int kTN = NB * Blk::kDim;
  constexpr int kHalf0 = NH * kHeadDim;  // first tile column of the shared half
  constexpr int kHStep = THREADS / 4;    // rows of one half pass (4 threads per row)
  constexpr int kHPasses = BM / kHStep;
  static_assert(BM % kHStep == 0, "the half passes must cover the tile");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int c4 = tid & 3;
  float* ep = reinterpret_cast<float*>(smem);
  __shared__ uint32_t xword;
  int proj, hh;
  split_head(h_pair + NH, e.Hq, e.Hkv, proj, hh);
  const bool qk = e.qkv == 1 && proj != 2;
  const int head0 = h_pair + side * (NH + 1);
  // RoPE table rows and paged-KV-cache slots of the whole-head epilogue's rows
  // (tid / 8 + q * THREADS / 8)
#pragma unroll
  for (int q = 0; q < BM / (THREADS / 8); ++q) {
    const int64_t t = m0 + (tid >> 3) + q * (THREADS / 8);
    prow[q] = (e.qkv && t < p.M) ? int32_t(rope_row(e, t)) : 0;
    cslot[q] = (e.qkv && t < p.M) ? paged_slot(e, t) : -1;
  }

  // the half's accumulator columns -> ep[row][0, 64)
  auto stage_half = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = wn * kTN + nb * Blk::kDim;
      if (col >= kHalf0) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < Blk::kElems; ++i) {
            const int row = wm * kTM + mb * Blk::kDim + Blk::row(i, lane);
            ep[row * kEpiPitch + (col - kHalf0) + Blk::col(lane)] = acc[mb][nb][i];
          }
      }
    }
  };
  // this thread's runs of row r: half columns [8*c4, +8) and [32 + 8*c4, +8)
  auto read_row = [&](int r, float (&lo)[8], float (&hi)[8]) __attribute__((always_inline)) {
    const float* rowp = ep + r * kEpiPitch;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const f32x4_t a = *reinterpret_cast<const f32x4_t*>(rowp + 8 * c4 + 4 * v);
      const f32x4_t b = *reinterpret_cast<const f32x4_t*>(rowp + 32 + 8 * c4 + 4 * v);
      lo[4 * v] = a.x; lo[4 * v + 1] = a.y; lo[4 * v + 2] = a.z; lo[4 * v + 3] = a.w;
      hi[4 * v] = b.x; hi[4 * v + 1] = b.y; hi[4 * v + 2] = b.z; hi[4 * v + 3] = b.w;
    }
  };
  // sum of squares of the row's half: run_sumsq, then head_sum's first two levels
  auto half_sumsq = [&](const float (&lo)[8], const float (&hi)[8]) __attribute__((always_inline)) {
    float v = run_sumsq(lo, hi);
    v += dpp_move<0xB1>(v);  // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);  // quad_perm [2,3,0,1]
    return v;
  };
  // norm (qk: with the other half's sums `other`), RoPE and stores of side s's half from ep
  auto finish_half = [&](int s, const float* other) __attribute__((always_inline)) {
    const PairRuns pr = pair_runs(4 * s + c4, kHeadDim);
#pragma unroll
    for (int q = 0; q < kHPasses; ++q) {
      const int r = (tid >> 2) + q * kHStep;
      const int64_t t = m0 + r;
      const bool valid = t < p.M;
      float lo[8], hi[8];
      read_row(r, lo, hi);
      if (qk) {
#pragma clang fp contract(off)
        const float own = half_sumsq(lo, hi);
        const float ss = own + __hip_atomic_load(other + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float rms = head_rms(ss, e.eps, kHeadDim);
        const int64_t base = (valid ? rope_row(e, t) : 0) * kHeadDim;
        u32x4_t c2[2], s2[2];
        c2[0] = *reinterpret_cast<const u32x4_t*>(e.cos + base + pr.dim_lo);
        c2[1] = *reinterpret_cast<const u32x4_t*>(e.cos + base + pr.dim_hi);
        s2[0] = *reinterpret_cast<const u32x4_t*>(e.sin + base + pr.dim_lo);
        s2[1] = *reinterpret_cast<const u32x4_t*>(e.sin + base + pr.dim_hi);
        const uint16_t* gam = pick3<const uint16_t>(proj, e.q_gamma, e.k_gamma, e.k_gamma);
        const u32x4_t g0 = *reinterpret_cast<const u32x4_t*>(gam + pr.dim_lo);
        const u32x4_t g1 = *reinterpret_cast<const u32x4_t*>(gam + pr.dim_hi);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int wd = i >> 1, sh = (i & 1) * 16;
          norm_rope_pair(lo[i], hi[i], rms, bf16_to_f32((g0[wd] >> sh) & 0xFFFFu),
                         bf16_to_f32((g1[wd] >> sh) & 0xFFFFu), c2, s2, wd, sh);
        }
      }
      if (!valid) continue;
      u32x4_t o1, o2;
      o1.x = pack_bf16x2(lo[0], lo[1]); o1.y = pack_bf16x2(lo[2], lo[3]);
      o1.z = pack_bf16x2(lo[4], lo[5]); o1.w = pack_bf16x2(lo[6], lo[7]);
      o2.x = pack_bf16x2(hi[0], hi[1]); o2.y = pack_bf16x2(hi[2], hi[3]);
      o2.z = pack_bf16x2(hi[4], hi[5]); o2.w = pack_bf16x2(hi[6], hi[7]);
      const int H = proj == 0 ? e.Hq : e.Hkv;
      uint16_t* obase = pick3<uint16_t>(proj, e.q, e.k, e.v);  // k / v may be null (cache only)
      if (obase) {
        uint16_t* dst = obase + (t * H + hh) * kHeadDim;
        __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(dst + pr.dim_lo));
        __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(dst + pr.dim_hi));
      }
      const int64_t slot = proj != 0 ? paged_slot(e, t) : -1;
      if (slot >= 0) {
        uint16_t* crow = paged_row(e, slot, proj, hh);
        __builtin_nontemporal_store(o1, reinterpret_cast<u32x4_t*>(crow + pr.dim_lo));
        __builtin_nontemporal_store(o2, reinterpret_cast<u32x4_t*>(crow + pr.dim_hi));
      }
    }
  };

  if (!qk) {  // a V head: each side stores its half as it is
    tile_epilogue<BM, NH, WM, WN, THREADS>(acc, prow, cslot, head0, m0, p, e, smem);
    stage_half();
    __syncthreads();
    finish_half(side, nullptr);
    return;
  }
  uint32_t* word = px.words + size_t(pair) * (kSplitLineBytes / 4);
  float* const ss_mine = px.sumsq + (size_t(pair) * 2 + side) * BM;
  float* const ss_other = px.sumsq + (size_t(pair) * 2 + (side ^ 1)) * BM;
  const uint32_t p_other = 1u << (side ^ 1), h_other = 4u << (side ^ 1);
  // ---- publish this half's sums of squares --------------------------------------
  if (side == 1)
    for (int n = 0; n < px.hold; ++n) __builtin_amdgcn_s_sleep(127);
  stage_half();
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kHPasses; ++q) {
    const int r = (tid >> 2) + q * kHStep;
    float lo[8], hi[8];
    read_row(r, lo, hi);
    const float v = half_sumsq(lo, hi);
    if (c4 == 0) __hip_atomic_store(ss_mine + r, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's sums have been written
  __syncthreads();                                    // ... and every thread's
  if (tid == 0) xword = __hip_atomic_fetch_or(word, 1u << side, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const uint32_t seen = xword;
  // ---- the whole heads (their barriers separate the reads of xword from its next write)
  tile_epilogue<BM, NH, WM, WN, THREADS>(acc, prow, cslot, head0, m0, p, e, smem);
  bool other_half = false, clear = false;
  if (seen & p_other) {
    // the partner published first: it clears the word, unless it handed its half over
    other_half = (seen & h_other) != 0;
    clear = other_half;
  } else {
    if (tid == 0) {
      uint32_t v = 0;
      for (int n = 0;; ++n) {
        v = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((v & p_other) || n >= px.max_spins) break;
        __builtin_amdgcn_s_sleep(2);
      }
      xword = v;
    }
    __syncthreads();
    if (!(xword & p_other)) {
      // no partner yet: hand this half over (values, then the bit)
      stage_half();
      __syncthreads();
      float* dst = px.handoff + size_t(pair) * BM * 64;
#pragma unroll
      for (int q = 0; q < kHPasses; ++q) {
        const int r = (tid >> 2) + q * kHStep;
        float lo[8], hi[8];
        read_row(r, lo, hi);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __hip_atomic_store(dst + r * 64 + 8 * c4 + i, lo[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(dst + r * 64 + 32 + 8 * c4 + i, hi[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) xword = __hip_atomic_fetch_or(word, 4u << side, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      if (!(xword & p_other)) return;  // the partner will finish this half
    }
    clear = true;  // the partner has published and no longer reads the word
  }
  // ---- finish this half (and the partner's, if it handed it over) -------------------
  stage_half();
  __syncthreads();
  finish_half(side, ss_other);
  if (other_half) {
    __syncthreads();  // ep is reloaded with the partner's values
    const float* src = px.handoff + size_t(pair) * BM * 64;
#pragma unroll
    for (int q = 0; q < kHPasses; ++q) {
      const int r = (tid >> 2) + q * kHStep;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ep[r * kEpiPitch + 8 * c4 + i] =
            __hip_atomic_load(src + r * 64 + 8 * c4 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ep[r * kEpiPitch + 32 + 8 * c4 + i] =
            __hip_atomic_load(src + r * 64 + 32 + 8 * c4 + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    finish_half(side ^ 1, ss_mine);
  }
  if (clear && tid == 0) __hip_atomic_store(word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The pipelined tile kernel.  XC == 0: one workgroup per BM x (NH*128) tile of
// whole heads (px unused).  XC == 64: a pair tile: the heads
// [h0, h0 + 2*NH + 1) of a pair are covered by two workgroups, side 0 holding
// heads h0 .. h0+NH-1 and half of head h0+NH, side 1 the other half of that head
// and heads h0+NH+1 .. h0+2NH; pair_epilogue finishes the shared head.
template <int BM, int NH, int WM, int WN, int NS, int SBK, int XC = 0>
__global__ void __launch_bounds__(WM* WN * 64)
tile_dma_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int group_m, PairX px) {
  using S = DmaShape<BM, NH, WM, WN, NS, SBK, XC>;
  constexpr int kRowBytes = S::kRowBytes;
  __shared__ __attribute__((aligned(16))) unsigned char smem[S::kLdsBytes];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (uniform: load bases and LDS offsets in SGPRs)
  const int wm = wave % WM;
  const int wn = wave / WM;

  // ---- tile coordinates: XCD-contiguous ids, grouped along M ------------------
  // (pair tiles: the two sides of a pair are consecutive tile ids, so they share
  // an XCD and a round of the grid; the grouping runs over pairs)
  const int n_mt = int((p.M + BM - 1) / BM);
  const int n_ht = XC ? p.n_tiles / (2 * NH + 1) : p.n_tiles / NH;
  const int tile0 = (XC && px.cross) ? int(blockIdx.x) : xcd_tile_id(blockIdx.x, gridDim.x, p.xcds);
  const int side = XC ? (tile0 & 1) : 0;
  const int tile = XC ? (tile0 >> 1) : tile0;
  const int per_group = group_m * n_ht;
  const int grp = tile / per_group;
  const int first_m = grp * group_m;
  const int gsz = min(group_m, n_mt - first_m);
  const int rr = tile - grp * per_group;
  const int mt = first_m + rr % gsz;
  const int ht = rr / gsz;  // (pair tiles: the pair's index along the heads)
  const int64_t m0 = int64_t(mt) * BM;
  // first head of the tile's whole heads, and (pair tiles) the shared head
  const int h_pair = ht * (2 * NH + 1);
  const int head0 = XC ? h_pair + side * (NH + 1) : ht * NH;

  // Epilogue geometry: thread -> rows (tid / 8) + q * kRowStep and the column pairs
  // [8c, 8c+8) / [64+8c, +8) of every head.  The RoPE table row of each of its
  // rows (a positions[] load in positions mode) is read now, under the main loop.
  constexpr int kRowStep = S::kThreads / 8;
  constexpr int kPasses = BM / kRowStep;
  // (vector types: indexed in registers even where the compiler merges the
  // per-row code paths, where a plain array would go to scratch memory)
  typedef int32_t RowV __attribute__((ext_vector_type(kPasses)));
  // (pair tiles: 32-bit slots, so that the epilogue's row state fits beside the
  // accumulators; their launch requires caches of fewer than 2^31 slots)
  typedef typename std::conditional<XC != 0, int32_t, int64_t>::type SlotT;
  typedef SlotT SlotV __attribute__((ext_vector_type(kPasses)));
  RowV prow;
  SlotV cslot;  // paged-KV-cache slot of the row (-1: none)
#pragma unroll
  for (int q = 0; q < kPasses; ++q) {
    const int64_t t = m0 + (tid >> 3) + q * kRowStep;
    // (pair tiles look the rows and slots up in their epilogue: held through the
    // main loop beside 160 accumulators they would spill)
    prow[q] = (!XC && e.qkv && t < p.M) ? int32_t(rope_row(e, t)) : 0;
    cslot[q] = (!XC && e.qkv && t < p.M) ? paged_slot(e, t) : -1;
  }
  const int64_t K = p.K;

  // ---- this lane's sources: load instruction i of a stage fills staged rows
  // [R*(wave + i*W), +R), R = rows per load; lane -> row +lane/chunks, slot lane%chunks.
  // Each load's source is a wave-uniform base (the tile's first x row, or the first
  // weight row of the load's head) plus a small per-lane byte offset (at most the
  // tile's rows x K x 2 bytes) plus the stage's k offset; loads i < kALoads fill x
  // rows, the others weight rows of one head each.
  uint32_t voff[S::kLoadsPerWave];
  const uint16_t* lbase[S::kLoadsPerWave];  // the load's base (x: the tile's first row; weights: the head's)
  uint32_t dst_off[S::kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < S::kLoadsPerWave; ++i) {
    const int row0 = S::kRowsPerLoad * (wave + i * S::kWaves);
    const int row = row0 + lane / S::kChunks;
    const int chunk = stage_slot<SBK>(row, lane % S::kChunks);  // global chunk stored in slot lane % chunks
    if (i < S::kALoads) {
      int64_t grow = m0 + row;
      grow = grow < p.M ? grow : p.M - 1;  // rows past M re-read the last row; never stored
      lbase[i] = p.x + m0 * K;
      voff[i] = uint32_t(((grow - m0) * K + chunk * 8) * 2);
    } else {
      const int brow = row - BM;
      int proj, hh, head = head0 + brow / kHeadDim, dim = brow % kHeadDim;
      if (XC && brow >= NH * kHeadDim) {  // the shared head's half: dims 32*side + [0, 32) and + [64, 96)
        const int u = brow - NH * kHeadDim;
        head = h_pair + NH;
        dim = (u < 32 ? u : u + 32) + 32 * side;
      }
      split_head(head, e.Hq, e.Hkv, proj, hh);
      int64_t col = int64_t(hh) * kHeadDim + dim;
      col = col < w.n_cols[proj] ? col : w.n_cols[proj] - 1;
      // (one head's rows per load: its base, the head's first row, is wave-uniform)
      const uint16_t* hb = pick3<const uint16_t>(proj, w.w[0], w.w[1], w.w[2]) + int64_t(hh) * kHeadDim * K;
      lbase[i] = hb;
      voff[i] = uint32_t(((col - int64_t(hh) * kHeadDim) * K + chunk * 8) * 2);
    }
    dst_off[i] = uint32_t(row0 * kRowBytes);
  }
  // input RMSNorm: scale of the x row and k offset of the chunk each of this
  // lane's x loads brings in (load i < kALoads, row0 + lane / chunks, slot lane % chunks)
  const bool in_norm = p.in_gamma != nullptr;
  float a_scale[S::kALoads];
  int a_koff[S::kALoads];
#pragma unroll
  for (int i = 0; i < S::kALoads; ++i) {
    const int row = S::kRowsPerLoad * (wave + i * S::kWaves) + lane / S::kChunks;
    int64_t grow = m0 + row;
    grow = grow < p.M ? grow : p.M - 1;
    a_scale[i] = in_norm ? p.in_scale[grow] : 1.f;
    a_koff[i] = stage_slot<SBK>(row, lane % S::kChunks) * 8;
  }
  if (in_norm) {
    stage_gamma<S::kThreads>(p);
    __syncthreads();
  }
  auto issue = [&](int kt) {
    const uint32_t base = lds0 + uint32_t((kt % NS) * S::kStageBytes);
    const uint32_t koff = uint32_t(kt) * (SBK * 2);
#pragma unroll
    for (int i = 0; i < S::kLoadsPerWave; ++i)
      dma16(reinterpret_cast<const char*>(lbase[i]) + voff[i] + koff, base + dst_off[i]);
  };

  // ---- main loop -------------------------------------------------------------------
  // 16 x 16 accumulator blocks (v_mfma_f32_16x16x32_bf16): measured on MI355X, this
  // loop alone ran 6-7 % faster than with 32 x 32 blocks (2 % for the whole kernel
  // on config 2, 5 % on config 4), with the same results
  constexpr int kMB = S::kTM / 16, kNB = S::kTN / 16;
  f32x4_t acc[kMB][kNB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) acc[mb][nb] = f32x4_t{};

  const int c16 = lane & 15;
  const int kq = lane >> 4;
  const int nkt = int(K / SBK);
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nkt) issue(s);

  for (int kt = 0; kt < nkt; ++kt) {
    const int ahead = min(NS - 2, nkt - 1 - kt);  // stages already issued after kt
    wait_stage<NS, S::kLoadsPerWave>(ahead);
    if (in_norm) {  // this wave's x chunks of stage kt have landed: normalise them in place
#pragma unroll
      for (int i = 0; i < S::kALoads; ++i)
        norm_chunk(smem + (kt % NS) * S::kStageBytes + dst_off[i] + lane * 16, int64_t(kt) * SBK + a_koff[i],
                   a_scale[i]);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    barrier();
    if (kt + NS - 1 < nkt) issue(kt + NS - 1);
    const unsigned char* st = smem + (kt % NS) * S::kStageBytes;
#pragma unroll
    for (int ks = 0; ks < SBK / 32; ++ks) {
      const int chunk = 4 * ks + kq;  // this lane's 8 k of the 32-wide step
      u32x4_t af[kMB], bf[kNB];
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        const int row = wm * S::kTM + mb * 16 + c16;
        af[mb] = *reinterpret_cast<const u32x4_t*>(st + row * kRowBytes + stage_slot<SBK>(row, chunk) * 16);
      }
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb) {
        const int row = BM + wn * S::kTN + nb * 16 + c16;
        bf[nb] = *reinterpret_cast<const u32x4_t*>(st + row * kRowBytes + stage_slot<SBK>(row, chunk) * 16);
      }
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb) acc[mb][nb] = mfma_16x16x32(af[mb], bf[nb], acc[mb][nb]);
    }
  }
  barrier();  // every wave is done with the ring; the epilogue reuses the LDS

  if constexpr (XC != 0)
    pair_epilogue<BM, NH, WM, WN, S::kThreads>(acc, prow, cslot, h_pair, side, mt * n_ht + ht, m0, p, e, smem, px);
  else
    tile_epilogue<BM, NH, WM, WN, S::kThreads>(acc, prow, cslot, head0, m0, p, e, smem);
}

// The split-K launch of the pipelined kernel (a separate kernel, so that the
// one-workgroup-per-tile kernel above keeps its own register allocation).
template <int BM, int NH, int WM, int WN, int NS, int SBK, bool INORM>
__global__ void __launch_bounds__(WM* WN * 64)
tile_dma_split_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, TileSplit sp) {
  using S = DmaShape<BM, NH, WM, WN, NS, SBK>;
  constexpr int kRowBytes = S::kRowBytes;
  constexpr int BN = S::kBN;
  static_assert(S::kTM % 32 == 0 && S::kTN % 32 == 0, "wave tile (32 x 32 accumulator blocks)");
  __shared__ __attribute__((aligned(16))) unsigned char smem[S::kLdsBytes];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;

  // ---- tile and split of this workgroup ----------------------------------------
  const int n_mt = int((p.M + BM - 1) / BM);
  const int n_ht = p.n_tiles / NH;
  int mt, ht, split = 0, tile = 0;
  int hw_xcd = 0;
  {
    // Workgroups go round-robin over the X XCDs (from a starting XCD that depends
    // on the hardware queue), so the workgroups b with one b % X share an XCD.
    // That group takes tiles [x*tpx, (x+1)*tpx), x = b % X, all splits of each (so
    // a tile's partials meet in one L2); row tiles vary fastest, so an XCD's
    // tiles share weight panels.
    const int X = p.xcds;
    const int tiles = n_mt * n_ht;
    const int tpx = (tiles + X - 1) / X;
    const int xcd = int(blockIdx.x) % X;
    const int l = int(blockIdx.x) / X;
    split = l % sp.ksplit;
    const int slot = l / sp.ksplit;
    tile = xcd * tpx + slot;
    if (slot >= tpx || tile >= tiles) return;  // grid padding
    mt = tile % n_mt;
    ht = tile / n_mt;
    hw_xcd = hw_xcc_id() % X;
  }
  const int64_t m0 = int64_t(mt) * BM;

  const int64_t K = p.K;

  // ---- this lane's sources: load instruction i of a stage fills staged rows
  // [R*(wave + i*W), +R), R = rows per load; lane -> row +lane/chunks, slot lane%chunks
  const uint16_t* src[S::kLoadsPerWave];
  uint32_t dst_off[S::kLoadsPerWave];
#pragma unroll
  for (int i = 0; i < S::kLoadsPerWave; ++i) {
    const int row0 = S::kRowsPerLoad * (wave + i * S::kWaves);
    const int row = row0 + lane / S::kChunks;
    const int chunk = stage_slot<SBK>(row, lane % S::kChunks);  // global chunk stored in slot lane % chunks
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
  // input RMSNorm: scale of the x row and k offset of the chunk each of this
  // lane's x loads brings in (load i < kALoads, row0 + lane / chunks, slot lane % chunks)
  constexpr bool in_norm = INORM;  // (p.in_gamma != nullptr: a template switch keeps its registers out of the plain kernel)
  float a_scale[S::kALoads];
  int a_koff[S::kALoads];
#pragma unroll
  for (int i = 0; i < S::kALoads; ++i) {
    const int row = S::kRowsPerLoad * (wave + i * S::kWaves) + lane / S::kChunks;
    int64_t grow = m0 + row;
    grow = grow < p.M ? grow : p.M - 1;
    a_scale[i] = in_norm ? p.in_scale[grow] : 1.f;
    a_koff[i] = stage_slot<SBK>(row, lane % S::kChunks) * 8;
  }
  if (in_norm) {
    stage_gamma<S::kThreads>(p);
    __syncthreads();
  }
  // stage j of a k range starting at stage kt0 goes to ring slot j % NS
  auto issue = [&](int kt0, int j) {
    const uint32_t base = lds0 + uint32_t((j % NS) * S::kStageBytes);
#pragma unroll
    for (int i = 0; i < S::kLoadsPerWave; ++i) {
      dma16(src[i] + int64_t(kt0 + j) * SBK, base + dst_off[i]);
    }
  };

  // ---- main loop over stages [kt0, kt0 + nkt) -------------------------------------
  f32x16_t acc[S::kMB][S::kNB];
  const int c32 = lane & 31;
  const int khalf = lane >> 5;
  auto run_range = [&](int kt0, int nkt) {
#pragma unroll
    for (int mb = 0; mb < S::kMB; ++mb)
#pragma unroll
      for (int nb = 0; nb < S::kNB; ++nb) acc[mb][nb] = f32x16_t{};
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
      if (s < nkt) issue(kt0, s);

    for (int kt = 0; kt < nkt; ++kt) {
      const int ahead = min(NS - 2, nkt - 1 - kt);  // stages already issued after kt
      wait_stage<NS, S::kLoadsPerWave>(ahead);
      if (in_norm) {  // this wave's x chunks of stage kt have landed: normalise them in place
#pragma unroll
        for (int i = 0; i < S::kALoads; ++i)
          norm_chunk(smem + (kt % NS) * S::kStageBytes + dst_off[i] + lane * 16,
                     int64_t(kt0 + kt) * SBK + a_koff[i], a_scale[i]);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
      barrier();
      if (kt + NS - 1 < nkt) issue(kt0, kt + NS - 1);
      const unsigned char* st = smem + (kt % NS) * S::kStageBytes;
#pragma unroll
      for (int ks = 0; ks < SBK / 16; ++ks) {
        const int chunk = 2 * ks + khalf;
        u32x4_t af[S::kMB], bf[S::kNB];
#pragma unroll
        for (int mb = 0; mb < S::kMB; ++mb) {
          const int row = wm * S::kTM + mb * 32 + c32;
          af[mb] = *reinterpret_cast<const u32x4_t*>(st + row * kRowBytes + stage_slot<SBK>(row, chunk) * 16);
        }
#pragma unroll
        for (int nb = 0; nb < S::kNB; ++nb) {
          const int row = BM + wn * S::kTN + nb * 32 + c32;
          bf[nb] = *reinterpret_cast<const u32x4_t*>(st + row * kRowBytes + stage_slot<SBK>(row, chunk) * 16);
        }
#pragma unroll
        for (int mb = 0; mb < S::kMB; ++mb)
#pragma unroll
          for (int nb = 0; nb < S::kNB; ++nb) {
            acc[mb][nb] = mfma_32x32x16(af[mb], bf[nb], acc[mb][nb]);
          }
      }
    }
    barrier();  // every wave is done with the ring; the epilogue (or the next range) reuses the LDS
  };

  const int nkt_all = int(K / SBK);
  {  // ---- split-K: this split's range, its partial, the arrival, the finish ----
    constexpr int kChunks = S::kMB * S::kNB * 4;  // f32x4 chunks of a thread's accumulators
    const int ns = sp.ksplit;
    auto range_of = [&](int sidx, int& kt0, int& nk) {
      kt0 = int((int64_t(sidx) * nkt_all) / ns);
      nk = int((int64_t(sidx + 1) * nkt_all) / ns) - kt0;
    };
    // chunk c of this thread in split sidx's partial: 16-byte stores / loads,
    // 1 KB contiguous per wave instruction
    auto part_at = [&](int sidx, int c) {
      return reinterpret_cast<f32x4_t*>(sp.part) + ((int64_t(tile) * ns + sidx) * kChunks + c) * S::kThreads + tid;
    };
    // skip: units whose rows this workgroup finishes itself (not written)
    auto publish = [&](int sidx, uint32_t skip) {
#pragma unroll
      for (int mb = 0; mb < S::kMB; ++mb)
        if (!((skip >> (wm * S::kMB + mb)) & 1u))
#pragma unroll
        for (int nb = 0; nb < S::kNB; ++nb)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *part_at(sidx, (mb * S::kNB + nb) * 4 + q) =
                f32x4_t{acc[mb][nb][4 * q], acc[mb][nb][4 * q + 1], acc[mb][nb][4 * q + 2], acc[mb][nb][4 * q + 3]};
    };
    // ---- this split's range and partial, then the arrival --------------------------
    // The tile's rows form U = WM * MB units of 32 (unit u: rows [32u, 32u+32),
    // held by waves wm = u / MB in accumulator block mb = u % MB).  Split s
    // finishes units [s*U/ns, (s+1)*U/ns) once every split has arrived, reading
    // only those rows of the ns partials.  Arrival word (64-bit): bits 0-7 count
    // the splits, bits 8-23 mark splits whose wait ran out (their units go to the
    // last arrival), bits 24-31 count splits forced onto the recompute path, and
    // bits 32-49 sum the splits' XCDs and their squares; when some split ran on
    // another XCD than the others (or was forced), the last arrival recomputes the
    // whole tile and the others leave.  The
    // recomputation reuses the one main loop below (a second inlined copy of it
    // would spill).
    constexpr int U = WM * S::kMB;
    uint64_t* arrive_word =
        reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(sp.counters) + kSplitWordsOffset + tile * kSplitLineBytes);
    uint32_t* exit_word = reinterpret_cast<uint32_t*>(arrive_word + 1);
    __shared__ uint64_t seen_word;
    // Every split leaves through here once it no longer reads the arrival word;
    // the last to leave re-arms both words for the next launch.
    auto leave = [&]() {
      if (tid == 0 && __hip_atomic_fetch_add(exit_word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u ==
                          uint32_t(ns)) {
        __hip_atomic_store(arrive_word, uint64_t(0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(exit_word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    };
    auto arrived = [&](uint64_t w_) { return (w_ & 0xFFu) == uint64_t(ns); };
    // some split ran on another XCD than the others, or was forced to recompute:
    // the arrival sums the splits' XCDs x (bits 32-39) and x * x (bits 40-49), and
    // n * sum(x^2) == sum(x)^2 exactly when all n values are equal
    auto misplaced = [&](uint64_t w_) {
      const uint64_t sx = (w_ >> 32) & 0xFFu, sxx = (w_ >> 40) & 0x3FFu;
      return ((w_ >> 24) & 0xFFu) != 0 || uint64_t(ns) * sxx != sx * sx;
    };
    auto units_of = [&](int sidx) {
      const int u0 = sidx * U / ns, u1 = (sidx + 1) * U / ns;
      return u1 > u0 ? ((1u << u1) - 1u) & ~((1u << u0) - 1u) : 0u;
    };
    uint32_t units = 0;
    bool recompute = false;
    int sidx = split;
#pragma unroll 1
    for (;;) {
      int kt0, nk;
      range_of(sidx, kt0, nk);
      run_range(kt0, nk);
      publish(sidx, recompute ? 0u : units_of(split));
      __builtin_amdgcn_s_waitcnt(0);  // this thread's partial has reached the L2
      if (recompute) {
        if (++sidx < ns) continue;
        units = (1u << U) - 1u;
        break;
      }
      __syncthreads();  // ... and every thread's
      const uint64_t inc = 1u + ((sp.ctl & 1) ? kSplitForced : 0u) + (uint64_t(hw_xcd) << 32) +
                           (uint64_t(hw_xcd * hw_xcd) << 40);
      if (tid == 0)
        seen_word = __hip_atomic_fetch_add(arrive_word, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
      __syncthreads();
      uint64_t v = seen_word;
      units = units_of(split);
      if (!arrived(v)) {
        if (units == 0) {  // nothing of this tile to finish here
          leave();
          return;
        }
        if (tid == 0) {
          // bounded wait for the other splits (they are normally resident and close)
          for (int spin = 0; !arrived(v) && spin < sp.max_spins; ++spin) {
            __builtin_amdgcn_s_sleep(2);
            v = __hip_atomic_load(arrive_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          seen_word = v;
        }
        __syncthreads();
        v = seen_word;
        if (!arrived(v)) {
          // hand this split's units to the last arrival: publish their rows too, then
          // mark the hand-off (unless the last split arrived meanwhile)
          publish(split, ~units);
          __builtin_amdgcn_s_waitcnt(0);
          __syncthreads();
          if (tid == 0)
            seen_word = __hip_atomic_fetch_or(arrive_word, uint64_t(1) << (8 + split), __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
          __syncthreads();
          v = seen_word;
        }
        if (!arrived(v) || misplaced(v)) {  // handed off, or the last arrival recomputes
          leave();
          return;
        }
        break;
      }
      if (misplaced(v)) {
        // A split ran on another XCD, so its partial may not be visible through
        // this L2: recompute every split here and publish each into this L2.
        if (tid == 0)
          __hip_atomic_fetch_add(sp.counters + kDecodeRecomputeWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        recompute = true;
        sidx = 0;
        continue;
      }
      for (int s2 = 0; s2 < ns; ++s2)
        if ((v >> (8 + s2)) & 1u) units |= units_of(s2);  // splits that handed off
      break;
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    leave();
    // ---- finish the units: every thread sums a share of a unit's fragment chunks
    // over the partials in split order into an LDS tile [32 rows][BN], then the
    // unit's rows get norm, RoPE and 16-byte stores.  This split's own rows come
    // from its registers through LDS (it did not publish them), except on the
    // recompute path, where every split was published.
    const int mine = recompute ? -1 : split;
    const uint32_t own_units = recompute ? 0u : units_of(split);
    constexpr int kUC = S::kNB * 4;              // f32x4 chunks per thread of a unit's waves
    constexpr int kUThreads = WN * 64;           // threads holding one unit (one wm)
    constexpr int kItems = kUC * kUThreads;      // f32x4 chunks of a unit
    static_assert(kItems % S::kThreads == 0, "unit chunks per thread");
    constexpr int kPer = kItems / S::kThreads;
    constexpr int kBatch = 1;                    // splits whose loads are in flight together (2 spill)
    constexpr int kTPitch = BN + 4;              // fp32 pitch of the unit tile
    f32x4_t* own_buf = reinterpret_cast<f32x4_t*>(smem);                  // [kUC][kUThreads]
    float* utile = reinterpret_cast<float*>(smem + size_t(kItems) * 16);  // [32][kTPitch]
    static_assert(size_t(kItems) * 16 + 32 * kTPitch * 4 <= size_t(S::kLdsBytes), "unit finish LDS");
    // a unit chunk item -> (chunk c, thread r of the unit's waves)
    auto item_src = [&](int it, int sidx) {
      const int c = it / kUThreads, r = it % kUThreads;
      return reinterpret_cast<const f32x4_t*>(sp.part) +
             ((int64_t(tile) * ns + sidx) * kChunks + c) * S::kThreads + r;  // r is offset below
    };
#pragma unroll 1
    for (int u = 0; u < U; ++u) {
      if (!((units >> u) & 1u)) continue;
      const int uwm = u / S::kMB, umb = u % S::kMB;
      const bool own = (own_units >> u) & 1u;
      if (own && wm == uwm) {
#pragma unroll
        for (int mb = 0; mb < S::kMB; ++mb)  // (compile-time indices: acc stays in registers)
          if (mb == umb)
#pragma unroll
            for (int nb = 0; nb < S::kNB; ++nb)
#pragma unroll
              for (int q = 0; q < 4; ++q)
                own_buf[(nb * 4 + q) * kUThreads + wn * 64 + lane] =
                    f32x4_t{acc[mb][nb][4 * q], acc[mb][nb][4 * q + 1], acc[mb][nb][4 * q + 2], acc[mb][nb][4 * q + 3]};
      }
      __syncthreads();
      // the unit's threads sit at workgroup thread wn * 64 * WM ... : thread index of
      // (wave wm = uwm, wn) lane L is (wn * WM + uwm) * 64 + L
      f32x4_t v[kPer];
#pragma unroll 1
      for (int s0 = 0; s0 < ns; s0 += kBatch) {
        f32x4_t t[kBatch][kPer];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const int sidx = s0 + b;
#pragma unroll
          for (int i = 0; i < kPer; ++i) {
            const int it = tid + i * S::kThreads;
            const int c = it / kUThreads, r = it % kUThreads;
            if (sidx < ns && !(own && sidx == mine)) {
              const int th = ((r >> 6) * WM + uwm) * 64 + (r & 63);
              t[b][i] = *(reinterpret_cast<const f32x4_t*>(sp.part) +
                          ((int64_t(tile) * ns + sidx) * kChunks + umb * kUC + c) * S::kThreads + th);
            } else if (sidx < ns) {
              t[b][i] = own_buf[c * kUThreads + r];
            }
          }
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
#pragma unroll
          for (int i = 0; i < kPer; ++i)
            if (s0 + b < ns) v[i] = (s0 + b == 0) ? t[b][i] : v[i] + t[b][i];
      }
      // chunk c = nb*4 + q of unit thread r (wave wn = r / 64, lane L = r % 64) holds
      // rows 8q + 4*(L >> 5) + 0..3, column wn*TN + nb*32 + (L & 31) of the unit
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int it = tid + i * S::kThreads;
        const int c = it / kUThreads, r = it % kUThreads;
        const int nb = c >> 2, q = c & 3, L = r & 63;
        const int row = 8 * q + 4 * (L >> 5);
        const int col = (r >> 6) * S::kTN + nb * 32 + (L & 31);
        float* d = utile + row * kTPitch + col;
        d[0] = v[i].x;
        d[kTPitch] = v[i].y;
        d[2 * kTPitch] = v[i].z;
        d[3 * kTPitch] = v[i].w;
      }
      __syncthreads();
      finish_unit_rows<NH, S::kThreads>(utile, kTPitch, m0 + u * 32, ht, p, e);
      __syncthreads();  // the next unit reuses the LDS
    }
    (void)item_src;
  }
}

template <int BM, int NH, int WM, int WN, int NS, int SBK = 32>
hipError_t launch_dma(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                      hipStream_t stream) {
  using S = DmaShape<BM, NH, WM, WN, NS, SBK>;
  const int n_mt = int((p.M + BM - 1) / BM);
  const int blocks = n_mt * (p.n_tiles / NH);
  const size_t dyn = p.in_gamma ? size_t(p.K) * 2 : 0;
  if (S::kLdsBytes + dyn > 160 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL((tile_dma_kernel<BM, NH, WM, WN, NS, SBK>), dim3(blocks), dim3(S::kThreads), dyn, stream, p, w, e,
                     group_m < 1 ? 1 : group_m, PairX{});
  return hipGetLastError();
}

template <int BM, int NH, int WM, int WN, int NS, int SBK>
size_t split_part_bytes(int64_t M, int n_tiles, int ksplit) {
  using S = DmaShape<BM, NH, WM, WN, NS, SBK>;
  const int64_t tiles = (M + BM - 1) / BM * (n_tiles / NH);
  return size_t(tiles) * ksplit * S::kMB * S::kNB * 4 * S::kThreads * 16;
}

template <int BM, int NH, int WM, int WN, int NS, int SBK>
hipError_t launch_dma_split(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int ksplit,
                            int force_recompute, int max_spins, void* workspace, hipStream_t stream) {
  using S = DmaShape<BM, NH, WM, WN, NS, SBK>;
  const int n_mt = int((p.M + BM - 1) / BM);
  const int tiles = n_mt * (p.n_tiles / NH);
  const int X = p.xcds > 0 ? p.xcds : 1;
  const int tpx = (tiles + X - 1) / X;
  const size_t dyn = p.in_gamma ? size_t(p.K) * 2 : 0;
  // (p.xcds <= 8: the arrival word's XCD sums hold x < 8)
  if (S::kLdsBytes + dyn > 160 * 1024 || ksplit < 2 || ksplit > 16 || tiles > kSplitMaxTiles || p.xcds > 8 ||
      p.K / SBK < ksplit)
    return hipErrorInvalidValue;
  TileSplit sp;
  sp.ksplit = ksplit;
  sp.ctl = force_recompute ? 1 : 0;
  sp.max_spins = max_spins;
  sp.counters = static_cast<uint32_t*>(workspace);
  sp.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kDecodeCounterBytes);
  if (p.in_gamma) {
    // (no input-norm form of the 256-row tiles: its registers would spill)
    if constexpr (BM > 128) return hipErrorInvalidValue;
    else
      hipLaunchKernelGGL((tile_dma_split_kernel<BM, NH, WM, WN, NS, SBK, true>), dim3(X * ksplit * tpx),
                         dim3(S::kThreads), dyn, stream, p, w, e, sp);
  } else {
    hipLaunchKernelGGL((tile_dma_split_kernel<BM, NH, WM, WN, NS, SBK, false>), dim3(X * ksplit * tpx),
                       dim3(S::kThreads), dyn, stream, p, w, e, sp);
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// W4A16: the same pipeline with int4 weights.  A stage (64 k) holds the x rows
// (128-byte rows, as above), the packed weight words of its 8 k-groups
// ([k-group][BN] int32, 512-byte runs per head), and the scale and packed zero
// of every column (a stage lies inside one quantisation group: group % 64 == 0).
// Everything is filled with direct L2 -> LDS loads; the weights are dequantised
// ((q - z) * s in fp32, one bf16 rounding) from the LDS word right before the
// MFMA.  Weights take a quarter of the bf16 bytes, so the ring is deeper.
// ---------------------------------------------------------------------------
template <int BM, int NH, int WM, int WN, int NS>
struct W4Shape {
  static constexpr int kBN = NH * kHeadDim;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kTM = BM / WM;
  static constexpr int kTN = kBN / WN;
  static constexpr int kMB = kTM / 32;
  static constexpr int kNB = kTN / 32;
  static constexpr int kABytes = BM * 128;            // x: BM rows x 64 k
  static constexpr int kBBytes = 8 * kBN * 4;         // 8 k-groups x BN packed words
  static constexpr int kSBytes = kBN * 2;             // scales of the stage's group
  static constexpr int kZBytes = kBN / 2;             // zeros of the stage's group (nibbles)
  static constexpr int kStageBytes = (kABytes + kBBytes + kSBytes + kZBytes + 1023) / 1024 * 1024;
  static constexpr int kNA = BM / 8;                  // 1 KB loads: 8 x rows each
  static constexpr int kNW = kBN / 32;                // 1 KB loads: two 512-byte (k-group, head) runs
  static constexpr int kLoads = kNA + kNW + 2;        // + one for the scales, one for the zeros (4-byte loads)
  static constexpr int kMaxPerWave = (kLoads + kWaves - 1) / kWaves;
  static constexpr int kRingBytes = NS * kStageBytes;
  static constexpr int kEpiBytes = BM * kEpiPitch * 4;
  static constexpr int kLdsBytes = kRingBytes > kEpiBytes ? kRingBytes : kEpiBytes;
  static_assert(kTM % 32 == 0 && kTN % 32 == 0, "wave tile");
  static_assert(kBN / 8 <= 64, "the scale and the zero loads fit one instruction each");
  static_assert(NS >= 2 && NS <= 8 && kMaxPerWave * (NS - 2) <= 63, "stages");
  static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

template <int BM, int NH, int WM, int WN, int NS>
__global__ void __launch_bounds__(WM* WN * 64)
tile_dma_w4_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int group_m) {
  using S = W4Shape<BM, NH, WM, WN, NS>;
  constexpr int BN = S::kBN;
  __shared__ __attribute__((aligned(16))) unsigned char smem[S::kLdsBytes];
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WM;
  const int wn = wave / WM;

  // ---- tile coordinates (as the bf16 kernel) ------------------------------------------
  const int n_mt = int((p.M + BM - 1) / BM);
  const int n_ht = p.n_tiles / NH;
  const int tile = xcd_tile_id(blockIdx.x, gridDim.x, p.xcds);
  const int per_group = group_m * n_ht;
  const int grp = tile / per_group;
  const int first_m = grp * group_m;
  const int gsz = min(group_m, n_mt - first_m);
  const int rr = tile - grp * per_group;
  const int mt = first_m + rr % gsz;
  const int ht = rr / gsz;
  const int64_t m0 = int64_t(mt) * BM;
  const int64_t K = p.K;

  constexpr int kRowStep = S::kThreads / 8;
  constexpr int kPasses = BM / kRowStep;
  // (vector types: indexed in registers even where the compiler merges the
  // per-row code paths, where a plain array would go to scratch memory)
  typedef int32_t RowV __attribute__((ext_vector_type(kPasses)));
  typedef int64_t SlotV __attribute__((ext_vector_type(kPasses)));
  RowV prow;
  SlotV cslot;  // paged-KV-cache slot of the row (-1: none)
#pragma unroll
  for (int q = 0; q < kPasses; ++q) {
    const int64_t t = m0 + (tid >> 3) + q * kRowStep;
    prow[q] = (e.qkv && t < p.M) ? int32_t(rope_row(e, t)) : 0;
    cslot[q] = (e.qkv && t < p.M) ? paged_slot(e, t) : -1;
  }

  // ---- load slots: slot g of a stage is issued by wave g % W --------------------------
  // kind 0: x rows; 1: packed weights; 2: scales; 3: zeros.  Source of stage kt =
  // base + step(kt) * stride, step = kt (kinds 0, 1) or the group index (2, 3).
  const char* base[S::kMaxPerWave];
  int64_t stride[S::kMaxPerWave];
  uint32_t dst[S::kMaxPerWave];
  int kind[S::kMaxPerWave];
  bool active[S::kMaxPerWave];
  const int nslots = (S::kLoads - wave + S::kWaves - 1) / S::kWaves;
#pragma unroll
  for (int i = 0; i < S::kMaxPerWave; ++i) {
    const int g = wave + i * S::kWaves;
    base[i] = nullptr;
    stride[i] = 0;
    dst[i] = 0;
    kind[i] = 0;
    active[i] = false;
    if (g < S::kNA) {
      const int row = 8 * g + (lane >> 3);
      const int chunk = stage_slot<64>(row, lane & 7);
      int64_t grow = m0 + row;
      grow = grow < p.M ? grow : p.M - 1;  // rows past M re-read the last row; never stored
      base[i] = reinterpret_cast<const char*>(p.x + grow * K + chunk * 8);
      stride[i] = 128;
      dst[i] = uint32_t(g * 1024);
      active[i] = true;
    } else if (g < S::kNA + S::kNW) {
      const int sg = 2 * (g - S::kNA) + (lane >> 5);  // (k-group, head) run
      const int kg = sg / NH, j = sg % NH;
      int proj, hh;
      split_head(ht * NH + j, e.Hq, e.Hkv, proj, hh);
      const int64_t n = w.n_cols[proj];
      // (a plain GEMM's last tile may pass N: its columns past N, whole 16-byte
      // chunks as N % 8 == 0, re-read the last chunk and are never stored)
      int64_t c4 = int64_t(hh) * kHeadDim + (lane & 31) * 4;
      c4 = c4 + 4 <= n ? c4 : n - 4;
      base[i] = reinterpret_cast<const char*>(w.qw[proj] + kg * n + c4);
      stride[i] = 8 * n * 4;
      dst[i] = uint32_t(S::kABytes + (g - S::kNA) * 1024);
      kind[i] = 1;
      active[i] = true;
    } else if (g == S::kNA + S::kNW) {
      const int j = lane / 16;  // 16 lanes x 8 scales per head
      if (j < NH) {
        int proj, hh;
        split_head(ht * NH + j, e.Hq, e.Hkv, proj, hh);
        const int64_t n = w.n_cols[proj];
        int64_t c8 = int64_t(hh) * kHeadDim + (lane % 16) * 8;
        c8 = c8 + 8 <= n ? c8 : n - 8;
        base[i] = reinterpret_cast<const char*>(static_cast<const uint16_t*>(w.sc[proj]) + c8);
        stride[i] = n * 2;
        active[i] = true;
      }
      dst[i] = uint32_t(S::kABytes + S::kBBytes);
      kind[i] = 2;
    } else if (g == S::kNA + S::kNW + 1) {
      // zeros: one packed word (8 columns) per lane, 16 lanes per head (4-byte
      // loads, so a last tile past N never shifts a valid column's word)
      const int j = lane / 16;
      if (j < NH) {
        int proj, hh;
        split_head(ht * NH + j, e.Hq, e.Hkv, proj, hh);
        const int64_t n = w.n_cols[proj];
        int64_t wd = int64_t(hh) * (kHeadDim / 8) + (lane % 16);
        wd = wd < n / 8 ? wd : n / 8 - 1;
        base[i] = reinterpret_cast<const char*>(w.qz[proj] + wd);
        stride[i] = (n / 8) * 4;
        active[i] = true;
      }
      dst[i] = uint32_t(S::kABytes + S::kBBytes + S::kSBytes);
      kind[i] = 3;
    }
  }
  // input RMSNorm: scale of the x row and k offset of the chunk of each x load slot
  const bool in_norm = p.in_gamma != nullptr;
  float a_scale[S::kMaxPerWave];
  int a_koff[S::kMaxPerWave];
#pragma unroll
  for (int i = 0; i < S::kMaxPerWave; ++i) {
    const int g = wave + i * S::kWaves;
    const int row = 8 * g + (lane >> 3);
    int64_t grow = m0 + (row < BM ? row : 0);
    grow = grow < p.M ? grow : p.M - 1;
    a_scale[i] = (in_norm && g < S::kNA) ? p.in_scale[grow] : 1.f;
    a_koff[i] = stage_slot<64>(row, lane & 7) * 8;
  }
  if (in_norm) {
    stage_gamma<S::kThreads>(p);
    __syncthreads();
  }
  const int group = w.group;
  auto issue = [&](int kt) {
    const uint32_t sbase = lds0 + uint32_t((kt % NS) * S::kStageBytes);
    const int64_t gstep = (int64_t(kt) * 64) / group;
#pragma unroll
    for (int i = 0; i < S::kMaxPerWave; ++i) {
      if (i < nslots) {
        const int64_t stp = kind[i] >= 2 ? gstep : int64_t(kt);
        if (active[i]) {
          if (kind[i] == 3) dma4(base[i] + stp * stride[i], sbase + dst[i]);
          else dma16(base[i] + stp * stride[i], sbase + dst[i]);
        }
      }
    }
  };

  // 16 x 16 accumulator blocks (v_mfma_f32_16x16x32_bf16), as the bf16 tile kernel
  constexpr int kMB = S::kTM / 16, kNB = S::kTN / 16;
  f32x4_t acc[kMB][kNB];
#pragma unroll
  for (int mb = 0; mb < kMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) acc[mb][nb] = f32x4_t{};

  const int c16 = lane & 15;
  const int kq = lane >> 4;
  const bool fp16 = w.scale_fp16 != 0;
  const int nkt = int(K / 64);
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nkt) issue(s);

  for (int kt = 0; kt < nkt; ++kt) {
    const int ahead = min(NS - 2, nkt - 1 - kt);  // stages already issued after kt
    wait_vm_n(ahead * nslots);
    if (in_norm) {  // this wave's x chunks of stage kt have landed: normalise them in place
#pragma unroll
      for (int i = 0; i < S::kMaxPerWave; ++i)
        if (wave + i * S::kWaves < S::kNA)
          norm_chunk(smem + (kt % NS) * S::kStageBytes + dst[i] + lane * 16, int64_t(kt) * 64 + a_koff[i],
                     a_scale[i]);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    barrier();
    if (kt + NS - 1 < nkt) issue(kt + NS - 1);
    const unsigned char* st = smem + (kt % NS) * S::kStageBytes;
    float scl[kNB], zro[kNB];
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const int col = wn * S::kTN + nb * 16 + c16;
      const uint32_t sraw = *reinterpret_cast<const uint16_t*>(st + S::kABytes + S::kBBytes + col * 2);
      const uint32_t zw = *reinterpret_cast<const uint32_t*>(st + S::kABytes + S::kBBytes + S::kSBytes + (col / 8) * 4);
      scl[nb] = fp16 ? f16_to_f32(sraw) : bf16_to_f32(sraw);
      zro[nb] = float((zw >> ((col % 8) * 4)) & 0xFu);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int chunk = 4 * ks + kq;  // x chunk == weight k-group of this lane
      u32x4_t bf[kNB];
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb) {
        const int col = wn * S::kTN + nb * 16 + c16;
        const uint32_t word = *reinterpret_cast<const uint32_t*>(st + S::kABytes + (chunk * BN + col) * 4);
        bf[nb] = dequant_int4x8(word, zro[nb], scl[nb]);
      }
#pragma unroll
      for (int mb = 0; mb < kMB; ++mb) {
        const int row = wm * S::kTM + mb * 16 + c16;
        const u32x4_t af = *reinterpret_cast<const u32x4_t*>(st + row * 128 + stage_slot<64>(row, chunk) * 16);
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb) acc[mb][nb] = mfma_16x16x32(af, bf[nb], acc[mb][nb]);
      }
    }
  }
  barrier();  // every wave is done with the ring; the epilogue reuses the LDS
  tile_epilogue<BM, NH, WM, WN, S::kThreads>(acc, prow, cslot, ht * NH, m0, p, e, smem);
}

template <int BM, int NH, int WM, int WN, int NS, int SBK>
size_t pair_bytes(int64_t M, int n_tiles) {
  const int64_t pairs = (M + BM - 1) / BM * (n_tiles / (2 * NH + 1));
  return kDecodeCounterBytes + size_t(pairs) * (2 * BM + BM * 64) * sizeof(float);
}

template <int BM, int NH, int WM, int WN, int NS, int SBK>
hipError_t launch_pair(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                       void* workspace, int max_spins, hipStream_t stream) {
  using S = DmaShape<BM, NH, WM, WN, NS, SBK, 64>;
  if (p.n_tiles % (2 * NH + 1) != 0 || !workspace || e.head_dim != kHeadDim) return hipErrorInvalidValue;
  const int64_t pairs = (p.M + BM - 1) / BM * (p.n_tiles / (2 * NH + 1));
  if (pairs > kSplitMaxTiles) return hipErrorInvalidValue;
  const size_t dyn = p.in_gamma ? size_t(p.K) * 2 : 0;
  if (S::kLdsBytes + 16 + dyn > 160 * 1024) return hipErrorInvalidValue;  // (+ the exchange word)
  char* ws = static_cast<char*>(workspace);
  PairX px;
  px.words = reinterpret_cast<uint32_t*>(ws + kSplitWordsOffset);
  px.sumsq = reinterpret_cast<float*>(ws + kDecodeCounterBytes);
  px.handoff = px.sumsq + size_t(pairs) * 2 * BM;
  px.max_spins = max_spins < 0 ? 0 : max_spins;
  px.hold = g_pair_hold & 0xFFFF;
  px.cross = g_pair_hold >> 16;
  hipLaunchKernelGGL((tile_dma_kernel<BM, NH, WM, WN, NS, SBK, 64>), dim3(unsigned(pairs * 2)), dim3(S::kThreads), dyn,
                     stream, p, w, e, group_m < 1 ? 1 : group_m, px);
  return hipGetLastError();
}

template <int BM, int NH, int WM, int WN, int NS>
hipError_t launch_dma_w4(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                         hipStream_t stream) {
  using S = W4Shape<BM, NH, WM, WN, NS>;
  const int n_mt = int((p.M + BM - 1) / BM);
  const int blocks = n_mt * (p.n_tiles / NH);
  const size_t dyn = p.in_gamma ? size_t(p.K) * 2 : 0;
  if (S::kLdsBytes + dyn > 160 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL((tile_dma_w4_kernel<BM, NH, WM, WN, NS>), dim3(blocks), dim3(S::kThreads), dyn, stream, p, w,
                     e, group_m < 1 ? 1 : group_m);
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
    case 16: return launch_dma<128, 3, 2, 4, 2, 64>(p, w, e, group_m, stream);  // 128x384, 2 stages of 64 k
    case 17: return launch_dma<256, 2, 4, 2, 2, 64>(p, w, e, group_m, stream);  // 256x256, 2 stages of 64 k
    case 18: return launch_dma<256, 2, 2, 4, 2, 64>(p, w, e, group_m, stream);  // 256x256 (128x64 waves), 64 k
    case 19: return launch_dma<128, 1, 2, 2, 4, 64>(p, w, e, group_m, stream);  // 128x128, 4 waves, 4 stages of 64 k
    case 20: return launch_dma<64, 1, 1, 4, 4, 64>(p, w, e, group_m, stream);   // 64x128, 4 waves (64x32)
    case 21: return launch_dma<128, 1, 2, 4, 4, 64>(p, w, e, group_m, stream);  // 128x128, 8 waves (64x32)
    case 22: return launch_dma<256, 1, 4, 2, 3, 64>(p, w, e, group_m, stream);  // 256x128, 8 waves (64x64), 3 stages
    case 23: return launch_dma<128, 2, 2, 4, 3, 64>(p, w, e, group_m, stream);  // 128x256, 8 waves (64x64), 3 stages
    default: return hipErrorInvalidValue;
  }
}

int g_pair_hold = 0;

hipError_t launch_pair_tile(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                            void* workspace, int max_spins, hipStream_t stream) {
  switch (id) {
    case 24: return launch_pair<256, 1, 4, 2, 2, 64>(p, w, e, group_m, workspace, max_spins, stream);  // 256x192
    case 25: return launch_pair<256, 2, 4, 2, 2, 64>(p, w, e, group_m, workspace, max_spins, stream);  // 256x320
    case 26: return launch_pair<128, 1, 4, 2, 3, 64>(p, w, e, group_m, workspace, max_spins, stream);  // 128x192
    case 27: return launch_pair<128, 2, 4, 2, 2, 64>(p, w, e, group_m, workspace, max_spins, stream);  // 128x320
    case 28: return launch_pair<192, 1, 3, 2, 3, 64>(p, w, e, group_m, workspace, max_spins, stream);  // 192x192
    default: return hipErrorInvalidValue;
  }
}

size_t pair_tile_workspace_bytes(int id, int64_t M, int n_tiles) {
  switch (id) {
    case 24: return pair_bytes<256, 1, 4, 2, 2, 64>(M, n_tiles);
    case 25: return pair_bytes<256, 2, 4, 2, 2, 64>(M, n_tiles);
    case 26: return pair_bytes<128, 1, 4, 2, 3, 64>(M, n_tiles);
    case 27: return pair_bytes<128, 2, 4, 2, 2, 64>(M, n_tiles);
    case 28: return pair_bytes<192, 1, 3, 2, 3, 64>(M, n_tiles);
    default: return 0;
  }
}

// (pair tiles: their epilogue's exchange word adds one 16-byte LDS allocation)
constexpr int kPairWordLds = 16;

int tile_dma_lds_bytes(int id) {
  switch (id) {
    case 24: return DmaShape<256, 1, 4, 2, 2, 64, 64>::kLdsBytes + kPairWordLds;
    case 25: return DmaShape<256, 2, 4, 2, 2, 64, 64>::kLdsBytes + kPairWordLds;
    case 26: return DmaShape<128, 1, 4, 2, 3, 64, 64>::kLdsBytes + kPairWordLds;
    case 27: return DmaShape<128, 2, 4, 2, 2, 64, 64>::kLdsBytes + kPairWordLds;
    case 28: return DmaShape<192, 1, 3, 2, 3, 64, 64>::kLdsBytes + kPairWordLds;
    case 10: return DmaShape<256, 2, 4, 2, 4, 32>::kLdsBytes;
    case 11: return DmaShape<128, 3, 2, 4, 4, 32>::kLdsBytes;
    case 12: return DmaShape<256, 1, 4, 1, 4, 32>::kLdsBytes;
    case 13: return DmaShape<128, 2, 2, 2, 4, 32>::kLdsBytes;
    case 14: return DmaShape<256, 2, 2, 4, 4, 32>::kLdsBytes;
    case 15: return DmaShape<128, 3, 2, 4, 5, 32>::kLdsBytes;
    case 16: return DmaShape<128, 3, 2, 4, 2, 64>::kLdsBytes;
    case 17: return DmaShape<256, 2, 4, 2, 2, 64>::kLdsBytes;
    case 18: return DmaShape<256, 2, 2, 4, 2, 64>::kLdsBytes;
    case 19: return DmaShape<128, 1, 2, 2, 4, 64>::kLdsBytes;
    case 20: return DmaShape<64, 1, 1, 4, 4, 64>::kLdsBytes;
    case 21: return DmaShape<128, 1, 2, 4, 4, 64>::kLdsBytes;
    case 22: return DmaShape<256, 1, 4, 2, 3, 64>::kLdsBytes;
    case 23: return DmaShape<128, 2, 2, 4, 3, 64>::kLdsBytes;
    case 30: return W4Shape<128, 3, 2, 4, 4>::kLdsBytes;
    case 31: return W4Shape<256, 2, 2, 4, 3>::kLdsBytes;
    case 32: return W4Shape<128, 2, 2, 2, 4>::kLdsBytes;
    case 33: return W4Shape<256, 2, 1, 8, 3>::kLdsBytes;
    case 34: return W4Shape<128, 1, 2, 4, 4>::kLdsBytes;
    case 35: return W4Shape<64, 1, 1, 4, 4>::kLdsBytes;
    default: return 0;
  }
}

hipError_t launch_tile_dma_split(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                                 int ksplit, int force_recompute, int max_spins, void* workspace, hipStream_t stream) {
  switch (id) {
    case 16:
      return launch_dma_split<128, 3, 2, 4, 2, 64>(p, w, e, ksplit, force_recompute, max_spins, workspace, stream);
    case 18:
      return launch_dma_split<256, 2, 2, 4, 2, 64>(p, w, e, ksplit, force_recompute, max_spins, workspace, stream);
    default: return hipErrorInvalidValue;
  }
}

size_t tile_split_part_bytes(int id, int64_t M, int n_tiles, int ksplit) {
  switch (id) {
    case 16: return split_part_bytes<128, 3, 2, 4, 2, 64>(M, n_tiles, ksplit);
    case 18: return split_part_bytes<256, 2, 2, 4, 2, 64>(M, n_tiles, ksplit);
    default: return 0;
  }
}

hipError_t launch_tile_dma_w4(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                              int group_m, hipStream_t stream) {
  switch (id) {
    case 30: return launch_dma_w4<128, 3, 2, 4, 4>(p, w, e, group_m, stream);  // 128x384, 4 stages
    case 31: return launch_dma_w4<256, 2, 2, 4, 3>(p, w, e, group_m, stream);  // 256x256, 3 stages
    case 32: return launch_dma_w4<128, 2, 2, 2, 4>(p, w, e, group_m, stream);  // 128x256, 4 waves
    case 33: return launch_dma_w4<256, 2, 1, 8, 3>(p, w, e, group_m, stream);  // 256x256, 256x32 waves
    case 34: return launch_dma_w4<128, 1, 2, 4, 4>(p, w, e, group_m, stream);  // 128x128, 8 waves (64x32)
    case 35: return launch_dma_w4<64, 1, 1, 4, 4>(p, w, e, group_m, stream);   // 64x128, 4 waves (64x32)
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mqk
