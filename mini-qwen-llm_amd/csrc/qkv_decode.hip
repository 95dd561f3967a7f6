// Split-K projection for small token counts (decode steps, T <= 64, and up to
// four 64-row blocks per launch at mid T) with the
// per-head norm + RoPE applied once the split partial sums are combined.
//
// At decode the op is weight-read bound: Qwen3-8B's 50 MB of projection
// weights against 64 tokens.  Measured on MI355X: one CU sustains only a few
// tens of GB/s of reads, so every CU must stream its share of the weights;
// splitting a head's columns (instead of K) would re-read the activations from
// L2 per workgroup, which measured 3-4x slower than the weight stream itself;
// and two workgroups sharing a CU finish twice as late as one alone.  Hence:
//   * one 512-thread workgroup per CU (its activation slice in LDS is larger
//     than half the LDS, so the hardware cannot co-schedule two);
//   * each head is split along K into S = floor(CUs per XCD / heads per XCD)
//     k-ranges, and the grid maps all splits of head h to XCD h % 8
//     (workgroup b runs on XCD b % 8), so every XCD gets the same number of
//     workgroups, at most one per CU;
//   * inside a workgroup, wave w owns columns [16w, 16w+16) of the head over
//     the split's whole k-range, for all 64 token rows (v_mfma_f32_16x16x32_bf16,
//     4 row blocks, so each weight fragment feeds 4 MFMAs and no reduction
//     between waves is needed).  The activation slice is staged once in LDS
//     with direct L2 -> LDS loads; the wave's weight slice streams HBM -> VGPR,
//     all of it issued up front, and each 64-wide k tile is multiplied as soon
//     as its fragments land.
// Combining the splits: each workgroup writes its fp32 partial tile [64 x 128]
// (in MFMA fragment order, 16-byte stores) with plain stores, which stay in (or are written back from) the L2 of its
// XCD, and bumps the head's arrival counter; the workgroup that arrives last
// reads the other partials with plain loads -- all of them were written
// through the same L2 -- adds them in split order, applies RMSNorm over the
// head (fused_qkv_rope.py:98-100) and rotate-half RoPE (:102-118), writes
// bf16 q/k (or v unchanged) and resets the counter for the next call.
// Device-coherent (sc1) accesses measured ~0.5 TB/s and an agent-scope fence
// pair (L2 writeback + invalidate) ~2x the whole op, so neither is used.
//
// Each workgroup checks the XCD it actually runs on (hardware register
// XCC_ID).  If any split of a head ran elsewhere, its partial may sit in a
// different L2, so the last workgroup instead recomputes every split of the
// head itself, with the same per-split arithmetic and summation order: slower,
// bit-identical, and correct whatever the dispatch order.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {

namespace {

constexpr int kDecRows = 64;            // token rows per block (one block per call when T <= 64)
constexpr int kDecMaxPasses = 4;        // most 64-row blocks one launch streams the weights for
constexpr int kDecThreads = 512;        // 8 waves; wave w owns columns [16w, 16w+16) of the head
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kDecMaxNK = 16;           // largest k-range of one split, in 64-wide tiles
constexpr int kDecLookahead = 6;        // weight tiles in flight per wave
constexpr int kDecKc = kDecMaxNK * kBK;     // LDS row length of the x slice (bf16), 2 KB
constexpr int kMaxHeads = kDecodeMaxHeads;
constexpr int kCounterBytes = int(kDecodeCounterBytes);
constexpr int kTileFloats = kDecRows * kHeadDim;
constexpr int kPitch = kHeadDim + 4;    // fp32 pitch of the finisher's LDS head tile
constexpr uint32_t kForeignUnit = 1u << 16;  // arrival-counter increment of a misplaced split

static_assert(kDecRows * kDecKc * 2 > 160 * 1024 / 2, "x slice must keep one workgroup per CU");
static_assert(kDecRows * 8 == kDecThreads, "one 16-byte x chunk per thread per k tile");
static_assert(kDecRows * kPitch * 4 <= kDecRows * kDecKc * 2, "the head tile aliases the x slice");
static_assert(kDecWaves * 16 == kHeadDim, "one 16-column group per wave");

// x slice layout in LDS: tile-major, [k tile t][row 0..63][8 chunks of 16 B]
// (8 KB per 64-wide k tile); chunk c of row r is stored in slot c ^ ((r >> 1) & 7),
// so the 16 rows one quarter-wave reads (8 even rows in one half of the banks, 8
// odd rows in the other) hit 16 different bank groups.
__device__ __forceinline__ int dec_lds_off(int t, int row, int chunk) {
  return t * (kDecRows * 64) + row * 64 + ((chunk ^ ((row >> 1) & 7)) << 3);  // in bf16 elements
}

__device__ __forceinline__ int xcc_id() {
  return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));  // hwreg(HW_REG_XCC_ID, 0, 4)
}

// k-tile range [kt0, kt0 + nk) of split s of S over nkt tiles (balanced).
__device__ __forceinline__ void split_range(int s, int S, int nkt, int& kt0, int& nk) {
  kt0 = int((int64_t(s) * nkt) / S);
  nk = int((int64_t(s + 1) * nkt) / S) - kt0;
}

// One direct L2 -> LDS load per wave stages k tile t of the x slice of the
// 64-row block starting at launch row r0: wave w fills rows [8w, 8w+8) (1 KB,
// contiguous in LDS); lane L takes row 8w + L/8 and LDS slot L % 8, i.e. global
// chunk (L % 8) ^ ((row >> 1) & 7).  Rows >= M re-read row M-1; those LDS rows
// only feed output rows that are never stored.
__device__ __forceinline__ void stage_x_tile(const ProblemArgs& p, int64_t kbeg, int t, uint32_t xs_lds, int r0 = 0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = wave * 8 + (lane >> 3);
  const int gq = (lane & 7) ^ ((row >> 1) & 7);
  const int grow = r0 + row < int(p.M) ? r0 + row : int(p.M) - 1;
  dma16(p.x + int64_t(grow) * p.K + kbeg + t * kBK + gq * 8,
        xs_lds + uint32_t(t * kDecRows * 128 + wave * 1024));
}

// Input RMSNorm (ProblemArgs::in_gamma): gamma is staged in the dynamic LDS that
// follows the x slice, and each wave normalises the x chunks its own direct
// loads brought in (rows [8w, 8w+8) of every tile: lane L holds row 8w + L/8,
// slot L % 8), in place, once they have landed.
extern __shared__ __attribute__((aligned(16))) unsigned char g_dec_dyn_lds[];
constexpr int kGamPerThread = 4;  // gamma chunks per thread: hidden <= 4 * 512 * 8

// Issue this thread's gamma loads (registers); stored to LDS by gamma_to_lds.
__device__ __forceinline__ void gamma_load(const ProblemArgs& p, u32x4_t (&gv)[kGamPerThread]) {
#pragma unroll
  for (int j = 0; j < kGamPerThread; ++j) {
    const int64_t c = threadIdx.x + j * kDecThreads;
    gv[j] = c < p.K / 8 ? *reinterpret_cast<const u32x4_t*>(p.in_gamma + c * 8) : u32x4_t{0, 0, 0, 0};
  }
}

__device__ __forceinline__ void gamma_to_lds(const ProblemArgs& p, const u32x4_t (&gv)[kGamPerThread]) {
#pragma unroll
  for (int j = 0; j < kGamPerThread; ++j) {
    const int64_t c = threadIdx.x + j * kDecThreads;
    if (c < p.K / 8) *reinterpret_cast<u32x4_t*>(g_dec_dyn_lds + c * 16) = gv[j];
  }
}

// Normalise this wave's chunks of x tiles [0, nk) of the slice starting at k = kbeg
// (gamma must be in LDS); ends with this wave's LDS writes complete.
__device__ __forceinline__ void norm_x_tiles(const ProblemArgs& p, uint16_t* xs, int64_t kbeg, int nk, int r0 = 0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = wave * 8 + (lane >> 3);
  const int gq = (lane & 7) ^ ((row >> 1) & 7);
  const float scale = p.in_scale[r0 + row < int(p.M) ? r0 + row : int(p.M) - 1];
  unsigned char* base = reinterpret_cast<unsigned char*>(xs) + wave * 1024 + lane * 16;
  for (int t = 0; t < nk; ++t) {
    u32x4_t* q = reinterpret_cast<u32x4_t*>(base + t * kDecRows * 128);
    const u32x4_t g = *reinterpret_cast<const u32x4_t*>(g_dec_dyn_lds + (kbeg + t * kBK + gq * 8) * 2);
    *q = input_norm8(*q, scale, g);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// 16x16x32 operand layout: lane (c, g) = (lane & 15, lane >> 4) holds column c
// of the wave's 16 (B) / row c of a 16-row block (A) and 8 k values; inside a
// 64-wide k tile, block kk (0, 1) of 32 and lane group g give k = kk*32 + g*8.
// acc[mb][j] = C[mb*16 + 4g + j][16*wave + c].
__device__ __forceinline__ void mma_tile(const uint16_t* xs, int t, const u32x4_t (&b)[2], f32x4_t (&acc)[4]) {
  const int lane = threadIdx.x & 63;
  const int c16 = lane & 15, g4 = lane >> 4;
  u32x4_t a[2][4];  // all 8 activation fragments of the tile in flight before the first MFMA
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
      a[kk][mb] = *reinterpret_cast<const u32x4_t*>(xs + dec_lds_off(t, mb * 16 + c16, kk * 4 + g4));
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[mb] = mfma_16x16x32(a[kk][mb], b[kk], acc[mb]);
}

// 8 consecutive bf16 (16 bytes, 16-byte aligned: the launcher checks gamma / cos / sin).
__device__ __forceinline__ u32x4_t load8_bf16(const uint16_t* ptr) { return *reinterpret_cast<const u32x4_t*>(ptr); }

// Element i (0..7) of 8 packed bf16, as float.
__device__ __forceinline__ float bf16_lane(const u32x4_t& v, int i) {
  const uint32_t wd = i < 2 ? v.x : (i < 4 ? v.y : (i < 6 ? v.z : v.w));
  return __uint_as_float((i & 1) ? (wd & 0xFFFF0000u) : (wd << 16));
}

// Weight fragment load: non-temporal, so the weight stream does not evict the
// split partials and the x slice from the L2.
__device__ __forceinline__ u32x4_t wload(const uint16_t* ptr) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(ptr));
}

struct Int4Col {  // this lane's column of an int4 projection
  const int32_t* qw;
  const uint16_t* sc;
  const int32_t* qz;
  int64_t n;      // columns of the projection
  int64_t col;
  int group;
  bool fp16;
};

__device__ __forceinline__ Int4Col int4_col(const WeightArgs& w, int proj, int64_t col) {
  return Int4Col{w.qw[proj], static_cast<const uint16_t*>(w.sc[proj]), w.qz[proj], w.n_cols[proj], col,
                 w.group, w.scale_fp16 != 0};
}

__device__ __forceinline__ void dequant_tile(const Int4Col& ic, const uint32_t (&q)[2], uint32_t sraw, uint32_t zw,
                                             u32x4_t (&b)[2]) {
  const float scale = ic.fp16 ? f16_to_f32(sraw) : bf16_to_f32(sraw);
  const float zero = float((zw >> ((ic.col % 8) * 4)) & 0xFu);
  b[0] = dequant_int4x8(q[0], zero, scale);
  b[1] = dequant_int4x8(q[1], zero, scale);
}

// The split partial of one wave over k tiles [kt0, kt0 + NK).
// bf16: per tile, the wave issues the x tile's direct load, then its two weight
// fragments (HBM -> VGPR, non-temporal so the weight stream does not evict the
// split partials from the L2).  Tile t is multiplied once the x tile has landed
// in every wave (own wait: the 3*(NK-1-t)+2 later loads may still be pending;
// then a barrier) and its weight fragments have arrived (the compiler's per-use
// waits), so the MFMAs run under the rest of the stream.
// With NP > 1 the launch covers NP blocks of 64 rows: block 0 as above, then
// for each later block the x slice of its rows is staged in the same LDS and
// multiplied by the weight fragments this wave still holds in registers, so the
// weights are streamed from HBM once for all NP * 64 rows (accs[pp] = block pp).
template <bool INT4, bool INORM, int NK, int NP>
__device__ __forceinline__ void partial_fixed(const ProblemArgs& p, const WeightArgs& w, int proj, int hh,
                                              int kt0, const uint16_t* xs, uint32_t xs_lds,
                                              f32x4_t (&accs)[NP][4]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int64_t kbeg = int64_t(kt0) * kBK;
  const int64_t col = int64_t(hh) * kHeadDim + wave * 16 + c16;
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) accs[pp][mb] = f32x4_t{};
  f32x4_t(&acc)[4] = accs[0];
  // rows [64 pp, 64 pp + 64): stage their x slice once every wave is done with the
  // previous block's (the normalising gamma, if any, is already in LDS)
  auto stage_block = [&](int pp) {
    barrier();
#pragma unroll
    for (int t = 0; t < NK; ++t) stage_x_tile(p, kbeg, t, xs_lds, pp * kDecRows);
    wait_vm<0>();
    if (INORM) norm_x_tiles(p, const_cast<uint16_t*>(xs), kbeg, NK, pp * kDecRows);
    barrier();
  };
  if constexpr (!INT4) {
    // The x slice (L2-resident) is requested first, then the first kLook weight
    // tiles; each later tile is requested one tile before the MFMAs that free
    // the lookahead slot, so about kLook tiles (16 KB per tile per CU) stay in
    // flight and early tiles land early instead of the whole stream landing at
    // once.
    constexpr int kLook = NK < kDecLookahead ? NK : kDecLookahead;
    const uint16_t* wp = w.w[proj] + col * p.K + kbeg + g4 * 8;
    u32x4_t b[NK][2];
    u32x4_t gv[kGamPerThread];
    if (INORM) gamma_load(p, gv);
#pragma unroll
    for (int t = 0; t < NK; ++t) stage_x_tile(p, kbeg, t, xs_lds);
#pragma unroll
    for (int t = 0; t < kLook; ++t)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        b[t][kk] = wload(wp + t * kBK + kk * 32);
    wait_vm<2 * kLook>();  // the x slice has landed (older than the weight loads) ...
    if (INORM) {           // (gamma too: loaded before it)
      gamma_to_lds(p, gv);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier();
      norm_x_tiles(p, const_cast<uint16_t*>(xs), kbeg, NK);
    }
    barrier();             // ... in every wave
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      if (t + kLook < NK) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          b[t + kLook][kk] =
              wload(wp + (t + kLook) * kBK + kk * 32);
      }
      mma_tile(xs, t, b[t], acc);
    }
#pragma unroll
    for (int pp = 1; pp < NP; ++pp) {
      stage_block(pp);
#pragma unroll
      for (int t = 0; t < NK; ++t) mma_tile(xs, t, b[t], accs[pp]);
    }
  } else {
    // int4 weights are 4x smaller: load them with their scales and zeros, then
    // the x slice, and wait for everything
    const Int4Col ic = int4_col(w, proj, col);
    uint32_t q[NK][2], sraw[NK], zw[NK];
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      const int64_t k0 = kbeg + int64_t(t) * kBK;
      const int64_t grp = k0 / ic.group;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) q[t][kk] = uint32_t(ic.qw[(k0 / 8 + kk * 4 + g4) * ic.n + col]);
      sraw[t] = ic.sc[grp * ic.n + col];
      zw[t] = uint32_t(ic.qz[grp * (ic.n / 8) + col / 8]);
    }
    u32x4_t gv[kGamPerThread];
    if (INORM) gamma_load(p, gv);
#pragma unroll
    for (int t = 0; t < NK; ++t) stage_x_tile(p, kbeg, t, xs_lds);
    wait_vm<0>();
    if (INORM) {
      gamma_to_lds(p, gv);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier();
      norm_x_tiles(p, const_cast<uint16_t*>(xs), kbeg, NK);
    }
    barrier();
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      u32x4_t b[2];
      dequant_tile(ic, q[t], sraw[t], zw[t], b);
      mma_tile(xs, t, b, acc);
    }
#pragma unroll
    for (int pp = 1; pp < NP; ++pp) {
      stage_block(pp);
#pragma unroll
      for (int t = 0; t < NK; ++t) {
        u32x4_t b[2];
        dequant_tile(ic, q[t], sraw[t], zw[t], b);
        mma_tile(xs, t, b, accs[pp]);
      }
    }
  }
}

// The same partial with a run-time k-range and one tile's loads at a time: the
// arithmetic (per-tile dequant, MFMA order) is identical to partial_fixed, so
// its result is bit-identical.  Used by the recompute path only.
template <bool INT4, bool INORM>
__device__ void partial_any(const ProblemArgs& p, const WeightArgs& w, int proj, int hh, int kt0, int nk,
                            const uint16_t* xs, uint32_t xs_lds, f32x4_t (&acc)[4], int r0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int64_t kbeg = int64_t(kt0) * kBK;
  const int64_t col = int64_t(hh) * kHeadDim + wave * 16 + c16;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4_t{};
  for (int t = 0; t < nk; ++t) stage_x_tile(p, kbeg, t, xs_lds, r0);
  wait_vm<0>();
  if (INORM) norm_x_tiles(p, const_cast<uint16_t*>(xs), kbeg, nk, r0);  // gamma is in LDS already
  barrier();
  for (int t = 0; t < nk; ++t) {
    const int64_t k0 = kbeg + int64_t(t) * kBK;
    u32x4_t b[2];
    if constexpr (!INT4) {
      const uint16_t* wp = w.w[proj] + col * p.K + k0 + g4 * 8;
      b[0] = *reinterpret_cast<const u32x4_t*>(wp);
      b[1] = *reinterpret_cast<const u32x4_t*>(wp + 32);
    } else {
      const Int4Col ic = int4_col(w, proj, col);
      const int64_t grp = k0 / ic.group;
      const uint32_t q[2] = {uint32_t(ic.qw[(k0 / 8 + g4) * ic.n + col]),
                             uint32_t(ic.qw[(k0 / 8 + 4 + g4) * ic.n + col])};
      dequant_tile(ic, q, ic.sc[grp * ic.n + col], uint32_t(ic.qz[grp * (ic.n / 8) + col / 8]), b);
    }
    mma_tile(xs, t, b, acc);
  }
}

template <bool INT4, bool INORM, int NP>
__device__ __forceinline__ void partial_dispatch(const ProblemArgs& p, const WeightArgs& w, int proj, int hh,
                                                 int kt0, int nk, const uint16_t* xs, uint32_t xs_lds,
                                                 f32x4_t (&acc)[NP][4]) {
  switch (nk) {
#define MQK_DEC_CASE(n) \
  case n: partial_fixed<INT4, INORM, n, NP>(p, w, proj, hh, kt0, xs, xs_lds, acc); break;
    MQK_DEC_CASE(1) MQK_DEC_CASE(2) MQK_DEC_CASE(3) MQK_DEC_CASE(4)
    MQK_DEC_CASE(5) MQK_DEC_CASE(6) MQK_DEC_CASE(7) MQK_DEC_CASE(8)
    MQK_DEC_CASE(9) MQK_DEC_CASE(10) MQK_DEC_CASE(11) MQK_DEC_CASE(12)
    MQK_DEC_CASE(13) MQK_DEC_CASE(14) MQK_DEC_CASE(15) MQK_DEC_CASE(16)
#undef MQK_DEC_CASE
    default: break;  // the launcher guarantees 1 <= nk <= kDecMaxNK
  }
}

template <bool INT4, bool INORM, int NP>
__global__ void __launch_bounds__(kDecThreads, 1)
decode_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int splits, float* __restrict__ part,
              uint32_t* __restrict__ counters, int force_recompute) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kDecRows * kDecKc];
  __shared__ uint32_t arrival;
  const uint32_t xs_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xs));
  float* tile = reinterpret_cast<float*>(xs);  // the finisher's head tile aliases the x slice

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n_tiles = p.n_tiles;
  const int bid = blockIdx.x;
  const int xcds = p.xcds;
  const int q = bid / xcds;
  const int split = q % splits;
  const int head = (q / splits) * xcds + bid % xcds;
  if (head >= n_tiles) return;  // padding workgroup
  const int M = int(p.M);
  const int nkt = int(p.K / kBK);
  int proj, hh;
  split_head(head, e.Hq, e.Hkv, proj, hh);

  // RoPE table row of this thread's finisher row (tid / 8) of each 64-row block,
  // read now: a positions[] load here is off every critical path
  int64_t prow[NP], cslot[NP];  // cslot: paged-KV-cache slot
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
    const int rr = pp * kDecRows + (tid >> 3);
    prow[pp] = (proj != 2 && rr < M) ? rope_row(e, rr) * kHeadDim : 0;
    cslot[pp] = (proj != 0 && rr < M) ? paged_slot(e, rr) : -1;
  }

  int kt0, nk;
  split_range(split, splits, nkt, kt0, nk);
  f32x4_t acc[NP][4];
  partial_dispatch<INT4, INORM, NP>(p, w, proj, hh, kt0, nk, xs, xs_lds, acc);

  // ---- publish the partials in fragment order: part[split][block][head][wave][mb][lane] ----
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
    f32x4_t* mine = reinterpret_cast<f32x4_t*>(part) +
                    (((int64_t(split) * NP + pp) * n_tiles + head) * kDecWaves + wave) * 4 * 64 + lane;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) mine[mb * 64] = acc[pp][mb];
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have reached the L2
  __syncthreads();                // ... and every thread's
  if (tid == 0) {
    // (XCC_ID is the physical XCD; a partition of the GPU holds xcds of them)
    const bool foreign = force_recompute || xcc_id() % xcds != bid % xcds;
    const uint32_t inc = 1u + (foreign ? kForeignUnit : 0u);
    arrival = __hip_atomic_fetch_add(counters + head, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
  }
  __syncthreads();
  const uint32_t seen = arrival;
  if ((seen & (kForeignUnit - 1)) != uint32_t(splits)) return;  // not the last split to arrive
  const bool recompute = (seen >> 16) != 0;
  if (recompute && tid == 0)  // statistics: heads finished on the recompute path
    __hip_atomic_fetch_add(counters + kDecodeRecomputeWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // thread -> row r = tid / 8, c = tid % 8 of the head tile: columns [8c, 8c+8)
  // and [64+8c, 64+8c+8), so every RoPE pair (d, d+64) is thread-local.  Its
  // gamma / cos / sin operands are loaded under the partial reads; its RoPE row
  // (prow, which may need a positions[] load) was read at kernel start so that
  // no dependent load stalls the finisher.
  const int r = tid >> 3;
  const int c = tid & 7;
#pragma unroll
  for (int pp = 0; pp < NP; ++pp) {
    if (pp > 0) __syncthreads();  // the previous block's epilogue is done with the LDS
    const int rr = pp * kDecRows + r;  // this thread's row of the launch
    u32x4_t g_lo{}, g_hi{}, c_lo{}, c_hi{}, s_lo{}, s_hi{};
    auto load_operands = [&]() {
      if (proj != 2 && rr < M) {
        const uint16_t* gamma = proj == 0 ? e.q_gamma : e.k_gamma;
        g_lo = load8_bf16(gamma + 8 * c);
        g_hi = load8_bf16(gamma + kHalfDim + 8 * c);
        c_lo = load8_bf16(e.cos + prow[pp] + 8 * c);
        c_hi = load8_bf16(e.cos + prow[pp] + kHalfDim + 8 * c);
        s_lo = load8_bf16(e.sin + prow[pp] + 8 * c);
        s_hi = load8_bf16(e.sin + prow[pp] + kHalfDim + 8 * c);
      }
    };

    // ---- last arrival: sum the partials in split order ---------------------------------
    f32x4_t sum[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) sum[mb] = f32x4_t{};
    if (!recompute) {
      // The other splits' fragments of this wave are pulled into LDS with direct
      // L2 -> LDS loads (a CU fetches faster that way than into VGPRs), up to four
      // splits per batch in the x slice's space, which no wave reads any more; each
      // wave reads back only the 4 KB regions it loaded itself, so its own vmcnt
      // wait is the only synchronisation.  Summation is in split order.
      const char* frag = reinterpret_cast<const char*>(part) +
                         (((int64_t(pp) * n_tiles + head) * kDecWaves + wave) * 4 * 64) * sizeof(f32x4_t);
      const int64_t split_stride = int64_t(NP) * n_tiles * kTileFloats * sizeof(float);
      const uint32_t slot0 = xs_lds + uint32_t(wave * 4096);
      const char* slot0_ptr = reinterpret_cast<const char*>(xs) + wave * 4096;
      load_operands();
      int slot = 0, first = 0;
#pragma unroll 1
      for (int q = 0; q < splits; ++q) {
        if (q != split) {
          const char* src = frag + q * split_stride + lane * 16;
#pragma unroll
          for (int mb = 0; mb < 4; ++mb)
            dma16(src + mb * 1024, slot0 + uint32_t(slot * kDecWaves * 4096 + mb * 1024));
          ++slot;
        }
        if (slot == 4 || q == splits - 1) {  // four slots filled, or the last split: add in split order
          wait_vm<0>();
          int u_slot = 0;
#pragma unroll 1
          for (int u = first; u <= q; ++u) {
            if (u == split) {
#pragma unroll
              for (int mb = 0; mb < 4; ++mb) sum[mb] += acc[pp][mb];
            } else {
#pragma unroll
              for (int mb = 0; mb < 4; ++mb)
                sum[mb] += *reinterpret_cast<const f32x4_t*>(slot0_ptr + u_slot * kDecWaves * 4096 + mb * 1024 +
                                                             lane * 16);
              ++u_slot;
            }
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads done before the next batch overwrites
          slot = 0;
          first = q + 1;
        }
      }
    } else {
      // Some split ran on another XCD: its partial may not be visible through this
      // L2.  Recompute every split here (same arithmetic, same order).
      load_operands();
      for (int s = 0; s < splits; ++s) {
        int s_kt0, s_nk;
        split_range(s, splits, nkt, s_kt0, s_nk);
        __syncthreads();  // every wave is done with the x slice of the previous split
        f32x4_t part_s[4];
        partial_any<INT4, INORM>(p, w, proj, hh, s_kt0, s_nk, xs, xs_lds, part_s, pp * kDecRows);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) sum[mb] += part_s[mb];
      }
    }

    // ---- head tile to LDS (fp32 [64][kPitch]); the x slice is no longer read ----------
    __syncthreads();
    {
      const int c16 = lane & 15, g4 = lane >> 4;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) tile[(mb * 16 + g4 * 4 + j) * kPitch + wave * 16 + c16] = sum[mb][j];
    }
    __syncthreads();

    float lo[8], hi[8];
    {
      const float* src = tile + r * kPitch;
      const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(src + 8 * c);
      const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(src + 8 * c + 4);
      const f32x4_t b0 = *reinterpret_cast<const f32x4_t*>(src + kHalfDim + 8 * c);
      const f32x4_t b1 = *reinterpret_cast<const f32x4_t*>(src + kHalfDim + 8 * c + 4);
      lo[0] = a0.x; lo[1] = a0.y; lo[2] = a0.z; lo[3] = a0.w;
      lo[4] = a1.x; lo[5] = a1.y; lo[6] = a1.z; lo[7] = a1.w;
      hi[0] = b0.x; hi[1] = b0.y; hi[2] = b0.z; hi[3] = b0.w;
      hi[4] = b1.x; hi[5] = b1.y; hi[6] = b1.z; hi[7] = b1.w;
    }

    if (proj != 2) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += lo[i] * lo[i] + hi[i] * hi[i];
      ss = sum8_lanes(ss);
      const float rms = rsqrtf(ss * (1.0f / float(kHeadDim)) + e.eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x1n = lo[i] * rms * bf16_lane(g_lo, i);
        const float x2n = hi[i] * rms * bf16_lane(g_hi, i);
        const float t1 = x1n * bf16_lane(c_lo, i) - x2n * bf16_lane(s_lo, i);
        const float t2 = x2n * bf16_lane(c_hi, i) + x1n * bf16_lane(s_hi, i);
        lo[i] = t1;
        hi[i] = t2;
      }
    }
    if (rr < M) {
      const int H = proj == 0 ? e.Hq : e.Hkv;
      u32x4_t o1, o2;
      o1.x = pack_bf16x2(lo[0], lo[1]);
      o1.y = pack_bf16x2(lo[2], lo[3]);
      o1.z = pack_bf16x2(lo[4], lo[5]);
      o1.w = pack_bf16x2(lo[6], lo[7]);
      o2.x = pack_bf16x2(hi[0], hi[1]);
      o2.y = pack_bf16x2(hi[2], hi[3]);
      o2.z = pack_bf16x2(hi[4], hi[5]);
      o2.w = pack_bf16x2(hi[6], hi[7]);
      uint16_t* base = proj == 0 ? e.q : (proj == 1 ? e.k : e.v);  // k / v may be null (cache only)
      if (base) {
        uint16_t* dst = base + (int64_t(rr) * H + hh) * kHeadDim;
        *reinterpret_cast<u32x4_t*>(dst + 8 * c) = o1;
        *reinterpret_cast<u32x4_t*>(dst + kHalfDim + 8 * c) = o2;
      }
      if (cslot[pp] >= 0) {
        uint16_t* crow = paged_row(e, cslot[pp], proj, hh);
        *reinterpret_cast<u32x4_t*>(crow + 8 * c) = o1;
        *reinterpret_cast<u32x4_t*>(crow + kHalfDim + 8 * c) = o2;
      }
    }
  }  // 64-row blocks
  if (tid == 0) __hip_atomic_store(counters + head, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

int g_decode_force_recompute = 0;

int decode_splits_for(int64_t M, int64_t K, int n_tiles, int requested, int cus, int xcds) {
  (void)M;
  const int nkt = int(K / kBK);
  if (nkt < 1) return 0;
  const int min_splits = (nkt + kDecMaxNK - 1) / kDecMaxNK;  // LDS bound on a split's k-range
  int s = requested;
  if (s <= 0) {
    // one workgroup per CU: (heads per XCD) x splits <= CUs per XCD
    xcds = xcds < 1 ? 1 : xcds;
    const int heads_per_xcd = (n_tiles + xcds - 1) / xcds;
    s = (cus / xcds) / heads_per_xcd;
    if (s > nkt) s = nkt;  // small hidden: at most one k tile per split
    if (s < min_splits) s = min_splits;
  }
  if (s < min_splits || s > nkt || s > kDecMaxNK) return 0;
  return s;
}

size_t decode_counter_bytes() { return size_t(kCounterBytes); }

size_t decode_workspace_bytes(int n_tiles, int splits, int passes) {
  return size_t(kCounterBytes) + size_t(splits) * passes * n_tiles * kTileFloats * sizeof(float);
}

hipError_t launch_decode(int int4, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                         int splits, void* workspace, hipStream_t stream) {
  const int nkt = int(p.K / kBK);
  const int passes = int((p.M + kDecRows - 1) / kDecRows);  // 64-row blocks of this launch
  if (splits < 1 || splits > kDecMaxNK || splits > nkt || (nkt + splits - 1) / splits > kDecMaxNK ||
      p.n_tiles > kMaxHeads || passes < 1 || passes > kDecMaxPasses)
    return hipErrorInvalidValue;
  uint32_t* counters = static_cast<uint32_t*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  if (p.xcds < 1) return hipErrorInvalidValue;
  const dim3 grid(((p.n_tiles + p.xcds - 1) / p.xcds) * p.xcds * splits);
  const int fr = g_decode_force_recompute;
  auto a16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; };
  if (!(a16(e.q_gamma) && a16(e.k_gamma) && a16(e.cos) && a16(e.sin))) return hipErrorInvalidValue;
  const size_t dyn = p.in_gamma ? size_t(p.K) * 2 : 0;
  if (p.in_gamma && (p.K / 8 > int64_t(kGamPerThread) * kDecThreads ||
                     kDecRows * kDecKc * 2 + 16 + dyn > 160 * 1024 || !a16(p.in_gamma)))
    return hipErrorInvalidValue;
  // (the input norm and the block count are template switches: the plain one-block
  // kernels carry none of their code)
  using Kernel = void (*)(ProblemArgs, WeightArgs, EpilogueArgs, int, float*, uint32_t*, int);
#define MQK_DEC_KERNELS(NP)                                                                   \
  {decode_kernel<false, false, NP>, decode_kernel<false, true, NP>, decode_kernel<true, false, NP>, \
   decode_kernel<true, true, NP>}
  static const Kernel kernels[kDecMaxPasses][4] = {MQK_DEC_KERNELS(1), MQK_DEC_KERNELS(2), MQK_DEC_KERNELS(3),
                                                   MQK_DEC_KERNELS(4)};
#undef MQK_DEC_KERNELS
  Kernel kernel = kernels[passes - 1][(int4 ? 2 : 0) + (p.in_gamma ? 1 : 0)];
  hipLaunchKernelGGL(kernel, grid, dim3(kDecThreads), dyn, stream, p, w, e, splits, part, counters, fr);
  return hipGetLastError();
}

}  // namespace mqk
