// Split-K projection for small token counts (decode steps, T <= 64, and up to
// sixteen 64-row blocks per launch at mid T) with the per-head norm + RoPE
// applied once the split partial sums of a block are combined.
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
#include <utility>

#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {

namespace {

constexpr int kDecRows = 64;            // token rows per block (one block per call when T <= 64)
constexpr int kDecMaxBlocks = 16;       // most 64-row blocks one launch streams the weights for
constexpr int kDecThreads = 512;        // 8 waves; wave w owns columns [16w, 16w+16) of the head
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kDecMaxNK = 16;           // k tiles of one x slice in LDS (64-wide tiles)
// Longest k range of a split in a launch of one block: two x slices, staged
// one after the other (wider models, e.g. hidden 5120 with 56 heads, then keep
// one workgroup per CU with 4 splits of 20 tiles instead of 5 splits over two
// rounds).
constexpr int kDecLongMaxNK = 2 * kDecMaxNK;
constexpr int kDecLookahead = 6;        // weight tiles in flight per wave
// Longest k range (in 64-wide tiles) of a split in a launch of several blocks:
// beyond it the held weights and the finisher no longer fit the 256 VGPRs of a
// wave without spilling, and such launches run one block each.  (int4 weights
// with the input norm: one tile less.)
constexpr int kDecMultiMaxNK = 13;
constexpr int kDecMultiMaxNKInt4Norm = 12;
constexpr int kDecKc = kDecMaxNK * kBK;     // LDS row length of the x slice (bf16), 2 KB
constexpr int kMaxHeads = kDecodeMaxHeads;
constexpr int kCounterBytes = int(kDecodeCounterBytes);
constexpr int kTileFloats = kDecRows * kHeadDim;
constexpr int kPitch = kHeadDim + 4;    // fp32 pitch of the finisher's LDS head tile
constexpr int kDecMaxSpins = 1 << 14;   // default polls (s_sleep 2 apart, ~1 ms) before a wait is handed off

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

template <int NK, int... T>
__device__ __forceinline__ void stage_x_step(const uint16_t* src, uint32_t dst, std::integer_sequence<int, T...>) {
  (dma16_at<T * kBK * 2>(src, dst + uint32_t(T * kDecRows * 128)), ...);
}

// stage_x_tile for tiles 0 .. NK-1 at once: one address per lane, the tiles'
// 128-byte steps as instruction offsets.
template <int NK>
__device__ __forceinline__ void stage_x_slice(const ProblemArgs& p, int64_t kbeg, uint32_t xs_lds, int r0 = 0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = wave * 8 + (lane >> 3);
  const int gq = (lane & 7) ^ ((row >> 1) & 7);
  const int grow = r0 + row < int(p.M) ? r0 + row : int(p.M) - 1;
  const uint16_t* src = p.x + int64_t(grow) * p.K + kbeg + gq * 8;
  const uint32_t dst = xs_lds + uint32_t(wave * 1024);
  stage_x_step<NK>(src, dst, std::make_integer_sequence<int, NK>{});
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
__device__ __forceinline__ void norm_x_tiles(const ProblemArgs& p, uint16_t* xs, int64_t kbeg, int nk, int r0 = 0,
                                             int t0 = 0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = wave * 8 + (lane >> 3);
  const int gq = (lane & 7) ^ ((row >> 1) & 7);
  const float scale = p.in_scale[r0 + row < int(p.M) ? r0 + row : int(p.M) - 1];
  unsigned char* base = reinterpret_cast<unsigned char*>(xs) + wave * 1024 + lane * 16;
  for (int t = t0; t < nk; ++t) {
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

__device__ __forceinline__ void zero_acc(f32x4_t (&acc)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x4_t{};
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

// The same partial with a run-time k-range and one tile's loads at a time: the
// arithmetic (per-tile dequant, MFMA order) is identical to run_split, so
// its result is bit-identical.  Used by the recompute path only.
template <bool INT4, bool INORM>
__device__ void partial_any(const ProblemArgs& p, const WeightArgs& w, int proj, int hh, int kt0, int nk,
                            const uint16_t* xs, uint32_t xs_lds, f32x4_t (&acc)[4], int r0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int64_t kbeg = int64_t(kt0) * kBK;
  const int64_t col = int64_t(hh) * kHeadDim + wave * 16 + c16;
  zero_acc(acc);
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

// partial_any over a range longer than one x slice: slices of kDecMaxNK tiles,
// each staged once every wave is done with the previous one, the tiles
// accumulated in order into one sum (the arithmetic of the two-slice split).
// (A function of its own rather than a loop in partial_any: that keeps the code
// of the one-slice kernels, C3's among them, exactly as it was.)
template <bool INT4, bool INORM>
__device__ void partial_any_long(const ProblemArgs& p, const WeightArgs& w, int proj, int hh, int kt0, int nk,
                                 const uint16_t* xs, uint32_t xs_lds, f32x4_t (&acc)[4], int r0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  const int64_t col = int64_t(hh) * kHeadDim + wave * 16 + c16;
  zero_acc(acc);
  for (int c0 = 0; c0 < nk; c0 += kDecMaxNK) {
    const int cn = nk - c0 < kDecMaxNK ? nk - c0 : kDecMaxNK;
    const int64_t kbeg = int64_t(kt0 + c0) * kBK;
    if (c0 > 0) barrier();  // every wave is done with the previous slice
    for (int t = 0; t < cn; ++t) stage_x_tile(p, kbeg, t, xs_lds, r0);
    wait_vm<0>();
    if (INORM) norm_x_tiles(p, const_cast<uint16_t*>(xs), kbeg, cn, r0);  // gamma is in LDS already
    barrier();
    for (int t = 0; t < cn; ++t) {
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
}

// What a workgroup works on: split `split` of head (128-column tile) `head`,
// projection `proj` / head `hh` inside it, for the launch's `nblk` 64-row blocks.
struct DecWork {
  int head, split, splits, proj, hh, nblk;
  uint32_t inc;  // this split's arrival increment (its XCD, and the forced flag for tests)
  int max_spins;  // polls of a designated finisher's final wait before it hands the block off
  int H;                  // heads of the projection (row stride of its output, in heads)
  const uint16_t* gamma;  // QK-Norm weights of the projection (Q or K)
  uint16_t* out;          // q / k / v (may be null: cache only)
};

// Arrival counter of a (head, block), one atomic add per split: bits 0-4 count
// the splits that have published (at most 16), bits 5-12 sum their XCDs x and
// bits 13-22 sum x * x, bits 23-27 count splits forced onto the recompute path
// (tests), and bit 30 marks a block whose designated finisher gave up waiting
// for the others (see run_split).  The splits of a head are dispatched to one
// XCD (workgroups go round-robin over the XCDs, from a starting XCD that
// depends on the hardware queue), so their partials meet in one L2; the last
// arrival checks that they did: n * sum(x^2) == sum(x)^2 exactly when all n
// values of x are equal.
constexpr uint32_t kAbandoned = 1u << 30;
constexpr uint32_t kForcedUnit = 1u << 23;
__device__ __forceinline__ uint32_t arrival_inc(int x, bool forced) {
  return 1u + (uint32_t(x) << 5) + (uint32_t(x * x) << 13) + (forced ? kForcedUnit : 0u);
}
__device__ __forceinline__ bool all_arrived(uint32_t v, int splits) { return (v & 0x1Fu) == uint32_t(splits); }
// some split ran on another XCD than the others (or was forced to recompute)
__device__ __forceinline__ bool any_foreign(uint32_t v, int splits) {
  v = __builtin_amdgcn_readfirstlane(v);  // (the same in every lane: scalar arithmetic)
  const uint32_t sx = (v >> 5) & 0xFFu, sxx = (v >> 13) & 0x3FFu;
  return ((v >> 23) & 0x1Fu) != 0 || uint32_t(splits) * sxx != sx * sx;
}

// Finishes 64-row block `blk` of the workgroup's head: sums every split's partial
// in split order (RECOMPUTE: recomputes them all), applies RMSNorm + RoPE (Q/K),
// stores the bf16 rows and resets the block's arrival counter.  prow / cslot:
// RoPE-table offset and paged-cache slot of this thread's row of the block.
template <bool INT4, bool INORM, bool MULTI, bool RECOMPUTE, bool LONG = false>
__device__ __forceinline__ void finish_block(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                                             const DecWork& d, int blk, const f32x4_t (&acc)[4], int64_t prow,
                                             int64_t cslot, uint16_t* xs, float* __restrict__ part,
                                             uint32_t* __restrict__ counters) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n_tiles = p.n_tiles;
  const int M = int(p.M);
  const uint32_t xs_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xs));
  float* tile = reinterpret_cast<float*>(xs);  // the finisher's head tile aliases the x slice
  uint32_t* counter = counters + blk * n_tiles + d.head;
  if (RECOMPUTE && tid == 0)  // statistics: heads finished on the recompute path
    __hip_atomic_fetch_add(counters + kDecodeRecomputeWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // thread -> row r = tid / 8, c = tid % 8 of the head tile: columns [8c, 8c+8)
  // and [64+8c, 64+8c+8), so every RoPE pair (d, d+64) is thread-local.  Its
  // gamma / cos / sin operands are loaded under the partial reads; its RoPE row
  // was read when the block started, so no dependent load stalls the finisher.
  const int r = tid >> 3;
  const int c = tid & 7;
  const int hd = e.head_dim;
  const PairRuns pr = pair_runs(c, hd);  // (head_dim 64: two heads per block, see pair_runs)
  const int rr = blk * kDecRows + r;  // this thread's row of the launch
  const bool qk = e.qkv == 1 && d.proj != 2;  // (qkv 2: q and k stored as projected)
  f32x4_t sum[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) sum[mb] = f32x4_t{};
  if constexpr (!RECOMPUTE) {
    // The other splits' fragments of this wave are pulled into LDS with direct
    // L2 -> LDS loads (a CU fetches faster that way than into VGPRs), up to four
    // splits per batch in the x slice's space, which no wave reads any more; each
    // wave reads back only the 4 KB regions it loaded itself, so its own vmcnt
    // wait is the only synchronisation.  Summation is in split order.  In a
    // launch of several blocks the finisher reads its own partial back as well:
    // its registers then hold the weights of the later blocks instead.
    const char* frag = reinterpret_cast<const char*>(part) +
                       (((int64_t(blk) * n_tiles + d.head) * kDecWaves + wave) * 4 * 64) * sizeof(f32x4_t);
    const int64_t split_stride = int64_t(d.nblk) * n_tiles * kTileFloats * sizeof(float);
    const uint32_t slot0 = xs_lds + uint32_t(wave * 4096);
    const char* slot0_ptr = reinterpret_cast<const char*>(xs) + wave * 4096;
    int slot = 0, first = 0;
#pragma unroll 1
    for (int q = 0; q < d.splits; ++q) {
      if (MULTI || q != d.split) {  // (MULTI: this split's partial too, see below)
        const char* src = frag + q * split_stride + lane * 16;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
          dma16(src + mb * 1024, slot0 + uint32_t(slot * kDecWaves * 4096 + mb * 1024));
        ++slot;
      }
      if (slot == 4 || q == d.splits - 1) {  // four slots filled, or the last split: add in split order
        wait_vm<0>();
        int u_slot = 0;
#pragma unroll 1
        for (int u = first; u <= q; ++u) {
          if (!MULTI && u == d.split) {
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) sum[mb] += acc[mb];
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
    const int nkt = int(p.K / kBK);
    for (int s = 0; s < d.splits; ++s) {
      int s_kt0, s_nk;
      split_range(s, d.splits, nkt, s_kt0, s_nk);
      __syncthreads();  // every wave is done with the x slice of the previous split
      f32x4_t part_s[4];
      if constexpr (LONG) partial_any_long<INT4, INORM>(p, w, d.proj, d.hh, s_kt0, s_nk, xs, xs_lds, part_s, blk * kDecRows);
      else partial_any<INT4, INORM>(p, w, d.proj, d.hh, s_kt0, s_nk, xs, xs_lds, part_s, blk * kDecRows);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) sum[mb] += part_s[mb];
    }
  }

  // (loaded only now: during the partial sums the registers hold the weights of later blocks)
  u32x4_t g_lo{}, g_hi{}, c_lo{}, c_hi{}, s_lo{}, s_hi{};
  if (qk && rr < M) {
    const uint16_t* gamma = d.gamma;
    g_lo = load8_bf16(gamma + pr.dim_lo);
    g_hi = load8_bf16(gamma + pr.dim_hi);
    c_lo = load8_bf16(e.cos + prow + pr.dim_lo);
    c_hi = load8_bf16(e.cos + prow + pr.dim_hi);
    s_lo = load8_bf16(e.sin + prow + pr.dim_lo);
    s_hi = load8_bf16(e.sin + prow + pr.dim_hi);
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
    const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(src + pr.col_lo);
    const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(src + pr.col_lo + 4);
    const f32x4_t b0 = *reinterpret_cast<const f32x4_t*>(src + pr.col_hi);
    const f32x4_t b1 = *reinterpret_cast<const f32x4_t*>(src + pr.col_hi + 4);
    lo[0] = a0.x; lo[1] = a0.y; lo[2] = a0.z; lo[3] = a0.w;
    lo[4] = a1.x; lo[5] = a1.y; lo[6] = a1.z; lo[7] = a1.w;
    hi[0] = b0.x; hi[1] = b0.y; hi[2] = b0.z; hi[3] = b0.w;
    hi[4] = b1.x; hi[5] = b1.y; hi[6] = b1.z; hi[7] = b1.w;
  }
  if (qk) {
    // RMSNorm over the head (fused_qkv_rope.py:98-100), then rotate-half RoPE
    // (:102-118).  Every fused multiply-add is explicit and nothing else is
    // contracted, so each instantiation of this code (the finish from partials
    // and the recompute finish) rounds identically.
#pragma clang fp contract(off)
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(hi[i], hi[i], __builtin_fmaf(lo[i], lo[i], ss));
    ss = head_sum(ss, hd);
    const float rms = head_rms(ss, e.eps, hd);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x1n = lo[i] * rms * bf16_lane(g_lo, i);
      const float x2n = hi[i] * rms * bf16_lane(g_hi, i);
      const float t1 = __builtin_fmaf(x1n, bf16_lane(c_lo, i), -(x2n * bf16_lane(s_lo, i)));
      const float t2 = __builtin_fmaf(x2n, bf16_lane(c_hi, i), x1n * bf16_lane(s_hi, i));
      lo[i] = t1;
      hi[i] = t2;
    }
  }
  if (rr < M) {
    u32x4_t o1, o2;
    o1.x = pack_bf16x2(lo[0], lo[1]);
    o1.y = pack_bf16x2(lo[2], lo[3]);
    o1.z = pack_bf16x2(lo[4], lo[5]);
    o1.w = pack_bf16x2(lo[6], lo[7]);
    o2.x = pack_bf16x2(hi[0], hi[1]);
    o2.y = pack_bf16x2(hi[2], hi[3]);
    o2.z = pack_bf16x2(hi[4], hi[5]);
    o2.w = pack_bf16x2(hi[6], hi[7]);
    if (e.qkv) {
      const int H = d.H;
      uint16_t* base = d.out;
      if (base) {
        uint16_t* dst = base + (int64_t(rr) * H + d.hh) * kHeadDim;
        *reinterpret_cast<u32x4_t*>(dst + pr.col_lo) = o1;
        *reinterpret_cast<u32x4_t*>(dst + pr.col_hi) = o2;
      }
      if (cslot >= 0) {
        uint16_t* crow = paged_row(e, cslot, d.proj, d.hh);
        *reinterpret_cast<u32x4_t*>(crow + pr.col_lo) = o1;
        *reinterpret_cast<u32x4_t*>(crow + pr.col_hi) = o2;
      }
    } else {  // plain GEMM output [M, N] (whole 128-column tiles: N % 128 == 0)
      uint16_t* dst = e.out + int64_t(rr) * e.N + int64_t(d.head) * kHeadDim;
      *reinterpret_cast<u32x4_t*>(dst + pr.col_lo) = o1;
      *reinterpret_cast<u32x4_t*>(dst + pr.col_hi) = o2;
    }
  }
  if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The weights of a wave's 16 columns over its split of NK k tiles as bf16 MFMA
// fragments, held in registers (int4 weights dequantised once, in block 0).
template <int NK>
struct HeldWeights {
  u32x4_t b[NK][2];
};

// Block 0: streams the wave's weight slice from HBM into registers (bf16: each
// tile's two fragments are requested about kDecLookahead tiles ahead of its
// MFMAs, after the x slice, so early tiles land early; int4: the packed words
// with their scales and zeros) and multiplies each 64-wide k tile as soon as it
// has landed.
template <bool INT4, bool INORM, int NK>
__device__ __forceinline__ void first_block(const ProblemArgs& p, const WeightArgs& w, const DecWork& d,
                                            int kt0, uint16_t* xs, HeldWeights<NK>& hw, f32x4_t (&acc)[4]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15, g4 = lane >> 4;
  const uint32_t xs_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xs));
  const int64_t kbeg = int64_t(kt0) * kBK;
  const int64_t col = int64_t(d.hh) * kHeadDim + wave * 16 + c16;
  constexpr int kLook = NK < kDecLookahead ? NK : kDecLookahead;
  u32x4_t gv[kGamPerThread];
  if (INORM) gamma_load(p, gv);
  if constexpr (!INT4) {
    const uint16_t* wp = w.w[d.proj] + col * p.K + kbeg + g4 * 8;
    stage_x_slice<NK>(p, kbeg, xs_lds);
#pragma unroll
    for (int t = 0; t < kLook; ++t)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) hw.b[t][kk] = wload(wp + t * kBK + kk * 32);
    wait_vm<2 * kLook>();  // the x slice (and gamma) have landed (older than the weight loads) ...
    if (INORM) {
      gamma_to_lds(p, gv);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier();
      norm_x_tiles(p, xs, kbeg, NK);
    }
    barrier();  // ... in every wave
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      if (t + kLook < NK) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) hw.b[t + kLook][kk] = wload(wp + (t + kLook) * kBK + kk * 32);
      }
      mma_tile(xs, t, hw.b[t], acc);
    }
  } else {
    // int4 weights are 4x smaller: load them with their scales and zeros, then
    // the x slice, and wait for everything
    const Int4Col ic = int4_col(w, d.proj, col);
    uint32_t q4[NK][2], sraw[NK], zw[NK];
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      const int64_t k0 = kbeg + int64_t(t) * kBK;
      const int64_t grp = k0 / ic.group;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) q4[t][kk] = uint32_t(ic.qw[(k0 / 8 + kk * 4 + g4) * ic.n + col]);
      sraw[t] = ic.sc[grp * ic.n + col];
      zw[t] = uint32_t(ic.qz[grp * (ic.n / 8) + col / 8]);
    }
    stage_x_slice<NK>(p, kbeg, xs_lds);
    wait_vm<0>();
    if (INORM) {
      gamma_to_lds(p, gv);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      barrier();
      norm_x_tiles(p, xs, kbeg, NK);
    }
    barrier();
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      dequant_tile(ic, q4[t], sraw[t], zw[t], hw.b[t]);
      mma_tile(xs, t, hw.b[t], acc);
    }
  }
}

// Tiles per barrier when a later block consumes its x slice: the MFMAs of a
// group start once its tiles have landed, under the loads of the next groups.
constexpr int kDecGroup = 4;

// A later block at row r0: stages its x slice (NK direct loads per thread, in
// tile order) and multiplies it by the held weights, group by group as the tiles
// land.  After the first group's wait and barrier -- when every memory operation
// each thread issued before the call (e.g. a partial's stores) has completed --
// it calls after_first_wait() in every thread.
template <bool INORM, int NK, class F>
__device__ __forceinline__ void later_block(const ProblemArgs& p, int64_t kbeg, int r0, uint16_t* xs,
                                            const HeldWeights<NK>& hw, f32x4_t (&acc)[4], F&& after_first_wait) {
  const uint32_t xs_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xs));
  stage_x_slice<NK>(p, kbeg, xs_lds, r0);
#pragma unroll
  for (int g0 = 0; g0 < NK; g0 += kDecGroup) {
    const int g1 = g0 + kDecGroup < NK ? g0 + kDecGroup : NK;
    wait_vm_n(NK - g1);  // (the loads of the later groups may stay in flight)
    if (INORM) norm_x_tiles(p, xs, kbeg, g1, r0, g0);
    barrier();
    if (g0 == 0) after_first_wait();
#pragma unroll
    for (int t = g0; t < g1; ++t) mma_tile(xs, t, hw.b[t], acc);
  }
}

// This wave's fp32 partial of block `blk` to part[split][blk][head][wave][mb][lane]
// (fragment order, 16-byte stores; not waited for here).
__device__ __forceinline__ void publish_partial(const ProblemArgs& p, const DecWork& d, int blk,
                                                const f32x4_t (&acc)[4], float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  f32x4_t* mine = reinterpret_cast<f32x4_t*>(part) +
                  (((int64_t(d.split) * d.nblk + blk) * p.n_tiles + d.head) * kDecWaves + wave) * 4 * 64 + lane;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) mine[mb * 64] = acc[mb];
}

__device__ __forceinline__ uint32_t arrive(uint32_t* counter, const DecWork& d) {
  return __hip_atomic_fetch_add(counter, d.inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + d.inc;
}

// RoPE-table offset and paged-cache slot of this thread's row (tid / 8) of block b.
__device__ __forceinline__ void block_rows(const EpilogueArgs& e, const DecWork& d, int M, int b, int64_t& prow,
                                           int64_t& cslot) {
  const int rr = b * kDecRows + (threadIdx.x >> 3);
  prow = (e.qkv == 1 && d.proj != 2 && rr < M) ? rope_row(e, rr) * e.head_dim : 0;
  cslot = (e.qkv && d.proj != 0 && rr < M) ? paged_slot(e, rr) : -1;
}

// One 64-row block (T <= 64): the split's partial, then the last split to arrive
// finishes the head (from the partials, or by recomputation when some split ran
// on another XCD).
// A split of NK + NK2 tiles (NK2 > 0) runs as two slices: the second x slice is
// staged once every wave is done with the first, and its tiles accumulate after
// the first's, so the order of the sums is that of one NK + NK2 slice.
// (LONG: some split of the launch is longer than one x slice, so the recompute
// path runs every split's range in slices.)
template <bool INT4, bool INORM, int NK, int NK2 = 0, bool LONG = (NK2 > 0)>
__device__ __forceinline__ void run_split_single(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                                                 const DecWork& d, int kt0, uint16_t* xs, uint32_t* arrival,
                                                 float* __restrict__ part, uint32_t* __restrict__ counters) {
  int64_t prow, cslot;  // read now: a positions[] load here is off every critical path
  block_rows(e, d, int(p.M), 0, prow, cslot);
  HeldWeights<NK> hw;
  f32x4_t acc[4];
  zero_acc(acc);
  first_block<INT4, INORM, NK>(p, w, d, kt0, xs, hw, acc);
  if constexpr (NK2 > 0) {
    __syncthreads();  // every wave is done with the first x slice
    HeldWeights<NK2> hw2;
    first_block<INT4, INORM, NK2>(p, w, d, kt0 + NK, xs, hw2, acc);
  }
  publish_partial(p, d, 0, acc, part);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have reached the L2
  __syncthreads();                // ... and every thread's
  if (threadIdx.x == 0) arrival[0] = arrive(counters + d.head, d);
  __syncthreads();
  const uint32_t seen = arrival[0];
  if (!all_arrived(seen, d.splits)) return;
  if (any_foreign(seen, d.splits)) finish_block<INT4, INORM, false, true, LONG>(p, w, e, d, 0, acc, prow, cslot, xs, part, counters);
  else finish_block<INT4, INORM, false, false, LONG>(p, w, e, d, 0, acc, prow, cslot, xs, part, counters);
}

// Several 64-row blocks.  Block 0 streams the weights into registers; each later
// block stages its rows' x slice in the same LDS and multiplies it by the held
// weights, so the weights are read from HBM once per launch.
//
// Block b is finished by its designated split b % splits.  (Were the last split
// to arrive to finish it, the slowest split would finish every block and fall
// further behind each time.)  A block's arrival is counted one block later: the
// staging of the next block already waits for all outstanding memory operations,
// the partial's stores included, so the counter increment needs no wait of its
// own and its latency hides under the next block's MFMAs.  The designated split
// finishes a block when it arrives last; otherwise it notes the block and checks
// its counter again, without waiting, at its next blocks, and waits for what is
// still open after its last block.  That wait is bounded: on time-out the block is
// marked kAbandoned and its last split to arrive finishes it instead, so no
// workgroup waits on one that cannot start before it exits.  Blocks whose splits
// did not all run on the XCD the grid assumes are recomputed after the block
// loop, when the held weights no longer need their registers.
template <bool INT4, bool INORM, int NK>
__device__ __forceinline__ void run_split_multi(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                                                const DecWork& d, int kt0, uint16_t* xs, uint32_t* arrival,
                                                float* __restrict__ part, uint32_t* __restrict__ counters) {
  const uint32_t xs_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xs));
  const int64_t kbeg = int64_t(kt0) * kBK;
  const int M = int(p.M);
  const int nblk = d.nblk;
  const int n_tiles = p.n_tiles;
  const bool tid0 = threadIdx.x == 0;
  const f32x4_t no_acc[4] = {};
  uint32_t deferred = 0;  // blocks to finish by recomputation after the loop
  uint32_t pending = 0;   // designated blocks noted, not yet finished
  HeldWeights<NK> hw;

  // Finish block b (counter value v, every split arrived), or defer it.
  auto finish_or_defer = [&](int b, uint32_t v) {
    if (any_foreign(v, d.splits)) {
      deferred |= 1u << b;
    } else {
      int64_t b_prow, b_cslot;
      block_rows(e, d, M, b, b_prow, b_cslot);
      finish_block<INT4, INORM, true, false>(p, w, e, d, b, no_acc, b_prow, b_cslot, xs, part, counters);
    }
  };
  // The counter value of block b after this split's arrival (seen) and the value
  // of the oldest noted block read at the same time (probed, probe_blk >= 0):
  // finish what this split is due to finish.
  auto decide = [&](int b, uint32_t seen, int probe_blk, uint32_t probed) {
    const bool mine = b % d.splits == d.split;
    if (all_arrived(seen, d.splits) && (mine || (seen & kAbandoned))) finish_or_defer(b, seen);
    else if (mine) pending |= 1u << b;
    if (probe_blk >= 0 && probe_blk != b && all_arrived(probed, d.splits)) {
      pending &= ~(1u << probe_blk);
      finish_or_defer(probe_blk, probed);
    }
  };

#pragma unroll 1
  for (int blk = 0; blk < nblk; ++blk) {
    f32x4_t acc[4];
    zero_acc(acc);
    if (blk == 0) {
      first_block<INT4, INORM, NK>(p, w, d, kt0, xs, hw, acc);
      publish_partial(p, d, 0, acc, part);
      continue;
    }
    // this block's x slice in the same LDS once every wave is done with it (the
    // previous block's MFMAs or a finish); the normalising gamma stays in LDS.
    // Once its first tiles have landed, so have the previous block's partial
    // stores (issued earlier): then that block's arrival is counted and the
    // counter of the oldest noted block read; both values are used after this
    // block's MFMAs.
    barrier();
    const int probe_blk = pending != 0 ? __builtin_ctz(pending) : -1;
    uint32_t seen = 0, probed = 0;
    later_block<INORM, NK>(p, kbeg, blk * kDecRows, xs, hw, acc, [&]() {
      if (tid0) {
        seen = arrive(counters + (blk - 1) * n_tiles + d.head, d);
        if (probe_blk >= 0)
          probed = __hip_atomic_load(counters + probe_blk * n_tiles + d.head, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
      }
    });
    publish_partial(p, d, blk, acc, part);
    if (tid0) {
      arrival[0] = seen;
      arrival[1] = probed;
    }
    __syncthreads();
    seen = arrival[0];
    probed = arrival[1];
    __syncthreads();  // (arrival is rewritten by the next block)
    decide(blk - 1, seen, probe_blk, probed);
  }
  // the last block's arrival
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid0) arrival[0] = arrive(counters + (nblk - 1) * n_tiles + d.head, d);
  __syncthreads();
  const uint32_t last_seen = arrival[0];
  __syncthreads();
  decide(nblk - 1, last_seen, -1, 0);

  // the noted blocks still open
#pragma unroll 1
  while (pending != 0) {
    const int b = __builtin_ctz(pending);
    pending &= pending - 1u;
    uint32_t* counter = counters + b * n_tiles + d.head;
    if (tid0) {
      uint32_t v = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int spin = 0; !all_arrived(v, d.splits) && spin < d.max_spins; ++spin) {
        __builtin_amdgcn_s_sleep(2);
        v = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // give up: the last split to arrive sees kAbandoned and finishes the block;
      // if every split arrived meanwhile, the fetch-or returns a full count
      if (!all_arrived(v, d.splits))
        v = __hip_atomic_fetch_or(counter, kAbandoned, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      arrival[0] = v;
    }
    __syncthreads();
    const uint32_t v = arrival[0];
    __syncthreads();
    if (all_arrived(v, d.splits)) finish_or_defer(b, v);
  }
#pragma unroll 1
  for (int b = 0; b < nblk; ++b) {
    if (!(deferred >> b & 1u)) continue;
    int64_t b_prow, b_cslot;
    block_rows(e, d, M, b, b_prow, b_cslot);
    __syncthreads();  // every wave is done with the LDS
    finish_block<INT4, INORM, true, true>(p, w, e, d, b, no_acc, b_prow, b_cslot, xs, part, counters);
  }
}

// The workgroup's split: grid position -> (head, split), XCD check, k range.
__device__ __forceinline__ DecWork dec_work(const ProblemArgs& p, const EpilogueArgs& e, int splits,
                                            int ctl, int& kt0, int& nk) {
  const int bid = blockIdx.x;
  const int xcds = p.xcds;
  const int q = bid / xcds;
  DecWork d;
  d.split = q % splits;
  d.head = (q / splits) * xcds + bid % xcds;
  d.splits = splits;
  d.nblk = int((p.M + kDecRows - 1) / kDecRows);
  split_head(d.head, e.Hq, e.Hkv, d.proj, d.hh);
  d.H = d.proj == 0 ? e.Hq : e.Hkv;
  d.gamma = pick3(d.proj, e.q_gamma, e.k_gamma, e.k_gamma);
  d.out = pick3(d.proj, e.q, e.k, e.v);
  // (XCC_ID is the physical XCD; a partition of the GPU holds xcds of them)
  d.inc = arrival_inc(xcc_id() % xcds, (ctl & 1) != 0);
  d.max_spins = ctl >> 1;
  split_range(d.split, splits, int(p.K / kBK), kt0, nk);
  return d;
}

// One 64-row block (T <= 64: decode steps, tails).
template <bool INT4, bool INORM>
__global__ void __launch_bounds__(kDecThreads, 1)
decode_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int splits, float* __restrict__ part,
              uint32_t* __restrict__ counters, int ctl) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kDecRows * kDecKc];
  __shared__ uint32_t arrival[2];
  if ((blockIdx.x / p.xcds / splits) * p.xcds + blockIdx.x % p.xcds >= p.n_tiles) return;  // padding
  int kt0, nk;
  const DecWork d = dec_work(p, e, splits, ctl, kt0, nk);
  switch (nk) {
#define MQK_DEC_CASE(n) \
  case n: run_split_single<INT4, INORM, n>(p, w, e, d, kt0, xs, arrival, part, counters); break;
    MQK_DEC_CASE(1) MQK_DEC_CASE(2) MQK_DEC_CASE(3) MQK_DEC_CASE(4)
    MQK_DEC_CASE(5) MQK_DEC_CASE(6) MQK_DEC_CASE(7) MQK_DEC_CASE(8)
    MQK_DEC_CASE(9) MQK_DEC_CASE(10) MQK_DEC_CASE(11) MQK_DEC_CASE(12)
    MQK_DEC_CASE(13) MQK_DEC_CASE(14) MQK_DEC_CASE(15) MQK_DEC_CASE(16)
#undef MQK_DEC_CASE
    default: break;  // the launcher guarantees 1 <= nk <= kDecMaxNK
  }
}

// One 64-row block whose splits are longer than one x slice
// (kDecMaxNK < nk <= kDecLongMaxNK for the longest): a kernel of its own, so
// that the kernel above keeps its code and register allocation.
template <bool INT4, bool INORM>
__global__ void __launch_bounds__(kDecThreads, 1)
decode_long_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int splits, float* __restrict__ part,
                   uint32_t* __restrict__ counters, int ctl) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kDecRows * kDecKc];
  __shared__ uint32_t arrival[2];
  if ((blockIdx.x / p.xcds / splits) * p.xcds + blockIdx.x % p.xcds >= p.n_tiles) return;  // padding
  int kt0, nk;
  const DecWork d = dec_work(p, e, splits, ctl, kt0, nk);
  // bf16: a first slice of kDecMaxNK tiles; int4: two halves (a 16-tile first
  // slice keeps too many packed words live and spills)
  constexpr auto first = [](int n) { return INT4 ? (n + 1) / 2 : (n > kDecMaxNK ? kDecMaxNK : n); };
  switch (nk) {
    // (balanced ranges: a launch whose longest split exceeds one slice has splits
    // of at least kDecMaxNK tiles)
#define MQK_DEC_LONG(n)                                                                                          \
  case n:                                                                                                         \
    run_split_single<INT4, INORM, first(n), n - first(n), true>(p, w, e, d, kt0, xs, arrival, part, counters);   \
    break;
    MQK_DEC_LONG(16) MQK_DEC_LONG(17) MQK_DEC_LONG(18) MQK_DEC_LONG(19) MQK_DEC_LONG(20)
    MQK_DEC_LONG(21) MQK_DEC_LONG(22) MQK_DEC_LONG(23) MQK_DEC_LONG(24)
    MQK_DEC_LONG(25) MQK_DEC_LONG(26) MQK_DEC_LONG(27) MQK_DEC_LONG(28)
    MQK_DEC_LONG(29) MQK_DEC_LONG(30) MQK_DEC_LONG(31) MQK_DEC_LONG(32)
#undef MQK_DEC_LONG
    default: break;  // the launcher guarantees kDecMaxNK <= nk <= kDecLongMaxNK
  }
}

// Several 64-row blocks, the weights held in registers across them.  Its splits
// cover NKC or NKC - 1 k tiles (balanced ranges), and each NKC is its own kernel
// so that the register allocation of the held weights fits the actual k range.
template <bool INT4, bool INORM, int NKC>
__global__ void __launch_bounds__(kDecThreads, 1)
decode_multi_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int splits, float* __restrict__ part,
                    uint32_t* __restrict__ counters, int ctl) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kDecRows * kDecKc];
  __shared__ uint32_t arrival[2];
  if ((blockIdx.x / p.xcds / splits) * p.xcds + blockIdx.x % p.xcds >= p.n_tiles) return;  // padding
  int kt0, nk;
  const DecWork d = dec_work(p, e, splits, ctl, kt0, nk);
  if (nk == NKC) run_split_multi<INT4, INORM, NKC>(p, w, e, d, kt0, xs, arrival, part, counters);
  else if constexpr (NKC > 1) run_split_multi<INT4, INORM, NKC - 1>(p, w, e, d, kt0, xs, arrival, part, counters);
}

}  // namespace

int g_decode_force_recompute = 0;
int g_decode_max_spins = kDecMaxSpins;

int decode_splits_for(int64_t M, int64_t K, int n_tiles, int requested, int cus, int xcds) {
  (void)M;
  const int nkt = int(K / kBK);
  if (nkt < 1) return 0;
  const int max_nk = kDecLongMaxNK;  // (both weight formats: splits of up to two x slices)
  const int min_splits = (nkt + max_nk - 1) / max_nk;  // bound on a split's k-range
  int s = requested;
  if (s <= 0) {
    // one workgroup per CU: (heads per XCD) x splits <= CUs per XCD
    xcds = xcds < 1 ? 1 : xcds;
    const int heads_per_xcd = (n_tiles + xcds - 1) / xcds;
    s = (cus / xcds) / heads_per_xcd;
    // at least four k tiles per split: with little to stream per split, the
    // finisher's partial reads cost more than the extra CUs save (measured at
    // hidden 1024: 9.2-10 us with four splits against 10.6-11.4 us with eight)
    if (s > nkt / 4) s = nkt / 4;
    if (s < min_splits) s = min_splits;
  }
  if (s < min_splits || s > nkt || s > kDecMaxNK) return 0;
  return s;
}

size_t decode_counter_bytes() { return size_t(kCounterBytes); }

size_t decode_workspace_bytes(int n_tiles, int splits, int blocks) {
  return size_t(kCounterBytes) + size_t(splits) * blocks * n_tiles * kTileFloats * sizeof(float);
}

int decode_max_blocks(int n_tiles, int64_t K, int splits, bool int4_norm) {
  const int max_nk = int4_norm ? kDecMultiMaxNKInt4Norm : kDecMultiMaxNK;
  if (splits < 1 || (K / kBK + splits - 1) / splits > max_nk) return 1;
  const int by_counters = kMaxHeads / (n_tiles < 1 ? 1 : n_tiles);
  return by_counters < kDecMaxBlocks ? by_counters : kDecMaxBlocks;
}

namespace {
using DecKernel = void (*)(ProblemArgs, WeightArgs, EpilogueArgs, int, float*, uint32_t*, int);
// the int4 + input-norm kernel of several blocks, where it exists
template <int N>
constexpr DecKernel int4_norm_multi() {
  if constexpr (N <= kDecMultiMaxNKInt4Norm) return decode_multi_kernel<true, true, N>;
  else return nullptr;
}
}  // namespace

hipError_t launch_decode(int int4, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                         int splits, void* workspace, hipStream_t stream) {
  const int nkt = int(p.K / kBK);
  const int blocks = int((p.M + kDecRows - 1) / kDecRows);  // 64-row blocks of this launch
  // (p.xcds <= 8: the arrival counter's XCD sums hold x < 8)
  if (splits < 1 || splits > kDecMaxNK || splits > nkt || p.xcds > 8 ||
      (nkt + splits - 1) / splits > (blocks > 1 ? kDecMultiMaxNK : kDecLongMaxNK) ||
      p.n_tiles > kMaxHeads || blocks < 1 || blocks > decode_max_blocks(p.n_tiles, p.K, splits, int4 && p.in_gamma) || p.xcds < 1)
    return hipErrorInvalidValue;
  uint32_t* counters = static_cast<uint32_t*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  const dim3 grid(((p.n_tiles + p.xcds - 1) / p.xcds) * p.xcds * splits);
  // ctl: bit 0 forces the recompute path, the rest is the final wait's poll limit
  const int fr = (g_decode_force_recompute ? 1 : 0) | (g_decode_max_spins << 1);
  auto a16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; };
  if (e.qkv && !(a16(e.q_gamma) && a16(e.k_gamma) && a16(e.cos) && a16(e.sin))) return hipErrorInvalidValue;
  if (!e.qkv && (e.N % kHeadDim != 0 || !a16(e.out) || int64_t(p.n_tiles) * kHeadDim != e.N))
    return hipErrorInvalidValue;
  const size_t dyn = p.in_gamma ? size_t(p.K) * 2 : 0;
  if (p.in_gamma && (p.K / 8 > int64_t(kGamPerThread) * kDecThreads ||
                     kDecRows * kDecKc * 2 + 16 + dyn > 160 * 1024 || !a16(p.in_gamma)))
    return hipErrorInvalidValue;
  // (the input norm and several blocks are template switches: the plain one-block
  // kernels carry none of their code)
  using Kernel = void (*)(ProblemArgs, WeightArgs, EpilogueArgs, int, float*, uint32_t*, int);
  static const Kernel single[4] = {decode_kernel<false, false>, decode_kernel<false, true>,
                                   decode_kernel<true, false>, decode_kernel<true, true>};
#define MQK_MULTI(n)                                                                              \
  {decode_multi_kernel<false, false, n>, decode_multi_kernel<false, true, n>,                      \
   decode_multi_kernel<true, false, n>, int4_norm_multi<n>()}
  static const Kernel multi[kDecMultiMaxNK][4] = {
      MQK_MULTI(1), MQK_MULTI(2), MQK_MULTI(3), MQK_MULTI(4),  MQK_MULTI(5),  MQK_MULTI(6),  MQK_MULTI(7),
      MQK_MULTI(8), MQK_MULTI(9), MQK_MULTI(10), MQK_MULTI(11), MQK_MULTI(12), MQK_MULTI(13)};
#undef MQK_MULTI
  const int variant = (int4 ? 2 : 0) + (p.in_gamma ? 1 : 0);
  const int nkc = (nkt + splits - 1) / splits;  // longest k range of a split, in tiles
  static const Kernel longk[4] = {decode_long_kernel<false, false>, decode_long_kernel<false, true>,
                                  decode_long_kernel<true, false>, decode_long_kernel<true, true>};
  Kernel kernel = blocks > 1 ? multi[nkc - 1][variant] : (nkc > kDecMaxNK ? longk[variant] : single[variant]);
  if (!kernel) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kernel, grid, dim3(kDecThreads), dyn, stream, p, w, e, splits, part, counters, fr);
  return hipGetLastError();
}

}  // namespace mqk
