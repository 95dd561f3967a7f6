// Host-side launch interface between the C ABI (mqk_api.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mqk {

constexpr int kHeadDimDefault = 128;

// Weight source of the projection.  A 128-column tile h (one head) belongs to
// projection 0 (Q) for h < Hq, 1 (K) for h < Hq + Hkv, else 2 (V); for a plain
// GEMM (w4a16_gemm) every tile belongs to projection 0 and Hq is the tile count.
struct WeightArgs {
  // bf16: w[p] is [n_cols[p], K] row-major (nn.Linear layout).
  const uint16_t* w[3];
  // int4: qw[p] [K/8, n_cols[p]] int32, sc[p] [K/group, n_cols[p]] (bf16 or fp16),
  //       qz[p] [K/group, n_cols[p]/8] int32.
  const int32_t* qw[3];
  const void* sc[3];
  const int32_t* qz[3];
  int64_t n_cols[3];
  int group;
  int scale_fp16;
};

// Output side.  qkv == 1: per-head norm + RoPE for Q/K tiles, plain store for V,
// outputs q [T, Hq, 128], k/v [T, Hkv, 128].  qkv == 0: plain [M, N] store into out.
struct EpilogueArgs {
  int qkv;
  int Hq, Hkv;
  const uint16_t* q_gamma;
  const uint16_t* k_gamma;
  const uint16_t* cos;
  const uint16_t* sin;
  const int32_t* positions;
  int64_t S;
  int64_t cos_rows;
  float eps;
  uint16_t* q;
  uint16_t* k;
  uint16_t* v;
  uint16_t* out;   // plain GEMM output
  int64_t N;       // plain GEMM width
  // Paged KV cache (null k_cache: none).  K / V row of token t also goes to
  // cache[(block * block_size + slot) * Hkv + head] (see paged_slot).
  uint16_t* k_cache;
  uint16_t* v_cache;
  const int32_t* block_table;  // [bt_rows, bt_cols]
  const int32_t* kv_seq;       // [T] or null: t / kv_len
  const int32_t* kv_pos;       // [T] or null: t % kv_len
  int64_t bt_rows, bt_cols, num_blocks, kv_len;
  int block_size;
  // Varlen mode (non-null cu_seqlens): token t is in sequence s with
  // cu_seqlens[s] <= t < cu_seqlens[s+1], at position t - cu_seqlens[s] (+ seq_pos0[s]);
  // that position selects its RoPE row and (with no kv_seq / kv_pos) its cache slot.
  const int32_t* cu_seqlens;
  const int32_t* seq_pos0;
  int64_t n_seqs;
  // Token index of the launch's row 0 within the call (a call's tokens may be
  // split over two launches); positions, slots and varlen offsets are indexed by
  // the call's token index, outputs and x by the launch's rows.
  int64_t t0;
  // Head dim, 128 or 64.  Hq / Hkv above (and the problem's n_tiles) count
  // 128-column blocks, Hq * head_dim / 128 of them: two heads of 64 per block.
  // gamma has head_dim entries and the cos / sin rows are head_dim apart.
  int head_dim = kHeadDimDefault;
};

struct ProblemArgs {
  const uint16_t* x;   // [M, K] bf16
  int64_t M;
  int64_t K;
  int n_tiles;         // number of 128-column tiles (heads)
  // Input RMSNorm (null in_gamma: none): the projection reads
  // bf16(in_gamma[k] * bf16(x[m, k] * in_scale[m])) instead of x (input_norm8).
  const uint16_t* in_gamma;  // [K] bf16
  const float* in_scale;     // [M] rsqrt(mean(x^2) + eps), from launch_row_scale
  // Topology of the device the launch runs on (hipDeviceGetAttribute): compute
  // units, and XCDs, each with its own L2; workgroup b is dispatched to XCD
  // b % xcds.
  int cus;
  int xcds;
};

// One tile-kernel variant: BM rows x (HPT*128) columns per workgroup, with KZ
// waves splitting each staged K tile.
struct TileVariant {
  int id;
  int bm;
  int hpt;
  int kz;
  int threads;
};

int tile_variant_count();
const TileVariant* tile_variant(int index);
// Picks a variant for the problem (id 0 = automatic).
// allow_pair: the pair-tile variants (24-28) may be chosen (bf16 q/k/v outputs
// with head_dim 128 and a workspace for their exchange).
const TileVariant* choose_tile_variant(int requested_id, int64_t M, int n_tiles, int int4, int cus,
                                       bool allow_pair = false);
// Workgroups of one launch of variant v over M rows and n_tiles heads.
int64_t tile_count(const TileVariant& v, int64_t M, int n_tiles);
hipError_t launch_tile(const TileVariant& v, int int4, const ProblemArgs& p, const WeightArgs& w,
                       const EpilogueArgs& e, int group_m, hipStream_t stream);
// Direct-to-LDS pipelined tile kernel (variant ids >= 10, bf16 weights).
hipError_t launch_tile_dma(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                           hipStream_t stream);
// Split-K launch of a pipelined bf16 variant (16: 128x384, 18: 256x256) for
// problems with fewer tiles than CUs: each tile's K range is cut into ksplit
// balanced ranges, run by ksplit workgroups on one XCD; each publishes its fp32
// accumulators and counts its arrival in counters[tile]; once all have arrived,
// each finishes its share of the tile's 32-row units (partials summed in split
// order, then the tile epilogue on those rows).  A split whose bounded wait
// (max_spins polls) runs out hands its units to the last arrival.  If a split
// ran on another XCD (or force_recompute), the last arrival recomputes every
// split (same arithmetic, same order) and finishes the whole tile.  The
// workspace: kDecodeCounterBytes of counters (zero; the tile words at
// kSplitWordsOffset, re-armed by the launch), then tile_split_part_bytes(...)
// of partials.
hipError_t launch_tile_dma_split(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                                 int ksplit, int force_recompute, int max_spins, void* workspace, hipStream_t stream);
size_t tile_split_part_bytes(int id, int64_t M, int n_tiles, int ksplit);
// Pair tiles (ids 24: 256 x 192, 25: 256 x 320, 26: 128 x 192, 27: 128 x 320,
// 28: 192 x 192; bf16 weights, head_dim 128): two workgroups cover 2 * hpt + 1 heads
// of BM = 256, 128 or 192 rows (hpt = 1 or 2 whole heads each, and half of the head they share).  The sides
// exchange the shared head's row sums of squares through the workspace:
// kDecodeCounterBytes of counters (the pair words reuse the split-K tile lines, zero
// between launches), then per pair 2 * BM floats of sums and a BM x 64 float
// hand-over area;
// pair_tile_workspace_bytes(id, M, n_tiles) in all.  max_spins bounds a side's
// wait for its partner before it hands its half over.
hipError_t launch_pair_tile(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e, int group_m,
                            void* workspace, int max_spins, hipStream_t stream);
size_t pair_tile_workspace_bytes(int id, int64_t M, int n_tiles);
inline bool is_pair_variant(int id) { return id >= 24 && id <= 28; }
// (tests) bits 0-15: side 1 of every pair waits this many ~4 us intervals before it
// publishes, which sends side 0 down the hand-over path once its bounded wait runs
// out; bit 16: the sides take adjacent workgroup ids (different XCDs).
extern int g_pair_hold;
// int4-weight (W4A16) variant of the pipelined kernel, ids 30-33.
hipError_t launch_tile_dma_w4(int id, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                              int group_m, hipStream_t stream);

// Split-K decode kernel for T <= 64.  decode_splits_for returns 0 when no
// valid split count exists (each split covers at most 16 64-wide k tiles);
// the caller then uses the tile kernel.
// LDS bytes (static) of pipelined tile variant id (10..32); 0 for other ids.
int tile_dma_lds_bytes(int id);

// Input RMSNorm pre-pass: scale[m] = rsqrt(mean(x[m, :]^2) + eps) for x [M, K] bf16.
hipError_t launch_row_scale(const uint16_t* x, int64_t M, int64_t K, float eps, float* scale,
                            hipStream_t stream);

int decode_splits_for(int64_t M, int64_t K, int n_tiles, int requested, int cus, int xcds);
size_t decode_workspace_bytes(int n_tiles, int splits, int blocks = 1);
// Most 64-row blocks one decode launch may cover with this many heads and splits
// (one arrival counter per (head, block) in the workspace's counter region; one
// block when a split's k range is too long to hold its weights in registers).
int decode_max_blocks(int n_tiles, int64_t K, int splits, bool int4_norm);
// The decode kernel's counters open every workspace: one arrival counter per
// head (kDecodeMaxHeads), then a statistics line whose first word counts the
// heads finished on the recompute path (a split ran on an unexpected XCD), then
// the split-K tile launch's words: one 128-byte line per tile (its arrival word,
// then its exit word), so that the splits of different tiles never contend for
// a line.
constexpr int kDecodeMaxHeads = 1024;
constexpr size_t kSplitWordsOffset = size_t(kDecodeMaxHeads) * 4 + 256;
constexpr int kSplitMaxTiles = 512;
constexpr size_t kSplitLineBytes = 128;
constexpr size_t kDecodeCounterBytes = kSplitWordsOffset + size_t(kSplitMaxTiles) * kSplitLineBytes;
constexpr int kDecodeRecomputeWord = kDecodeMaxHeads;
size_t decode_counter_bytes();
// The split-K decode kernel on the launch's p.M rows: ceil(M / 64) <=
// decode_max_blocks(n_tiles) blocks of 64 rows share one stream of the weights;
// the workspace holds decode_workspace_bytes(n_tiles, splits, blocks).  With
// e.qkv == 0 it writes the plain product to e.out ([M, N], N = 128 * n_tiles).
hipError_t launch_decode(int int4, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                         int splits, void* workspace, hipStream_t stream);

// 1: the last workgroup of every head recomputes all splits itself (the path
// taken when a split ran on an unexpected XCD); for tests.
extern int g_decode_force_recompute;
// Polls a designated finisher makes for the last splits of its block before it
// hands the block to the last split to arrive (several-block launches); tests
// set it low to exercise the hand-off.
extern int g_decode_max_spins;

// W4A16 GEMM for small M (1 <= M <= kGemvMaxM): out[M, N] = x[M, K] @ dequant(W)
// with w.qw[0] / sc[0] / qz[0] / n_cols[0] = N / group / scale_fp16; fp32
// dequantisation and accumulation, one bf16 rounding; no workspace (w4_gemv.hip).
constexpr int kGemvMaxM = 16;
hipError_t launch_w4_gemv(const uint16_t* x, const WeightArgs& w, int64_t M, int64_t K, uint16_t* out,
                          hipStream_t stream);

// HBM read-rate probe (bench.py): reads `bytes` (16-byte aligned) once over
// `blocks` workgroups of 512 threads and writes one word per workgroup to out.
hipError_t launch_read_probe(const void* src, size_t bytes, int blocks, uint32_t* out, hipStream_t stream);
// Shader clock probe (bench.py): out[0..2] = shader clocks and 100 MHz ticks over a
// dependent chain of `spins` FMAs, and the chain's result.
hipError_t launch_clock_probe(uint64_t* out, int spins, hipStream_t stream);

// Standalone QK-norm + RoPE.
// QK-Norm + RoPE in place on already-projected q [T, Hq, D] / k [T, Hkv, D] (e.q, e.k)
// for a head_dim D that is a multiple of 8 up to 512 (e.head_dim).
hipError_t launch_norm_rope_any(const EpilogueArgs& e, int64_t T, hipStream_t stream);
hipError_t launch_norm_rope(const uint16_t* q_raw, const uint16_t* k_raw, const EpilogueArgs& e,
                            int64_t T, hipStream_t stream);

// fp32 / fp16 front: x, weights, norm weights and RoPE tables all fp32 (or all
// fp16), outputs in the same type; products and sums in fp32.
struct F32Args {
  const void* x;        // [M, K]
  const void* w[3];     // w_q [Hq*128, K], w_k / w_v [Hkv*128, K]
  const void* q_gamma;
  const void* k_gamma;
  const void* cos;      // [cos_rows, 128]
  const void* sin;
  const int32_t* positions;  // [M] or null: prefill, token t uses row t % S
  int64_t M, K, S, cos_rows;
  int Hq, Hkv;
  float eps;
  void* q;              // [M, Hq, 128]
  void* k;              // [M, Hkv, 128]
  void* v;              // [M, Hkv, 128]
  // (fields read by rope_row: no varlen, launch row 0 is token 0)
  const int32_t* cu_seqlens = nullptr;
  const int32_t* seq_pos0 = nullptr;
  int64_t n_seqs = 0;
  int64_t t0 = 0;
  // head dim, 128 or 64 (Hq / Hkv then count 128-column blocks of two heads)
  int head_dim = kHeadDimDefault;
};
constexpr int kF32BK = 32;       // k extent of one staged tile of the fp32 / fp16 front
// rows: token rows per workgroup, 32 or 16; half: fp16 elements (else fp32)
hipError_t launch_f32_qkv(const F32Args& a, int rows, bool half, int xcds, hipStream_t stream);

}  // namespace mqk
