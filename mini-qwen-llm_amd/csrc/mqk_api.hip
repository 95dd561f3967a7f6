// C ABI of libmqk.so: argument validation, kernel selection and launch.
// Declarations and the contract of every entry point: include/mqk.h.
#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/mqk.h"
#include "mqk_device.h"
#include "mqk_kernels.h"

using namespace mqk;

namespace {

thread_local char g_detail[256] = "";

int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_detail, sizeof(g_detail), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_detail[0] = '\0';
  return MQK_OK;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return ok();
  return fail(MQK_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }
size_t align_up(size_t n, size_t a) { return (n + a - 1) / a * a; }

// Process-wide knobs (mqk_set_option).
std::atomic<int64_t> g_prefill_tile{0};
std::atomic<int64_t> g_decode_max_t{64};
std::atomic<int64_t> g_decode_splits{0};
std::atomic<int64_t> g_group_m{8};
std::atomic<int64_t> g_tail_split{1};
std::atomic<int64_t> g_decode_blocks{16};  // most 64-row decode blocks for one call (T > 64)
std::atomic<int64_t> g_decode_cost_model{1};  // 0: decode blocks whenever eligible (measurements)
std::atomic<int64_t> g_decode_passes{16};  // most 64-row blocks one decode launch covers (1..16)
std::atomic<int64_t> g_head_tiles{1};  // one round of single-head tiles where the planner models them fastest
std::atomic<int64_t> g_tile_ksplit{1};  // split-K tile launches: 0 off, 1 by cost model, >= 2 that split count
std::atomic<int64_t> g_gemv_max_m{kGemvMaxM};  // W4A16 GEMMs with M up to this run the column-parallel kernel
std::atomic<int64_t> g_pair_tiles{1};  // pair-tile variants (24-28) as planner candidates
std::atomic<int64_t> g_pair_max_spins{1 << 14};  // a pair side's polls for its partner before it hands its half over

constexpr int kMaxTiles = 1024;  // arrival counters available in the workspace (per head)

// Shared validation of the position / table / gamma arguments.
int check_rope_args(const void* q_gamma, const void* k_gamma, const void* cos, const void* sin,
                    int64_t S, int64_t cos_rows, const int32_t* positions, float eps, bool varlen = false) {
  if (!q_gamma || !k_gamma || !cos || !sin)
    return fail(MQK_ERR_NULL_POINTER, "q_gamma/k_gamma/cos/sin must be non-NULL");
  if (cos_rows <= 0) return fail(MQK_ERR_BAD_SHAPE, "cos_rows must be > 0 (got %lld)", (long long)cos_rows);
  if (!positions && !varlen && S <= 0)
    return fail(MQK_ERR_BAD_SHAPE, "prefill mode (positions == NULL) needs S > 0 (got %lld)", (long long)S);
  if (!(eps >= 0.0f)) return fail(MQK_ERR_BAD_SHAPE, "eps must be >= 0");
  return MQK_OK;
}

EpilogueArgs make_qkv_epilogue(const mqk_bf16* q_gamma, const mqk_bf16* k_gamma, const mqk_bf16* cos,
                               const mqk_bf16* sin, const int32_t* positions, int64_t S,
                               int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                               int Hq, int Hkv) {
  EpilogueArgs e{};
  e.qkv = 1;
  e.Hq = Hq;
  e.Hkv = Hkv;
  e.q_gamma = q_gamma;
  e.k_gamma = k_gamma;
  e.cos = cos;
  e.sin = sin;
  e.positions = positions;
  e.S = positions ? 1 : S;
  e.cos_rows = cos_rows;
  e.eps = eps;
  e.q = q;
  e.k = k;
  e.v = v;
  return e;
}

bool int4_aligned(const WeightArgs& w) {
  for (int i = 0; i < 3; ++i)
    if (!aligned16(w.qw[i]) || !aligned16(w.sc[i]) || !aligned16(w.qz[i])) return false;
  return true;
}

bool use_decode(int64_t T) { return T >= 1 && T <= g_decode_max_t.load() && T <= 64; }

// The split-K decode kernel and the pipelined tile variants read gamma / cos /
// sin rows with 16-byte loads.
bool epilogue_aligned(const EpilogueArgs& e) {
  return aligned16(e.q_gamma) && aligned16(e.k_gamma) && aligned16(e.cos) && aligned16(e.sin);
}

// Compute units and XCDs of the calling thread's current device, queried once
// per device (an MI355X has 256 CUs in 8 XCDs; a partitioned one fewer).
struct Topology {
  int cus = 256;
  int xcds = 8;
};
constexpr int kMaxTopoDevices = 64;
std::mutex g_topo_mu;
Topology g_topo[kMaxTopoDevices];
bool g_topo_known[kMaxTopoDevices] = {};

Topology device_topology() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxTopoDevices) {
    (void)hipGetLastError();
    return Topology{};
  }
  std::lock_guard<std::mutex> lock(g_topo_mu);
  if (!g_topo_known[dev]) {
    Topology t;
    int cus = 0, xcds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0)
      t.cus = cus;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess && xcds > 0 &&
        t.cus % xcds == 0)
      t.xcds = xcds;
    else
      t.xcds = t.cus % 8 == 0 ? 8 : 1;
    (void)hipGetLastError();
    g_topo[dev] = t;
    g_topo_known[dev] = true;
  }
  return g_topo[dev];
}

// How a call's T tokens are split over kernels.  T <= 64: the split-K decode
// kernel alone.  Otherwise a tile kernel; when the rows of its last, partial
// row tile (at most 64) would cost a whole extra round of tiles over the CUs,
// those rows go to the decode kernel in a second launch instead (e.g. 8214
// tokens in 256-row tiles: three full rounds plus 22 rows).
struct Plan {
  const TileVariant* v = nullptr;  // tile variant (null: decode only)
  int64_t tail = 0;                // rows run by the decode kernel after the tile rows
  int splits = 0;                  // decode kernel split-K factor (0: no decode launch)
  int passes = 1;                  // 64-row blocks per decode launch
  int ksplit = 0;                  // tile launch split over K (0: one workgroup per tile)
};

// Split-K tile launch for problems with fewer tiles than CUs (bf16 weights):
// variant 16 (128 x 384) when the heads tile by 3, else 18 (256 x 256).  Returns
// the split count (0: none fits) and its modelled kernel time, fitted on MI355X:
// a fixed cost (launch and waits), a cost per 64-k stage of the busiest split, per
// MB of fp32 partials published and read back, and per 32-row unit of a tile that
// the busiest split finishes (ceil(units / splits)).
//   128 x 384 (hidden 4096, T = 129 .. 1024, 2 to 8 splits; within ~1.5 us):
//     9.5 us, 1.13 us per stage, 0.24 us per MB, 5.2 us per unit.
//   256 x 256 (hidden 1024 / 2048 / 5120 with 32 / 40 / 56 heads, T = 128 .. 1536,
//     2 to 8 splits; rms error 1.5 us): 12.6 us, 1.6 us per stage of
//     ceil(stages / splits), 0.195 us per MB, 0.35 us per unit.
// (The 256 x 256 split kernel has no input-norm form: with the norm's registers it
// would spill.)
int plan_tile_split(int64_t M, int64_t K, int n_tiles, const Topology& topo, bool in_norm, const TileVariant*& v,
                    double& us) {
  v = nullptr;
  us = 1e30;
  const int64_t req = g_tile_ksplit.load();
  if (req == 0 || g_prefill_tile.load() != 0) return 0;
  const int id = n_tiles % 3 == 0 ? 16 : (n_tiles % 2 == 0 && !in_norm ? 18 : 0);
  if (id == 0) return 0;
  for (int i = 0; i < tile_variant_count(); ++i)
    if (tile_variant(i)->id == id) v = tile_variant(i);
  if (!v) return 0;
  const int64_t tiles = (M + v->bm - 1) / v->bm * (n_tiles / v->hpt);
  const int64_t X = topo.xcds;
  const int64_t slots = (tiles + X - 1) / X * X;  // tiles padded to whole XCD shares
  const int64_t nkt = K / 64;
  const double fixed_us = id == 16 ? 9.5 : 12.6, stage_us = id == 16 ? 1.13 : 1.6;
  const double mb_us = id == 16 ? 0.24 : 0.195, unit_us = id == 16 ? 5.2 : 0.35;
  const double part_mb = (id == 16 ? 196608.0 : 262144.0) * 1e-6;  // one workgroup's partial
  const int units = id == 16 ? 4 : 8;
  int best = 0;
  const int lo = req >= 2 ? int(req) : 2, hi = req >= 2 ? int(req) : 8;
  for (int s = lo; s <= hi; ++s) {
    if (slots * s > topo.cus || nkt < 4 * int64_t(s) || tiles > kSplitMaxTiles) break;
    const double stages = id == 16 ? double(nkt) / s : double((nkt + s - 1) / s);
    const double t = fixed_us + stages * stage_us + mb_us * part_mb * double(tiles) * s +
                     unit_us * double((units + s - 1) / s);
    if (t < us) {
      us = t;
      best = s;
    }
  }
  return best;
}

Plan plan_fused(int int4, int64_t M, int64_t K, int n_tiles, bool aligned, const Topology& topo,
                bool allow_blocks = true, bool in_norm = false, bool allow_split = true, bool allow_pair = false) {
  allow_pair = allow_pair && !int4 && aligned && g_pair_tiles.load() != 0;
  Plan pl;
  const int64_t cus = topo.cus;
  if (use_decode(M) && aligned) {
    pl.splits = decode_splits_for(M, K, n_tiles, int(g_decode_splits.load()), topo.cus, topo.xcds);
    if (pl.splits > 0) {
      pl.tail = M;
      return pl;
    }
  }
  // A few 64-row blocks: a decode launch streams the weights over every CU once
  // for up to sixteen blocks (holding them in registers), which beats a tile
  // launch whose few tiles leave most CUs idle and stream their panels at a
  // single CU's rate.  Measured at hidden 4096 (kernel times): the first block
  // of a launch ~19 us bf16 / ~17 us int4 (the weight stream), each further
  // block ~5 us (its x slice staged, multiplied, published and finished by its
  // designated split: T = 128 / 256 / 512 / 1024 take 25.6 / 39.3 / 56.9 / 93.5 us
  // bf16), against ~83 us (bf16) and ~138 us (int4) for the best tile variant at
  // T = 65..1024.  The models below follow those measurements; at hidden 4096 bf16
  // runs as blocks up to T = 832, int4 up to T = 1024.  The bf16 block costs were
  // refitted over hidden 1024 / 2048 / 4096 (32 / 40 / 48 heads, T = 128 .. 1024;
  // within ~2.5 us): the first block ~14.2 us + 0.187 us per MB of weights, each
  // further block 2.17 + 0.584 * K/1024 us.  The one-workgroup-per-tile launch
  // costs ~1.15 us per 64-k stage with 128 x 384 tiles, ~1.27 us with the others.
  // int4, refitted over the same shapes and hidden 5120 (40/8 heads): the first
  // block max(14.5, 1.45 * k tiles per split) us, each further block
  // 1.95 + 0.71 * K/1024 us, the tile kernel 2.1 us per stage + 7 us.
  const int64_t nblk = (M + 63) / 64;
  const int blk_splits = decode_splits_for(64, K, n_tiles, int(g_decode_splits.load()), topo.cus, topo.xcds);
  const int64_t per_launch = std::max<int64_t>(
      1, std::min<int64_t>(g_decode_passes.load(), decode_max_blocks(n_tiles, K, blk_splits, int4 && in_norm)));
  const int64_t launches = (nblk + per_launch - 1) / per_launch;
  const double w_bytes = double(n_tiles) * kHeadDim * double(K) * (int4 ? 0.5 : 2.0);
  // (int4's first block is bound by the 64-k tiles each split dequantises and
  // multiplies, ~1.45 us each, over a ~14.5 us floor)
  const int64_t split_kt = blk_splits > 0 ? (K / 64 + blk_splits - 1) / blk_splits : 0;
  // (splits longer than a launch of several blocks takes run one block per launch,
  // each ~7.5 + 0.65 us per k tile: 20.5 / 21.3 / 25.1 us at 20 / 22 / 27 tiles)
  const double dec_us = !int4 ? 14.2 + 0.187 * w_bytes * 1e-6
                              : (split_kt > 13 ? 7.5 + 0.65 * double(split_kt) : std::max(14.5, 1.45 * double(split_kt)));
  const double pass_us = int4 ? 1.95 + 0.71 * double(K) / 1024.0 : 2.17 + 0.584 * double(K) / 1024.0;
  const double blocks_us = double(launches) * dec_us + double(nblk - launches) * pass_us;
  const double tile_us = int4 ? double(K) / 64.0 * 2.1 + 7.0 : double(K) / 64.0 * (n_tiles % 3 == 0 ? 1.15 : 1.27) + 5.0;
  // split-K tile launch (bf16): taken when its model beats both the one-workgroup-
  // per-tile launch and the decode blocks
  const TileVariant* sv = nullptr;
  double split_us = 1e30;
  const int ksplit = (!int4 && aligned && allow_split && M > 64) ? plan_tile_split(M, K, n_tiles, topo, in_norm, sv, split_us) : 0;
  // One round of single-head tiles: 64 x 128 while ceil(M/64) x heads fit the CUs,
  // else 128 x 128 with 8 waves while ceil(M/128) x heads do.  Neither needs a
  // partial exchange.  Fitted on MI355X over hidden 2048 / 4096 / 5120 (40 / 48 / 56
  // heads, T = 128 .. 1024; within ~6 %), per 64-k stage:
  //   bf16 (ids 20 / 21): 2 + 0.5 us, and 2.5 + (0.6 + 0.0002 * tiles) us;
  //   int4 (ids 35 / 34): 3.5 + 1.0 us, and 2.5 + 1.2 us (the dequantisation bounds
  //   them: they win only where the decode blocks' long splits run one block per
  //   launch, e.g. hidden 5120 at T = 384 / 512: 98 us against 119 / 158).
  const TileVariant* hv = nullptr;
  double head_us = 1e30;
  if (aligned && M > 64 && g_prefill_tile.load() == 0 && g_head_tiles.load() != 0) {
    const int64_t t64 = (M + 63) / 64 * n_tiles, t128 = (M + 127) / 128 * n_tiles;
    const double stages = double(K / 64);
    const bool one64 = t64 <= cus, one128 = t128 <= cus;
    const int id = one64 ? (int4 ? 35 : 20) : (one128 ? (int4 ? 34 : 21) : 0);
    for (int i = 0; id != 0 && i < tile_variant_count(); ++i)
      if (tile_variant(i)->id == id) hv = tile_variant(i);
    if (hv) {
      if (int4) head_us = one64 ? 3.5 + 1.0 * stages : 2.5 + 1.2 * stages;
      else head_us = one64 ? 2.0 + 0.5 * stages : 2.5 + stages * (0.6 + 0.0002 * double(t128));
    }
  }
  // One round of 128-row pair tiles (26: 2 x 128 x 192 per 3 heads) over more than
  // half of the CUs, which no whole-head shape fills at these T, against the split-K,
  // single-head and decode-block launches.  Fitted on MI355X (hidden 2560 / 4096,
  // 48 heads, T = 576 .. 1024, within ~2 us): 15 us + (0.465 + 0.001 * workgroups) us
  // per 64-k stage.  (The 2-stage 128 x 320 form 27 and the 192-row form 28 win only
  // against whole-head tiles; the tile chooser ranks them.)
  const TileVariant* pv = nullptr;
  double pair_us = 1e30;
  if (allow_pair && M > 64 && g_prefill_tile.load() == 0 && n_tiles % 3 == 0) {
    for (int i = 0; i < tile_variant_count(); ++i)
      if (tile_variant(i)->id == 26) pv = tile_variant(i);
    const int64_t wgs = pv ? tile_count(*pv, M, n_tiles) : 0;
    if (pv && 2 * wgs > cus && wgs <= cus && wgs / 2 <= kSplitMaxTiles &&
        !(in_norm && tile_dma_lds_bytes(26) + K * 2 > 160 * 1024)) {
      pair_us = 15.0 + double(K / 64) * (0.465 + 0.001 * double(wgs));
    } else {
      pv = nullptr;
    }
  }
  const bool blocks_ok = allow_blocks && aligned && M > 64 && g_prefill_tile.load() == 0 &&
                         g_decode_max_t.load() >= 64 && nblk <= g_decode_blocks.load() && blk_splits > 0;
  const bool forced_split = ksplit > 0 && g_tile_ksplit.load() >= 2;
  if (blocks_ok && !forced_split &&
      (!g_decode_cost_model.load() ||
       (blocks_us <= tile_us && blocks_us <= split_us && blocks_us <= head_us && blocks_us <= pair_us))) {
    pl.splits = blk_splits;
    pl.tail = M;
    pl.passes = int(std::min<int64_t>(per_launch, nblk));
    return pl;
  }
  if (ksplit > 0 && (forced_split || (split_us < tile_us && split_us <= head_us && split_us <= pair_us))) {
    pl.v = sv;
    pl.ksplit = ksplit;
    return pl;
  }
  if (hv && head_us < tile_us && head_us <= pair_us) {
    pl.v = hv;
    return pl;
  }
  if (pv && pair_us < tile_us) {
    pl.v = pv;
    return pl;
  }
  pl.v = choose_tile_variant(int(g_prefill_tile.load()), M, n_tiles, int4, topo.cus, allow_pair);
  if (!pl.v || !g_tail_split.load() || !aligned || M <= 64) return pl;
  const int64_t r = M % pl.v->bm;
  if (r == 0 || r > 64 || !use_decode(r)) return pl;
  const int64_t rounds_all = (tile_count(*pl.v, M, n_tiles) + cus - 1) / cus;
  const int64_t rounds_main = (tile_count(*pl.v, M - r, n_tiles) + cus - 1) / cus;
  if (rounds_main >= rounds_all) return pl;
  const int splits = decode_splits_for(r, K, n_tiles, int(g_decode_splits.load()), topo.cus, topo.xcds);
  if (splits > 0) {
    pl.tail = r;
    pl.splits = splits;
  }
  return pl;
}

// Common launcher of the fused op (bf16 or int4 weights).  With an input norm
// (p.in_gamma set, epsilon in_eps), the per-token scales go to the workspace
// after the decode kernel's region and are computed by a pre-pass first.
int run_fused(int int4, ProblemArgs p, const WeightArgs& w, const EpilogueArgs& e, float in_eps,
              void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (p.M == 0) return ok();
  const Topology topo = device_topology();
  p.cus = topo.cus;
  p.xcds = topo.xcds;
  // pair tiles: q/k/v outputs with head_dim 128 (their epilogue splits a head in
  // 32-dim runs) and paged-cache slots below 2^31 (held in 32 bits)
  const bool pair_ok = e.qkv && e.head_dim == kHeadDim &&
                       (!e.k_cache || double(e.num_blocks) * double(e.block_size) < 2147483647.0);
  Plan pl = plan_fused(int4, p.M, p.K, p.n_tiles, epilogue_aligned(e), topo, true, p.in_gamma != nullptr, true, pair_ok);
  if (!pl.v && pl.splits == 0)
    return fail(MQK_ERR_BAD_OPTION, "prefill_tile variant %lld cannot run this problem (%d heads%s)",
                (long long)g_prefill_tile.load(), p.n_tiles, int4 ? ", int4 weights" : "");
  // (the decode kernel's arrival counters open every workspace and must stay zero,
  // so the scales never start before them, whichever kernel runs this call)
  auto region = [&](const Plan& q) {
    if (q.ksplit > 0) return kDecodeCounterBytes + tile_split_part_bytes(q.v->id, p.M, p.n_tiles, q.ksplit);
    if (q.v && is_pair_variant(q.v->id))
      return std::max(pair_tile_workspace_bytes(q.v->id, p.M - q.tail, p.n_tiles),
                      q.splits > 0 ? decode_workspace_bytes(p.n_tiles, q.splits, q.passes) : size_t(0));
    return q.splits > 0 ? decode_workspace_bytes(p.n_tiles, q.splits, q.passes) : decode_counter_bytes();
  };
  size_t base = region(pl);
  // bytes the plan needs: the decode (or split-tile) region, then (input norm) the per-token scales
  const size_t scale_bytes = p.in_gamma ? align_up(size_t(p.M) * sizeof(float), 256) : 0;
  auto fits = [&](size_t b) { return workspace && ws_bytes >= align_up(b, 256) + scale_bytes; };
  const bool split_ok = epilogue_aligned(e) && !(p.in_gamma && pl.v && tile_dma_lds_bytes(pl.v->id) + p.K * 2 > 160 * 1024);
  if (pl.ksplit > 0 && (!fits(base) || !split_ok)) {
    // a workspace sized without the split-K tile launch (or operands it cannot take): plan without it
    pl = plan_fused(int4, p.M, p.K, p.n_tiles, epilogue_aligned(e), topo, true, p.in_gamma != nullptr, false, pair_ok);
    base = region(pl);
  }
  if (pl.v && is_pair_variant(pl.v->id) &&
      (!fits(base) || (p.in_gamma && tile_dma_lds_bytes(pl.v->id) + p.K * 2 > 160 * 1024))) {
    // a workspace sized without the pair tiles' exchange area, or an input norm whose
    // gamma does not fit the LDS beside their ring: plan without them
    pl = plan_fused(int4, p.M, p.K, p.n_tiles, epilogue_aligned(e), topo, true, p.in_gamma != nullptr, false, false);
    base = region(pl);
  }
  while (!pl.v && pl.passes > 1 && !fits(base)) {
    pl.passes = (pl.passes + 1) / 2;  // a workspace sized for fewer blocks per launch
    base = decode_workspace_bytes(p.n_tiles, pl.splits, pl.passes);
  }
  if (!pl.v && p.M > 64 && !fits(base)) {
    // decode blocks planned, but a workspace sized without them: the tile kernel
    pl = plan_fused(int4, p.M, p.K, p.n_tiles, epilogue_aligned(e), topo, false, p.in_gamma != nullptr, false);
    base = region(pl);
  }
  if (pl.v && pl.splits > 0 && !fits(base)) {
    pl.tail = 0;  // a workspace sized without the tail launch: run the tile kernel on every row
    pl.splits = 0;
    base = decode_counter_bytes();
  }
  const size_t scale_off = align_up(base, 256);
  const bool pair = pl.v && is_pair_variant(pl.v->id);
  const size_t need = p.in_gamma ? scale_off + size_t(p.M) * sizeof(float)
                                 : ((pl.splits > 0 || pl.ksplit > 0 || pair) ? base : 0);
  if (need > 0 && (!workspace || ws_bytes < need))
    return fail(MQK_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given%s", need, ws_bytes,
                workspace ? "" : " (NULL)");
  if (p.in_gamma) {
    float* scale = reinterpret_cast<float*>(static_cast<char*>(workspace) + scale_off);
    const int st = hip_status(launch_row_scale(p.x, p.M, p.K, in_eps, scale, stream), "input norm pre-pass launch");
    if (st != MQK_OK) return st;
    p.in_scale = scale;
  }
  if (pl.ksplit > 0)
    return hip_status(launch_tile_dma_split(pl.v->id, p, w, e, pl.ksplit, g_decode_force_recompute,
                                            g_decode_max_spins, workspace, stream),
                      "split-K tile kernel launch");
  if (pl.v) {
    const TileVariant* v = pl.v;
    // The pipelined variants (ids >= 10) read every operand with 16-byte direct loads,
    // and with an input norm hold gamma in LDS next to their ring.
    if (v->id >= 10 && (!(epilogue_aligned(e) && (!int4 || int4_aligned(w))) ||
                        (p.in_gamma && tile_dma_lds_bytes(v->id) + p.K * 2 > 160 * 1024)))
      v = choose_tile_variant(p.n_tiles % 2 == 0 ? 4 : 1, p.M, p.n_tiles, int4, p.cus);
    ProblemArgs pm = p;
    pm.M = p.M - pl.tail;
    const int st =
        is_pair_variant(v->id)
            ? hip_status(launch_pair_tile(v->id, pm, w, e, int(g_group_m.load()), workspace,
                                          int(g_pair_max_spins.load()), stream),
                         "pair tile kernel launch")
            : hip_status(launch_tile(*v, int4, pm, w, e, int(g_group_m.load()), stream), "tile kernel launch");
    if (st != MQK_OK || pl.tail == 0) return st;
  }
  // the decode kernel on the last pl.tail rows (all of them when there is no tile
  // launch), pl.passes blocks of 64 rows per launch; the launches share the
  // workspace in stream order
  const int64_t rows_per_launch = 64 * int64_t(pl.passes);
  for (int64_t t0 = p.M - pl.tail; t0 < p.M; t0 += rows_per_launch) {
    ProblemArgs pt = p;
    pt.M = std::min<int64_t>(rows_per_launch, p.M - t0);
    pt.x = p.x + t0 * p.K;
    if (p.in_scale) pt.in_scale = p.in_scale + t0;
    EpilogueArgs et = e;
    et.t0 = t0;
    auto shift = [&](uint16_t* ptr, int heads) { return ptr ? ptr + t0 * heads * kHeadDim : ptr; };
    et.q = shift(e.q, e.Hq);
    et.k = shift(e.k, e.Hkv);
    et.v = shift(e.v, e.Hkv);
    if (e.out) et.out = e.out + t0 * e.N;  // plain GEMM output [M, N]
    const int st = hip_status(launch_decode(int4, pt, w, et, pl.splits, workspace, stream), "decode kernel launch");
    if (st != MQK_OK) return st;
  }
  return ok();
}

}  // namespace

extern "C" {

int mqk_version(void) { return 100; }  // 0.1.0

const char* mqk_error_string(int status) {
  switch (status) {
    case MQK_OK: return "ok";
    case MQK_ERR_NULL_POINTER: return "null pointer argument";
    case MQK_ERR_BAD_SHAPE: return "invalid shape or size";
    case MQK_ERR_UNSUPPORTED: return "unsupported shape";
    case MQK_ERR_MISALIGNED: return "pointer not 16-byte aligned";
    case MQK_ERR_WORKSPACE: return "workspace missing or too small";
    case MQK_ERR_HIP: return "HIP runtime error";
    case MQK_ERR_BAD_OPTION: return "bad option";
    default: return "unknown mqk status";
  }
}

const char* mqk_last_error_detail(void) { return g_detail; }

// Workspace bytes run_fused's plan of `tiles` 128-column blocks needs (before
// any input-norm scales): a plain GEMM (bf16 or int4 weights, no pair tiles), or
// with allow_pair the q/k/v launch of the generic head sizes.
static size_t plan_bytes(int int4, int64_t M, int64_t K, int tiles, const Topology& topo, bool in_norm,
                         bool allow_pair) {
  if (tiles > kMaxTiles) return ~size_t(0);
  const Plan pl = plan_fused(int4, M, K, tiles, true, topo, true, in_norm, true, allow_pair);
  size_t n = 0;
  if (pl.splits > 0) n = std::max(n, decode_workspace_bytes(tiles, pl.splits, pl.passes));
  if (pl.ksplit > 0) n = std::max(n, kDecodeCounterBytes + tile_split_part_bytes(pl.v->id, M, tiles, pl.ksplit));
  if (pl.v && is_pair_variant(pl.v->id)) n = std::max(n, pair_tile_workspace_bytes(pl.v->id, M - pl.tail, tiles));
  return n;
}

static size_t plain_plan_bytes(int int4, int64_t M, int64_t K, int tiles, const Topology& topo) {
  if (int4 && M <= g_gemv_max_m.load()) return 0;  // the column-parallel kernel needs none
  return plan_bytes(int4, M, K, tiles, topo, false, false);
}

size_t mqk_fused_qkv_rope_workspace_size(int64_t T, int Hq, int Hkv, int64_t hidden) {
  if (T <= 0 || Hq <= 0 || Hkv <= 0 || hidden <= 0 || hidden % kBK != 0) return 0;
  const int tiles = Hq + 2 * Hkv;
  size_t n = 0;
  for (int int4 = 0; int4 < 2; ++int4) {  // the same size serves both weight formats
    const Plan pl = plan_fused(int4, T, hidden, tiles, true, device_topology(), true, false, true, true);
    if (pl.splits > 0) n = std::max(n, decode_workspace_bytes(tiles, pl.splits, pl.passes));
    if (pl.v && is_pair_variant(pl.v->id)) n = std::max(n, pair_tile_workspace_bytes(pl.v->id, T - pl.tail, tiles));
    if (pl.ksplit > 0) n = std::max(n, kDecodeCounterBytes + tile_split_part_bytes(pl.v->id, T, tiles, pl.ksplit));
  }
  return n;
}

size_t mqk_fused_qkv_rope_workspace_size_hd(int64_t T, int Hq, int Hkv, int64_t hidden, int head_dim) {
  if (T <= 0 || Hq <= 0 || Hkv <= 0 || hidden <= 0 || hidden % kBK != 0 || head_dim <= 0) return 0;
  if (head_dim == kHeadDim || head_dim == 64)
    return mqk_fused_qkv_rope_workspace_size(T, int(int64_t(Hq) * head_dim / kHeadDim),
                                             int(int64_t(Hkv) * head_dim / kHeadDim), hidden);
  // other head sizes: q and k/v widths of whole 128-column blocks run all three
  // projections in one launch of the fused kernels' plan; otherwise each
  // projection of whole blocks is planned on its own
  const Topology topo = device_topology();
  size_t n = 0;
  if ((int64_t(Hq) * head_dim) % kHeadDim == 0 && (int64_t(Hkv) * head_dim) % kHeadDim == 0)
    for (int int4 = 0; int4 < 2; ++int4) {
      const int tiles = int((int64_t(Hq) + 2 * Hkv) * head_dim / kHeadDim);
      const size_t m = plan_bytes(int4, T, hidden, tiles, topo, false, true);
      if (m != ~size_t(0)) n = std::max(n, m);
      // (with the fused input RMSNorm: that plan, then the per-token scales)
      const size_t mn = plan_bytes(int4, T, hidden, tiles, topo, true, true);
      if (mn != ~size_t(0))
        n = std::max(n, align_up(mn > 0 ? mn : decode_counter_bytes(), 256) + align_up(size_t(T) * sizeof(float), 256));
    }
  for (int int4 = 0; int4 < 2; ++int4)
    for (int h : {Hq, Hkv}) {
      const int64_t N = int64_t(h) * head_dim;
      if (N % kHeadDim != 0 || N / kHeadDim > kMaxTiles) continue;
      n = std::max(n, plain_plan_bytes(int4, T, hidden, int(N / kHeadDim), topo));
    }
  return n;
}

size_t mqk_fused_qkv_rope_ex_workspace_size(int64_t T, int Hq, int Hkv, int64_t hidden,
                                            const mqk_fused_ext* ext) {
  size_t n = mqk_fused_qkv_rope_workspace_size(T, Hq, Hkv, hidden);
  if (ext && ext->in_gamma && T > 0)
    n = align_up(n > 0 ? n : decode_counter_bytes(), 256) + align_up(size_t(T) * sizeof(float), 256);
  return n;
}

// head_dim: 128, or 64 with even head counts (the kernels then run 128-column
// blocks of two heads each: Hq * D / 128 and Hkv * D / 128 of them).
static int check_head_dim(int D, int Hq, int Hkv) {
  if (D % 2 != 0) return fail(MQK_ERR_BAD_SHAPE, "head_dim must be even (RoPE rotate_half), got %d", D);
  if (D != kHeadDim && D != 64) return fail(MQK_ERR_UNSUPPORTED, "head_dim %d not supported (128 or 64)", D);
  if (D == 64 && (Hq % 2 != 0 || Hkv % 2 != 0))
    return fail(MQK_ERR_UNSUPPORTED, "head_dim 64 needs even head counts (got Hq=%d, Hkv=%d)", Hq, Hkv);
  return MQK_OK;
}

// Head counts -> 128-column block counts (identity for head_dim 128).
static void to_blocks(int D, int& Hq, int& Hkv) {
  Hq = Hq * D / kHeadDim;
  Hkv = Hkv * D / kHeadDim;
}

static int validate_fused_common(const mqk_bf16* x, int64_t T, int64_t S, int64_t hidden, int Hq,
                                 int Hkv, int D, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                                 bool kv_optional = false) {
  if (T < 0 || hidden <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0)
    return fail(MQK_ERR_BAD_SHAPE, "need T >= 0, hidden > 0, Hq > 0, Hkv > 0, D > 0");
  if (int st = check_head_dim(D, Hq, Hkv); st != MQK_OK) return st;
  if (hidden % kBK != 0)
    return fail(MQK_ERR_UNSUPPORTED, "hidden %lld must be a multiple of 64", (long long)hidden);
  if (Hq + 2 * Hkv > kMaxTiles) return fail(MQK_ERR_UNSUPPORTED, "Hq + 2*Hkv must be <= %d", kMaxTiles);
  if (T > (int64_t(1) << 31) / 2) return fail(MQK_ERR_UNSUPPORTED, "T too large");
  (void)S;
  if (T == 0) return MQK_OK;
  if (!x || !q) return fail(MQK_ERR_NULL_POINTER, "x/q must be non-NULL");
  if (!kv_optional && (!k || !v)) return fail(MQK_ERR_NULL_POINTER, "x/q/k/v must be non-NULL");
  if (!aligned16(x) || !aligned16(q) || !aligned16(k) || !aligned16(v))
    return fail(MQK_ERR_MISALIGNED, "x/q/k/v must be 16-byte aligned");
  return MQK_OK;
}

// Paged-KV-cache arguments -> epilogue fields (kv == NULL: no cache).
static int apply_paged(const mqk_paged_kv* kv, const int32_t* positions, int64_t S, int64_t T,
                       bool varlen, EpilogueArgs& e) {
  if (!kv) return MQK_OK;
  if (!kv->k_cache || !kv->v_cache || !kv->block_table)
    return fail(MQK_ERR_NULL_POINTER, "paged kv: k_cache/v_cache/block_table must be non-NULL");
  if (!aligned16(kv->k_cache) || !aligned16(kv->v_cache))
    return fail(MQK_ERR_MISALIGNED, "paged kv: caches must be 16-byte aligned");
  if (kv->block_size < 1 || kv->bt_rows < 1 || kv->bt_cols < 1 || kv->num_blocks < 1)
    return fail(MQK_ERR_BAD_SHAPE, "paged kv: block_size, bt_rows, bt_cols, num_blocks must be >= 1");
  if (positions && (!kv->kv_seq || !kv->kv_pos))
    return fail(MQK_ERR_NULL_POINTER, "paged kv: positions mode needs kv_seq and kv_pos");
  if (!positions && !varlen && S <= 0) return fail(MQK_ERR_BAD_SHAPE, "paged kv: S must be > 0");
  (void)T;
  e.k_cache = kv->k_cache;
  e.v_cache = kv->v_cache;
  e.block_table = kv->block_table;
  e.kv_seq = kv->kv_seq;
  e.kv_pos = kv->kv_pos;
  e.bt_rows = kv->bt_rows;
  e.bt_cols = kv->bt_cols;
  e.num_blocks = kv->num_blocks;
  e.kv_len = (positions || varlen) ? 1 : S;
  e.block_size = kv->block_size;
  return MQK_OK;
}

// Optional features of the _ex entry points -> epilogue / problem fields.
static int apply_ext(const mqk_fused_ext* ext, const int32_t* positions, int64_t S, int64_t T,
                     ProblemArgs& p, EpilogueArgs& e) {
  if (!ext) return MQK_OK;
  const bool varlen = ext->cu_seqlens != nullptr;
  if (varlen) {
    if (positions) return fail(MQK_ERR_BAD_SHAPE, "varlen mode (cu_seqlens) and positions are exclusive");
    if (ext->n_seqs < 1 || ext->n_seqs > (int64_t(1) << 30))
      return fail(MQK_ERR_BAD_SHAPE, "varlen mode needs 1 <= n_seqs (got %lld)", (long long)ext->n_seqs);
    e.cu_seqlens = ext->cu_seqlens;
    e.seq_pos0 = ext->seq_pos0;
    e.n_seqs = ext->n_seqs;
  } else if (ext->seq_pos0) {
    return fail(MQK_ERR_BAD_SHAPE, "seq_pos0 needs cu_seqlens");
  }
  if (ext->in_gamma) {
    if (!aligned16(ext->in_gamma)) return fail(MQK_ERR_MISALIGNED, "in_gamma must be 16-byte aligned");
    if (p.K > 16384) return fail(MQK_ERR_UNSUPPORTED, "input RMSNorm needs hidden <= 16384");
    if (!(ext->in_eps >= 0.0f)) return fail(MQK_ERR_BAD_SHAPE, "in_eps must be >= 0");
    p.in_gamma = ext->in_gamma;
  }
  return apply_paged(ext->kv, positions, S, T, varlen, e);
}

// Validation and the norm / RoPE arguments of the generic head-size path (below).
static int any_d_prepare(const mqk_bf16* x, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                         const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions, int64_t T,
                         int64_t S, int64_t hidden, int Hq, int Hkv, int D, int64_t cos_rows, float eps,
                         mqk_bf16* q, mqk_bf16* k, mqk_bf16* v, const mqk_fused_ext* ext, EpilogueArgs& er) {
  if (T < 0 || hidden <= 0 || Hq <= 0 || Hkv <= 0)
    return fail(MQK_ERR_BAD_SHAPE, "need T >= 0, hidden > 0, Hq > 0, Hkv > 0");
  if (D % 8 != 0 || D > 512)
    return fail(MQK_ERR_UNSUPPORTED, "head_dim %d not supported (64, 128, or a multiple of 8 up to 512)", D);
  if (hidden % kBK != 0)
    return fail(MQK_ERR_UNSUPPORTED, "hidden %lld must be a multiple of 64", (long long)hidden);
  const int64_t n_max = int64_t(Hq > Hkv ? Hq : Hkv) * D;
  if ((n_max + kHeadDim - 1) / kHeadDim > kMaxTiles)
    return fail(MQK_ERR_UNSUPPORTED, "Hq * head_dim must be <= %d", kMaxTiles * kHeadDim);
  if (T > (int64_t(1) << 31) / 2) return fail(MQK_ERR_UNSUPPORTED, "T too large");
  if (T == 0) return MQK_OK;
  // (k and v are written even with a paged cache: the cache rows are copied from them)
  if (!x || !q || !k || !v) return fail(MQK_ERR_NULL_POINTER, "x/q/k/v must be non-NULL");
  if (!aligned16(x) || !aligned16(q) || !aligned16(k) || !aligned16(v))
    return fail(MQK_ERR_MISALIGNED, "x/q/k/v must be 16-byte aligned");
  int st = check_rope_args(q_gamma, k_gamma, cos, sin, S, cos_rows, positions, eps, ext && ext->cu_seqlens);
  if (st != MQK_OK) return st;
  er = make_qkv_epilogue(q_gamma, k_gamma, cos, sin, positions, S, cos_rows, eps, q, k, v, Hq, Hkv);
  er.head_dim = D;
  ProblemArgs pr{x, T, hidden, 0};
  return apply_ext(ext, positions, S, T, pr, er);
}

// Head sizes the fused kernels do not tile (a multiple of 8 up to 512, other than
// 64 and 128): the three projections are written straight into q, k and v, then
// launch_norm_rope_any normalises and rotates q and k in place.  When the q and
// k / v widths are whole 128-column blocks they run as one launch of the fused
// op's plan over those blocks (run_fused with qkv 2: q and k stored as
// projected); otherwise a projection of whole blocks goes through the planner on
// its own (run_fused, plain epilogue), and the others, and the fused input RMSNorm
// of that route, run on the tile kernels.  A planned form runs only when the
// workspace holds what its plan needs.  Like the reference's own
// composition (a vendor GEMM into bf16 q / k, then its norm + RoPE kernel,
// fused_qkv_rope.py:166-190), the projections are rounded to bf16 before the
// norm.  The fused input RMSNorm runs in the GEMMs as in the fused path (per-token
// scales from the pre-pass, in the workspace after its arrival counters); the
// paged-cache rows are written by the norm + RoPE launch.
static int fused_bf16_any_d(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                            const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                            const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                            int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                            int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                            const mqk_fused_ext* ext, void* workspace, size_t ws_bytes, void* stream) {
  EpilogueArgs er{};
  int st = any_d_prepare(x, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D, cos_rows, eps, q, k,
                         v, ext, er);
  if (st != MQK_OK || T == 0) return st == MQK_OK ? ok() : st;
  if (!w_q || !w_k || !w_v) return fail(MQK_ERR_NULL_POINTER, "w_q/w_k/w_v must be non-NULL");
  if (!aligned16(w_q) || !aligned16(w_k) || !aligned16(w_v))
    return fail(MQK_ERR_MISALIGNED, "weights must be 16-byte aligned");
  const Topology topo = device_topology();
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  const int64_t nq = int64_t(Hq) * D, nkv = int64_t(Hkv) * D;
  if (nq % kHeadDim == 0 && nkv % kHeadDim == 0) {
    // q and k/v widths of whole 128-column blocks: one launch of the fused
    // kernels' plan for all three projections over those blocks, q and k stored
    // as projected (qkv 2), when the workspace holds what that plan needs
    const bool in_norm = ext && ext->in_gamma;
    const int tiles = int((nq + 2 * nkv) / kHeadDim);
    const size_t need = plan_bytes(0, T, hidden, tiles, topo, in_norm, true);
    const size_t scales = in_norm ? align_up(size_t(T) * sizeof(float), 256) : 0;
    const bool fits = need != ~size_t(0) &&
                      ((need == 0 && !in_norm) ||
                       (workspace && align_up(need > 0 ? need : decode_counter_bytes(), 256) + scales <= ws_bytes));
    if (fits) {
      ProblemArgs pr{x, T, hidden, tiles};
      pr.in_gamma = in_norm ? ext->in_gamma : nullptr;
      WeightArgs w{};
      w.w[0] = w_q;
      w.w[1] = w_k;
      w.w[2] = w_v;
      w.n_cols[0] = nq;
      w.n_cols[1] = nkv;
      w.n_cols[2] = nkv;
      EpilogueArgs e = er;
      e.qkv = 2;
      e.Hq = int(nq / kHeadDim);
      e.Hkv = int(nkv / kHeadDim);
      e.head_dim = kHeadDim;
      e.k_cache = nullptr;  // (the paged rows are written by the norm + RoPE launch)
      e.v_cache = nullptr;
      if ((st = run_fused(0, pr, w, e, in_norm ? ext->in_eps : 0.f, workspace, ws_bytes, hs)) != MQK_OK) return st;
      return hip_status(launch_norm_rope_any(er, T, hs), "norm + RoPE launch");
    }
  }
  ProblemArgs pn{x, T, hidden, 0};
  if (ext && ext->in_gamma) {
    if ((st = apply_ext(ext, positions, S, T, pn, er)) != MQK_OK) return st;  // (in_gamma checks)
    // the scales after the workspace's arrival counters, which other calls on it need at zero
    const size_t off = align_up(decode_counter_bytes(), 256);
    if (!workspace || ws_bytes < off + size_t(T) * sizeof(float))
      return fail(MQK_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given%s", off + size_t(T) * sizeof(float),
                  ws_bytes, workspace ? "" : " (NULL)");
    float* scale = reinterpret_cast<float*>(static_cast<char*>(workspace) + off);
    st = hip_status(launch_row_scale(x, T, hidden, ext->in_eps, scale, hs), "input norm pre-pass launch");
    if (st != MQK_OK) return st;
    pn.in_scale = scale;
  }
  const mqk_bf16* wts[3] = {w_q, w_k, w_v};
  mqk_bf16* outs[3] = {q, k, v};
  const int heads[3] = {Hq, Hkv, Hkv};
  for (int i = 0; i < 3; ++i) {
    const int64_t N = int64_t(heads[i]) * D;  // N % 8 == 0: the tiles store whole 8-column runs below N
    const int tiles = int((N + kHeadDim - 1) / kHeadDim);
    if (!pn.in_gamma && N % kHeadDim == 0 && aligned16(outs[i]) &&
        plain_plan_bytes(0, T, hidden, tiles, topo) <= (workspace ? ws_bytes : 0)) {
      // whole 128-column blocks: the planner's launches for this projection
      // (decode blocks, split-K or single-head tiles where they are faster)
      ProblemArgs pp{x, T, hidden, tiles};
      WeightArgs w{};
      w.w[0] = wts[i];
      w.n_cols[0] = N;
      EpilogueArgs e{};
      e.qkv = 0;
      e.Hq = tiles;
      e.Hkv = 0;
      e.out = outs[i];
      e.N = N;
      e.head_dim = kHeadDim;
      if ((st = run_fused(0, pp, w, e, 0.f, workspace, ws_bytes, hs)) != MQK_OK) return st;
      continue;
    }
    ProblemArgs p{x, T, hidden, tiles};
    p.cus = topo.cus;
    p.xcds = topo.xcds;
    p.in_gamma = pn.in_gamma;
    p.in_scale = pn.in_scale;
    WeightArgs w{};
    w.w[0] = wts[i];
    w.n_cols[0] = N;
    EpilogueArgs e{};
    e.qkv = 0;
    e.Hq = tiles;
    e.Hkv = 0;
    e.out = outs[i];
    e.N = N;
    e.head_dim = kHeadDim;  // (plain output: the epilogue's 128-column blocks)
    const TileVariant* v = choose_tile_variant(0, T, tiles, 0, topo.cus);
    // (the pipelined tiles hold the input norm's gamma in LDS beside their ring)
    if (!v || (p.in_gamma && tile_dma_lds_bytes(v->id) + hidden * 2 > 160 * 1024))
      v = choose_tile_variant(1, T, tiles, 0, topo.cus);
    st = hip_status(launch_tile(*v, 0, p, w, e, int(g_group_m.load()), hs), "tile kernel launch (projection)");
    if (st != MQK_OK) return st;
  }
  return hip_status(launch_norm_rope_any(er, T, hs), "norm + RoPE launch");
}

static int fused_bf16_impl(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                           const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                           const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                           int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                           int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                           const mqk_fused_ext* ext, void* workspace, size_t ws_bytes, void* stream) {
  if (D > 0 && D % 2 == 0 && D != kHeadDim && D != 64)
    return fused_bf16_any_d(x, w_q, w_k, w_v, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D,
                            cos_rows, eps, q, k, v, ext, workspace, ws_bytes, stream);
  const bool varlen = ext && ext->cu_seqlens;
  int st = validate_fused_common(x, T, S, hidden, Hq, Hkv, D, q, k, v, ext && ext->kv);
  if (st != MQK_OK) return st;
  if (T == 0) return ok();
  if (!w_q || !w_k || !w_v) return fail(MQK_ERR_NULL_POINTER, "w_q/w_k/w_v must be non-NULL");
  if (!aligned16(w_q) || !aligned16(w_k) || !aligned16(w_v))
    return fail(MQK_ERR_MISALIGNED, "weights must be 16-byte aligned");
  st = check_rope_args(q_gamma, k_gamma, cos, sin, S, cos_rows, positions, eps, varlen);
  if (st != MQK_OK) return st;
  to_blocks(D, Hq, Hkv);

  ProblemArgs p{x, T, hidden, Hq + 2 * Hkv};
  WeightArgs w{};
  w.w[0] = w_q;
  w.w[1] = w_k;
  w.w[2] = w_v;
  w.n_cols[0] = int64_t(Hq) * kHeadDim;
  w.n_cols[1] = w.n_cols[2] = int64_t(Hkv) * kHeadDim;
  EpilogueArgs e = make_qkv_epilogue(q_gamma, k_gamma, cos, sin, positions, S, cos_rows, eps,
                                     q, k, v, Hq, Hkv);
  e.head_dim = D;
  if ((st = apply_ext(ext, positions, S, T, p, e)) != MQK_OK) return st;
  return run_fused(0, p, w, e, ext ? ext->in_eps : 0.f, workspace, ws_bytes, static_cast<hipStream_t>(stream));
}

int mqk_fused_qkv_rope_bf16(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                            const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                            const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                            int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                            int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                            void* workspace, size_t ws_bytes, void* stream) {
  return fused_bf16_impl(x, w_q, w_k, w_v, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D,
                         cos_rows, eps, q, k, v, nullptr, workspace, ws_bytes, stream);
}

static int fused_f32_impl(bool half, const void* x, const void* w_q, const void* w_k, const void* w_v,
                          const void* q_gamma, const void* k_gamma, const void* cos, const void* sin,
                          const int32_t* positions, int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                          int64_t cos_rows, float eps, void* q, void* k, void* v, void* stream) {
  if (T < 0 || hidden <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0)
    return fail(MQK_ERR_BAD_SHAPE, "need T >= 0, hidden > 0, Hq > 0, Hkv > 0, D > 0");
  if (int st = check_head_dim(D, Hq, Hkv); st != MQK_OK) return st;
  if (hidden % kF32BK != 0)
    return fail(MQK_ERR_UNSUPPORTED, "hidden %lld must be a multiple of %d", (long long)hidden, kF32BK);
  if (Hq + 2 * Hkv > kMaxTiles) return fail(MQK_ERR_UNSUPPORTED, "Hq + 2*Hkv must be <= %d", kMaxTiles);
  if (T > (int64_t(1) << 31) / 2) return fail(MQK_ERR_UNSUPPORTED, "T too large");
  if (T == 0) return ok();
  if (!x || !q || !k || !v) return fail(MQK_ERR_NULL_POINTER, "x/q/k/v must be non-NULL");
  if (!w_q || !w_k || !w_v) return fail(MQK_ERR_NULL_POINTER, "w_q/w_k/w_v must be non-NULL");
  if (!aligned16(x) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(w_q) ||
      !aligned16(w_k) || !aligned16(w_v))
    return fail(MQK_ERR_MISALIGNED, "x/q/k/v and the weights must be 16-byte aligned");
  int st = check_rope_args(q_gamma, k_gamma, cos, sin, S, cos_rows, positions, eps);
  if (st != MQK_OK) return st;
  to_blocks(D, Hq, Hkv);
  F32Args a{};
  a.head_dim = D;
  a.x = x;
  a.w[0] = w_q;
  a.w[1] = w_k;
  a.w[2] = w_v;
  a.q_gamma = q_gamma;
  a.k_gamma = k_gamma;
  a.cos = cos;
  a.sin = sin;
  a.positions = positions;
  a.M = T;
  a.K = hidden;
  a.S = positions ? 1 : S;
  a.cos_rows = cos_rows;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.eps = eps;
  a.q = q;
  a.k = k;
  a.v = v;
  // 16-row tiles when 32-row tiles would leave CUs idle
  const Topology topo = device_topology();
  const int rows = (T + 31) / 32 * (Hq + 2 * Hkv) < topo.cus ? 16 : 32;
  return hip_status(launch_f32_qkv(a, rows, half, topo.xcds, static_cast<hipStream_t>(stream)),
                    half ? "f16 front launch" : "f32 front launch");
}

int mqk_fused_qkv_rope_f32(const float* x, const float* w_q, const float* w_k, const float* w_v,
                           const float* q_gamma, const float* k_gamma, const float* cos, const float* sin,
                           const int32_t* positions, int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv,
                           int D, int64_t cos_rows, float eps, float* q, float* k, float* v, void* stream) {
  return fused_f32_impl(false, x, w_q, w_k, w_v, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D,
                        cos_rows, eps, q, k, v, stream);
}

int mqk_fused_qkv_rope_f16(const mqk_f16* x, const mqk_f16* w_q, const mqk_f16* w_k, const mqk_f16* w_v,
                           const mqk_f16* q_gamma, const mqk_f16* k_gamma, const mqk_f16* cos, const mqk_f16* sin,
                           const int32_t* positions, int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv,
                           int D, int64_t cos_rows, float eps, mqk_f16* q, mqk_f16* k, mqk_f16* v, void* stream) {
  return fused_f32_impl(true, x, w_q, w_k, w_v, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D,
                        cos_rows, eps, q, k, v, stream);
}

// ---- allocation-free variant of mqk_fused_qkv_rope_bf16 ---------------------------------
// The decode kernel's scratch (its arrival counters, then its fp32 split partials)
// lives in this file-scope device array instead of a caller workspace: 68.25 KiB
// of counters (the decode arrival counters, a statistics line and the split-K
// tile words) plus 8 MiB of partials, enough for one 64-row block of any head count
// up to one split per CU (e.g. 48 heads x 5 splits at hidden 4096: 7.5 MiB).
// Each GPU holds its own copy for the life of the process.  Host code never
// passes `scratch` itself to a kernel (in host code the name is a stand-in, not a
// device address): the device address comes from hipGetSymbolAddress, once per
// device, and only that address is used.
}  // extern "C"

static __device__ __align__(256) unsigned char scratch[mqk::kDecodeCounterBytes + (size_t(8) << 20)];

namespace {

constexpr size_t kScratchBytes = sizeof(scratch);
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ void clear_words_kernel(uint32_t* words, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) words[i] = 0u;
}

// Device address of this device's scratch (set up on the first call on a device).
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_status(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(MQK_ERR_UNSUPPORTED, "device %d beyond %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) return hip_status(err != hipSuccess ? err : hipErrorInvalidSymbol,
                                                     "hipGetSymbolAddress(scratch)");
    // The counters must start at zero (every call leaves them so).  Device
    // globals are zero when the code object loads; they are cleared once more
    // here with a fill kernel, unless the stream is being captured (the fill
    // would then run only at replay).
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    err = hipStreamIsCapturing(stream, &cs);
    if (err != hipSuccess) return hip_status(err, "hipStreamIsCapturing");
    if (cs == hipStreamCaptureStatusNone) {
      const int words = int(decode_counter_bytes() / 4);
      hipLaunchKernelGGL(clear_words_kernel, dim3((words + 255) / 256), dim3(256), 0, stream,
                         static_cast<uint32_t*>(ptr), words);
      err = hipGetLastError();
      if (err != hipSuccess) return hip_status(err, "scratch clear launch");
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MQK_OK;
}

}  // namespace

extern "C" {

int mqk_fused_qkv_rope_bf16_noalloc(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                                    const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                                    const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                                    int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                                    int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                                    void* stream) {
  void* ws = nullptr;
  if (T > 0) {
    const int st = scratch_address(static_cast<hipStream_t>(stream), &ws);
    if (st != MQK_OK) return st;
  }
  const int st = fused_bf16_impl(x, w_q, w_k, w_v, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv,
                                 D, cos_rows, eps, q, k, v, nullptr, ws, kScratchBytes, stream);
  if (st == MQK_ERR_WORKSPACE)
    return fail(MQK_ERR_WORKSPACE,
                "T=%lld with %d heads at hidden %lld needs more than the %zu-byte fixed scratch of "
                "mqk_fused_qkv_rope_bf16_noalloc (use mqk_fused_qkv_rope_bf16 with a workspace)",
                (long long)T, Hq + 2 * Hkv, (long long)hidden, kScratchBytes);
  return st;
}

int mqk_fused_qkv_rope_paged_bf16(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                                  const mqk_bf16* w_v, const mqk_bf16* q_gamma,
                                  const mqk_bf16* k_gamma, const mqk_bf16* cos, const mqk_bf16* sin,
                                  const int32_t* positions, int64_t T, int64_t S, int64_t hidden,
                                  int Hq, int Hkv, int D, int64_t cos_rows, float eps, mqk_bf16* q,
                                  mqk_bf16* k, mqk_bf16* v, const mqk_paged_kv* kv, void* workspace,
                                  size_t ws_bytes, void* stream) {
  if (!kv) return fail(MQK_ERR_NULL_POINTER, "paged kv descriptor is NULL");
  mqk_fused_ext ext{};
  ext.kv = kv;
  return fused_bf16_impl(x, w_q, w_k, w_v, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D,
                         cos_rows, eps, q, k, v, &ext, workspace, ws_bytes, stream);
}

int mqk_fused_qkv_rope_ex_bf16(const mqk_bf16* x, const mqk_bf16* w_q, const mqk_bf16* w_k,
                               const mqk_bf16* w_v, const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                               const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                               int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                               int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                               const mqk_fused_ext* ext, void* workspace, size_t ws_bytes, void* stream) {
  return fused_bf16_impl(x, w_q, w_k, w_v, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D,
                         cos_rows, eps, q, k, v, ext, workspace, ws_bytes, stream);
}

int mqk_qk_norm_rope_bf16(const mqk_bf16* q_raw, const mqk_bf16* k_raw, const mqk_bf16* q_gamma,
                          const mqk_bf16* k_gamma, const mqk_bf16* cos, const mqk_bf16* sin,
                          const int32_t* positions, int64_t T, int64_t S, int Hq, int Hkv, int D,
                          int64_t cos_rows, float eps, mqk_bf16* q_out, mqk_bf16* k_out,
                          void* stream) {
  if (T < 0 || Hq < 0 || Hkv < 0 || D <= 0) return fail(MQK_ERR_BAD_SHAPE, "negative size");
  if (int st = check_head_dim(D, Hq, Hkv); st != MQK_OK) return st;
  if (T == 0 || Hq + Hkv == 0) return ok();
  to_blocks(D, Hq, Hkv);
  if ((Hq > 0 && (!q_raw || !q_out)) || (Hkv > 0 && (!k_raw || !k_out)))
    return fail(MQK_ERR_NULL_POINTER, "q/k input or output is NULL");
  int st = check_rope_args(Hq ? q_gamma : k_gamma, Hkv ? k_gamma : q_gamma, cos, sin, S, cos_rows,
                           positions, eps);
  if (st != MQK_OK) return st;
  EpilogueArgs e = make_qkv_epilogue(q_gamma, k_gamma, cos, sin, positions, S, cos_rows, eps,
                                     q_out, k_out, nullptr, Hq, Hkv);
  e.head_dim = D;
  return hip_status(launch_norm_rope(q_raw, k_raw, e, T, static_cast<hipStream_t>(stream)),
                    "norm_rope kernel launch");
}

static int validate_int4(const int32_t* qw, const void* sc, const int32_t* qz, int64_t K, int64_t N,
                         int group, int scale_type, const char* which) {
  if (!qw || !sc || !qz) return fail(MQK_ERR_NULL_POINTER, "%s: qweight/scales/qzeros NULL", which);
  if (N <= 0 || N % 8 != 0) return fail(MQK_ERR_BAD_SHAPE, "%s: N=%lld must be a positive multiple of 8", which, (long long)N);
  if (group <= 0 || K % group != 0)
    return fail(MQK_ERR_BAD_SHAPE, "%s: K=%lld not divisible by group=%d", which, (long long)K, group);
  if (group % kBK != 0) return fail(MQK_ERR_UNSUPPORTED, "%s: group %d must be a multiple of 64", which, group);
  if (scale_type != MQK_SCALE_BF16 && scale_type != MQK_SCALE_FP16)
    return fail(MQK_ERR_BAD_SHAPE, "%s: scale_type %d unknown", which, scale_type);
  return MQK_OK;
}

}  // extern "C"

// The column-parallel kernel for small M (any N % 8 == 0, any operand alignment
// but x's): no workspace.
static int w4a16_gemv(const mqk_bf16* x, const int32_t* qweight, const void* scales, const int32_t* qzeros,
                      int64_t M, int64_t K, int64_t N, int group, int scale_type, mqk_bf16* out, void* stream) {
  WeightArgs w{};
  w.qw[0] = qweight;
  w.sc[0] = scales;
  w.qz[0] = qzeros;
  w.n_cols[0] = N;
  w.group = group;
  w.scale_fp16 = scale_type == MQK_SCALE_FP16;
  return hip_status(launch_w4_gemv(x, w, M, K, out, static_cast<hipStream_t>(stream)), "w4a16 GEMV launch");
}

extern "C" {

int mqk_w4a16_gemm(const mqk_bf16* x, const int32_t* qweight, const void* scales,
                   const int32_t* qzeros, int64_t M, int64_t K, int64_t N, int group,
                   int scale_type, mqk_bf16* out, void* stream) {
  if (M < 0 || K <= 0) return fail(MQK_ERR_BAD_SHAPE, "need M >= 0, K > 0");
  if (K % kBK != 0) return fail(MQK_ERR_UNSUPPORTED, "K=%lld must be a multiple of 64", (long long)K);
  int st = validate_int4(qweight, scales, qzeros, K, N, group, scale_type, "w4a16_gemm");
  if (st != MQK_OK) return st;
  if (M == 0) return ok();
  if (!x || !out) return fail(MQK_ERR_NULL_POINTER, "x/out must be non-NULL");
  if (!aligned16(x)) return fail(MQK_ERR_MISALIGNED, "x must be 16-byte aligned");
  if (M <= g_gemv_max_m.load()) return w4a16_gemv(x, qweight, scales, qzeros, M, K, N, group, scale_type, out, stream);
  const int tiles = int((N + kHeadDim - 1) / kHeadDim);
  ProblemArgs p{x, M, K, tiles};
  const Topology topo = device_topology();
  p.cus = topo.cus;
  p.xcds = topo.xcds;
  WeightArgs w{};
  w.qw[0] = qweight;
  w.sc[0] = scales;
  w.qz[0] = qzeros;
  w.n_cols[0] = N;
  w.group = group;
  w.scale_fp16 = scale_type == MQK_SCALE_FP16;
  EpilogueArgs e{};
  e.qkv = 0;
  e.Hq = tiles;
  e.Hkv = 0;
  e.out = out;
  e.N = N;
  // The pipelined int4 variants read qweight and scales with 16-byte loads (a last
  // tile past N re-reads whole in-range chunks, N % 8 == 0) and qzeros with 4-byte
  // loads; operands without that alignment take the register-staged kernel.
  const TileVariant* v = nullptr;
  if (aligned16(qweight) && aligned16(scales) && (reinterpret_cast<uintptr_t>(qzeros) & 3u) == 0)
    v = choose_tile_variant(int(g_prefill_tile.load()), M, tiles, 1, topo.cus);
  if (!v) v = choose_tile_variant(1, M, tiles, 1, topo.cus);
  return hip_status(launch_tile(*v, 1, p, w, e, int(g_group_m.load()), static_cast<hipStream_t>(stream)),
                    "w4a16 tile kernel launch");
}

size_t mqk_w4a16_gemm_workspace_size(int64_t M, int64_t K, int64_t N) {
  if (M <= g_gemv_max_m.load()) return 0;  // the column-parallel kernel needs none
  if (M <= 0 || K <= 0 || K % kBK != 0 || N <= 0 || N % kHeadDim != 0 || N / kHeadDim > kMaxTiles) return 0;
  const int tiles = int(N / kHeadDim);
  const Plan pl = plan_fused(1, M, K, tiles, true, device_topology());
  return pl.splits > 0 ? decode_workspace_bytes(tiles, pl.splits, pl.passes) : 0;
}

int mqk_w4a16_gemm_ex(const mqk_bf16* x, const int32_t* qweight, const void* scales, const int32_t* qzeros,
                      int64_t M, int64_t K, int64_t N, int group, int scale_type, mqk_bf16* out,
                      void* workspace, size_t ws_bytes, void* stream) {
  if (M < 0 || K <= 0) return fail(MQK_ERR_BAD_SHAPE, "need M >= 0, K > 0");
  if (K % kBK != 0) return fail(MQK_ERR_UNSUPPORTED, "K=%lld must be a multiple of 64", (long long)K);
  int st = validate_int4(qweight, scales, qzeros, K, N, group, scale_type, "w4a16_gemm");
  if (st != MQK_OK) return st;
  if (M == 0) return ok();
  if (!x || !out) return fail(MQK_ERR_NULL_POINTER, "x/out must be non-NULL");
  if (!aligned16(x)) return fail(MQK_ERR_MISALIGNED, "x must be 16-byte aligned");
  if (M <= g_gemv_max_m.load()) return w4a16_gemv(x, qweight, scales, qzeros, M, K, N, group, scale_type, out, stream);
  // the planned kernels (split-K decode kernel for small M) need whole 128-column
  // tiles and 16-byte aligned operands; anything else takes the tile kernels
  if (N % kHeadDim != 0 || N / kHeadDim > kMaxTiles || !aligned16(qweight) || !aligned16(scales) ||
      !aligned16(qzeros) || !aligned16(out))
    return mqk_w4a16_gemm(x, qweight, scales, qzeros, M, K, N, group, scale_type, out, stream);
  const int tiles = int(N / kHeadDim);
  ProblemArgs p{x, M, K, tiles};
  WeightArgs w{};
  w.qw[0] = qweight;
  w.sc[0] = scales;
  w.qz[0] = qzeros;
  w.n_cols[0] = N;
  w.group = group;
  w.scale_fp16 = scale_type == MQK_SCALE_FP16;
  EpilogueArgs e{};
  e.qkv = 0;
  e.Hq = tiles;
  e.Hkv = 0;
  e.out = out;
  e.N = N;
  return run_fused(1, p, w, e, 0.f, workspace, ws_bytes, static_cast<hipStream_t>(stream));
}

static int fused_w4a16_impl(const mqk_bf16* x, const int32_t* qw_q, const void* sc_q,
                            const int32_t* qz_q, const int32_t* qw_k, const void* sc_k,
                            const int32_t* qz_k, const int32_t* qw_v, const void* sc_v,
                            const int32_t* qz_v, int group, int scale_type,
                            const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                            const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                            int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                            int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                            const mqk_fused_ext* ext, void* workspace, size_t ws_bytes, void* stream) {
  if (D > 0 && D % 2 == 0 && D != kHeadDim && D != 64) {
    // the generic head-size path, as fused_bf16_any_d, with int4 weights
    const bool in_norm = ext && ext->in_gamma;
    EpilogueArgs er{};
    int st = any_d_prepare(x, q_gamma, k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D, cos_rows, eps, q,
                           k, v, ext, er);
    if (st != MQK_OK || T == 0) return st == MQK_OK ? ok() : st;
    const int32_t* qws[3] = {qw_q, qw_k, qw_v};
    const void* scs[3] = {sc_q, sc_k, sc_v};
    const int32_t* qzs[3] = {qz_q, qz_k, qz_v};
    mqk_bf16* outs[3] = {q, k, v};
    const int heads[3] = {Hq, Hkv, Hkv};
    const Topology topo = device_topology();
    const int64_t nq = int64_t(Hq) * D, nkv = int64_t(Hkv) * D;
    if (nq % kHeadDim == 0 && nkv % kHeadDim == 0) {
      // whole 128-column widths: one launch of the fused int4 plan for all three
      // projections, q and k stored as projected (qkv 2), when the workspace holds
      // what that plan needs (at T = 8, hidden 4096 it beats three column-parallel
      // GEMMs, whose few workgroups each run the whole K, 20 us against 43)
      const char* names[3] = {"q_proj", "k_proj", "v_proj"};
      for (int i = 0; i < 3; ++i)
        if ((st = validate_int4(qws[i], scs[i], qzs[i], hidden, i == 0 ? nq : nkv, group, scale_type, names[i])) !=
            MQK_OK)
          return st;
      const int tiles = int((nq + 2 * nkv) / kHeadDim);
      const size_t need = plan_bytes(1, T, hidden, tiles, topo, in_norm, true);
      const size_t scales = in_norm ? align_up(size_t(T) * sizeof(float), 256) : 0;
      if (need != ~size_t(0) &&
          ((need == 0 && !in_norm) ||
           (workspace && align_up(need > 0 ? need : decode_counter_bytes(), 256) + scales <= ws_bytes))) {
        ProblemArgs pr{x, T, hidden, tiles};
        pr.in_gamma = in_norm ? ext->in_gamma : nullptr;
        WeightArgs w{};
        for (int i = 0; i < 3; ++i) {
          w.qw[i] = qws[i];
          w.sc[i] = scs[i];
          w.qz[i] = qzs[i];
        }
        w.n_cols[0] = nq;
        w.n_cols[1] = w.n_cols[2] = nkv;
        w.group = group;
        w.scale_fp16 = scale_type == MQK_SCALE_FP16;
        EpilogueArgs e = er;
        e.qkv = 2;
        e.Hq = int(nq / kHeadDim);
        e.Hkv = int(nkv / kHeadDim);
        e.head_dim = kHeadDim;
        e.k_cache = nullptr;  // (the paged rows are written by the norm + RoPE launch)
        e.v_cache = nullptr;
        const hipStream_t hs = static_cast<hipStream_t>(stream);
        if ((st = run_fused(1, pr, w, e, in_norm ? ext->in_eps : 0.f, workspace, ws_bytes, hs)) != MQK_OK) return st;
        return hip_status(launch_norm_rope_any(er, T, hs), "norm + RoPE launch");
      }
    }
    // (the per-projection W4A16 GEMMs take no input norm)
    if (in_norm)
      return fail(MQK_ERR_UNSUPPORTED,
                  "head_dim %d: the W4A16 front's input RMSNorm needs Hq * head_dim and Hkv * head_dim to be "
                  "multiples of 128 and a workspace of mqk_fused_qkv_rope_ex_workspace_size bytes",
                  D);
    for (int i = 0; i < 3; ++i) {
      // whole 128-column blocks with the workspace their plan needs: the planned
      // launches (mqk_w4a16_gemm_ex: decode kernel, decode blocks, tiles); else the
      // column-parallel kernel (M <= 16) or the tile kernels
      const int64_t N = int64_t(heads[i]) * D;
      const bool planned = N % kHeadDim == 0 &&
                           plain_plan_bytes(1, T, hidden, int(N / kHeadDim), topo) <= (workspace ? ws_bytes : 0);
      st = planned ? mqk_w4a16_gemm_ex(x, qws[i], scs[i], qzs[i], T, hidden, N, group, scale_type, outs[i],
                                       workspace, ws_bytes, stream)
                   : mqk_w4a16_gemm(x, qws[i], scs[i], qzs[i], T, hidden, N, group, scale_type, outs[i], stream);
      if (st != MQK_OK) return st;
    }
    return hip_status(launch_norm_rope_any(er, T, static_cast<hipStream_t>(stream)), "norm + RoPE launch");
  }
  const bool varlen = ext && ext->cu_seqlens;
  int st = validate_fused_common(x, T, S, hidden, Hq, Hkv, D, q, k, v, ext && ext->kv);
  if (st != MQK_OK) return st;
  if (T == 0) return ok();
  to_blocks(D, Hq, Hkv);
  const int64_t nq = int64_t(Hq) * kHeadDim, nkv = int64_t(Hkv) * kHeadDim;
  if ((st = validate_int4(qw_q, sc_q, qz_q, hidden, nq, group, scale_type, "q_proj")) != MQK_OK) return st;
  if ((st = validate_int4(qw_k, sc_k, qz_k, hidden, nkv, group, scale_type, "k_proj")) != MQK_OK) return st;
  if ((st = validate_int4(qw_v, sc_v, qz_v, hidden, nkv, group, scale_type, "v_proj")) != MQK_OK) return st;
  st = check_rope_args(q_gamma, k_gamma, cos, sin, S, cos_rows, positions, eps, varlen);
  if (st != MQK_OK) return st;

  ProblemArgs p{x, T, hidden, Hq + 2 * Hkv};
  WeightArgs w{};
  const int32_t* qws[3] = {qw_q, qw_k, qw_v};
  const void* scs[3] = {sc_q, sc_k, sc_v};
  const int32_t* qzs[3] = {qz_q, qz_k, qz_v};
  for (int i = 0; i < 3; ++i) {
    w.qw[i] = qws[i];
    w.sc[i] = scs[i];
    w.qz[i] = qzs[i];
  }
  w.n_cols[0] = nq;
  w.n_cols[1] = w.n_cols[2] = nkv;
  w.group = group;
  w.scale_fp16 = scale_type == MQK_SCALE_FP16;
  EpilogueArgs e = make_qkv_epilogue(q_gamma, k_gamma, cos, sin, positions, S, cos_rows, eps,
                                     q, k, v, Hq, Hkv);
  e.head_dim = D;
  if ((st = apply_ext(ext, positions, S, T, p, e)) != MQK_OK) return st;
  return run_fused(1, p, w, e, ext ? ext->in_eps : 0.f, workspace, ws_bytes, static_cast<hipStream_t>(stream));
}

int mqk_fused_qkv_rope_w4a16(const mqk_bf16* x, const int32_t* qw_q, const void* sc_q,
                             const int32_t* qz_q, const int32_t* qw_k, const void* sc_k,
                             const int32_t* qz_k, const int32_t* qw_v, const void* sc_v,
                             const int32_t* qz_v, int group, int scale_type,
                             const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                             const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                             int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                             int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                             void* workspace, size_t ws_bytes, void* stream) {
  return fused_w4a16_impl(x, qw_q, sc_q, qz_q, qw_k, sc_k, qz_k, qw_v, sc_v, qz_v, group, scale_type, q_gamma,
                          k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D, cos_rows, eps, q, k, v, nullptr,
                          workspace, ws_bytes, stream);
}

int mqk_fused_qkv_rope_paged_w4a16(const mqk_bf16* x, const int32_t* qw_q, const void* sc_q,
                                   const int32_t* qz_q, const int32_t* qw_k, const void* sc_k,
                                   const int32_t* qz_k, const int32_t* qw_v, const void* sc_v,
                                   const int32_t* qz_v, int group, int scale_type,
                                   const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                                   const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                                   int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                                   int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                                   const mqk_paged_kv* kv, void* workspace, size_t ws_bytes,
                                   void* stream) {
  if (!kv) return fail(MQK_ERR_NULL_POINTER, "paged kv descriptor is NULL");
  mqk_fused_ext ext{};
  ext.kv = kv;
  return fused_w4a16_impl(x, qw_q, sc_q, qz_q, qw_k, sc_k, qz_k, qw_v, sc_v, qz_v, group, scale_type, q_gamma,
                          k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D, cos_rows, eps, q, k, v, &ext,
                          workspace, ws_bytes, stream);
}

int mqk_fused_qkv_rope_ex_w4a16(const mqk_bf16* x, const int32_t* qw_q, const void* sc_q,
                                const int32_t* qz_q, const int32_t* qw_k, const void* sc_k,
                                const int32_t* qz_k, const int32_t* qw_v, const void* sc_v,
                                const int32_t* qz_v, int group, int scale_type,
                                const mqk_bf16* q_gamma, const mqk_bf16* k_gamma,
                                const mqk_bf16* cos, const mqk_bf16* sin, const int32_t* positions,
                                int64_t T, int64_t S, int64_t hidden, int Hq, int Hkv, int D,
                                int64_t cos_rows, float eps, mqk_bf16* q, mqk_bf16* k, mqk_bf16* v,
                                const mqk_fused_ext* ext, void* workspace, size_t ws_bytes,
                                void* stream) {
  return fused_w4a16_impl(x, qw_q, sc_q, qz_q, qw_k, sc_k, qz_k, qw_v, sc_v, qz_v, group, scale_type, q_gamma,
                          k_gamma, cos, sin, positions, T, S, hidden, Hq, Hkv, D, cos_rows, eps, q, k, v, ext,
                          workspace, ws_bytes, stream);
}

int mqk_set_option(const char* name, int64_t value) {
  if (!name) return fail(MQK_ERR_BAD_OPTION, "option name is NULL");
  if (!strcmp(name, "prefill_tile")) {
    if (value < 0) return fail(MQK_ERR_BAD_OPTION, "prefill_tile must be >= 0");
    if (value > 0) {
      bool found = false;
      for (int i = 0; i < tile_variant_count(); ++i) found |= tile_variant(i)->id == value;
      if (!found) return fail(MQK_ERR_BAD_OPTION, "unknown prefill_tile %lld", (long long)value);
    }
    g_prefill_tile = value;
  } else if (!strcmp(name, "decode_max_t")) {
    if (value < 0 || value > 64) return fail(MQK_ERR_BAD_OPTION, "decode_max_t must be in [0, 64]");
    g_decode_max_t = value;
  } else if (!strcmp(name, "decode_splits")) {
    if (value < 0 || value > 4096) return fail(MQK_ERR_BAD_OPTION, "decode_splits must be in [0, 4096]");
    g_decode_splits = value;
  } else if (!strcmp(name, "decode_max_spins")) {
    if (value < 0 || value > (1 << 24)) return fail(MQK_ERR_BAD_OPTION, "decode_max_spins must be in [0, 2^24]");
    g_decode_max_spins = int(value);
  } else if (!strcmp(name, "decode_force_recompute")) {
    if (value != 0 && value != 1) return fail(MQK_ERR_BAD_OPTION, "decode_force_recompute must be 0 or 1");
    g_decode_force_recompute = int(value);
  } else if (!strcmp(name, "tail_split")) {
    if (value != 0 && value != 1) return fail(MQK_ERR_BAD_OPTION, "tail_split must be 0 or 1");
    g_tail_split = value;
  } else if (!strcmp(name, "decode_blocks")) {
    if (value < 0 || value > 64) return fail(MQK_ERR_BAD_OPTION, "decode_blocks must be in [0, 64]");
    g_decode_blocks = value;
  } else if (!strcmp(name, "decode_passes")) {
    if (value < 1 || value > 16) return fail(MQK_ERR_BAD_OPTION, "decode_passes must be in [1, 16]");
    g_decode_passes = value;
  } else if (!strcmp(name, "decode_cost_model")) {
    if (value != 0 && value != 1) return fail(MQK_ERR_BAD_OPTION, "decode_cost_model must be 0 or 1");
    g_decode_cost_model = value;
  } else if (!strcmp(name, "head_tiles")) {
    if (value != 0 && value != 1) return fail(MQK_ERR_BAD_OPTION, "head_tiles must be 0 or 1");
    g_head_tiles = value;
  } else if (!strcmp(name, "tile_ksplit")) {
    if (value < 0 || value > 16) return fail(MQK_ERR_BAD_OPTION, "tile_ksplit must be in [0, 16]");
    g_tile_ksplit = value;
  } else if (!strcmp(name, "group_m")) {
    if (value < 1 || value > 1024) return fail(MQK_ERR_BAD_OPTION, "group_m must be in [1, 1024]");
    g_group_m = value;
  } else if (!strcmp(name, "pair_tiles")) {
    if (value < 0 || value > 1) return fail(MQK_ERR_BAD_OPTION, "pair_tiles must be 0 or 1");
    g_pair_tiles = value;
  } else if (!strcmp(name, "pair_max_spins")) {
    if (value < 0 || value > (1 << 24)) return fail(MQK_ERR_BAD_OPTION, "pair_max_spins must be in [0, 2^24]");
    g_pair_max_spins = value;
  } else if (!strcmp(name, "pair_hold")) {
    if (value < 0 || value > 4096) return fail(MQK_ERR_BAD_OPTION, "pair_hold must be in [0, 4096]");
    g_pair_hold = (g_pair_hold & ~0xFFFF) | int(value);
  } else if (!strcmp(name, "pair_cross_xcd")) {
    if (value != 0 && value != 1) return fail(MQK_ERR_BAD_OPTION, "pair_cross_xcd must be 0 or 1");
    g_pair_hold = (g_pair_hold & 0xFFFF) | (int(value) << 16);
  } else if (!strcmp(name, "gemv_max_m")) {
    if (value < 0 || value > kGemvMaxM) return fail(MQK_ERR_BAD_OPTION, "gemv_max_m must be in [0, %d]", kGemvMaxM);
    g_gemv_max_m = value;
  } else {
    return fail(MQK_ERR_BAD_OPTION, "unknown option '%s'", name);
  }
  return ok();
}

int64_t mqk_get_option(const char* name) {
  if (!name) return -1;
  if (!strcmp(name, "prefill_tile")) return g_prefill_tile.load();
  if (!strcmp(name, "decode_max_t")) return g_decode_max_t.load();
  if (!strcmp(name, "decode_splits")) return g_decode_splits.load();
  if (!strcmp(name, "group_m")) return g_group_m.load();
  if (!strcmp(name, "tail_split")) return g_tail_split.load();
  if (!strcmp(name, "decode_blocks")) return g_decode_blocks.load();
  if (!strcmp(name, "decode_passes")) return g_decode_passes.load();
  if (!strcmp(name, "decode_cost_model")) return g_decode_cost_model.load();
  if (!strcmp(name, "tile_ksplit")) return g_tile_ksplit.load();
  if (!strcmp(name, "head_tiles")) return g_head_tiles.load();
  if (!strcmp(name, "gemv_max_m")) return g_gemv_max_m.load();
  if (!strcmp(name, "pair_tiles")) return g_pair_tiles.load();
  if (!strcmp(name, "pair_max_spins")) return g_pair_max_spins.load();
  if (!strcmp(name, "pair_hold")) return g_pair_hold & 0xFFFF;
  if (!strcmp(name, "pair_cross_xcd")) return g_pair_hold >> 16;
  if (!strcmp(name, "decode_force_recompute")) return g_decode_force_recompute;
  if (!strcmp(name, "decode_max_spins")) return g_decode_max_spins;
  if (!strcmp(name, "device_cus")) return device_topology().cus;    // read-only: the current device's
  if (!strcmp(name, "device_xcds")) return device_topology().xcds;  // topology as the planner uses it
  return -1;
}

int mqk_read_probe(const void* src, size_t bytes, int blocks, uint32_t* out, void* stream) {
  return hip_status(launch_read_probe(src, bytes, blocks, out, static_cast<hipStream_t>(stream)), "read probe launch");
}

int mqk_clock_probe(uint64_t* out, int spins, void* stream) {
  return hip_status(launch_clock_probe(out, spins, static_cast<hipStream_t>(stream)), "clock probe launch");
}

const char* mqk_tile_variants(void) {
  static const char* const text = [] {
    static char buf[512];
    size_t n = 0;
    buf[0] = '\0';
    for (int i = 0; i < tile_variant_count(); ++i) {
      const TileVariant* v = tile_variant(i);
      // (a pair variant's hpt counts the heads of both workgroups of a pair)
      n += snprintf(buf + n, sizeof(buf) - n, "%s%d:%dx%d/%dw", i ? ";" : "", v->id, v->bm,
                    is_pair_variant(v->id) ? v->hpt * kHeadDim / 2 : v->hpt * kHeadDim, v->threads / 64);
    }
    return buf;
  }();
  return text;
}

}  // extern "C"
