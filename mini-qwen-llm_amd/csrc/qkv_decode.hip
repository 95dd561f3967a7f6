// Split-K projection for small token counts (decode steps, T <= 64) with the
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
//   * inside a workgroup, wave (cg, kq) owns columns [64cg, 64cg+64) of the
//     head and a quarter of the split's k-range, for all 64 token rows
//     (v_mfma_f32_16x16x32_bf16, 4 x 4 blocks, so each activation fragment read
//     from LDS feeds 4 MFMAs).  Its weight slice is loaded HBM -> VGPR before
//     the first MFMA; the activation slice is staged once in LDS with direct
//     global->LDS loads.  The four k-quarters are added through LDS.
// Combining the splits: each workgroup writes its fp32 partial tile [64 x 128]
// with plain stores, which stay in (or are written back from) the L2 of its
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

#ifdef MQK_DECODE_TRACE
// Diagnostic build only: per-workgroup phase timestamps (100 MHz s_memrealtime)
// written to a device buffer set with mqk_set_option("decode_trace", ptr).
__device__ int64_t* g_decode_trace = nullptr;
void set_decode_trace(void* ptr) {
  (void)hipMemcpyToSymbol(HIP_SYMBOL(g_decode_trace), &ptr, sizeof(ptr));
}
#define DECODE_TRACE(i)                                                   \
  if (g_decode_trace && threadIdx.x == 0)                                 \
    g_decode_trace[blockIdx.x * 8 + (i)] = __builtin_amdgcn_s_memrealtime();
#else
#define DECODE_TRACE(i)
#endif

namespace {

constexpr int kDecRows = 64;            // token rows per call (T <= 64)
constexpr int kDecThreads = 512;        // 8 waves: 2 column halves x 4 k-quarters
constexpr int kDecMaxNK = 16;           // largest k-range of one split, in 64-wide tiles
constexpr int kDecQuarterNK = kDecMaxNK / 4;
constexpr int kDecKc = kDecMaxNK * kBK;     // LDS row length of the x slice (bf16), 2 KB
constexpr int kMaxHeads = 1024;
constexpr int kCounterBytes = kMaxHeads * 4;
constexpr int kTileFloats = kDecRows * kHeadDim;
constexpr int kPitch = kHeadDim;        // LDS pitch (floats) of a partial tile
constexpr int kXcds = 8;                // MI355X: 8 XCDs, workgroup b dispatched to XCD b % 8
constexpr uint32_t kForeignUnit = 1u << 16;  // arrival-counter increment of a misplaced split

static_assert(kDecRows * kDecKc * 2 > 160 * 1024 / 2, "x slice must keep one workgroup per CU");
static_assert(4 * kDecRows * kPitch * 4 <= kDecRows * kDecKc * 2, "4 partial tiles alias the x slice");

__device__ __forceinline__ int dec_lds_off(int row, int chunk) {
  // row stride kDecKc bf16 (2 KB); 16-byte chunk index XOR-swizzled in its low
  // 4 bits so the 16 rows read by one quarter-wave hit 16 different bank groups
  return row * kDecKc + ((chunk ^ (row & 15)) << 3);
}

__device__ __forceinline__ int xcc_id() {
  return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));  // hwreg(HW_REG_XCC_ID, 0, 4)
}

// k-tile range [kt0, kt0 + nk) of split s of S over nkt tiles (balanced).
__device__ __forceinline__ void split_range(int s, int S, int nkt, int& kt0, int& nk) {
  kt0 = int((int64_t(s) * nkt) / S);
  nk = int((int64_t(s + 1) * nkt) / S) - kt0;
}

// Computes the partial tile of k-tiles [kt0, kt0 + nk) of one head into LDS
// `tile` (fp32 [64][kPitch], row-major), using `xs` as staging.  All threads of
// the workgroup call it; it ends with a barrier.
template <bool INT4>
__device__ void compute_partial(const ProblemArgs& p, const WeightArgs& w, int proj, int hh, int kt0,
                                int nk, uint16_t* xs, float* tile) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int cg = wave & 1;            // 64-column half of the head
  const int kq = wave >> 1;           // k-quarter of the split
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int M = int(p.M);
  const int64_t kbeg = int64_t(kt0) * kBK;
  // k-quarter kq covers tiles [kq*nk/4, (kq+1)*nk/4) of the split
  const int my_t0 = (kq * nk) >> 2;
  const int my_nt = (((kq + 1) * nk) >> 2) - my_t0;

  // 1. activation slice x[0:M, kbeg : kbeg + nk*64] -> LDS with direct
  // global->LDS loads (no VGPR staging).  One wave instruction fills half an
  // LDS row (64 chunks of 16 B); lane L writes LDS chunk slot half*64 + L, which
  // holds global chunk slot ^ (row & 15) (the swizzle of dec_lds_off).
  constexpr int kWaves = kDecThreads / 64;
#pragma unroll
  for (int i = 0; i < 2 * kDecRows / kWaves; ++i) {
    const int u = wave + kWaves * i;      // (row, half) unit, wave-uniform
    const int row = u >> 1, half = u & 1;
    const int gq = (half * 64 + lane) ^ (row & 15);
    if (row < M && gq < nk * 8)
      __builtin_amdgcn_global_load_lds(p.x + int64_t(row) * p.K + kbeg + gq * 8,
                                       xs + row * kDecKc + half * 64 * 8, 16, 0, 0);
  }

  // 2. this wave's weight slice, straight to registers.  16x16x32 operand
  // layout: lane (c, g) holds column c (B) / row c (A) and 8 k values; k order
  // inside a 64-wide tile: block kk (0,1) of 32, lane group g -> kk*32 + g*8.
  const int64_t col0 = int64_t(hh) * kHeadDim + cg * 64 + c16;  // column (nb = 0) inside the projection
  const int64_t qstride = w.n_cols[proj];
  u32x4_t wb[INT4 ? 1 : kDecQuarterNK][4][2];
  uint32_t wq[INT4 ? kDecQuarterNK : 1][4][2];
#pragma unroll
  for (int t = 0; t < kDecQuarterNK; ++t) {
    if (t < my_nt) {
      const int64_t k0 = kbeg + int64_t(my_t0 + t) * kBK;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int64_t col = col0 + nb * 16;
          if constexpr (!INT4)
            wb[t][nb][kk] = *reinterpret_cast<const u32x4_t*>(w.w[proj] + col * p.K + k0 + kk * 32 + g4 * 8);
          else
            wq[t][nb][kk] = uint32_t(w.qw[proj][(k0 / 8 + kk * 4 + g4) * qstride + col]);
        }
    }
  }

  // 3. wait for every load (the x slice must be in LDS before the barrier; the
  // compiler drains all loads before a barrier that follows LDS-DMA loads anyway)
  __builtin_amdgcn_s_waitcnt(0);
  DECODE_TRACE(1)
  __syncthreads();
  DECODE_TRACE(5)

  // 4. MFMAs.  Rows >= M of xs hold stale data; output row r depends only on
  // row r of x and rows >= M are never stored.
  f32x4_t acc[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4_t{};
#pragma unroll
  for (int t = 0; t < kDecQuarterNK; ++t) {
    if (t < my_nt) {
      u32x4_t b[4][2];
      if constexpr (!INT4) {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          b[nb][0] = wb[t][nb][0];
          b[nb][1] = wb[t][nb][1];
        }
      } else {
        const int64_t k0 = kbeg + int64_t(my_t0 + t) * kBK;
        const int grp = int(k0 / w.group);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const int64_t col = col0 + nb * 16;
          const uint32_t sraw = static_cast<const uint16_t*>(w.sc[proj])[grp * qstride + col];
          const float scale = w.scale_fp16 ? f16_to_f32(sraw) : bf16_to_f32(sraw);
          const uint32_t zw = uint32_t(w.qz[proj][grp * (qstride / 8) + col / 8]);
          const float zero = float((zw >> ((col % 8) * 4)) & 0xFu);
          b[nb][0] = dequant_int4x8(wq[t][nb][0], zero, scale);
          b[nb][1] = dequant_int4x8(wq[t][nb][1], zero, scale);
        }
      }
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int chunk = (my_t0 + t) * 8 + kk * 4 + g4;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xs + dec_lds_off(mb * 16 + c16, chunk));
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma_16x16x32(a, b[nb][kk], acc[mb][nb]);
        }
      }
    }
  }
  __syncthreads();  // xs no longer read; the quarter tiles alias it
  DECODE_TRACE(6)

  // 5. add the four k-quarters: wave (cg, kq) writes its block into quarter tile
  // kq, then every thread sums one 16-column strip of one row into tile 0.
  // acc[mb][nb][j] = C[mb*16 + 4g + j][cg*64 + nb*16 + c].
  float* qt = tile + kq * (kDecRows * kPitch);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        qt[(mb * 16 + g4 * 4 + j) * kPitch + cg * 64 + nb * 16 + c16] = acc[mb][nb][j];
  __syncthreads();
  {
    const int r = tid >> 3, c0 = (tid & 7) * 16;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      f32x4_t sum = *reinterpret_cast<const f32x4_t*>(tile + r * kPitch + c0 + 4 * v);
#pragma unroll
      for (int k = 1; k < 4; ++k)
        sum += *reinterpret_cast<const f32x4_t*>(tile + k * (kDecRows * kPitch) + r * kPitch + c0 + 4 * v);
      *reinterpret_cast<f32x4_t*>(tile + r * kPitch + c0 + 4 * v) = sum;
    }
  }
  __syncthreads();
}

template <bool INT4>
__global__ void __launch_bounds__(kDecThreads, 1)
decode_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int splits, float* __restrict__ part,
              uint32_t* __restrict__ counters, int force_recompute) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kDecRows * kDecKc];
  __shared__ uint32_t arrival;
  float* tile = reinterpret_cast<float*>(xs);  // partial tile aliases the x staging area

  const int tid = threadIdx.x;
  const int n_tiles = p.n_tiles;
  const int bid = blockIdx.x;
  const int q = bid / kXcds;
  const int split = q % splits;
  const int head = (q / splits) * kXcds + bid % kXcds;
  if (head >= n_tiles) return;  // padding workgroup
  const int M = int(p.M);
  const int nkt = int(p.K / kBK);
  int proj, hh;
  split_head(head, e.Hq, e.Hkv, proj, hh);
  DECODE_TRACE(0)

  int kt0, nk;
  split_range(split, splits, nkt, kt0, nk);
  compute_partial<INT4>(p, w, proj, hh, kt0, nk, xs, tile);

  DECODE_TRACE(2)
  // ---- publish the partial: part[split][head] = [64][128] fp32 row-major -------
  {
    const int r = tid >> 3, c0 = (tid & 7) * 16;  // row, 16 consecutive columns
    if (r < M) {
      float* dst = part + (int64_t(split) * n_tiles + head) * kTileFloats + r * kHeadDim + c0;
#pragma unroll
      for (int v = 0; v < 4; ++v)
        *reinterpret_cast<f32x4_t*>(dst + 4 * v) = *reinterpret_cast<const f32x4_t*>(tile + r * kPitch + c0 + 4 * v);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have reached the L2
  __syncthreads();                // ... and every thread's
  if (tid == 0) {
    const bool foreign = force_recompute || xcc_id() != bid % kXcds;
    const uint32_t inc = 1u + (foreign ? kForeignUnit : 0u);
    arrival = __hip_atomic_fetch_add(counters + head, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
  }
  __syncthreads();
  DECODE_TRACE(3)
  const uint32_t seen = arrival;
  if ((seen & (kForeignUnit - 1)) != uint32_t(splits)) return;  // not the last split to arrive
  const bool recompute = (seen >> 16) != 0;

  // ---- last arrival: sum the partials in split order -------------------------------
  // thread -> row r = tid / 8, c = tid % 8: columns [8c, 8c+8) and
  // [64+8c, 64+8c+8), so every RoPE pair (d, d+64) is thread-local.
  const int r = tid >> 3;
  const int c = tid & 7;
  float lo[8], hi[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) lo[i] = hi[i] = 0.f;
  auto add8 = [&](const float* src) {
    const f32x4_t a0 = *reinterpret_cast<const f32x4_t*>(src + 8 * c);
    const f32x4_t a1 = *reinterpret_cast<const f32x4_t*>(src + 8 * c + 4);
    const f32x4_t b0 = *reinterpret_cast<const f32x4_t*>(src + kHalfDim + 8 * c);
    const f32x4_t b1 = *reinterpret_cast<const f32x4_t*>(src + kHalfDim + 8 * c + 4);
    lo[0] += a0.x; lo[1] += a0.y; lo[2] += a0.z; lo[3] += a0.w;
    lo[4] += a1.x; lo[5] += a1.y; lo[6] += a1.z; lo[7] += a1.w;
    hi[0] += b0.x; hi[1] += b0.y; hi[2] += b0.z; hi[3] += b0.w;
    hi[4] += b1.x; hi[5] += b1.y; hi[6] += b1.z; hi[7] += b1.w;
  };
  if (!recompute) {
    if (r < M) {
      for (int s0 = 0; s0 < splits; s0 += 4) {
        f32x4_t buf[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int s = s0 + j < splits ? s0 + j : s0;  // padding slots re-read a valid tile
          const float* src = s == split ? tile + r * kPitch
                                        : part + (int64_t(s) * n_tiles + head) * kTileFloats + r * kHeadDim;
          buf[j][0] = *reinterpret_cast<const f32x4_t*>(src + 8 * c);
          buf[j][1] = *reinterpret_cast<const f32x4_t*>(src + 8 * c + 4);
          buf[j][2] = *reinterpret_cast<const f32x4_t*>(src + kHalfDim + 8 * c);
          buf[j][3] = *reinterpret_cast<const f32x4_t*>(src + kHalfDim + 8 * c + 4);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (s0 + j >= splits) break;
          lo[0] += buf[j][0].x; lo[1] += buf[j][0].y; lo[2] += buf[j][0].z; lo[3] += buf[j][0].w;
          lo[4] += buf[j][1].x; lo[5] += buf[j][1].y; lo[6] += buf[j][1].z; lo[7] += buf[j][1].w;
          hi[0] += buf[j][2].x; hi[1] += buf[j][2].y; hi[2] += buf[j][2].z; hi[3] += buf[j][2].w;
          hi[4] += buf[j][3].x; hi[5] += buf[j][3].y; hi[6] += buf[j][3].z; hi[7] += buf[j][3].w;
        }
      }
    }
  } else {
    // Some split ran on another XCD: its partial may not be visible through this
    // L2.  Recompute every split here (same arithmetic, same order).
    for (int s = 0; s < splits; ++s) {
      int s_kt0, s_nk;
      split_range(s, splits, nkt, s_kt0, s_nk);
      compute_partial<INT4>(p, w, proj, hh, s_kt0, s_nk, xs, tile);
      if (r < M) add8(tile + r * kPitch);
      __syncthreads();  // tile is rewritten by the next split
    }
  }

  if (proj != 2) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += lo[i] * lo[i] + hi[i] * hi[i];
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    const float rms = rsqrtf(ss * (1.0f / float(kHeadDim)) + e.eps);
    if (r < M) {
      const uint16_t* gamma = proj == 0 ? e.q_gamma : e.k_gamma;
      const int64_t prow = rope_row(e.positions, r, e.S, e.cos_rows) * kHeadDim;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int d = 8 * c + i;
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
    o.x = pack_bf16x2(lo[0], lo[1]);
    o.y = pack_bf16x2(lo[2], lo[3]);
    o.z = pack_bf16x2(lo[4], lo[5]);
    o.w = pack_bf16x2(lo[6], lo[7]);
    *reinterpret_cast<u32x4_t*>(dst + 8 * c) = o;
    o.x = pack_bf16x2(hi[0], hi[1]);
    o.y = pack_bf16x2(hi[2], hi[3]);
    o.z = pack_bf16x2(hi[4], hi[5]);
    o.w = pack_bf16x2(hi[6], hi[7]);
    *reinterpret_cast<u32x4_t*>(dst + kHalfDim + 8 * c) = o;
  }
  if (tid == 0) __hip_atomic_store(counters + head, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef MQK_DECODE_TRACE
  __builtin_amdgcn_s_waitcnt(0);
  DECODE_TRACE(4)
#endif
}

int g_cus_per_xcd = 0;  // queried once (single-device processes)

int cus_per_xcd() {
  if (g_cus_per_xcd <= 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus >= kXcds)
      g_cus_per_xcd = cus / kXcds;
    else
      g_cus_per_xcd = 32;  // MI355X: 256 CUs / 8 XCDs
    (void)hipGetLastError();
  }
  return g_cus_per_xcd;
}

}  // namespace

int g_decode_force_recompute = 0;

int decode_splits_for(int64_t M, int64_t K, int n_tiles, int requested) {
  (void)M;
  const int nkt = int(K / kBK);
  if (nkt < 1) return 0;
  const int min_splits = (nkt + kDecMaxNK - 1) / kDecMaxNK;  // LDS bound on a split's k-range
  int s = requested;
  if (s <= 0) {
    // one workgroup per CU: (heads per XCD) x splits <= CUs per XCD
    const int heads_per_xcd = (n_tiles + kXcds - 1) / kXcds;
    s = cus_per_xcd() / heads_per_xcd;
    if (s > nkt) s = nkt;  // small hidden: at most one k tile per split
    if (s < min_splits) s = min_splits;
  }
  if (s < min_splits || s > nkt || s > kDecMaxNK) return 0;
  return s;
}

size_t decode_workspace_bytes(int n_tiles, int splits) {
  return size_t(kCounterBytes) + size_t(splits) * n_tiles * kTileFloats * sizeof(float);
}

hipError_t launch_decode(int int4, const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                         int splits, void* workspace, hipStream_t stream) {
  const int nkt = int(p.K / kBK);
  if (splits < 1 || splits > kDecMaxNK || splits > nkt || (nkt + splits - 1) / splits > kDecMaxNK ||
      p.n_tiles > kMaxHeads)
    return hipErrorInvalidValue;
  uint32_t* counters = static_cast<uint32_t*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  const dim3 grid(((p.n_tiles + kXcds - 1) / kXcds) * kXcds * splits);
  const int fr = g_decode_force_recompute;
  if (int4)
    hipLaunchKernelGGL(decode_kernel<true>, grid, dim3(kDecThreads), 0, stream, p, w, e, splits, part, counters,
                       fr);
  else
    hipLaunchKernelGGL(decode_kernel<false>, grid, dim3(kDecThreads), 0, stream, p, w, e, splits, part,
                       counters, fr);
  return hipGetLastError();
}

}  // namespace mqk
