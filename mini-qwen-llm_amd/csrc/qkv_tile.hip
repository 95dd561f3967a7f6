// Tiled MFMA projection with a fused per-head epilogue (prefill / large-T path).
//
// One workgroup computes a BM x (HPT*128) tile of  x[M,K] @ W^T  where every
// 128-column slice is exactly one attention head (Q, K or V; the three weight
// matrices are addressed directly, no concatenated copy is made).  Waves own
// 64-row x 128-column sub-tiles, i.e. whole heads, so the epilogue -- sum of
// squares over the head, rsqrt, gamma, rotate-half RoPE -- runs on the fp32
// accumulators in registers and each output element is written to HBM once.
//
// Main loop: K is staged through LDS in 64-wide tiles, double buffered, with one
// barrier per tile.  Staging goes HBM -> VGPR -> LDS so the global loads of tile
// k+1 are in flight while the MFMAs of tile k run.  LDS rows are 128 bytes
// (8 chunks of 16 B); chunk c of row r is stored at slot c ^ (r & 7) so that the
// 16-byte fragment reads of 8 consecutive rows hit 8 different bank groups.
//
// KZ == 2 variants split each staged tile's four k16 steps between two waves
// that own the same output sub-tile; their partial sums are exchanged through
// LDS before the epilogue (each wave then finalises one of its two 32-row
// blocks).  This keeps 4 waves busy on a 128x128 tile without shrinking the
// per-wave register tile (which sets the LDS bytes read per MFMA).
//
// The int4 (W4A16) variant replaces the bf16 weight stage: packed int32 words
// of qweight [K/8, N] (8 consecutive k of one column) are loaded, dequantised
// (q - z) * s in fp32 and written to LDS as bf16 in the same layout.
#include "mqk_device.h"
#include "mqk_kernels.h"

namespace mqk {
namespace {

template <int BM, int HPT, int KZ>
struct TileShape {
  static constexpr int kWavesM = BM / 64;
  static constexpr int kWavesMN = kWavesM * HPT;
  static constexpr int kWaves = kWavesMN * KZ;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kBN = HPT * kHeadDim;
  static constexpr int kCA = BM * 8 / kThreads;       // A chunks (16 B) per thread per stage
  static constexpr int kCB = kBN * 8 / kThreads;      // B chunks per thread per stage
  static constexpr int kStage = (BM + kBN) * kBK;     // bf16 elements per stage
  static constexpr int kStepsPerWave = 4 / KZ;        // k16 MFMA steps per staged tile
  static_assert(BM % 64 == 0, "BM");
  static_assert((BM * 8) % kThreads == 0 && (kBN * 8) % kThreads == 0, "chunk split");
  static_assert(kThreads % kBN == 0, "int4 loader assigns one column per thread");
  static_assert(KZ == 1 || KZ == 2, "KZ");
  static_assert(KZ == 1 || kWavesMN * 2 * 4096 <= 2 * kStage * 2, "exchange fits in LDS");
};

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kBK + ((chunk ^ (row & 7)) << 3);
}

// Epilogue for one 32-row block of a wave's 64x128 sub-tile.  acc[nb][i] holds
// C[row_base + 8*(i/4) + 4*(lane>>5) + i%4][nb*32 + (lane&31)] of head h.
__device__ __forceinline__ void store_block(const f32x16_t (&acc)[4], int64_t row_base, int h,
                                           const ProblemArgs& p, const EpilogueArgs& e, int lane) {
  const int c32 = lane & 31;
  const int half = lane >> 5;
  int proj, hh;
  split_head(h, e.Hq, e.Hkv, proj, hh);

  if (!e.qkv) {  // plain GEMM output [M, N]
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int64_t col = int64_t(h) * kHeadDim + nb * 32 + c32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t t = row_base + 8 * (i >> 2) + 4 * half + (i & 3);
        if (t < p.M && col < e.N) e.out[t * e.N + col] = f32_to_bf16(acc[nb][i]);
      }
    }
    return;
  }

  const int H = proj == 0 ? e.Hq : e.Hkv;
  uint16_t* __restrict__ dst = pick3(proj, e.q, e.k, e.v);

  if (proj == 2 || e.qkv == 2) {  // V (fused_qkv_rope.py:169, :194), or any head with qkv 2: as projected
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t t = row_base + 8 * (i >> 2) + 4 * half + (i & 3);
      if (t < p.M) {
        const int64_t cs = paged_slot(e, t);
        uint16_t* o = dst ? dst + (t * H + hh) * kHeadDim + c32 : nullptr;  // v may be null (cache only)
        uint16_t* oc = cs >= 0 ? paged_row(e, cs, proj, hh) + c32 : nullptr;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const uint16_t b = f32_to_bf16(acc[nb][i]);
          if (o) o[nb * 32] = b;
          if (oc) oc[nb * 32] = b;
        }
      }
    }
    return;
  }

  // Q/K: RMSNorm over the head (fused_qkv_rope.py:98-100) then rotate-half RoPE
  // (:102-118).  Lane holds columns c32 + 32 nb (nb = 0..3) of the block.  Head dim
  // 128: one head, RoPE pairs (d, d+64) are nb (0,2) and (1,3).  Head dim 64: two
  // heads, columns 0-63 (nb 0, 1) and 64-127 (nb 2, 3), pairs (d, d+32) are nb
  // (0,1) and (2,3).  All in registers.
  const uint16_t* __restrict__ gamma = pick3(proj, e.q_gamma, e.k_gamma, e.k_gamma);
  const int hd = e.head_dim;
  const bool two = hd == 64;
  float g[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) g[nb] = bf16_to_f32(gamma[(two ? (nb & 1) : nb) * 32 + c32]);
  const float inv_d = two ? 1.0f / 64.0f : 1.0f / float(kHeadDim);

#pragma unroll
  for (int i = 0; i < 16; ++i) {
    // sums of squares over the 32 lanes that share this row (same lane>>5)
    float ss, ss2 = 0.f;
    if (!two) {
      ss = acc[0][i] * acc[0][i] + acc[1][i] * acc[1][i] + acc[2][i] * acc[2][i] + acc[3][i] * acc[3][i];
    } else {
      ss = acc[0][i] * acc[0][i] + acc[1][i] * acc[1][i];
      ss2 = acc[2][i] * acc[2][i] + acc[3][i] * acc[3][i];
    }
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) {
      ss += __shfl_xor(ss, m);
      if (two) ss2 += __shfl_xor(ss2, m);
    }
    const float rms = rsqrtf(ss * inv_d + e.eps);
    const float rms2 = two ? rsqrtf(ss2 * inv_d + e.eps) : rms;
    const int64_t t = row_base + 8 * (i >> 2) + 4 * half + (i & 3);
    if (t < p.M) {
      const int64_t prow = rope_row(e, t) * hd;
      const int64_t cs = proj == 1 ? paged_slot(e, t) : -1;
      uint16_t* o = dst ? dst + (t * H + hh) * kHeadDim : nullptr;  // k may be null (cache only)
      uint16_t* oc = cs >= 0 ? paged_row(e, cs, proj, hh) : nullptr;
#pragma unroll
      for (int pr = 0; pr < 2; ++pr) {
        // (lo, hi) accumulator blocks of the pair, its first dim, and its head's rms
        const int lo = two ? 2 * pr : pr, hi = two ? 2 * pr + 1 : pr + 2;
        const int d = two ? c32 : pr * 32 + c32;
        const int hd2 = hd / 2;
        const float r = pr == 1 ? rms2 : rms;
        const float x1n = acc[lo][i] * r * g[lo];
        const float x2n = acc[hi][i] * r * g[hi];
        const float c1 = bf16_to_f32(e.cos[prow + d]);
        const float c2 = bf16_to_f32(e.cos[prow + d + hd2]);
        const float s1 = bf16_to_f32(e.sin[prow + d]);
        const float s2 = bf16_to_f32(e.sin[prow + d + hd2]);
        const uint16_t b1 = f32_to_bf16(x1n * c1 - x2n * s1);
        const uint16_t b2 = f32_to_bf16(x2n * c2 + x1n * s2);
        if (o) {
          o[lo * 32 + c32] = b1;
          o[hi * 32 + c32] = b2;
        }
        if (oc) {
          oc[lo * 32 + c32] = b1;
          oc[hi * 32 + c32] = b2;
        }
      }
    }
  }
}

template <int BM, int HPT, int KZ, bool INT4>
__global__ void __launch_bounds__(BM / 64 * HPT * KZ * 64)
tile_kernel(ProblemArgs p, WeightArgs w, EpilogueArgs e, int group_m) {
  using TS = TileShape<BM, HPT, KZ>;
  constexpr int NT = TS::kThreads;
  constexpr int BN = TS::kBN;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * TS::kStage];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int kz = wave / TS::kWavesMN;
  const int wrem = wave % TS::kWavesMN;
  const int wm = wrem % TS::kWavesM;
  const int wh = wrem / TS::kWavesM;

  // ---- tile coordinates: XCD-contiguous ids, grouped along M -------------
  const int n_mt = int((p.M + BM - 1) / BM);
  const int n_ht = p.n_tiles / HPT;
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

  // ---- per-thread global sources and LDS slots ------------------------------
  const uint16_t* a_src[TS::kCA];
  int a_lds[TS::kCA];
  float a_scale[TS::kCA];  // input RMSNorm scale of the chunk's row
  int a_cc[TS::kCA];
  const bool in_norm = p.in_gamma != nullptr;
#pragma unroll
  for (int i = 0; i < TS::kCA; ++i) {
    const int ci = tid + i * NT;
    const int row = ci >> 3, cc = ci & 7;
    int64_t grow = m0 + row;
    grow = grow < p.M ? grow : p.M - 1;  // rows past M re-read the last row; never stored
    a_src[i] = p.x + grow * K + cc * 8;
    a_lds[i] = lds_off(row, cc);
    a_cc[i] = cc;
    a_scale[i] = in_norm ? p.in_scale[grow] : 1.f;
  }

  const uint16_t* b_src[INT4 ? 1 : TS::kCB];
  int b_lds[TS::kCB];
  // int4 staging state: one output column per thread.
  const int32_t* q_src = nullptr;
  const uint16_t* s_src = nullptr;
  const int32_t* z_src = nullptr;
  int64_t q_stride = 0, z_stride = 0;
  int z_shift = 0;
  if constexpr (!INT4) {
#pragma unroll
    for (int i = 0; i < TS::kCB; ++i) {
      const int ci = tid + i * NT;
      const int row = ci >> 3, cc = ci & 7;
      int proj, hh;
      split_head(ht * HPT + row / kHeadDim, e.Hq, e.Hkv, proj, hh);
      int64_t col = int64_t(hh) * kHeadDim + (row % kHeadDim);
      col = col < w.n_cols[proj] ? col : w.n_cols[proj] - 1;
      b_src[i] = w.w[proj] + col * K + cc * 8;
      b_lds[i] = lds_off(row, cc);
    }
  } else {
    const int cl = tid % BN;
    int proj, hh;
    split_head(ht * HPT + cl / kHeadDim, e.Hq, e.Hkv, proj, hh);
    int64_t col = int64_t(hh) * kHeadDim + (cl % kHeadDim);
    col = col < w.n_cols[proj] ? col : w.n_cols[proj] - 1;
    q_stride = w.n_cols[proj];
    z_stride = w.n_cols[proj] / 8;
    q_src = w.qw[proj] + col;
    s_src = static_cast<const uint16_t*>(w.sc[proj]) + col;
    z_src = w.qz[proj] + col / 8;
    z_shift = int(col % 8) * 4;
#pragma unroll
    for (int i = 0; i < TS::kCB; ++i) {
      const int j = tid / BN + i * (NT / BN);
      b_lds[i] = lds_off(cl, j);
    }
  }

  u32x4_t ra[TS::kCA];
  u32x4_t rg[TS::kCA];  // input-norm gamma of each A chunk
  u32x4_t rb[INT4 ? 1 : TS::kCB];
  uint32_t rq[INT4 ? TS::kCB : 1];
  uint32_t rs = 0, rz = 0;

  auto gload = [&](int kt) {
    const int64_t k0 = int64_t(kt) * kBK;
#pragma unroll
    for (int i = 0; i < TS::kCA; ++i) ra[i] = *reinterpret_cast<const u32x4_t*>(a_src[i] + k0);
    if (in_norm) {
#pragma unroll
      for (int i = 0; i < TS::kCA; ++i) rg[i] = *reinterpret_cast<const u32x4_t*>(p.in_gamma + k0 + a_cc[i] * 8);
    }
    if constexpr (!INT4) {
#pragma unroll
      for (int i = 0; i < TS::kCB; ++i) rb[i] = *reinterpret_cast<const u32x4_t*>(b_src[i] + k0);
    } else {
      const int64_t g = k0 / w.group;
      rs = s_src[g * q_stride];
      rz = uint32_t(z_src[g * z_stride]);
#pragma unroll
      for (int i = 0; i < TS::kCB; ++i) {
        const int j = tid / BN + i * (NT / BN);
        rq[i] = uint32_t(q_src[(k0 / 8 + j) * q_stride]);
      }
    }
  };
  auto sstore = [&](int buf) {
    uint16_t* sA = smem + buf * TS::kStage;
    uint16_t* sB = sA + BM * kBK;
    if (in_norm) {
#pragma unroll
      for (int i = 0; i < TS::kCA; ++i) ra[i] = input_norm8(ra[i], a_scale[i], rg[i]);
    }
#pragma unroll
    for (int i = 0; i < TS::kCA; ++i) *reinterpret_cast<u32x4_t*>(sA + a_lds[i]) = ra[i];
    if constexpr (!INT4) {
#pragma unroll
      for (int i = 0; i < TS::kCB; ++i) *reinterpret_cast<u32x4_t*>(sB + b_lds[i]) = rb[i];
    } else {
      const float scale = w.scale_fp16 ? f16_to_f32(rs) : bf16_to_f32(rs);
      const float zero = float((rz >> z_shift) & 0xFu);
#pragma unroll
      for (int i = 0; i < TS::kCB; ++i)
        *reinterpret_cast<u32x4_t*>(sB + b_lds[i]) = dequant_int4x8(rq[i], zero, scale);
    }
  };

  // ---- main loop ------------------------------------------------------------
  f32x16_t acc[2][4];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x16_t{};

  const int c32 = lane & 31;
  const int khalf = lane >> 5;
  const int swz = c32 & 7;  // row & 7 of every fragment row this lane reads
  const int a_row0 = (wm * 64 + c32) * kBK;
  const int b_row0 = (wh * kHeadDim + c32) * kBK;

  const int nkt = int(K / kBK);
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nkt; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nkt) gload(kt + 1);
    const uint16_t* sA = smem + cur * TS::kStage;
    const uint16_t* sB = sA + BM * kBK;
#pragma unroll
    for (int st = 0; st < TS::kStepsPerWave; ++st) {
      const int cc = 2 * (kz * TS::kStepsPerWave + st) + khalf;
      const int co = (cc ^ swz) << 3;
      u32x4_t af[2], bf[4];
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        af[mb] = *reinterpret_cast<const u32x4_t*>(sA + a_row0 + mb * 32 * kBK + co);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        bf[nb] = *reinterpret_cast<const u32x4_t*>(sB + b_row0 + nb * 32 * kBK + co);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = mfma_32x32x16(af[mb], bf[nb], acc[mb][nb]);
    }
    if (kt + 1 < nkt) sstore(cur ^ 1);
    __syncthreads();
  }

  // ---- combine the K-split halves (KZ == 2) ---------------------------------
  if constexpr (KZ == 2) {
    float* xch = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      float* mine = xch + (wrem * 2 + kz) * 1024;
      const float* other = xch + (wrem * 2 + (kz ^ 1)) * 1024;
      const f32x16_t send = kz == 0 ? acc[1][nb] : acc[0][nb];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4_t v4 = {send[4 * q], send[4 * q + 1], send[4 * q + 2], send[4 * q + 3]};
        *reinterpret_cast<f32x4_t*>(mine + (q * 64 + lane) * 4) = v4;
      }
      __syncthreads();
      f32x16_t recv;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(other + (q * 64 + lane) * 4);
        recv[4 * q] = v4.x;
        recv[4 * q + 1] = v4.y;
        recv[4 * q + 2] = v4.z;
        recv[4 * q + 3] = v4.w;
      }
      if (kz == 0) acc[0][nb] += recv;
      else acc[1][nb] += recv;
      __syncthreads();
    }
  }

  // ---- epilogue -------------------------------------------------------------
  const int head = ht * HPT + wh;
  if constexpr (KZ == 2) {
    // (the block is selected by value: indexing acc by the wave's kz would put the
    // accumulators in scratch memory)
    f32x16_t blk[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) blk[nb] = kz == 0 ? acc[0][nb] : acc[1][nb];
    store_block(blk, m0 + wm * 64 + kz * 32, head, p, e, lane);
  } else {
    store_block(acc[0], m0 + wm * 64, head, p, e, lane);
    store_block(acc[1], m0 + wm * 64 + 32, head, p, e, lane);
  }
}

template <int BM, int HPT, int KZ, bool INT4>
hipError_t launch_impl(const ProblemArgs& p, const WeightArgs& w, const EpilogueArgs& e,
                       int group_m, hipStream_t stream) {
  using TS = TileShape<BM, HPT, KZ>;
  const int n_mt = int((p.M + BM - 1) / BM);
  const int n_ht = p.n_tiles / HPT;
  const int blocks = n_mt * n_ht;
  if (group_m < 1) group_m = 1;
  hipLaunchKernelGGL((tile_kernel<BM, HPT, KZ, INT4>), dim3(blocks), dim3(TS::kThreads), 0,
                     stream, p, w, e, group_m);
  return hipGetLastError();
}

template <int BM, int HPT, int KZ>
hipError_t launch_dispatch(int int4, const ProblemArgs& p, const WeightArgs& w,
                           const EpilogueArgs& e, int group_m, hipStream_t stream) {
  return int4 ? launch_impl<BM, HPT, KZ, true>(p, w, e, group_m, stream)
              : launch_impl<BM, HPT, KZ, false>(p, w, e, group_m, stream);
}

// ids 1-5: register-staged kernel above (bf16 and int4 weights);
// ids 10-23: direct-to-LDS pipelined kernel (qkv_tile_dma.hip, bf16 weights only);
// ids 30-35: its int4-weight twin (W4A16 only).
const TileVariant kVariants[] = {
    {1, 128, 1, 2, 256},
    {2, 256, 1, 1, 256},
    {3, 128, 2, 1, 256},
    {4, 256, 2, 1, 512},
    {5, 128, 2, 2, 512},
    {10, 256, 2, 0, 512},
    {11, 128, 3, 0, 512},
    {12, 256, 1, 0, 256},
    {13, 128, 2, 0, 256},
    {14, 256, 2, 0, 512},
    {15, 128, 3, 0, 512},
    {16, 128, 3, 0, 512},
    {17, 256, 2, 0, 512},
    {18, 256, 2, 0, 512},
    {19, 128, 1, 0, 256},
    {20, 64, 1, 0, 256},
    {21, 128, 1, 0, 512},
    {22, 256, 1, 0, 512},
    {23, 128, 2, 0, 512},
    {24, 256, 3, 0, 512},  // pair tiles: hpt = heads per pair of workgroups (256 x 192 each)
    {25, 256, 5, 0, 512},  // (256 x 320 each)
    {26, 128, 3, 0, 512},  // (128 x 192 each)
    {27, 128, 5, 0, 512},  // (128 x 320 each)
    {28, 192, 3, 0, 384},  // (192 x 192 each)
    {30, 128, 3, 0, 512},
    {31, 256, 2, 0, 512},
    {32, 128, 2, 0, 256},
    {33, 256, 2, 0, 512},
    {34, 128, 1, 0, 512},
    {35, 64, 1, 0, 256},
};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

}  // namespace

int tile_variant_count() { return kNumVariants; }

const TileVariant* tile_variant(int index) {
  return (index >= 0 && index < kNumVariants) ? &kVariants[index] : nullptr;
}

const TileVariant* find_variant(int id) {
  for (const auto& v : kVariants)
    if (v.id == id) return &v;
  return nullptr;
}

// ids 1-5 take either weight type, 10-18 bf16 weights only, 30-33 int4 weights only
static bool supports(const TileVariant& v, int int4) {
  return v.id < 10 || (int4 ? v.id >= 30 : v.id < 30);
}

int64_t tile_count(const TileVariant& v, int64_t M, int n_tiles) {
  return ((M + v.bm - 1) / v.bm) * (n_tiles / v.hpt) * (is_pair_variant(v.id) ? 2 : 1);
}

const TileVariant* choose_tile_variant(int requested_id, int64_t M, int n_tiles, int int4, int cus_, bool allow_pair) {
  // (a pair launch has one exchange word per pair in the workspace's kSplitMaxTiles lines)
  auto pair_fits = [&](const TileVariant& v) { return allow_pair && tile_count(v, M, n_tiles) / 2 <= kSplitMaxTiles; };
  if (requested_id > 0) {
    const TileVariant* v = find_variant(requested_id);
    if (!v || n_tiles % v->hpt != 0 || !supports(*v, int4) || (is_pair_variant(v->id) && !pair_fits(*v)))
      return nullptr;
    return v;
  }
  // Score = relative per-tile speed (measured on MI355X) x fraction of the last
  // round of workgroups that is busy, assuming one workgroup per CU at a time
  // (cus_: the device's compute units).
  struct Cand { int id; float speed; };
  // (per-tile rates measured on MI355X: 64-wide k stages (16, 17, 18) beat 32-wide
  // ones; 128x384 wins when its tiles fill the chip, 256x256 otherwise)
  // The register-staged variants (1-5) are not candidates: with few tiles (small
  // T) their per-tile rate collapses (T = 65..1024 measured 3-6x slower than the
  // pipelined variants), so they serve only as the fallback for shapes no
  // pipelined variant tiles and for explicit requests.
  // (23, 128x256 with 8 waves and 3 stages of 64 k, measured ~1.2x the rate of 13:
  // the reference's published Qwen3-0.6B B=4 x S=512 call in 24.6 us against 30.3)
  // (pair tiles, 24 = 2 x 256 x 192 per 3 heads and 25 = 2 x 256 x 320 per 5 heads,
  // need the workspace and head_dim 128 (allow_pair).  Measured on MI355X: 24 no
  // faster than 16 at Qwen3-8B prefill (104.6-104.9 us against 104.5-105.6), so it
  // ranks just below it; 25 takes BASELINE config 4's 512 tiles in two rounds in
  // 170.5-171.7 us against 188.5-189.0 for variant 18's 640 tiles; the 128-row pairs
  // 26 (3 stages of 64 k) and 27 (2 stages) fill one round where the whole-head
  // tiles cannot: e.g. hidden 2560 (48 heads) T = 896 41.7 us against 48.5 for 23,
  // hidden 2048 (40 heads) T = 2048 49.5 against 58.0 for 18; the 192-row pair 28
  // (3 stages) where it fills nearly one round: hidden 4096 T = 1536 86 against 100
  // for 16, and 78-81 against 67-74 with 7 of 8 workgroups per CU, so it is
  // taken only beyond that)
  static const Cand bf16_cands[] = {{16, 1.00f}, {18, 1.27f}, {17, 1.26f}, {11, 0.94f}, {10, 1.19f},
                                    {23, 0.90f}, {13, 0.75f}, {12, 0.75f}, {25, 1.33f}, {24, 0.99f},
                                    {26, 0.82f}, {27, 0.87f}, {28, 0.91f}};
  // (33 is 31 with waves of 256 x 32, so every int4 weight is dequantised once per
  // workgroup instead of twice: 419 us against 447 us on the W4A16 ragged batch)
  static const Cand int4_cands[] = {{33, 1.07f}, {31, 1.00f}, {30, 0.75f}, {32, 0.54f}};
  const Cand* cands = int4 ? int4_cands : bf16_cands;
  const int ncand = int(int4 ? sizeof(int4_cands) / sizeof(int4_cands[0]) : sizeof(bf16_cands) / sizeof(bf16_cands[0]));
  const int64_t cus = cus_ > 0 ? cus_ : 256;
  const TileVariant* best = find_variant(1);
  float best_score = -1.f;
  for (int i = 0; i < ncand; ++i) {
    const TileVariant* v = find_variant(cands[i].id);
    if (!v || n_tiles % v->hpt != 0 || !supports(*v, int4) || (is_pair_variant(v->id) && !pair_fits(*v))) continue;
    const int64_t tiles = tile_count(*v, M, n_tiles);
    if (v->bm == 128 && is_pair_variant(v->id) && 2 * tiles <= cus) continue;  // (measured from half a round up)
    if (v->bm == 192 && (8 * tiles <= 7 * cus || tiles > cus)) continue;       // (and 28 in most of one round)
    const int64_t rounds = (tiles + cus - 1) / cus;
    const float util = float(tiles) / float(rounds * cus);
    // rows past M in the last row tile are wasted work
    const float fill = float(M) / float(((M + v->bm - 1) / v->bm) * v->bm);
    const float score = cands[i].speed * util * fill;
    if (score > best_score) {
      best_score = score;
      best = v;
    }
  }
  return best;
}

hipError_t launch_tile(const TileVariant& v, int int4, const ProblemArgs& p, const WeightArgs& w,
                       const EpilogueArgs& e, int group_m, hipStream_t stream) {
  if (v.id >= 30) return int4 ? launch_tile_dma_w4(v.id, p, w, e, group_m, stream) : hipErrorInvalidValue;
  if (v.id >= 10) return int4 ? hipErrorInvalidValue : launch_tile_dma(v.id, p, w, e, group_m, stream);
  switch (v.id) {
    case 1: return launch_dispatch<128, 1, 2>(int4, p, w, e, group_m, stream);
    case 2: return launch_dispatch<256, 1, 1>(int4, p, w, e, group_m, stream);
    case 3: return launch_dispatch<128, 2, 1>(int4, p, w, e, group_m, stream);
    case 4: return launch_dispatch<256, 2, 1>(int4, p, w, e, group_m, stream);
    case 5: return launch_dispatch<128, 2, 2>(int4, p, w, e, group_m, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mqk
