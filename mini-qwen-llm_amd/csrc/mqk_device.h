// Device-side building blocks shared by the mqk kernels (gfx950 / CDNA4).
//
// Conventions used throughout:
//   * bf16 tensors travel as uint16_t bit patterns; widening to fp32 is exact,
//     narrowing is round-to-nearest-even (the gfx950 v_cvt_pk_bf16_f32 path).
//   * MFMA operands are 8 bf16 values per lane packed in a u32x4.  Because the
//     projection is a sum over k, the hardware's assignment of k-slots to lanes
//     only has to be the same for the A (activation) and B (weight) operand of
//     one instruction; the kernels use that freedom to pick load-friendly k
//     orders.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mqk {

// The kernels tile the projection in 128-column blocks.  With head_dim 128 (every
// Qwen3 checkpoint) a block is one head; with head_dim 64 (the reference's
// default Qwen3Config) it is two heads, and the epilogues normalise and rotate
// each 64-column half on its own (pair_runs, head_sum, head_rms).
constexpr int kHeadDim = 128;   // columns of one block (one head of 128, or two of 64)
constexpr int kHalfDim = 64;
constexpr int kBK = 64;         // K extent of one staged tile (8 chunks of 16 bytes per row)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two floats -> packed bf16x2 (low half = a).
// Two floats -> two bf16 (round to nearest even) in one 32-bit word, low half first;
// one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  typedef float f32x2_v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_v){a, b}, bf16x2_v));
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// C[32x32] += A[32x16] * B[16x32]; lane l holds A row (l & 31), B column (l & 31),
// and k-slots 8*(l >> 5) .. +8 of each.  Output: acc[i] = C[8*(i/4) + 4*(l>>5) + i%4][l & 31].
__device__ __forceinline__ f32x16_t mfma_32x32x16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// C[16x16] += A[16x32] * B[32x16]; lane l holds A row (l & 15), B column (l & 15),
// k-slots 8*(l >> 4) .. +8.  Output: acc[j] = C[4*(l>>4) + j][l & 15].
__device__ __forceinline__ f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Dequantize one packed int32 (8 consecutive k of one output column) to 8 bf16:
// w = (q - z) * s, exact in fp32 (|q - z| <= 15 times an 8/11-bit mantissa),
// then one rounding to bf16.  Nibble e holds k = 8j + e (little-endian nibbles).
__device__ __forceinline__ u32x4_t dequant_int4x8(uint32_t packed, float zero, float scale) {
  // (q - z) * s with q, z in 0..15 and a 16-bit (bf16 / fp16) scale: q*s and z*s
  // have at most 15 significant bits, so fma(q, s, -z*s) is exact in fp32 and
  // equals (q - z) * s bit for bit; the nibbles are split into bytes so each
  // converts with one byte-to-float instruction.
  const float zs = zero * scale;
  const uint32_t even = packed & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6
  const uint32_t odd = (packed >> 4) & 0x0F0F0F0Fu;   // nibbles 1, 3, 5, 7
  float w[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    w[2 * b] = __builtin_fmaf(static_cast<float>((even >> (8 * b)) & 0xFFu), scale, -zs);
    w[2 * b + 1] = __builtin_fmaf(static_cast<float>((odd >> (8 * b)) & 0xFFu), scale, -zs);
  }
  u32x4_t r;
  r.x = pack_bf16x2(w[0], w[1]);
  r.y = pack_bf16x2(w[2], w[3]);
  r.z = pack_bf16x2(w[4], w[5]);
  r.w = pack_bf16x2(w[6], w[7]);
  return r;
}

// Varlen mode: sequence s of token t (cu_seqlens[s] <= t < cu_seqlens[s+1]) by
// binary search over the n_seqs + 1 offsets, and its position t - cu_seqlens[s]
// (+ seq_pos0[s]) -- the batch_ids / positions of paged_attn_prefill.py:188-199.
// Only offsets 0..n_seqs are read, whatever their values.
template <class E>
__device__ __forceinline__ void varlen_locate(const E& e, int64_t t, int64_t& seq, int64_t& pos) {
  int64_t lo = 0, hi = e.n_seqs;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (int64_t(e.cu_seqlens[mid]) <= t) lo = mid;
    else hi = mid;
  }
  seq = lo;
  pos = t - int64_t(e.cu_seqlens[lo]) + (e.seq_pos0 ? int64_t(e.seq_pos0[lo]) : 0);
}

// The decoder's input RMSNorm applied to 8 activations of one token
// (mini_qwen/model/layers/rms_norm.py:15-18): bf16(gamma * bf16(x * scale)) with
// scale = rsqrt(mean(x^2) + eps) of the token, i.e. the product is rounded to bf16
// before the gamma multiply, which is rounded again -- the bf16 operand the
// reference's projection reads.
__device__ __forceinline__ u32x4_t input_norm8(const u32x4_t& xv, float scale, const u32x4_t& gv) {
  u32x4_t r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t xw = xv[j], gw = gv[j];
    const uint32_t y = pack_bf16x2(bf16_to_f32(xw & 0xFFFFu) * scale, bf16_to_f32(xw >> 16) * scale);
    r[j] = pack_bf16x2(bf16_to_f32(y & 0xFFFFu) * bf16_to_f32(gw & 0xFFFFu),
                       bf16_to_f32(y >> 16) * bf16_to_f32(gw >> 16));
  }
  return r;
}

// Row of the RoPE table used by token t, clamped into [0, rows): prefill t % S
// (reference fused_qkv_rope.py:109), positions[t] (:107), or the varlen position.
template <class E>
__device__ __forceinline__ int64_t rope_row(const E& e, int64_t t) {
  t += e.t0;  // the launch's first row is token t0 of the call
  int64_t p;
  if (e.cu_seqlens) {
    int64_t s;
    varlen_locate(e, t, s, p);
  } else {
    p = e.positions ? static_cast<int64_t>(e.positions[t]) : (t % e.S);
  }
  p = p < 0 ? 0 : p;
  return p >= e.cos_rows ? e.cos_rows - 1 : p;
}

// Slot of token t in the paged KV cache (mini_qwen/kernels/paged_attn_prefill.py:45-50:
// page = pos / block_size, slot = pos % block_size, block = block_table[seq][page]),
// as block * block_size + slot, or -1 when there is no cache or the token's entry
// is out of range (such rows are not written rather than written out of bounds).
template <class E>
__device__ __forceinline__ int64_t paged_slot(const E& e, int64_t t) {
  if (!e.k_cache) return -1;
  t += e.t0;
  int64_t seq, pos;
  if (e.cu_seqlens && !(e.kv_seq && e.kv_pos)) {
    varlen_locate(e, t, seq, pos);
    if (e.kv_seq) seq = int64_t(e.kv_seq[t]);
    if (e.kv_pos) pos = int64_t(e.kv_pos[t]);
  } else {
    seq = e.kv_seq ? int64_t(e.kv_seq[t]) : t / e.kv_len;
    pos = e.kv_pos ? int64_t(e.kv_pos[t]) : t % e.kv_len;
  }
  if (seq < 0 || seq >= e.bt_rows || pos < 0) return -1;
  const int64_t page = pos / e.block_size;
  if (page >= e.bt_cols) return -1;
  const int64_t blk = e.block_table[seq * e.bt_cols + page];
  if (blk < 0 || blk >= e.num_blocks) return -1;
  return blk * e.block_size + pos % e.block_size;
}

// Cache row of head hh of projection proj (1 = K, 2 = V) for a slot from paged_slot.
template <class E>
__device__ __forceinline__ uint16_t* paged_row(const E& e, int64_t slot, int proj, int hh) {
  // arithmetic select of the two pointer values: a select of the two argument
  // fields' addresses would make the compiler copy them to scratch memory
  const uintptr_t kc = reinterpret_cast<uintptr_t>(e.k_cache), vc = reinterpret_cast<uintptr_t>(e.v_cache);
  uint16_t* const cache = reinterpret_cast<uint16_t*>(vc + (kc - vc) * uintptr_t(proj == 1));
  return cache + (slot * e.Hkv + hh) * kHeadDim;
}

// Element i (0, 1, 2) of three pointer values, selected arithmetically: a
// select between kernel-argument fields makes the compiler copy the whole
// argument struct to scratch memory to address the chosen field.
template <class T>
__device__ __forceinline__ T* pick3(int i, T* a, T* b, T* c) {
  const uintptr_t ua = reinterpret_cast<uintptr_t>(a), ub = reinterpret_cast<uintptr_t>(b),
                  uc = reinterpret_cast<uintptr_t>(c);
  return reinterpret_cast<T*>(ua * uintptr_t(i == 0) + ub * uintptr_t(i == 1) + uc * uintptr_t(i == 2));
}

// Which projection a 128-column tile belongs to: 0 = Q, 1 = K, 2 = V, and the
// tile's head index inside that projection.
__device__ __forceinline__ void split_head(int h, int Hq, int Hkv, int& proj, int& hh) {
  if (h < Hq) { proj = 0; hh = h; }
  else if (h < Hq + Hkv) { proj = 1; hh = h - Hq; }
  else { proj = 2; hh = h - Hq - Hkv; }
}

// Maps a linear workgroup id onto a tile id so that consecutive tile ids land on
// the same XCD (workgroups are dispatched round-robin over the device's XCDs,
// and each XCD has its own L2).
__device__ __forceinline__ int xcd_tile_id(int bid, int nblocks, int xcds) {
  if (xcds <= 1 || nblocks % xcds != 0) return bid;
  return (bid % xcds) * (nblocks / xcds) + bid / xcds;
}

// ---------------------------------------------------------------------------
// Direct L2 -> LDS loads and explicit waits (inline asm; see the kernels that use them)
// ---------------------------------------------------------------------------

// L2 -> LDS: this lane's 16 bytes at gptr go to LDS byte lds_base + 16 * lane
// (lds_base wave-uniform).  M0 carries the LDS base; it is saved and restored
// around the load because the compiler reserves it.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(gptr)
      : "memory");
}

// L2 -> LDS, 4 bytes per lane: this lane's word at gptr goes to LDS byte
// lds_base + 4 * lane (lds_base wave-uniform).
__device__ __forceinline__ void dma4(const void* gptr, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dword %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(gptr)
      : "memory");
}

// dma16 of the 16 bytes at gptr + OFF bytes (OFF an immediate of the instruction,
// 0 <= OFF < 4096), so a run of loads at fixed distances shares one address.  The
// instruction offset moves the LDS destination as well (M0 + offset + 16 * lane),
// so M0 is set to lds_base - OFF.
template <int OFF>
__device__ __forceinline__ void dma16_at(const void* gptr, uint32_t lds_base) {
  static_assert(OFF >= 0 && OFF < 4096, "global instruction offset");
  lds_base -= uint32_t(OFF);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, off offset:%3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(__builtin_amdgcn_readfirstlane(lds_base)), "v"(gptr), "n"(OFF)
      : "memory");
}

// Wait until at most n of this wave's vector-memory operations are pending.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait_vm with a count known only after unrolling (folds to one s_waitcnt when
// n is a constant; counts above 62 wait for nothing older than 63 operations).
__device__ __forceinline__ void wait_vm_n(int n) {
  switch (n) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<1>(); break;
    case 2: wait_vm<2>(); break;
    case 3: wait_vm<3>(); break;
    case 4: wait_vm<4>(); break;
    case 5: wait_vm<5>(); break;
    case 6: wait_vm<6>(); break;
    case 7: wait_vm<7>(); break;
    case 8: wait_vm<8>(); break;
    case 9: wait_vm<9>(); break;
    case 10: wait_vm<10>(); break;
    case 11: wait_vm<11>(); break;
    case 12: wait_vm<12>(); break;
    case 13: wait_vm<13>(); break;
    case 14: wait_vm<14>(); break;
    case 15: wait_vm<15>(); break;
    case 16: wait_vm<16>(); break;
    case 17: wait_vm<17>(); break;
    case 18: wait_vm<18>(); break;
    case 19: wait_vm<19>(); break;
    case 20: wait_vm<20>(); break;
    case 21: wait_vm<21>(); break;
    case 22: wait_vm<22>(); break;
    case 23: wait_vm<23>(); break;
    case 24: wait_vm<24>(); break;
    case 25: wait_vm<25>(); break;
    case 26: wait_vm<26>(); break;
    case 27: wait_vm<27>(); break;
    case 28: wait_vm<28>(); break;
    case 29: wait_vm<29>(); break;
    case 30: wait_vm<30>(); break;
    case 31: wait_vm<31>(); break;
    case 32: wait_vm<32>(); break;
    case 33: wait_vm<33>(); break;
    case 34: wait_vm<34>(); break;
    case 35: wait_vm<35>(); break;
    case 36: wait_vm<36>(); break;
    case 37: wait_vm<37>(); break;
    case 38: wait_vm<38>(); break;
    case 39: wait_vm<39>(); break;
    case 40: wait_vm<40>(); break;
    case 41: wait_vm<41>(); break;
    case 42: wait_vm<42>(); break;
    case 43: wait_vm<43>(); break;
    case 44: wait_vm<44>(); break;
    case 45: wait_vm<45>(); break;
    case 46: wait_vm<46>(); break;
    case 47: wait_vm<47>(); break;
    case 48: wait_vm<48>(); break;
    case 49: wait_vm<49>(); break;
    case 50: wait_vm<50>(); break;
    case 51: wait_vm<51>(); break;
    case 52: wait_vm<52>(); break;
    case 53: wait_vm<53>(); break;
    case 54: wait_vm<54>(); break;
    case 55: wait_vm<55>(); break;
    case 56: wait_vm<56>(); break;
    case 57: wait_vm<57>(); break;
    case 58: wait_vm<58>(); break;
    case 59: wait_vm<59>(); break;
    case 60: wait_vm<60>(); break;
    case 61: wait_vm<61>(); break;
    case 62: wait_vm<62>(); break;
    default: wait_vm<63>(); break;
  }
}

// Sum over each aligned group of 8 lanes, returned to all 8, with DPP lane
// moves (no LDS round trip): the xor-1 and xor-2 butterflies as quad
// permutations, then the other quad of the group via the half-row mirror.
// Every lane adds the same pairs as the xor-1/2/4 butterfly, so the result is
// the same bit for bit.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum8_lanes(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror: lane i <-> 7 - i within 8
  return v;
}

// The two runs of 8 columns that thread c (0..7) of a block row takes in the
// norm / RoPE epilogues, chosen so that column d of the first run and column
// d + D/2 of the second are a RoPE pair of one head, and the 8 (D = 128) or 4
// (D = 64) threads sharing a head are an aligned lane group:
//   D = 128: columns [8c, 8c+8) and [64+8c, +8); dims the same.
//   D = 64:  head h = c / 4 of the block, j = c % 4: columns 64h + [8j, +8) and
//            64h + 32 + [8j, +8); dims [8j, +8) and [32+8j, +8) of head h.
struct PairRuns {
  int col_lo, col_hi;  // column of the runs' first element within the 128-column block
  int dim_lo, dim_hi;  // head dim of the same (indexes gamma and the cos / sin rows)
};
__device__ __forceinline__ PairRuns pair_runs(int c, int head_dim) {
  if (head_dim == 64) {
    const int h = c >> 2, j = c & 3;
    return PairRuns{64 * h + 8 * j, 64 * h + 32 + 8 * j, 8 * j, 32 + 8 * j};
  }
  return PairRuns{8 * c, kHalfDim + 8 * c, 8 * c, kHalfDim + 8 * c};
}

// Sum over the lanes that hold one head's runs (pair_runs): the aligned group of
// 8 lanes for head_dim 128 (bit for bit sum8_lanes), of 4 lanes for head_dim 64.
__device__ __forceinline__ float head_sum(float v, int head_dim) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  if (head_dim != 64) v += dpp_move<0x141>(v);  // row_half_mirror: the other quad
  return v;
}

// Epilogue arithmetic with every rounding step written out (no contraction left
// to the compiler), so that each tile shape's instantiation gives identical bits
// for the same accumulators however the compiler schedules it.
//
// Sum of squares of one thread's 16 head dims d = 8c+i and 64+8c+i (i = 0..7).
__device__ __forceinline__ float run_sumsq(const float (&lo)[8], const float (&hi)[8]) {
#pragma clang fp contract(off)
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = ss + __builtin_fmaf(lo[i], lo[i], hi[i] * hi[i]);
  return ss;
}

// 1 / rms of a head from the sum of squares of its head_dim (128 or 64) dims.
__device__ __forceinline__ float head_rms(float ss, float eps, int head_dim = kHeadDim) {
#pragma clang fp contract(off)
  return rsqrtf(__builtin_fmaf(ss, head_dim == 64 ? 1.0f / 64.0f : 1.0f / float(kHeadDim), eps));
}

__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

}  // namespace mqk
