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

constexpr int kHeadDim = 128;   // head_dim handled by the kernels (all Qwen3 models)
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
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return uint32_t(f32_to_bf16(a)) | (uint32_t(f32_to_bf16(b)) << 16);
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
  float w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float q = static_cast<float>((packed >> (4 * e)) & 0xFu);
    w[e] = (q - zero) * scale;
  }
  u32x4_t r;
  r.x = pack_bf16x2(w[0], w[1]);
  r.y = pack_bf16x2(w[2], w[3]);
  r.z = pack_bf16x2(w[4], w[5]);
  r.w = pack_bf16x2(w[6], w[7]);
  return r;
}

// Row of the RoPE table used by token t (reference fused_qkv_rope.py:106-111),
// clamped into [0, rows).
__device__ __forceinline__ int64_t rope_row(const int32_t* __restrict__ positions, int64_t t,
                                            int64_t S, int64_t rows) {
  int64_t p = positions ? static_cast<int64_t>(positions[t]) : (t % S);
  p = p < 0 ? 0 : p;
  return p >= rows ? rows - 1 : p;
}

// Which projection a 128-column tile belongs to: 0 = Q, 1 = K, 2 = V, and the
// tile's head index inside that projection.
__device__ __forceinline__ void split_head(int h, int Hq, int Hkv, int& proj, int& hh) {
  if (h < Hq) { proj = 0; hh = h; }
  else if (h < Hq + Hkv) { proj = 1; hh = h - Hq; }
  else { proj = 2; hh = h - Hq - Hkv; }
}

// Maps a linear workgroup id onto a tile id so that consecutive tile ids land on
// the same XCD (workgroups are dispatched round-robin over the 8 XCDs, and
// each XCD has its own L2).
__device__ __forceinline__ int xcd_tile_id(int bid, int nblocks) {
  if ((nblocks & 7) != 0) return bid;
  return (bid & 7) * (nblocks >> 3) + (bid >> 3);
}

}  // namespace mqk
