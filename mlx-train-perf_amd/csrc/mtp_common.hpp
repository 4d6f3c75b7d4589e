// Shared CDNA4 (gfx950) building blocks for the mlx-train-perf hot-path kernels.
//
// Conventions used by every kernel in this library:
//  * bf16 operands, fp32 accumulation, v_mfma_f32_32x32x16_bf16 tiles.
//  * MFMA 32x32x16 lane layout (wave64): lane l supplies A[i = l%32][k = 8*(l/32) .. +7] and
//    B[k = 8*(l/32) .. +7][j = l%32]; the 16 fp32 results of lane l are
//    C[i = 8*(r/4) + 4*(l/32) + r%4][j = l%32] for r = 0..15.
//  * LDS operand tiles are stored row-major with 64 bf16 (128 bytes, eight 16-byte chunks) per
//    row; chunk c of row r lives at chunk slot c ^ swz(r), swz(r) = (r ^ (r >> 3)) & 7, which
//    keeps both the MFMA fragment reads (8 consecutive rows, same chunk) and the transposing
//    writes (rows 8 apart, same chunk) free of bank conflicts.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mtp {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t bf16_t;  // storage type for bf16 in global memory

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_to_f32(bf16_t v) { return __uint_as_float(((uint32_t)v) << 16); }
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }

// Byte offset of 16-byte chunk c of row `row` in a 128-byte-per-row swizzled LDS tile.
__device__ __forceinline__ int lds_off(int row, int c) { return row * 128 + ((c ^ swz(row)) << 4); }

__device__ __forceinline__ u32x4 lds_read16(const char* lds, int off) {
  return *reinterpret_cast<const u32x4*>(lds + off);
}
__device__ __forceinline__ void lds_write16(char* lds, int off, const u32x4& v) {
  *reinterpret_cast<u32x4*>(lds + off) = v;
}

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

// 8x8 transpose of bf16: in x[i] halfword j -> out y[j] halfword i.
__device__ __forceinline__ void transpose8x8(const u32x4 (&x)[8], u32x4 (&y)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // result = (lo16: x[2p].h[j], hi16: x[2p+1].h[j])
      y[j][p] = __builtin_amdgcn_perm(x[2 * p + 1][j >> 1], x[2 * p][j >> 1], sel);
    }
  }
}

// Dequantize one packed word (8 four-bit values, low nibble first) with an affine
// scale/bias into 8 bf16 values (w = scale * q + bias, computed in fp32).
// The even nibbles are spread into the bytes of one word and the odd ones into another, so each
// value converts with a single byte-to-float (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ u32x4 dequant8(uint32_t q, float s, float b) {
  uint32_t ev = q & 0x0F0F0F0Fu, od = (q >> 4) & 0x0F0F0F0Fu;
  // Hide the masks from the compiler, which would otherwise narrow each conversion to a 4-bit
  // field extract plus a byte-0 conversion (two instructions instead of one).
  asm("" : "+v"(ev), "+v"(od));
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float lo = __builtin_fmaf(s, (float)((ev >> (8 * p)) & 0xFFu), b);
    const float hi = __builtin_fmaf(s, (float)((od >> (8 * p)) & 0xFFu), b);
    r[p] = pack_bf16x2(lo, hi);
  }
  return r;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Merge two (max, sum-of-exp2) partials in the log2 domain; -inf maxima are handled so that an
// empty partial contributes nothing and two empty partials stay empty (no NaN).
__device__ __forceinline__ void lse2_merge(float& m, float& s, float mo, float so) {
  const float mn = fmaxf(m, mo);
  const float base = (mn == kNegInf) ? 0.f : mn;
  s = s * fast_exp2(m - base) + so * fast_exp2(mo - base);
  m = mn;
}

}  // namespace mtp
