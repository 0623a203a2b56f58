// Shared device helpers for the gfx950 (CDNA4) DSpark kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dspark {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int WAVE = 64;
constexpr int PAGE = 32;  // tokens per KV page (the reference's BlockTokens)

// D = A(16x32) * B(32x16) + C on the matrix cores. Lane l holds A row l%16 / B column l%16, k = 8*(l/16)+0..7;
// C/D: column l%16, rows 4*(l/16)+0..3.
__device__ __forceinline__ f32x4 mfma16x16x32(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8 as_half8(u32x4 u) {
  half8 h;
  __builtin_memcpy(&h, &u, 16);
  return h;
}

template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
  typedef __attribute__((address_space(1))) const T GT;
  return *(const GT*)p;
}

template <typename T>
__device__ __forceinline__ T ldg_nt(const T* p) {
  typedef __attribute__((address_space(1))) const T GT;
  return __builtin_nontemporal_load((const GT*)p);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt immediates (gfx9 encoding): vmcnt(n) with expcnt and lgkmcnt left at their maxima; lgkmcnt(0) alone.
__device__ __forceinline__ constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int LGKMCNT0_IMM = 0xC07F;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// quantize_pair (kernels/ops.hip:212-224) of a record's 128 values, one IEEE fp32 operation per step: the scale from
// the values' absolute maximum, and the int8 code of x with inv = 1 / scale.
__device__ __forceinline__ float rec_scale(float amax) { return fmaxf(__fdiv_rn(amax, 127.f), 1e-6f); }
__device__ __forceinline__ int rec_code(float x, float inv) {
  float a = __fmul_rn(x, inv);
  a = a >= 0.f ? __fadd_rn(a, 0.5f) : __fsub_rn(a, 0.5f);
  return (int)truncf(fminf(fmaxf(a, -128.f), 127.f));
}

// Argmax key (reference dspark.hip:967-971): ordered float bits above, 0xFFFFFFFF - index below. The maximum key is the
// largest value and, among equal values, the smallest index.
__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(0xffffffffu - idx);
}

// K/V page formats (one block of PAGE keys x D dims per (page, KV head)). K is stored in the operand order of
// v_mfma_f32_16x16x32_f16: key `slot` is row n = 4 (slot / 8) + slot % 4 of key block b = (slot / 4) % 2, and dim d sits
// in k-step d / 32 of lane n + 16 ((d % 32) / 8), element d % 8. V is stored transposed: [d][slot].
__device__ __forceinline__ int k_page_elem(int slot, int d, int D) {
  const int b = (slot >> 2) & 1, n = 4 * (slot >> 3) + (slot & 3);
  return ((b * (D / 32) + d / 32) * 64 + n + 16 * ((d % 32) / 8)) * 8 + d % 8;
}
__device__ __forceinline__ int v_page_elem(int slot, int d) { return d * PAGE + slot; }

// Activations a verify GEMM reads as X ([M][K] fp16, M <= 16 tbs) in the B-operand order of v_mfma_f32_16x16x32_f16:
// 1 KB blocks [K / 64 chunks][tbs token blocks][2 halves] of 64 lanes x 8 halves, lane 16 g + n holding token
// 16 tb + n, columns 64 c + 16 g + 8 h .. + 7. A wave's X operand load is then one contiguous 1 KB (row-major X
// gathers 64 bytes from each of 16 token rows). Four consecutive columns from a multiple of 4 stay contiguous.
__device__ __forceinline__ size_t xop_elem(int t, int k, int tbs) {
  return ((((size_t)(k >> 6) * tbs + (t >> 4)) * 2 + ((k >> 3) & 1)) * 64 + ((k >> 4) & 3) * 16 + (t & 15)) * 8 +
         (k & 7);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = shfl_xor_u64(v, o);
    v = w > v ? w : v;
  }
  return v;
}

}  // namespace dspark
