// Shared device/host definitions of the in-context sparse attention (ICSA) library.
//
// Target: gfx950 (MI355X / CDNA4) only.  wave64, MFMA bf16 32x32x16 and f32 32x32x2.
//
// Layout conventions used by every kernel (element strides, innermost dim contiguous):
//   token tensors   [B, S, H, D]  addressed by (sb, ss, sh); d is contiguous.
//   Vt              [B, H, D, Sp] bf16, d-major ("V transposed"), token contiguous.
//                   Inside every 16-token group the token order is permuted by
//                   swapping bit 2 and bit 3 of the token index (kv_slot()).  That
//                   order makes the 8 keys one lane needs for the PV MFMA B/A operand
//                   contiguous (see flash_attn.hip).
//   block sums      [B, H, NB, D] fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define ICSA_D 128          // head dim supported by the MFMA kernels
#define ICSA_BLOCK 64       // BLOCK_M of the reference (tokens per block)

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

enum IcsaDtype { ICSA_DT_BF16 = 0, ICSA_DT_F32 = 1 };

// ---------------------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------------------

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 f2bf(float x) { return (bf16)x; }   // RNE (v_cvt_pk_bf16_f32)

// position of token `tok` inside its 16-token group of a Vt row (involution).
__host__ __device__ __forceinline__ int kv_slot(int tok) {
  return (tok & ~12) | ((tok & 4) << 1) | ((tok & 8) >> 1);
}

// Load 8 consecutive elements of a row as fp32 (bf16 or fp32 storage).
template <typename T>
__device__ __forceinline__ void load8_f32(const T* p, float out[8]);

template <>
__device__ __forceinline__ void load8_f32<bf16>(const bf16* p, float out[8]) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (float)v[i];
}

template <>
__device__ __forceinline__ void load8_f32<float>(const float* p, float out[8]) {
  floatx4 a = *reinterpret_cast<const floatx4*>(p);
  floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) { out[i] = a[i]; out[4 + i] = b[i]; }
}

__device__ __forceinline__ bf16x8 pack8_bf16(const float v[8]) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (bf16)v[i];
  return r;
}

// Partner-lane (lane ^ 32) combine helpers built on v_permlane32_swap.
// swap(x, x) returns {lo-half copy in upper lanes, hi-half copy in lower lanes}; taking
// both components covers {x[l], x[l^32]} in every lane.
__device__ __forceinline__ float xhalf_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

// Order-preserving map float -> uint32 (larger float -> larger key).  NaN-free inputs.
__device__ __forceinline__ uint32_t f2key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}

// XCD-aware work mapping.  Workgroups are dispatched round-robin over the 8 XCDs
// (wg i -> XCD i % 8).  Remap so each XCD walks one contiguous range of the work list:
// neighbouring work items (same head) then share that XCD's L2.  Returns -1 for padding.
__device__ __forceinline__ int xcd_remap(int wg, int n_work) {
  const int nx = 8;
  int per = (n_work + nx - 1) / nx;
  int w = (wg % nx) * per + wg / nx;
  return w < n_work ? w : -1;
}
__host__ __forceinline__ int xcd_grid(int n_work) { return ((n_work + 7) / 8) * 8; }

// MFMA wrappers (gfx950).  Operand/result layouts (checked on the device):
//  32x32x16 bf16: A lane l holds A[l%32][8*(l/32)+i], B lane l holds B[8*(l/32)+i][l%32],
//                 C lane l element i is C[(i/4)*8 + (l/32)*4 + i%4][l%32].
//  32x32x2 f32:   A lane l holds A[l%32][l/32],       B lane l holds B[l/32][l%32],
//                 C as above.
__device__ __forceinline__ floatx16 mfma32x32x16(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 mfma32x32x2f32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row (within a 32-row MFMA tile) held by accumulator element i of lane l.
__device__ __forceinline__ int acc_row(int i, int lane) {
  return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
}

// Row 32 sub + acc_row(i, lane) of a 64-row tile held as two 32x32 accumulators is at or
// past `limit` iff the lane-independent part 32 sub + 8 (i / 4) + i % 4 reaches the
// threshold mask_threshold(limit, lane).  Testing against that threshold compares each
// element with a compile-time constant: no per-element row values are kept in registers
// (which the compiler would otherwise rematerialise on every tile, mask or not).
__device__ __forceinline__ int mask_threshold(int limit, int lane) { return limit - (lane >> 5) * 4; }
__device__ __forceinline__ constexpr int acc_row_const(int sub, int i) { return 32 * sub + 8 * (i >> 2) + (i & 3); }

// ---------------------------------------------------------------------------------------
// kernel parameter blocks (passed by value)
// ---------------------------------------------------------------------------------------

struct TokTensor {        // [B, S, H, D] style strided view, element strides
  const void* p;
  int64_t sb, ss, sh;
  int dtype;
};

struct AlphaView {        // residual weight alpha_2, broadcast to [B, S, H, D]
  const void* p;          // nullptr -> scalar
  int64_t sb, ss, sh, sd;
  int dtype;
  float scalar;
};

struct OutView {
  void* p;
  int64_t sb, ss, sh;
  int dtype;
};
