// Residual / LayerNorm / adaLN glue of the Wan DiT block around the attention path.
//
// Reference: WanAttentionBlock.forward, model.py:249-270, with WanLayerNorm (model.py:117-122):
//   y = self_attn(norm1(x).float() * (1 + e[1]) + e[0], ...)        norm1: no affine
//   x = x + y * e[2]
//   x = x + cross_attn(norm3(x), context, context_lens)            norm3: affine (weight, bias)
//   y = ffn(norm2(x).float() * (1 + e[4]) + e[3])
//   x = x + y * e[5]
// Every "x + y * g" followed by a LayerNorm is one pass here: one workgroup per token row
// keeps the fp32 row in registers, applies the gated residual update (written back to x),
// the LayerNorm (mean, then the variance of the centred row: two passes over registers),
// the optional affine and modulation, and writes the bf16 row the next GEMM reads (the
// model's autocast casts the fp32 result to bf16 at the Linear).
#include "icsa_kernels.h"

#define LNM_THREADS 256
#define LNM_MAX_PER_THREAD 24           // dim <= 256 * 24 = 6144 (Wan 14B: 5120)

__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();                                      // red reused across calls
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];             // fixed order
}

template <typename TX>
__global__ void __launch_bounds__(LNM_THREADS) icsa_wan_ln_mod_kernel(LnModParams p) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;                       // b * S + s
  const int b = (int)(row / p.S), s = (int)(row % p.S);
  const int t = threadIdx.x;
  const int nv = p.dim / 4;                             // float4 / 4-element groups per row
  const TX* xr = reinterpret_cast<const TX*>(p.x) + (int64_t)b * p.x_sb + (int64_t)s * p.x_ss;
  float v[LNM_MAX_PER_THREAD];
#pragma unroll
  for (int j = 0; j < LNM_MAX_PER_THREAD / 4; ++j) {
    const int c = t + j * LNM_THREADS;                  // 4-element group index
    if (c < nv) {
      if constexpr (sizeof(TX) == 4) {
        const floatx4 a = *reinterpret_cast<const floatx4*>(xr + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * j + e] = a[e];
      } else {
        const bf16x4 a = *reinterpret_cast<const bf16x4*>(xr + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * j + e] = (float)a[e];
      }
      if (p.y != nullptr) {                             // x = x + y * gate
        const bf16x4 yy = *reinterpret_cast<const bf16x4*>(p.y + (int64_t)b * p.y_sb + (int64_t)s * p.y_ss + 4 * c);
        const floatx4 g = *reinterpret_cast<const floatx4*>(p.gate + (int64_t)b * p.g_sb + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * j + e] = fmaf((float)yy[e], g[e], v[4 * j + e]);
        if (p.x_out != nullptr)
          *reinterpret_cast<floatx4*>(p.x_out + (int64_t)b * p.xo_sb + (int64_t)s * p.xo_ss + 4 * c) =
              floatx4{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
      }
    }
  }
  if (p.out == nullptr) return;                         // residual update only
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < LNM_MAX_PER_THREAD / 4; ++j)
    if (t + j * LNM_THREADS < nv)
#pragma unroll
      for (int e = 0; e < 4; ++e) sum += v[4 * j + e];
  const float mean = block_sum_256(sum, red) / (float)p.dim;
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < LNM_MAX_PER_THREAD / 4; ++j)
    if (t + j * LNM_THREADS < nv)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = v[4 * j + e] - mean;
        sq = fmaf(d, d, sq);
      }
  const float var = block_sum_256(sq, red) / (float)p.dim;
  const float rstd = 1.f / sqrtf(var + p.eps);
#pragma unroll
  for (int j = 0; j < LNM_MAX_PER_THREAD / 4; ++j) {
    const int c = t + j * LNM_THREADS;
    if (c >= nv) continue;
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (v[4 * j + e] - mean) * rstd;
    if (p.lw != nullptr) {                              // elementwise affine (norm3)
      const floatx4 w = *reinterpret_cast<const floatx4*>(p.lw + 4 * c);
      const floatx4 bb = *reinterpret_cast<const floatx4*>(p.lb + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = fmaf(o[e], w[e], bb[e]);
    }
    if constexpr (sizeof(TX) == 2) {                    // .type_as(x) of a bf16 x; after an
      if (p.y == nullptr) {                             // update x + y * gate is f32 (promotion)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (float)(bf16)o[e];
      }
    }
    if (p.scale != nullptr) {                           // * (1 + scale) + shift
      const floatx4 sc = *reinterpret_cast<const floatx4*>(p.scale + (int64_t)b * p.mod_sb + 4 * c);
      const floatx4 sh = *reinterpret_cast<const floatx4*>(p.shift + (int64_t)b * p.mod_sb + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = fmaf(o[e], 1.f + sc[e], sh[e]);
    }
    bf16x4 ob;
#pragma unroll
    for (int e = 0; e < 4; ++e) ob[e] = (bf16)o[e];
    *reinterpret_cast<bf16x4*>(p.out + (int64_t)b * p.o_sb + (int64_t)s * p.o_ss + 4 * c) = ob;
  }
}

hipError_t launch_ln_mod(const LnModParams& p, hipStream_t stream) {
  const int64_t rows = (int64_t)p.B * p.S;
  if (rows == 0) return hipSuccess;
  if (p.dim % 4 != 0 || p.dim > LNM_THREADS * LNM_MAX_PER_THREAD) return hipErrorInvalidValue;
  if (p.x_dtype == ICSA_DT_F32)
    hipLaunchKernelGGL(icsa_wan_ln_mod_kernel<float>, dim3((unsigned)rows), dim3(LNM_THREADS), 0, stream, p);
  else
    hipLaunchKernelGGL(icsa_wan_ln_mod_kernel<bf16>, dim3((unsigned)rows), dim3(LNM_THREADS), 0, stream, p);
  return hipGetLastError();
}
