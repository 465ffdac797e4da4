// Stage 1: BLOCK_M = 64 block pooling of Q/K/V (HBM streaming).
//
// Reference: editing_sparse_attention.py:89-111 (pad + block mean, compress_seq :37-55) and
// the block-sum kernels tilelang_kernels.py:33-120 / triton_kernels.py:16-119.
//
// One workgroup per (64-token block, b*h).  Each of the three inputs is read exactly once:
//   * fp32 block sums        -> sums[i]  [B, H, NB, D]   (means = sums / block size)
//   * optional bf16 copy     -> xb[i]    same strides as a contiguous [B, S, H, D]
//   * optional V transposed  -> vt       [B, H, D, Sp] bf16, kv_slot() order, zero padded
// Token rows at or beyond S read as zeros, so the partial last block sums only real tokens
// and the transposed copy is zero for padding tokens.
#include "icsa_kernels.h"

template <typename T>
__device__ __forceinline__ void pool_one(const PoolParams& p, int i, int n, int b, int h,
                                         float (*red)[ICSA_D + 4], bf16 (*vtile)[ICSA_D + 8]) {
  const int t = threadIdx.x;
  const int c = t & 15;          // 16 chunks of 8 elements across D = 128
  const int g = t >> 4;          // 16 row groups, 4 rows each
  const T* base = reinterpret_cast<const T*>(p.x[i].p) + (int64_t)b * p.x[i].sb + (int64_t)h * p.x[i].sh;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  const bool want_copy = p.xb[i] != nullptr;
  const bool want_vt = (p.vt != nullptr) && (i == p.vt_src);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = g + 16 * j;
    const int tok = n * ICSA_BLOCK + r;
    float v[8];
    if (tok < p.S) {
      load8_f32<T>(base + (int64_t)tok * p.x[i].ss + 8 * c, v);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += v[e];
    if (want_copy && tok < p.S) {
      bf16* dst = p.xb[i] + (int64_t)b * p.xb_sb + (int64_t)tok * p.xb_ss + (int64_t)h * p.xb_sh + 8 * c;
      *reinterpret_cast<bf16x8*>(dst) = pack8_bf16(v);
    }
    if (want_vt) {
      *reinterpret_cast<bf16x8*>(&vtile[r][8 * c]) = pack8_bf16(v);
    }
  }
  if (p.sums[i] != nullptr) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[g][8 * c + e] = acc[e];
  }
  __syncthreads();
  if (p.sums[i] != nullptr && t < ICSA_D) {
    float s = 0.f;
#pragma unroll
    for (int gg = 0; gg < 16; ++gg) s += red[gg][t];      // fixed order: deterministic
    p.sums[i][(((int64_t)b * p.H + h) * p.NB + n) * ICSA_D + t] = s;
  }
  if (want_vt) {
    // thread -> (d, half): 32 consecutive slots of Vt row d for this block
    const int d = t >> 1;
    const int half = t & 1;
    bf16* dst = p.vt + (int64_t)b * p.vt_sb + (int64_t)h * p.vt_sh + (int64_t)d * p.vt_sd
                + (int64_t)n * ICSA_BLOCK + 32 * half;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int slot = 32 * half + 8 * q4 + e;
        o[e] = vtile[kv_slot(slot)][d];
      }
      *reinterpret_cast<bf16x8*>(dst + 8 * q4) = o;
    }
  }
  __syncthreads();
}

template <typename T0, typename T1, typename T2>
__global__ void __launch_bounds__(256) icsa_pool_kernel(PoolParams p) {
  __shared__ float red[16][ICSA_D + 4];
  __shared__ bf16 vtile[ICSA_BLOCK][ICSA_D + 8];
  const int n = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  if (p.x[0].p) pool_one<T0>(p, 0, n, b, h, red, vtile);
  if (p.x[1].p) pool_one<T1>(p, 1, n, b, h, red, vtile);
  if (p.x[2].p) pool_one<T2>(p, 2, n, b, h, red, vtile);
}

// Host launcher: dtypes select the instantiation (bf16 / fp32 per input).
hipError_t launch_pool(const PoolParams& p, hipStream_t stream) {
  dim3 grid(p.NB, p.B * p.H);
  dim3 block(256);
  const int d0 = p.x[0].p ? p.x[0].dtype : ICSA_DT_BF16;
  const int d1 = p.x[1].p ? p.x[1].dtype : ICSA_DT_BF16;
  const int d2 = p.x[2].p ? p.x[2].dtype : ICSA_DT_BF16;
  const int code = d0 * 4 + d1 * 2 + d2;
  switch (code) {
#define ICSA_POOL_CASE(C, A, B_, C_) \
    case C: hipLaunchKernelGGL((icsa_pool_kernel<A, B_, C_>), grid, block, 0, stream, p); break;
    ICSA_POOL_CASE(0, bf16, bf16, bf16)
    ICSA_POOL_CASE(1, bf16, bf16, float)
    ICSA_POOL_CASE(2, bf16, float, bf16)
    ICSA_POOL_CASE(3, bf16, float, float)
    ICSA_POOL_CASE(4, float, bf16, bf16)
    ICSA_POOL_CASE(5, float, bf16, float)
    ICSA_POOL_CASE(6, float, float, bf16)
    ICSA_POOL_CASE(7, float, float, float)
#undef ICSA_POOL_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
