// Stage 1: BLOCK_M = 64 block pooling of Q/K/V (HBM streaming).
//
// Reference: editing_sparse_attention.py:89-111 (pad + block mean, compress_seq :37-55) and
// the block-sum kernels tilelang_kernels.py:33-120 / triton_kernels.py:16-119.
//
// One workgroup per (b*h, 64-token block), heads fastest.  Each input is read exactly once:
//   * fp32 block sums        -> sums[i]  [B, H, NB, D]   (means = sums / block size)
//   * optional bf16 copy     -> xb[i]    same strides as a contiguous [B, S, H, D]
//   * optional V transposed  -> vt       [B, H, D, Sp] bf16, kv_slot() order, zero padded;
//     with vt_limit only blocks n < vt_nblk (the pipeline's target blocks), and
//     icsa_vt_blocks_kernel transposes a list of further blocks (the selected source
//     blocks) once the selection is known
// Token rows at or beyond S read as zeros, so the partial last block sums only real tokens
// and the transposed copy is zero for padding tokens.
#include "icsa_kernels.h"

// Raw storage of 8 consecutive elements of one row (one thread's share of a 64-token row).
template <typename T> struct Raw8;
template <> struct Raw8<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (bf16)0.f;
  }
  __device__ __forceinline__ void to_f32(float o[8]) const {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (float)v[e];
  }
};
template <> struct Raw8<float> {
  floatx4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = *reinterpret_cast<const floatx4*>(p);
    b = *reinterpret_cast<const floatx4*>(p + 4);
  }
  __device__ __forceinline__ void zero() { a = floatx4{0.f, 0.f, 0.f, 0.f}; b = a; }
  __device__ __forceinline__ void to_f32(float o[8]) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) { o[e] = a[e]; o[4 + e] = b[e]; }
  }
};

// Thread t covers chunk c = t % 16 (8 of the 128 dims) of rows g + 16 j, g = t / 16.
template <typename T>
__device__ __forceinline__ void pool_load(const PoolParams& p, int i, int n, int b, int h, Raw8<T> (&r)[4]) {
  const int t = threadIdx.x;
  const int c = t & 15, g = t >> 4;
  const T* base = reinterpret_cast<const T*>(p.x[i].p) + (int64_t)b * p.x[i].sb + (int64_t)h * p.x[i].sh;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tok = n * ICSA_BLOCK + g + 16 * j;
    if (tok < p.S) r[j].load(base + (int64_t)tok * p.x[i].ss + 8 * c);
    else r[j].zero();
  }
}

// V^T of block n from the staged rows vtile[token][d]: thread -> (d, half), 32 consecutive
// slots of V^T row d, in kv_slot order
__device__ __forceinline__ void vt_store(const PoolParams& p, int n, int b, int h,
                                         const bf16 (*vtile)[ICSA_D + 8]) {
  const int t = threadIdx.x;
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

template <typename T>
__device__ __forceinline__ void pool_one(const PoolParams& p, int i, int n, int b, int h, const Raw8<T> (&rows)[4],
                                         float (*red)[ICSA_D + 4], bf16 (*vtile)[ICSA_D + 8]) {
  const int t = threadIdx.x;
  const int c = t & 15;          // 16 chunks of 8 elements across D = 128
  const int g = t >> 4;          // 16 row groups, 4 rows each
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  const bool want_copy = p.xb[i] != nullptr;
  const bool want_vt = (p.vt != nullptr) && (i == p.vt_src) && !(p.vt_limit && n >= p.vt_nblk);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = g + 16 * j;
    const int tok = n * ICSA_BLOCK + r;
    float v[8];
    rows[j].to_f32(v);           // rows past S were loaded as zeros
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
  if (want_vt) vt_store(p, n, b, h, vtile);
  __syncthreads();
}

template <typename T0, typename T1, typename T2>
__global__ void __launch_bounds__(256) icsa_pool_kernel(PoolParams p) {
  __shared__ float red[16][ICSA_D + 4];
  __shared__ bf16 vtile[ICSA_BLOCK][ICSA_D + 8];
  const int bh = blockIdx.x;          // heads fastest: neighbouring workgroups read adjacent
  const int n = blockIdx.y;           // 256-byte head rows of the same tokens
  const int b = bh / p.H, h = bh % p.H;
  // every present input's rows are requested before any is reduced
  Raw8<T0> r0[4];
  Raw8<T1> r1[4];
  Raw8<T2> r2[4];
  if (p.x[0].p) pool_load<T0>(p, 0, n, b, h, r0);
  if (p.x[1].p) pool_load<T1>(p, 1, n, b, h, r1);
  if (p.x[2].p) pool_load<T2>(p, 2, n, b, h, r2);
  if (p.x[0].p) pool_one<T0>(p, 0, n, b, h, r0, red, vtile);
  if (p.x[1].p) pool_one<T1>(p, 1, n, b, h, r1, red, vtile);
  if (p.x[2].p) pool_one<T2>(p, 2, n, b, h, r2, red, vtile);
}

// Host launcher: dtypes select the instantiation (bf16 / fp32 per input).
hipError_t launch_pool(const PoolParams& p, hipStream_t stream) {
  dim3 grid(p.B * p.H, p.NB);
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

// V^T of listed blocks: one workgroup per (b*h, list entry r), stored as V^T block dst0 + r
// (an entry outside [0, NB) stores a zero block, so no column keeps stale workspace data)
template <typename T>
__global__ void __launch_bounds__(256) icsa_vt_blocks_kernel(PoolParams p, const int* list, int base,
                                                             int stride, int dst0) {
  __shared__ bf16 vtile[ICSA_BLOCK][ICSA_D + 8];
  const int bh = blockIdx.x, r = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int n = base + list[(int64_t)bh * stride + r];
  const bool real = n >= 0 && n < p.NB;            // uniform for the workgroup
  Raw8<T> rows[4];
  if (real) {
    pool_load<T>(p, p.vt_src, n, b, h, rows);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) rows[j].zero();
  }
  const int c = threadIdx.x & 15, g = threadIdx.x >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v[8];
    rows[j].to_f32(v);
    *reinterpret_cast<bf16x8*>(&vtile[g + 16 * j][8 * c]) = pack8_bf16(v);
  }
  __syncthreads();
  vt_store(p, dst0 + r, b, h, vtile);
}

hipError_t launch_vt_blocks(const PoolParams& p, const int* list, int base, int stride, int n,
                            int dst0, hipStream_t stream) {
  if (n <= 0 || p.B * p.H == 0) return hipSuccess;
  if (!p.vt || !p.x[p.vt_src].p) return hipErrorInvalidValue;
  dim3 grid(p.B * p.H, n);
  if (p.x[p.vt_src].dtype == ICSA_DT_F32)
    hipLaunchKernelGGL(icsa_vt_blocks_kernel<float>, grid, dim3(256), 0, stream, p, list, base, stride, dst0);
  else
    hipLaunchKernelGGL(icsa_vt_blocks_kernel<bf16>, grid, dim3(256), 0, stream, p, list, base, stride, dst0);
  return hipGetLastError();
}
