// Stage 2: compressed (block-level) attention, per-head source retrieval, sharpness split,
// new-KV block sums and per-query-block (level-3) top-k selection.
//
// Reference:
//   editing_sparse_attention.py:58-64, 113-123  compressed attention + out_c residual
//   editing_sparse_attention.py:125-136          per-head source top-k (column mass)
//   editing_sparse_attention.py:161-172          sharpness split (peaked / diffuse halves)
//   tilelang_host.py:163-173                     new-KV block sums, top_k per query block
//
// Every ranked decision uses the rule "larger value first, lower index first on ties".
// All score arithmetic is fp32 with fixed reduction orders, so repeated runs are bitwise
// identical and no float atomics are used.
#include "icsa_kernels.h"

#define ICSA_MAX_NT 4096     // longest target-column row held in LDS by the softmax kernel
#define ICSA_MAX_SORT 4096   // longest list ranked by the select kernel
#define ICSA_L3_ROWS 8       // query blocks per workgroup in the level-3 kernel
#define ICSA_MAX_NKV 2048    // longest level-3 score row held in LDS

__device__ __forceinline__ float block_size_f(int blk, int NB, int S) {
  return blk < NB - 1 ? (float)ICSA_BLOCK : (float)(S - (NB - 1) * ICSA_BLOCK);
}

// ---------------------------------------------------------------------------------------
// (a) logits L = (Qs/size) (Ks/size)^T / sqrt(D), one 64x64 tile per workgroup (fp32 MFMA)
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) icsa_compressed_logits_kernel(CompressedParams p) {
  __shared__ float qs[64][132];
  __shared__ float ks[64][132];
  const int ct = blockIdx.x, rt = blockIdx.y, bh = blockIdx.z;
  const int NB = p.NB;
  const float* qbase = p.qsum + (int64_t)bh * NB * ICSA_D;
  const float* kbase = p.ksum + (int64_t)bh * NB * ICSA_D;
  for (int e = threadIdx.x; e < 64 * 32; e += 256) {
    const int r = e >> 5, c4 = e & 31;
    floatx4 qv = {0.f, 0.f, 0.f, 0.f}, kv = {0.f, 0.f, 0.f, 0.f};
    const int qrow = rt * 64 + r, krow = ct * 64 + r;
    if (qrow < NB) {
      qv = *reinterpret_cast<const floatx4*>(qbase + (int64_t)qrow * ICSA_D + 4 * c4);
      const float sz = block_size_f(qrow, NB, p.S);
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = qv[i] / sz;
    }
    if (krow < NB) {
      kv = *reinterpret_cast<const floatx4*>(kbase + (int64_t)krow * ICSA_D + 4 * c4);
      const float sz = block_size_f(krow, NB, p.S);
#pragma unroll
      for (int i = 0; i < 4; ++i) kv[i] = kv[i] / sz;
    }
    *reinterpret_cast<floatx4*>(&qs[r][4 * c4]) = qv;
    *reinterpret_cast<floatx4*>(&ks[r][4 * c4]) = kv;
  }
  __syncthreads();
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int li = l & 31, hl = l >> 5;
  const int r0 = 32 * (w & 1), c0 = 32 * (w >> 1);
  floatx16 acc = {};
  // lane half hl contracts d in [64*hl, 64*hl + 64); A and B use the same split.
#pragma unroll 4
  for (int kk = 0; kk < 64; kk += 4) {
    const floatx4 a = *reinterpret_cast<const floatx4*>(&qs[r0 + li][64 * hl + kk]);
    const floatx4 b = *reinterpret_cast<const floatx4*>(&ks[c0 + li][64 * hl + kk]);
#pragma unroll
    for (int j = 0; j < 4; ++j) acc = mfma32x32x2f32(a[j], b[j], acc);
  }
  const float sq = sqrtf((float)ICSA_D);
  float* out = p.P + (int64_t)bh * NB * NB;
  const int col = ct * 64 + c0 + li;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = rt * 64 + r0 + acc_row(i, l);
    if (row < NB && col < NB) out[(int64_t)row * NB + col] = acc[i] / sq;
  }
}

// ---------------------------------------------------------------------------------------
// (b) row softmax in place + sharpness = sum of the k_sparsity largest P[i, :n_t]
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int wave_sum_i(int x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

__global__ void __launch_bounds__(256) icsa_compressed_softmax_kernel(CompressedParams p) {
  __shared__ float tgt[4][ICSA_MAX_NT];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;
  const bool active = row < (int64_t)p.BH * p.NB;
  const int NB = p.NB;
  const int n_t = p.n_t;
  if (active) {
    float* L = p.P + row * NB;
    float m = -INFINITY;
    for (int j = lane; j < NB; j += 64) m = fmaxf(m, L[j]);
    m = wave_max(m);
    float z = 0.f;
    for (int j = lane; j < NB; j += 64) z += expf(L[j] - m);
    z = wave_sum(z);
    for (int j = lane; j < NB; j += 64) {
      const float pv = expf(L[j] - m) / z;
      L[j] = pv;
      if (j < n_t) tgt[w][j] = pv;
    }
  }
  __syncthreads();
  if (!active) return;
  float sharp = 0.f;
  const int k = p.k_sparsity;
  if (n_t > 0) {
    // largest tau (bit pattern of a non-negative float) with count(P >= tau) >= k
    uint32_t lo = 0u, hi = 0x7f800000u;
    while (hi - lo > 1u) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      int c = 0;
      for (int j = lane; j < n_t; j += 64) c += (__float_as_uint(tgt[w][j]) >= mid) ? 1 : 0;
      c = wave_sum_i(c);
      if (c >= k) lo = mid; else hi = mid;
    }
    int cgt = 0;
    float s = 0.f;
    for (int j = lane; j < n_t; j += 64) {
      const float v = tgt[w][j];
      if (__float_as_uint(v) > lo) { ++cgt; s += v; }
    }
    cgt = wave_sum_i(cgt);
    s = wave_sum(s);
    sharp = s + (float)(k - cgt) * __uint_as_float(lo);
  }
  if (lane == 0) p.sharp[row] = sharp;
}

// ---------------------------------------------------------------------------------------
// (c) out_c = P (Vs/size), one 64-row tile per workgroup (fp32 MFMA)
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) icsa_compressed_pv_kernel(CompressedParams p) {
  __shared__ float ps[64][68];
  __shared__ float vs[64][132];
  const int rt = blockIdx.x, bh = blockIdx.y;
  const int NB = p.NB;
  const float* P = p.P + (int64_t)bh * NB * NB;
  const float* V = p.vsum + (int64_t)bh * NB * ICSA_D;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int li = l & 31, hl = l >> 5;
  const int r0 = 32 * (w & 1), c0 = 64 * (w >> 1);
  floatx16 acc0 = {}, acc1 = {};
  for (int k0 = 0; k0 < NB; k0 += 64) {
    for (int e = threadIdx.x; e < 64 * 64; e += 256) {
      const int r = e >> 6, kk = e & 63;
      const int row = rt * 64 + r, kc = k0 + kk;
      ps[r][kk] = (row < NB && kc < NB) ? P[(int64_t)row * NB + kc] : 0.f;
    }
    for (int e = threadIdx.x; e < 64 * 32; e += 256) {
      const int kk = e >> 5, c4 = e & 31;
      const int kc = k0 + kk;
      floatx4 v = {0.f, 0.f, 0.f, 0.f};
      if (kc < NB) {
        v = *reinterpret_cast<const floatx4*>(V + (int64_t)kc * ICSA_D + 4 * c4);
        const float sz = block_size_f(kc, NB, p.S);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = v[i] / sz;
      }
      *reinterpret_cast<floatx4*>(&vs[kk][4 * c4]) = v;
    }
    __syncthreads();
#pragma unroll 2
    for (int s = 0; s < 32; s += 4) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(&ps[r0 + li][32 * hl + s]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc0 = mfma32x32x2f32(a[j], vs[32 * hl + s + j][c0 + li], acc0);
        acc1 = mfma32x32x2f32(a[j], vs[32 * hl + s + j][c0 + 32 + li], acc1);
      }
    }
    __syncthreads();
  }
  float* out = p.out_c + (int64_t)bh * NB * ICSA_D;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = rt * 64 + r0 + acc_row(i, l);
    if (row < NB) {
      out[(int64_t)row * ICSA_D + c0 + li] = acc0[i];
      out[(int64_t)row * ICSA_D + c0 + 32 + li] = acc1[i];
    }
  }
}

hipError_t launch_compressed(const CompressedParams& p, hipStream_t stream) {
  if (p.n_t > ICSA_MAX_NT) return hipErrorInvalidValue;
  const int nt = (p.NB + 63) / 64;
  hipLaunchKernelGGL(icsa_compressed_logits_kernel, dim3(nt, nt, p.BH), dim3(256), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = (int64_t)p.BH * p.NB;
  hipLaunchKernelGGL(icsa_compressed_softmax_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(icsa_compressed_pv_kernel, dim3(nt, p.BH), dim3(256), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// (d) per-head selection: source column mass -> top-topK, sharpness ranking, new-KV map
// ---------------------------------------------------------------------------------------
__device__ void bitonic_sort_desc(unsigned long long* keys, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const unsigned long long a = keys[i], b = keys[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (a < b) : (a > b)) { keys[i] = b; keys[ixj] = a; }
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ unsigned long long rank_key(float v, int idx) {
  return ((unsigned long long)f2key(v) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ int rank_idx(unsigned long long key) {
  return (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
}

__global__ void __launch_bounds__(1024) icsa_select_kernel(SelectParams p) {
  __shared__ unsigned long long keys[ICSA_MAX_SORT];
  __shared__ int sel_l[ICSA_MAX_SORT];
  const int bh = blockIdx.x;
  const int NB = p.NB, n_t = p.n_t, n_s = p.n_s;
  const float* P = p.P + (int64_t)bh * NB * NB;
  int n1 = 1;
  while (n1 < n_s) n1 <<= 1;
  // column mass of source key blocks over target query blocks, sequential over rows
  for (int j = threadIdx.x; j < n1; j += blockDim.x) {
    if (j < n_s) {
      float s = 0.f;
      const float* col = P + n_t + j;
      int i = 0;
      for (; i + 8 <= n_t; i += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = col[(int64_t)(i + u) * NB];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
      }
      for (; i < n_t; ++i) s += col[(int64_t)i * NB];
      p.src_score[(int64_t)bh * n_s + j] = s;
      keys[j] = rank_key(s, j);
    } else {
      keys[j] = 0ull;
    }
  }
  __syncthreads();
  if (!p.inject_sel) {
    if (n_s > 0) bitonic_sort_desc(keys, n1);
    for (int r = threadIdx.x; r < p.topK; r += blockDim.x) {
      const int idx = rank_idx(keys[r]);
      sel_l[r] = idx;
      p.sel[(int64_t)bh * p.topK + r] = idx;
    }
  } else {
    for (int r = threadIdx.x; r < p.topK; r += blockDim.x) sel_l[r] = p.sel[(int64_t)bh * p.topK + r];
  }
  __syncthreads();
  if (!p.inject_order) {
    int n2 = 1;
    while (n2 < NB) n2 <<= 1;
    for (int i = threadIdx.x; i < n2; i += blockDim.x)
      keys[i] = i < NB ? rank_key(p.sharp[(int64_t)bh * NB + i], i) : 0ull;
    __syncthreads();
    bitonic_sort_desc(keys, n2);
    for (int r = threadIdx.x; r < NB; r += blockDim.x)
      p.order[(int64_t)bh * NB + r] = rank_idx(keys[r]);
  }
  // new-KV block j -> source block: target blocks, then the selected source blocks in
  // ranked order, then zero padding (-1).
  for (int j = threadIdx.x; j < p.NKV; j += blockDim.x) {
    int src;
    if (p.materialized) src = j;
    else if (j < n_t) src = j;
    else if (j < n_t + p.topK) src = n_t + sel_l[j - n_t];
    else src = -1;
    p.kvmap[(int64_t)bh * p.NKV + j] = src;
  }
}

hipError_t launch_select(const SelectParams& p, hipStream_t stream) {
  if (p.n_s > ICSA_MAX_SORT || p.NB > ICSA_MAX_SORT) return hipErrorInvalidValue;
  hipLaunchKernelGGL(icsa_select_kernel, dim3(p.BH), dim3(1024), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// (e) sums of the new-KV blocks (fp32 for scoring; bf16 rows / transposed for the kernel)
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(128) icsa_newkv_sums_kernel(NewKvSumsParams p) {
  const int j = blockIdx.x, bh = blockIdx.y, d = threadIdx.x;
  int src = -1;
  if (j < p.NKV) src = p.map_identity ? j : p.kvmap[(int64_t)bh * p.NKV + j];
  float ks = 0.f, vs = 0.f;
  if (src >= 0) {
    ks = p.ksum[((int64_t)bh * p.Nsrc + src) * ICSA_D + d];
    vs = p.vsum[((int64_t)bh * p.Nsrc + src) * ICSA_D + d];
  }
  if (j < p.NKV) p.kc32[((int64_t)bh * p.NKV + j) * ICSA_D + d] = ks;
  p.kc[((int64_t)bh * p.NKVp + j) * ICSA_D + d] = f2bf(ks);
  p.vct[((int64_t)bh * ICSA_D + d) * p.NKVp + (j & ~15) + kv_slot(j & 15)] = f2bf(vs);
}

hipError_t launch_newkv_sums(const NewKvSumsParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(icsa_newkv_sums_kernel, dim3(p.NKVp, p.BH), dim3(128), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// (f) level-3: per query block, top_k new-KV blocks by QCsum . KCsum (fp32), ascending list
// ---------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) icsa_level3_kernel(Level3Params p) {
  __shared__ float qrow[ICSA_L3_ROWS][ICSA_D];
  __shared__ float sc[ICSA_L3_ROWS][ICSA_MAX_NKV];
  const int bh = blockIdx.y;
  const int r0 = blockIdx.x * ICSA_L3_ROWS;
  const int NKV = p.NKV;
  for (int e = threadIdx.x; e < ICSA_L3_ROWS * ICSA_D; e += 256) {
    const int r = e / ICSA_D, d = e % ICSA_D;
    float v = 0.f;
    if (r0 + r < p.n_rows) {
      const int qb = p.rows ? p.rows[(int64_t)bh * p.rows_stride + p.rows_offset + r0 + r] : r0 + r;
      v = p.qsum[((int64_t)bh * p.NQsrc + qb) * ICSA_D + d];
    }
    qrow[r][d] = v;
  }
  __syncthreads();
  const float* kc = p.kc32 + (int64_t)bh * NKV * ICSA_D;
  for (int j = threadIdx.x; j < NKV; j += 256) {
    float acc[ICSA_L3_ROWS];
#pragma unroll
    for (int r = 0; r < ICSA_L3_ROWS; ++r) acc[r] = 0.f;
    for (int d = 0; d < ICSA_D; d += 4) {
      const floatx4 kv = *reinterpret_cast<const floatx4*>(kc + (int64_t)j * ICSA_D + d);
#pragma unroll
      for (int r = 0; r < ICSA_L3_ROWS; ++r) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[r] = fmaf(qrow[r][d + u], kv[u], acc[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < ICSA_L3_ROWS; ++r) sc[r][j] = acc[r];
  }
  __syncthreads();
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int k = p.top_k;
  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int rr = w; rr < ICSA_L3_ROWS; rr += 4) {
    const int r = r0 + rr;
    if (r >= p.n_rows) break;
    // largest key tau with count(key >= tau) >= k
    uint32_t lo = 0u, hi = 0xffffffffu;
    while (hi - lo > 1u) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      int c = 0;
      for (int j = lane; j < NKV; j += 64) c += (f2key(sc[rr][j]) >= mid) ? 1 : 0;
      c = wave_sum_i(c);
      if (c >= k) lo = mid; else hi = mid;
    }
    int cgt = 0;
    for (int j = lane; j < NKV; j += 64) cgt += (f2key(sc[rr][j]) > lo) ? 1 : 0;
    cgt = wave_sum_i(cgt);
    const int need_eq = k - cgt;
    int seen_eq = 0, taken = 0;
    int* out = p.idx + ((int64_t)bh * p.n_rows + r) * k;
    for (int base = 0; base < NKV; base += 64) {
      const int j = base + lane;
      uint32_t key = 0u;
      if (j < NKV) key = f2key(sc[rr][j]);
      const bool gt = (j < NKV) && key > lo;
      const bool eq = (j < NKV) && key == lo;
      const unsigned long long eqm = __ballot(eq);
      const int eq_before = seen_eq + __popcll(eqm & lt_mask);
      const bool take = gt || (eq && eq_before < need_eq);
      const unsigned long long tm = __ballot(take);
      const int pos = taken + __popcll(tm & lt_mask);
      if (take && pos < k) out[pos] = j;
      seen_eq += __popcll(eqm);
      taken += __popcll(tm);
    }
  }
}

hipError_t launch_level3(const Level3Params& p, hipStream_t stream) {
  if (p.NKV > ICSA_MAX_NKV || p.top_k > p.NKV || p.top_k < 1) return hipErrorInvalidValue;
  dim3 grid((p.n_rows + ICSA_L3_ROWS - 1) / ICSA_L3_ROWS, p.BH);
  hipLaunchKernelGGL(icsa_level3_kernel, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}
