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
#include "attn_tile.h"
#include "icsa_kernels.h"

#define ICSA_MAX_NB 4096     // longest P row held in registers by the strip kernel
#define ICSA_MAX_SORT 4096   // longest list ranked by the select kernel
#define ICSA_MAX_NKV 2048    // longest level-3 score row held in registers

__device__ __forceinline__ float block_size_f(int blk, int NB, int S) {
  return blk < NB - 1 ? (float)ICSA_BLOCK : (float)(S - (NB - 1) * ICSA_BLOCK);
}

// ---------------------------------------------------------------------------------------
// (a) logits L = (Qs/size) (Ks/size)^T / sqrt(D) at fp32 accuracy on the bf16 matrix pipe.
//     Every fp32 operand x is split exactly into three bf16 parts, x = xh + xm + xl + r with
//     |r| <= 2^-27 |x| (xh = bf16(x), xm = bf16(x - xh), xl = bf16(x - xh - xm)), and each
//     product is formed from the six part products down to 2^-18 of its size
//     (al bh + am bm + ah bl + am bh + ah bm + ah bh, small terms first); the dropped
//     ones are below 2^-25 of it, and every part product is exact in the fp32
//     accumulator.  So the logits carry fp32-level rounding while the matrix work takes
//     6 bf16 MFMAs (32x32x16, 32 cycles) per 16 dims instead of 8 fp32 ones (32x32x2, 64).
//     Workgroup = 4 waves = 128 query rows (wave w: rows 32 w .. 32 w + 31) against one of
//     LG_SPLIT column ranges.  A wave's split A operands stay in registers for the whole
//     range (lane (li, hl) holds row li's dims 16 s + 8 hl .. + 7, s = 0 .. 7); 32-column K
//     tiles pass through a double-buffered LDS ring of split tiles, the next tile prefetched
//     into registers while the current one is multiplied.  A fixed order of MFMAs, so
//     repeated runs are bitwise identical.
// ---------------------------------------------------------------------------------------
#define LG_SPLIT 3
#define LG_ROWS 128
#define LG_COLS 32
#define LG_KST 136            // bf16 row stride of a split K tile (272 B: conflict-free reads)

__device__ __forceinline__ void split3_bf16(float x, bf16& h, bf16& m, bf16& l) {
  h = f2bf(x);
  const float r1 = x - bf2f(h);
  m = f2bf(r1);
  l = f2bf(r1 - bf2f(m));
}

// The same fp32-accurate product for the logits and for the level-3 block scores:
// C[r][c] = (A_r / sa) . (B_c / sb) / div over D = 128, with A's rows optionally gathered
// through a list, and sa, sb the block sizes (logits) or 1 (level-3 scores: raw sums).
struct Split3Gemm {
  const float* A;           // [BH, a_rows, D]
  const int* rows;          // output row r reads A row rows[bh * rows_stride + rows_offset + r]
  int rows_stride, rows_offset, a_rows;
  int n_rows;               // output rows per head
  const float* B;           // [BH, n_cols, D]
  int n_cols;
  float* C;                 // [BH, n_rows, n_cols]
  int NB, S;                // block sizes (block_mean)
  float div;
};

template <bool BLOCK_MEAN>
__global__ void __launch_bounds__(256) icsa_split3_gemm_kernel(Split3Gemm g) {
  __shared__ __attribute__((aligned(16))) bf16 ks[2][3][LG_COLS][LG_KST];
  const int rt = blockIdx.x, cs = blockIdx.y, bh = blockIdx.z;
  const int NC = g.n_cols;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int li = l & 31, hl = l >> 5;
  const float* qbase = g.A + (int64_t)bh * g.a_rows * ICSA_D;
  const float* kbase = g.B + (int64_t)bh * NC * ICSA_D;

  // A operands: this lane's row (divided by its block size for the logits), split in three
  bf16x8 ah[8], am[8], al[8];
  {
    const int r = rt * LG_ROWS + 32 * w + li;
    const bool ok = r < g.n_rows;
    const int row = !ok ? 0 : (g.rows ? g.rows[(int64_t)bh * g.rows_stride + g.rows_offset + r] : r);
    const float sz = (BLOCK_MEAN && ok) ? block_size_f(row, g.NB, g.S) : 1.f;
    const float* src = qbase + (int64_t)row * ICSA_D + 8 * hl;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      floatx4 v0 = {0.f, 0.f, 0.f, 0.f}, v1 = v0;
      if (ok) {
        v0 = *reinterpret_cast<const floatx4*>(src + 16 * st);
        v1 = *reinterpret_cast<const floatx4*>(src + 16 * st + 4);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bf16 h, m, lo;
        const float x = e < 4 ? v0[e] : v1[e - 4];
        split3_bf16(BLOCK_MEAN ? x / sz : x, h, m, lo);
        ah[st][e] = h;
        am[st][e] = m;
        al[st][e] = lo;
      }
    }
  }

  const int n_ct = (NC + LG_COLS - 1) / LG_COLS;
  const int per = (n_ct + LG_SPLIT - 1) / LG_SPLIT;
  const int t0 = cs * per, t1 = min(n_ct, t0 + per);
  if (t0 >= t1) return;                                // uniform for the workgroup

  // K tile staging: thread -> (column tid / 8, 16 dims from 16 (tid % 8))
  const int kc = tid >> 3, kd = 16 * (tid & 7);
  floatx4 pre[4];
  auto load_tile = [&](int t) {
    const int col = t * LG_COLS + kc;
    if (col < NC) {
      const float sz = BLOCK_MEAN ? block_size_f(col, g.NB, g.S) : 1.f;
      const float* src = kbase + (int64_t)col * ICSA_D + kd;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pre[q] = *reinterpret_cast<const floatx4*>(src + 4 * q);
        if (BLOCK_MEAN) {
#pragma unroll
          for (int e = 0; e < 4; ++e) pre[q][e] = pre[q][e] / sz;
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) pre[q] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      bf16x8 h, m, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        bf16 a, b, c;
        split3_bf16(pre[2 * half + (e >> 2)][e & 3], a, b, c);
        h[e] = a;
        m[e] = b;
        lo[e] = c;
      }
      *reinterpret_cast<bf16x8*>(&ks[buf][0][kc][kd + 8 * half]) = h;
      *reinterpret_cast<bf16x8*>(&ks[buf][1][kc][kd + 8 * half]) = m;
      *reinterpret_cast<bf16x8*>(&ks[buf][2][kc][kd + 8 * half]) = lo;
    }
  };

  float* out = g.C + (int64_t)bh * g.n_rows * NC;
  load_tile(t0);
  store_tile(0);
  __syncthreads();
  for (int t = t0; t < t1; ++t) {
    const int buf = (t - t0) & 1;
    const bool more = t + 1 < t1;
    if (more) load_tile(t + 1);
    floatx16 acc = {};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const bf16x8 bh = *reinterpret_cast<const bf16x8*>(&ks[buf][0][li][16 * st + 8 * hl]);
      const bf16x8 bm = *reinterpret_cast<const bf16x8*>(&ks[buf][1][li][16 * st + 8 * hl]);
      const bf16x8 bl = *reinterpret_cast<const bf16x8*>(&ks[buf][2][li][16 * st + 8 * hl]);
      acc = mfma32x32x16(al[st], bh, acc);
      acc = mfma32x32x16(am[st], bm, acc);
      acc = mfma32x32x16(ah[st], bl, acc);
      acc = mfma32x32x16(am[st], bh, acc);
      acc = mfma32x32x16(ah[st], bm, acc);
      acc = mfma32x32x16(ah[st], bh, acc);
    }
    const int col = t * LG_COLS + li;
    if (col < NC) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = rt * LG_ROWS + 32 * w + acc_row(i, l);
        if (row < g.n_rows) out[(int64_t)row * NC + col] = acc[i] / g.div;
      }
    }
    if (more) store_tile(buf ^ 1);                     // that buffer was read in step t - 1
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------
// (b) row statistics, one wave per row of logits (held in registers, VPL per lane): row
//     max m, 1 / sum exp(L - m), and the sharpness = sum of the k_sparsity largest
//     P[i, :n_t].  exp is monotonic, so the k-th largest target probability is
//     exp(tau - m) / z for the k-th largest target logit tau, found by bisection over the
//     order-preserving float keys with ballot counts.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int wave_count(bool pred) { return __popcll(__ballot(pred)); }

// Whole-wave reductions over DPP lane moves (no LDS round trip): quad swaps, half-row and
// row mirrors leave every lane of a 16-lane row holding the row's result; two row
// broadcasts fold rows 0+1 and 2+3 and then the pairs into lane 63, which is read back as
// a wave-uniform value.  A fixed combination order, so sums are bitwise reproducible.
// Every lane of the wave must be active.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t old, uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)x, CTRL, ROWS, 0xf, false);
}
template <typename F>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t x, uint32_t ident, F op) {
  x = op(x, dpp_mov<0xb1, 0xf>(ident, x));     // quad_perm [1, 0, 3, 2]
  x = op(x, dpp_mov<0x4e, 0xf>(ident, x));     // quad_perm [2, 3, 0, 1]
  x = op(x, dpp_mov<0x141, 0xf>(ident, x));    // row_half_mirror
  x = op(x, dpp_mov<0x140, 0xf>(ident, x));    // row_mirror
  x = op(x, dpp_mov<0x142, 0xa>(ident, x));    // row_bcast:15 into rows 1 and 3
  x = op(x, dpp_mov<0x143, 0xc>(ident, x));    // row_bcast:31 into rows 2 and 3
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
__device__ __forceinline__ float wave_max_dpp(float x) {
  return __uint_as_float(wave_reduce(__float_as_uint(x), __float_as_uint(-INFINITY), [](uint32_t a, uint32_t b) {
    return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
  }));
}
__device__ __forceinline__ float wave_sum_dpp(float x) {
  return __uint_as_float(wave_reduce(__float_as_uint(x), 0u, [](uint32_t a, uint32_t b) {
    return __float_as_uint(__uint_as_float(a) + __uint_as_float(b));
  }));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  return wave_reduce(x, 0xffffffffu, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  return wave_reduce(x, 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}

// Largest key lo with count(key >= lo) >= k over the wave's keys (keys 0 = absent; requires
// at least k nonzero keys): the key of the k-th largest.  Only registers u < nu can hold
// nonzero keys; they are visited in groups of four (one uniform branch per group, the
// zero keys of a partly used group never count).  Bisection over the key range; as soon
// as a midpoint has exactly k keys at or above it, the answer is the smallest of those
// keys (one wave minimum), which for spread-out values ends the search long before the
// 32nd step.  The search starts from a bracket that the keys themselves give: every lane's
// largest key is at or above the smallest of the 64 lane maxima, so for k <= 64 that
// minimum has at least k keys at or above it, and no key lies above the wave's largest.
// The answer is the same key from any valid bracket; the narrower one saves steps.
template <int VPL>
__device__ __forceinline__ uint32_t kth_largest_key(const uint32_t (&key)[VPL], int k, int nu) {
  static_assert(VPL % 4 == 0, "registers are visited in groups of four");
  uint32_t lmax = 0u;
#pragma unroll
  for (int g = 0; g < VPL; g += 4)
    if (g < nu) {
#pragma unroll
      for (int u = g; u < g + 4; ++u) lmax = key[u] > lmax ? key[u] : lmax;
    }
  const uint32_t kmax = wave_max_u32(lmax);
  uint32_t lo = k <= 64 ? wave_min_u32(lmax) : 0u;
  uint32_t hi = kmax == 0xffffffffu ? kmax : kmax + 1u;
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    int c = 0;
#pragma unroll
    for (int g = 0; g < VPL; g += 4)
      if (g < nu) {
#pragma unroll
        for (int u = g; u < g + 4; ++u) c += wave_count(key[u] >= mid);
      }
    if (c == k) {
      uint32_t mn = 0xffffffffu;
#pragma unroll
      for (int g = 0; g < VPL; g += 4)
        if (g < nu) {
#pragma unroll
          for (int u = g; u < g + 4; ++u)
            if (key[u] >= mid && key[u] < mn) mn = key[u];
        }
      return wave_min_u32(mn);
    }
    if (c > k) lo = mid; else hi = mid;
  }
  return lo;
}

template <int VPL>   // logits per lane: NB <= 64 * VPL
__global__ void __launch_bounds__(256) icsa_compressed_stats_kernel(CompressedParams p) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;          // over BH * NB rows
  if (row >= (int64_t)p.BH * p.NB) return;
  const int NB = p.NB, n_t = p.n_t;
  const float* L = p.L + row * NB;
  float v[VPL];
  uint32_t key[VPL];                              // order keys of the target logits (0: none)
  float m = -INFINITY;
#pragma unroll
  for (int u = 0; u < VPL; ++u) {
    const int j = lane + 64 * u;
    v[u] = j < NB ? L[j] : -INFINITY;
    key[u] = j < n_t ? f2key(v[u]) : 0u;
    m = fmaxf(m, v[u]);
  }
  m = wave_max_dpp(m);
  float z = 0.f;
#pragma unroll
  for (int u = 0; u < VPL; ++u) {
    v[u] = expf(v[u] - m);                        // v now holds exp(L - m)
    z += v[u];
  }
  z = wave_sum_dpp(z);
  float sharp = 0.f;
  if (n_t > 0) {
    const int k = p.k_sparsity;
    const int nu = (n_t + 63) / 64;
    const uint32_t lo = kth_largest_key<VPL>(key, k, nu);
    int cgt = 0;
    float sa = 0.f;
#pragma unroll
    for (int g = 0; g < VPL; g += 4)
      if (g < nu) {
#pragma unroll
        for (int u = g; u < g + 4; ++u) {
          const bool in = key[u] > lo;
          cgt += wave_count(in);
          sa += in ? v[u] : 0.f;
        }
      }
    sa = wave_sum_dpp(sa);
    sharp = (sa + (float)(k - cgt) * expf(key2f(lo) - m)) / z;
  }
  if (lane == 0) {
    p.rstat[2 * row] = m;
    p.rstat[2 * row + 1] = 1.f / z;
    p.sharp[row] = sharp;
  }
}

// ---------------------------------------------------------------------------------------
// (c) one 64-row strip of P per workgroup of 8 waves, in 32-key chunks: out_c = P Vm with
//     P = exp(L - m) / z, on the bf16 matrix pipe from split operands.  Per chunk:
//       * the chunk's logits (64 x 32 fp32) and its split, transposed value means (two bf16
//         planes of 128 dims x 32 keys, icsa_vmean_split_kernel) arrive by LDS DMA, double
//         buffered: chunk c + 1 is in flight while chunk c is computed, and two workgroups
//         share each CU (65 KB of LDS each);
//       * P is formed once in fp32 and kept as its two bf16 parts P = Ph + Pl (to 2^-17 of
//         P), and, for strips holding target rows, also in fp32 for the column sums of the
//         source columns over those rows (rows in order: the strip's partial, summed across
//         strips by the select kernel);
//       * wave w adds Pl Vh + Ph Vl + Ph Vh over the chunk's two 16-key steps into output
//         rows 32 (w % 2) .. + 31, columns 32 (w / 2) .. + 31 (the dropped Pl Vl is below
//         2^-16 of each product).
//     Fixed orders throughout, so repeated runs are bitwise identical.
// ---------------------------------------------------------------------------------------
#define RW_PB_LD 36                             // floats per P row in LDS (16-byte skew)

// Vm = Vsum / block size, transposed and split in two bf16 parts:
// vmt[((bh * 2 + part) * D + d) * NBp + key], zero for keys >= NB.
__global__ void __launch_bounds__(256) icsa_vmean_split_kernel(CompressedParams p, int NBp) {
  __shared__ float tile[64][ICSA_D + 4];
  const int k0 = blockIdx.x * 64, bh = blockIdx.y;
  const int NB = p.NB, t = threadIdx.x;
  const float* V = p.vsum + (int64_t)bh * NB * ICSA_D;
  floatx4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {                 // float4 f = t + 256 j: key f / 32, dims 4 (f % 32)
    const int f = t + 256 * j, key = k0 + (f >> 5);
    v[j] = key < NB ? *reinterpret_cast<const floatx4*>(V + (int64_t)key * ICSA_D + 4 * (f & 31))
                    : floatx4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int f = t + 256 * j, key = k0 + (f >> 5);
    if (key < NB) {
      const float inv = 1.f / block_size_f(key, NB, p.S);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[j][e] *= inv;
    }
    *reinterpret_cast<floatx4*>(&tile[f >> 5][4 * (f & 31)]) = v[j];
  }
  __syncthreads();
  const int d = t >> 1, kh = t & 1;             // dim d, keys 32 kh .. + 31
  bf16* dst = p.vmt + ((int64_t)bh * 2 * ICSA_D + d) * NBp + k0 + 32 * kh;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    bf16x8 hi, lo;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = tile[32 * kh + 8 * g + i][d];
      const bf16 h = f2bf(x);
      hi[i] = h;
      lo[i] = f2bf(x - bf2f(h));
    }
    *reinterpret_cast<bf16x8*>(dst + 8 * g) = hi;
    *reinterpret_cast<bf16x8*>(dst + (int64_t)ICSA_D * NBp + 8 * g) = lo;
  }
}

// LDS DMA issued from inline assembly: the compiler does not track these loads, so it
// inserts no waits for them before LDS reads of the other stage; the kernel waits itself
// (vmcnt(0) before the barrier that opens each chunk).  Lane l of one instruction lands at
// lds_addr + 16 l.  The resource words are those of make_rsrc (raw buffer, no stride).
__device__ __forceinline__ u32x4 rw_rsrc(const void* base, int64_t bytes) {
  const unsigned long long a = (unsigned long long)base;
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (int)(bytes < 0 ? 0 : bytes);
  u32x4 r;
  r[0] = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)a);
  r[1] = (unsigned)__builtin_amdgcn_readfirstlane((int)((unsigned)(a >> 32) & 0xffffu));
  r[2] = (unsigned)__builtin_amdgcn_readfirstlane(n);
  r[3] = 0x00020000u;
  return r;
}
__device__ __forceinline__ void rw_dma16(unsigned lds_addr, int voff, u32x4 rs) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds_addr), "v"(voff), "s"(rs) : "memory", "m0");
}
__device__ __forceinline__ unsigned lds_u32(const void* p) {
  return (unsigned)__builtin_amdgcn_readfirstlane(
      (int)(unsigned)(size_t)(const __attribute__((address_space(3))) void*)p);
}

__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
icsa_compressed_rows_kernel(CompressedParams p, int NBp) {
  // two stages of the chunk operands as separate objects; 65 KB in all, two workgroups per CU
  __shared__ __attribute__((aligned(16))) float lc0[64 * 32], lc1[64 * 32];          // logits
  __shared__ __attribute__((aligned(16))) bf16 vc0[2 * ICSA_D * 32], vc1[2 * ICSA_D * 32];  // Vm^T planes
  __shared__ __attribute__((aligned(16))) float pb[64 * RW_PB_LD];   // P as [Ph x 8 | Pl x 8] per 8 keys
  __shared__ __attribute__((aligned(16))) float pf[64 * 32];         // fp32 P (target strips)
  __shared__ float row_m[64], row_iz[64];
  const int strip = blockIdx.x, bh = blockIdx.y;
  const int NB = p.NB, n_t = p.n_t;
  const int r_base = strip * 64;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  if (tid < 64) {
    const int row = r_base + tid;
    row_m[tid] = row < NB ? p.rstat[2 * ((int64_t)bh * NB + row)] : 0.f;
    row_iz[tid] = row < NB ? p.rstat[2 * ((int64_t)bh * NB + row) + 1] : 0.f;
  }
  const int n_ts = (n_t + ICSA_BLOCK - 1) / ICSA_BLOCK;
  const int tgt_rows = min(64, n_t - r_base);          // > 0 only for target strips
  const int nch = NBp / 32;                            // even

  // DMA sources: the strip's logit rows (rows past NB and keys past the last row are
  // outside the resource: no load, and P is zero there) and the head's value planes
  const float* Lbh = p.L + (int64_t)bh * NB * NB;
  const u32x4 rs_l = rw_rsrc(Lbh + (int64_t)r_base * NB, (int64_t)max(0, min(64, NB - r_base)) * NB * 4);
  const u32x4 rs_v = rw_rsrc(p.vmt + (int64_t)bh * 2 * ICSA_D * NBp, (int64_t)2 * ICSA_D * NBp * 2);
  // logits: wave w moves rows 8 w .. + 7 (128 bytes each), 16 bytes per lane
  const int l_off = ((8 * w + (lane >> 3)) * NB + 4 * (lane & 7)) * 4;
  // value planes: instruction j (0, 1) of wave w moves rows R = 16 (2 w + j) .. + 15 of the
  // 256 (plane R / 128, dim R % 128), 64 bytes each; physical 16-byte unit lane % 4 of row R
  // holds logical unit (lane % 4) ^ (R % 4)
  int v_off[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int R = 16 * (2 * w + j) + (lane >> 2);
    v_off[j] = ((R >> 7) * ICSA_D + (R & 127)) * NBp * 2 + 16 * ((lane & 3) ^ (R & 3));
  }
  auto issue = [&](int c, float* lc, bf16* vc) {
    rw_dma16(lds_u32(lc + 256 * w), l_off + 128 * c, rs_l);
#pragma unroll
    for (int j = 0; j < 2; ++j) rw_dma16(lds_u32(vc + 512 * (2 * w + j)), v_off[j] + 64 * c, rs_v);
  };

  const int li = lane & 31, hl = lane >> 5;
  const int rh = w & 1, dc = 32 * (w >> 1);
  floatx16 acc = {};
  // one chunk of 32 keys: P from lc (thread: row t / 8, keys 4 (t % 8) .. + 3), then the
  // MFMAs on vc
  auto chunk = [&](int c, const float* lc, const bf16* vc) {
    const int k0 = 32 * c;
    const bool want_cs = tgt_rows > 0 && k0 + 32 > n_t;   // uniform
    {
      const int r = tid >> 3, q = tid & 7, row = r_base + r;
      const floatx4 a = *reinterpret_cast<const floatx4*>(lc + r * 32 + 4 * q);
      const float m = row_m[r], iz = row_iz[r];
      float pv[4];
      bf16x4 hi, lo;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = k0 + 4 * q + i;
        pv[i] = (row < NB && col < NB) ? expf(a[i] - m) * iz : 0.f;
        const bf16 h = f2bf(pv[i]);
        hi[i] = h;
        lo[i] = f2bf(pv[i] - bf2f(h));
      }
      // 8-key group q / 2, half q % 2: Ph at floats 8 (q / 2) + 2 (q % 2), Pl 4 floats on
      float* dst = pb + r * RW_PB_LD + 8 * (q >> 1) + 2 * (q & 1);
      *reinterpret_cast<bf16x4*>(dst) = hi;
      *reinterpret_cast<bf16x4*>(dst + 4) = lo;
      if (want_cs) *reinterpret_cast<floatx4*>(pf + r * 32 + 4 * q) = floatx4{pv[0], pv[1], pv[2], pv[3]};
    }
    ATT_BARRIER();                                   // P of the chunk ready
    if (want_cs && tid < 32) {
      const int col = k0 + tid;
      if (col >= n_t && col < NB) {
        float cs = 0.f;
        for (int r = 0; r < tgt_rows; ++r) cs += pf[r * 32 + tid];
        p.colpart[((int64_t)bh * n_ts + strip) * p.n_s + (col - n_t)] = cs;
      }
    }
    const float* prow = pb + (32 * rh + li) * RW_PB_LD;
    const int d = dc + li;
    const bf16* vh = vc + d * 32;
    const bf16* vl = vc + (ICSA_D + d) * 32;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int u = 2 * s + hl;                      // logical 16-byte unit: keys 8 u .. + 7
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(prow + 8 * u);
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(prow + 8 * u + 4);
      const int pu = (u ^ (d & 3)) * 8;
      const bf16x8 bh_ = *reinterpret_cast<const bf16x8*>(vh + pu);
      const bf16x8 bl_ = *reinterpret_cast<const bf16x8*>(vl + pu);
      acc = mfma32x32x16(al, bh_, acc);
      acc = mfma32x32x16(ah, bl_, acc);
      acc = mfma32x32x16(ah, bh_, acc);
    }
  };

  __syncthreads();                                   // row statistics in LDS
  issue(0, lc0, vc0);
  for (int c = 0; c < nch; c += 2) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // chunk c (and this wave's older stores)
    ATT_BARRIER();                                   // chunk c in LDS; chunk c - 1 consumed
    issue(c + 1, lc1, vc1);                          // nch is even
    chunk(c, lc0, vc0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    ATT_BARRIER();
    if (c + 2 < nch) issue(c + 2, lc0, vc0);
    chunk(c + 1, lc1, vc1);
  }
  float* out = p.out_c + (int64_t)bh * NB * ICSA_D;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = r_base + 32 * rh + acc_row(i, lane);
    if (row < NB) out[(int64_t)row * ICSA_D + dc + li] = acc[i];
  }
}

hipError_t launch_compressed(const CompressedParams& p, hipStream_t stream) {
  if (p.NB > ICSA_MAX_NB || p.vmt == nullptr) return hipErrorInvalidValue;
  const int nt = (p.NB + 63) / 64;
  Split3Gemm g;
  g.A = p.qsum; g.rows = nullptr; g.rows_stride = 0; g.rows_offset = 0; g.a_rows = p.NB;
  g.n_rows = p.NB; g.B = p.ksum; g.n_cols = p.NB; g.C = p.L; g.NB = p.NB; g.S = p.S;
  g.div = sqrtf((float)ICSA_D);
  hipLaunchKernelGGL(icsa_split3_gemm_kernel<true>, dim3((p.NB + LG_ROWS - 1) / LG_ROWS, LG_SPLIT, p.BH),
                     dim3(256), 0, stream, g);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = (int64_t)p.BH * p.NB;
  const dim3 sgrid((unsigned)((rows + 3) / 4));
  if (p.NB <= 256)
    hipLaunchKernelGGL(icsa_compressed_stats_kernel<4>, sgrid, dim3(256), 0, stream, p);
  else if (p.NB <= 512)
    hipLaunchKernelGGL(icsa_compressed_stats_kernel<8>, sgrid, dim3(256), 0, stream, p);
  else if (p.NB <= 1024)
    hipLaunchKernelGGL(icsa_compressed_stats_kernel<16>, sgrid, dim3(256), 0, stream, p);
  else if (p.NB <= 2048)
    hipLaunchKernelGGL(icsa_compressed_stats_kernel<32>, sgrid, dim3(256), 0, stream, p);
  else if (p.NB <= 2560)                             // configuration 5: NB = 2363
    hipLaunchKernelGGL(icsa_compressed_stats_kernel<40>, sgrid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(icsa_compressed_stats_kernel<64>, sgrid, dim3(256), 0, stream, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int NBp = compressed_nbp(p.NB);
  hipLaunchKernelGGL(icsa_vmean_split_kernel, dim3(NBp / 64, p.BH), dim3(256), 0, stream, p, NBp);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(icsa_compressed_rows_kernel, dim3(nt, p.BH), dim3(512), 0, stream, p, NBp);
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

// Two workgroups per head (blockIdx.y): 0 ranks the source blocks and builds the new-KV
// map, 1 ranks the query blocks by sharpness; the two rankings are independent.
__global__ void __launch_bounds__(1024) icsa_select_kernel(SelectParams p) {
  __shared__ unsigned long long keys[ICSA_MAX_SORT];
  __shared__ int sel_l[ICSA_MAX_SORT];
  const int bh = blockIdx.x;
  const int NB = p.NB, n_t = p.n_t, n_s = p.n_s;
  if (blockIdx.y == 1) {                       // uniform for the workgroup
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
    return;
  }
  int n1 = 1;
  while (n1 < n_s) n1 <<= 1;
  // column mass of source key blocks over target query blocks: the per-strip partial
  // sums of the strip kernel, added in strip order
  const int n_ts = (n_t + ICSA_BLOCK - 1) / ICSA_BLOCK;
  const float* part = p.colpart + (int64_t)bh * n_ts * n_s;
  for (int j = threadIdx.x; j < n1; j += blockDim.x) {
    if (j < n_s) {
      float s = 0.f;
      for (int st = 0; st < n_ts; ++st) s += part[(int64_t)st * n_s + j];
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
  // new-KV block j -> source block: target blocks, then the selected source blocks in
  // ranked order, then zero padding (-1).  With t % 64 != 0 the blocks from n_t on straddle
  // two of these (the kernels take the first t % 64 rows from the block before).
  for (int j = threadIdx.x; j < p.NKV; j += blockDim.x) {
    int src;
    if (j < n_t) src = j;
    else if (j < n_t + p.topK) src = n_t + sel_l[j - n_t];
    else src = -1;
    p.kvmap[(int64_t)bh * p.NKV + j] = src;
  }
}

hipError_t launch_select(const SelectParams& p, hipStream_t stream) {
  if (p.n_s > ICSA_MAX_SORT || p.NB > ICSA_MAX_SORT) return hipErrorInvalidValue;
  hipLaunchKernelGGL(icsa_select_kernel, dim3(p.BH, 2), dim3(1024), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// (e) sums of the new-KV blocks (fp32 for scoring; bf16 rows / transposed for the kernel)
// ---------------------------------------------------------------------------------------
// One workgroup per 16 consecutive new-KV blocks, thread d: dim d of each (the 32 source
// sums of a thread are requested together).  The 16 blocks' V sums of dim d are one
// 16-slot group of V^T row d, written as 32 contiguous bytes in kv_slot() order (kv_slot
// swaps two index bits, so it is its own inverse).
__global__ void __launch_bounds__(128) icsa_newkv_sums_kernel(NewKvSumsParams p) {
  const int j0 = 16 * blockIdx.x, bh = blockIdx.y, d = threadIdx.x;
  float ks[16], vs[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int j = j0 + i;
    int src = -1;
    if (j < p.NKV) src = p.map_identity ? j : p.kvmap[(int64_t)bh * p.NKV + j];
    ks[i] = 0.f;
    vs[i] = 0.f;
    if (src >= 0) {
      ks[i] = p.ksum[((int64_t)bh * p.Nsrc + src) * ICSA_D + d];
      vs[i] = p.vsum[((int64_t)bh * p.Nsrc + src) * ICSA_D + d];
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int j = j0 + i;
    if (p.seg_a > 0 && j >= p.seg_from && j < p.NKV) continue;   // icsa_newkv_straddle_kernel
    if (j < p.NKV) p.kc32[((int64_t)bh * p.NKV + j) * ICSA_D + d] = ks[i];
    p.kc[((int64_t)bh * p.NKVp + j) * ICSA_D + d] = f2bf(ks[i]);
    if (p.vc) p.vc[((int64_t)bh * p.NKVp + j) * ICSA_D + d] = f2bf(vs[i]);
  }
  if (p.vct) {                    // no straddling blocks where V^T sums are wanted (seg_a == 0)
    bf16x8 a, b;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      a[s] = f2bf(vs[kv_slot(s)]);
      b[s] = f2bf(vs[kv_slot(s + 8)]);
    }
    bf16* dst = p.vct + ((int64_t)bh * ICSA_D + d) * p.NKVp + j0;
    *reinterpret_cast<bf16x8*>(dst) = a;
    *reinterpret_cast<bf16x8*>(dst + 8) = b;
  }
}

// Straddling new-KV block j (the pipeline's new KV when t % 64 != 0; see SparseParams):
// rows r < a from tokens segA + r, rows r >= a from 64 kvmap[j] + r - a, summed straight
// from the token rows.  Thread t: 8 dims 8 (t % 16) .. + 7 of rows t / 16 + 8 m; the 8
// row groups are added in fixed order.
template <typename TK, typename TV>
__global__ void __launch_bounds__(128) icsa_newkv_straddle_kernel(NewKvSumsParams p) {
  __shared__ float red[2][8][ICSA_D + 4];
  const int j = p.seg_from + blockIdx.x, bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int t = threadIdx.x, c = t & 15, g = t >> 4;
  const int a = p.seg_a;
  const int* map = p.kvmap + (int64_t)bh * p.NKV;
  int tokA = -1;
  if (j == p.seg_from) tokA = ICSA_BLOCK * p.seg_from;
  else if (map[j - 1] >= 0) tokA = ICSA_BLOCK * map[j - 1] + ICSA_BLOCK - a;
  const int tokB = map[j] >= 0 ? ICSA_BLOCK * map[j] - a : -1;    // token of row r >= a: tokB + r
  const TK* kb = reinterpret_cast<const TK*>(p.k.p) + (int64_t)b * p.k.sb + (int64_t)h * p.k.sh;
  const TV* vb = reinterpret_cast<const TV*>(p.v.p) + (int64_t)b * p.v.sb + (int64_t)h * p.v.sh;
  float ks[8], vs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) { ks[e] = 0.f; vs[e] = 0.f; }
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const int r = g + 8 * m;
    const int tok = r < a ? (tokA < 0 ? -1 : tokA + r) : (tokB < 0 ? -1 : tokB + r);
    if (tok >= 0 && tok < p.S) {
      float x[8];
      load8_f32(kb + (int64_t)tok * p.k.ss + 8 * c, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) ks[e] += x[e];
      load8_f32(vb + (int64_t)tok * p.v.ss + 8 * c, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) vs[e] += x[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) { red[0][g][8 * c + e] = ks[e]; red[1][g][8 * c + e] = vs[e]; }
  __syncthreads();
  const int d = t;
  float k_sum = 0.f, v_sum = 0.f;
#pragma unroll
  for (int gg = 0; gg < 8; ++gg) { k_sum += red[0][gg][d]; v_sum += red[1][gg][d]; }
  p.kc32[((int64_t)bh * p.NKV + j) * ICSA_D + d] = k_sum;
  p.kc[((int64_t)bh * p.NKVp + j) * ICSA_D + d] = f2bf(k_sum);
  if (p.vct) p.vct[((int64_t)bh * ICSA_D + d) * p.NKVp + (j & ~15) + kv_slot(j & 15)] = f2bf(v_sum);
  if (p.vc) p.vc[((int64_t)bh * p.NKVp + j) * ICSA_D + d] = f2bf(v_sum);
}

hipError_t launch_newkv_sums(const NewKvSumsParams& p, hipStream_t stream) {
  if (p.NKVp % 16 != 0 || (p.vct && p.seg_a > 0)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(icsa_newkv_sums_kernel, dim3(p.NKVp / 16, p.BH), dim3(128), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.seg_a <= 0 || p.seg_from >= p.NKV) return e;
  if (!p.kvmap || !p.k.p || !p.v.p) return hipErrorInvalidValue;
  const dim3 grid(p.NKV - p.seg_from, p.BH);
  const bool kf = p.k.dtype == ICSA_DT_F32, vf = p.v.dtype == ICSA_DT_F32;
  if (kf && vf) hipLaunchKernelGGL((icsa_newkv_straddle_kernel<float, float>), grid, dim3(128), 0, stream, p);
  else if (kf) hipLaunchKernelGGL((icsa_newkv_straddle_kernel<float, bf16>), grid, dim3(128), 0, stream, p);
  else if (vf) hipLaunchKernelGGL((icsa_newkv_straddle_kernel<bf16, float>), grid, dim3(128), 0, stream, p);
  else hipLaunchKernelGGL((icsa_newkv_straddle_kernel<bf16, bf16>), grid, dim3(128), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// (f) level-3: per query block, top_k new-KV blocks by QCsum . KCsum (fp32), ascending list.
//     Scores: the fp32-accurate split-bf16 product of (a) on the raw sums (128 query blocks
//     of the list per workgroup, a third of the new-KV blocks), written to a scratch row
//     per query block.  Selection: one wave per query block, bisection over the float keys
//     (ballot counts), then compaction in ascending block order.
// ---------------------------------------------------------------------------------------
template <int VPL>   // scores per lane: NKV <= 64 * VPL
__global__ void __launch_bounds__(256) icsa_level3_select_kernel(Level3Params p) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;          // over BH * n_rows
  if (row >= (int64_t)p.BH * p.n_rows) return;
  const int NKV = p.NKV, k = p.top_k;
  const float* srow = p.scores + row * NKV;
  uint32_t key[VPL];
#pragma unroll
  for (int u = 0; u < VPL; ++u) {
    const int j = lane + 64 * u;
    key[u] = j < NKV ? f2key(srow[j]) : 0u;         // 0 is below every real key
  }
  const int nu = (NKV + 63) / 64;
  const uint32_t lo = kth_largest_key<VPL>(key, k, nu);
  int cgt = 0;
#pragma unroll
  for (int g = 0; g < VPL; g += 4)
    if (g < nu) {
#pragma unroll
      for (int u = g; u < g + 4; ++u) cgt += wave_count(key[u] > lo);
    }
  const int need_eq = k - cgt;
  const unsigned long long lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int seen_eq = 0, taken = 0;
  int* out = p.idx + row * k;
#pragma unroll
  for (int g = 0; g < VPL; g += 4)
    if (g < nu) {
#pragma unroll
      for (int u = g; u < g + 4; ++u) {
        const int j = lane + 64 * u;
        const bool gt = key[u] > lo;
        const bool eq = key[u] == lo && j < NKV;
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
  if (p.n_rows <= 0) return hipSuccess;
  Split3Gemm g;
  g.A = p.qsum; g.rows = p.rows; g.rows_stride = p.rows_stride; g.rows_offset = p.rows_offset;
  g.a_rows = p.NQsrc; g.n_rows = p.n_rows; g.B = p.kc32; g.n_cols = p.NKV; g.C = p.scores;
  g.NB = 0; g.S = 0; g.div = 1.f;
  hipLaunchKernelGGL(icsa_split3_gemm_kernel<false>, dim3((p.n_rows + LG_ROWS - 1) / LG_ROWS, LG_SPLIT, p.BH),
                     dim3(256), 0, stream, g);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = (int64_t)p.BH * p.n_rows;
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (p.NKV <= 256)
    hipLaunchKernelGGL(icsa_level3_select_kernel<4>, grid, dim3(256), 0, stream, p);
  else if (p.NKV <= 512)
    hipLaunchKernelGGL(icsa_level3_select_kernel<8>, grid, dim3(256), 0, stream, p);
  else if (p.NKV <= 1024)
    hipLaunchKernelGGL(icsa_level3_select_kernel<16>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(icsa_level3_select_kernel<32>, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}
