// Backward of the sparse piecewise attention with the first-order interval approximation.
//
// Reference: sparse_piecewise_attn_1st_intervals_bwd_kernel (triton_kernels.py:265-486) and
// SparsePiecewiseAttn1stIntervalsFunction.backward (:541-598).  With D = rowsum(dO * O)
// and P = exp2(s - lse) (scores in log2-scaled units, lse saved by the forward):
//   exact blocks (the top_k selected per query block):
//     dS = P (dO V^T - D);  dq += dS K scale;  dk += dS^T q scale;  dv += P^T dO
//   interval blocks (every unselected block c < NKV, block sums KC / VC):
//     s = q KC^T scale / 64;  dS = P (dO VC^T - 64 D);  dq += dS KC scale / 64;
//     each key row of block c gets dKC_c / 64 = (dS^T q)_c scale / 64 and dVC_c = (P^T dO)_c.
//
// The reference adds dk / dv (and dq) with fp32 atomics, so its sums depend on timing.  Here
// every gradient is a fixed-order sum:
//   * icsa_sparse_bwd_dq_kernel: one workgroup per query block (dq rows are owned);
//   * icsa_sparse_bwd_dkv_kernel<true>: one workgroup per (chunk of 64 compressed blocks,
//     range of query blocks) -> interval partials dKC / dVC, summed later in split order;
//   * icsa_sparse_bwd_dkv_kernel<false>: one workgroup per key block; it walks the query
//     blocks that selected it in ascending order (from the selection bitmap) and adds the
//     interval partials in its epilogue.
//
// MFMA orientation (v_mfma_f32_32x32x16_bf16, the tile toolkit of the forward):
//   dq kernel: S^T = K Q^T and dP^T = V dO^T with the K / V rows in LDS and Q, dO of the
//     wave's 32 queries in registers; dQ^T += K^T dS^T with K^T (kv_slot order) in LDS.
//   dk / dv kernel, the roles swapped: S = Q K^T and dP = dO V^T with the Q / dO rows in
//     LDS and K, V of the wave's 32 keys in registers; dV^T += dO^T P and dK^T += Q^T dS
//     with the transposed Q / dO tiles in LDS.
// P and dS are rounded to bf16 for the MFMA (the reference rounds P for dv and uses fp32
// dots for dq / dk).  Workgroup = 2 waves; wave w owns queries (or keys) 32 w .. 32 w + 31.
#include "attn_tile.h"
#include "icsa_kernels.h"

#define BW_THREADS 128
#define BW_MAX_TOPK 512
#define BW_MAX_CHUNKS 32                 // NKV <= 2048
#define BW_MAX_NQ 4096
#define BW_STAGE_BYTES (32 * O_LDS_STRIDE * 4)   // one wave's fp32 staging rows

// 64 x 128 bf16 row tile (rows at src, row stride rs elements) -> LDS, XOR-swizzled as a K tile.
__device__ __forceinline__ void bw_row_tile(bf16* dst, const bf16* src, int64_t rs) {
  const int t = threadIdx.x;
  const int c = t & 15;
  u32x4 r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = *reinterpret_cast<const u32x4*>(src + (int64_t)((t >> 4) + 8 * i) * rs + 8 * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(dst + k_lds_off((t >> 4) + 8 * i, c)) = r[i];
}

// [128 d][64 slots] bf16 transposed tile (d rows at src, d stride ds elements) -> LDS,
// XOR-swizzled as a V^T tile.
__device__ __forceinline__ void bw_t_tile(bf16* dst, const bf16* src, int64_t ds) {
  const int t = threadIdx.x;
  const int c = t & 7;
  u32x4 r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = *reinterpret_cast<const u32x4*>(src + (int64_t)((t >> 3) + 16 * i) * ds + 8 * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(dst + v_lds_off((t >> 3) + 16 * i, c)) = r[i];
}

// ------------------------------------------------------------------------------------------
// prep: D = rowsum(dO * O) per query row and the selection bitmap of each query block
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) icsa_sparse_bwd_rows_kernel(SparseBwdParams p) {
  __shared__ unsigned long long sel[BW_MAX_CHUNKS];
  const int i = blockIdx.x, bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int t = threadIdx.x;
  if (t < p.nc) sel[t] = 0ull;
  __syncthreads();
  const int* row = p.idx + ((int64_t)bh * p.NQ + i) * p.top_k;
  for (int u = t; u < p.top_k; u += 256) {
    const int j = row[u];
    if (j >= 0 && j < p.NKV) atomicOr(&sel[j >> 6], 1ull << (j & 63));
  }
  const int r = t >> 2, qq = t & 3;               // row, quarter of D (32 elements)
  const int tok = i * ICSA_BLOCK + r;
  const bf16* dor = p.dout + (int64_t)b * p.do_sb + (int64_t)h * p.do_sh + (int64_t)tok * p.do_st + 32 * qq;
  const bf16* orr = p.out + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)tok * p.o_st + 32 * qq;
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(dor + 8 * c);
    const bf16x8 o = *reinterpret_cast<const bf16x8*>(orr + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf((float)a[e], (float)o[e], acc);
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  if (qq == 0) p.dvec[(int64_t)bh * p.TQ + tok] = acc;
  __syncthreads();
  if (t < p.nc) p.selbits[((int64_t)bh * p.NQ + i) * p.nc + t] = sel[t];
}

// prep: bf16 block sums (rows, and transposed in kv_slot order) from the f32 sums
__global__ void __launch_bounds__(256) icsa_sparse_bwd_sums_kernel(SparseBwdParams p) {
  __shared__ bf16 tile[ICSA_BLOCK][ICSA_D + 8];
  const int ch = blockIdx.x, bh = blockIdx.y;
  const int t = threadIdx.x;
  const int r = t >> 2, qq = t & 3;
  const int c = ch * ICSA_BLOCK + r;              // block index (< NKVp)
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const float* src = (part == 0 ? p.ksum : p.vsum) + ((int64_t)bh * p.NKV + c) * ICSA_D + 32 * qq;
    bf16* dst = (part == 0 ? p.kcb : p.vcb) + ((int64_t)bh * p.NKVp + c) * ICSA_D + 32 * qq;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float v[8];
      if (c < p.NKV) {
        load8_f32<float>(src + 8 * g, v);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
      const bf16x8 o = pack8_bf16(v);
      *reinterpret_cast<bf16x8*>(dst + 8 * g) = o;
      if (part == 0) *reinterpret_cast<bf16x8*>(&tile[r][32 * qq + 8 * g]) = o;
    }
  }
  __syncthreads();
  const int d = t >> 1, half = t & 1;
  bf16* dst = p.kct + ((int64_t)bh * ICSA_D + d) * p.NKVp + (int64_t)ch * ICSA_BLOCK + 32 * half;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = tile[kv_slot(32 * half + 8 * q4 + e)][d];
    *reinterpret_cast<bf16x8*>(dst + 8 * q4) = o;
  }
}

// ------------------------------------------------------------------------------------------
// dq: one workgroup per query block
// ------------------------------------------------------------------------------------------
__global__ void __launch_bounds__(BW_THREADS) icsa_sparse_bwd_dq_kernel(SparseBwdParams p) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[3 * K_TILE_BYTES];
  __shared__ int src_l[BW_MAX_TOPK];
  __shared__ unsigned long long sel_l[BW_MAX_CHUNKS];
  bf16* ks = reinterpret_cast<bf16*>(smem);
  bf16* vs = reinterpret_cast<bf16*>(smem + K_TILE_BYTES);
  bf16* kts = reinterpret_cast<bf16*>(smem + 2 * K_TILE_BYTES);

  const int n_work = p.B * p.H * p.NQ;
  const int work = xcd_remap(blockIdx.x, n_work);
  if (work < 0) return;
  const int bh = work / p.NQ, qb = work % p.NQ;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 31;
  const int qtok0 = qb * ICSA_BLOCK + 32 * wave;

  for (int c = tid; c < p.nc; c += BW_THREADS) sel_l[c] = p.selbits[((int64_t)bh * p.NQ + qb) * p.nc + c];
  for (int u = tid; u < p.top_k; u += BW_THREADS) {
    const int j = p.idx[((int64_t)bh * p.NQ + qb) * p.top_k + u];
    src_l[u] = (j >= 0 && j < p.NKV) ? j : -1;    // out-of-range entries: zero blocks, no gradient
  }
  bf16x8 qf[8], dof[8];
  load_q_frags(qf, p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)qtok0 * p.q_st, p.q_st, 32);
  load_q_frags(dof, p.dout + (int64_t)b * p.do_sb + (int64_t)h * p.do_sh + (int64_t)qtok0 * p.do_st, p.do_st, 32);
  const float lse = p.lse[(int64_t)bh * p.TQ + qtok0 + li];
  const float dd = p.dvec[(int64_t)bh * p.TQ + qtok0 + li];
  __syncthreads();

  const bf16* kb = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  const bf16* ktb = p.kt + (int64_t)bh * ICSA_D * p.TKV;
  floatx16 dq[4] = {};
  floatx16 s[2], dp[2];
  bf16x8 dsf[4];

  // ---- exact blocks ----
  for (int t = 0; t < p.top_k; ++t) {
    const int j = src_l[t];
    if (j < 0) continue;
    __syncthreads();                                   // previous tiles consumed
    bw_row_tile(ks, kb + (int64_t)j * ICSA_BLOCK * p.k_st, p.k_st);
    bw_row_tile(vs, vb + (int64_t)j * ICSA_BLOCK * p.v_st, p.v_st);
    bw_t_tile(kts, ktb + (int64_t)j * ICSA_BLOCK, p.TKV);
    __syncthreads();
    qk_tile(s, ks, qf);
    qk_tile(dp, vs, dof);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float pr = __builtin_amdgcn_exp2f(fmaf(s[sub][e], p.scale_log2, -lse));
        dsf[2 * sub + (e >> 3)][e & 7] = (bf16)(pr * (dp[sub][e] - dd));
      }
    pv_tile(dq, kts, dsf);
  }

  // ---- interval chunks: unselected compressed blocks, score / 64, dS / 64 ----
  const float c64 = p.scale_log2 * (1.0f / 64.0f);
  for (int ch = 0; ch < p.nc; ++ch) {
    __syncthreads();
    bw_row_tile(ks, p.kcb + ((int64_t)bh * p.NKVp + ch * ICSA_BLOCK) * ICSA_D, ICSA_D);
    bw_row_tile(vs, p.vcb + ((int64_t)bh * p.NKVp + ch * ICSA_BLOCK) * ICSA_D, ICSA_D);
    bw_t_tile(kts, p.kct + (int64_t)bh * ICSA_D * p.NKVp + ch * ICSA_BLOCK, p.NKVp);
    __syncthreads();
    qk_tile(s, ks, qf);
    qk_tile(dp, vs, dof);
    const unsigned long long selm = sel_l[ch];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int jj = 32 * sub + acc_row(e, lane);
        const bool masked = (ch * ICSA_BLOCK + jj >= p.NKV) || ((selm >> jj) & 1ull);
        const float pr = masked ? 0.f : __builtin_amdgcn_exp2f(fmaf(s[sub][e], c64, -lse));
        dsf[2 * sub + (e >> 3)][e & 7] = (bf16)(pr * (dp[sub][e] - 64.0f * dd) * (1.0f / 64.0f));
      }
    pv_tile(dq, kts, dsf);
  }

  // ---- epilogue: dq = scale * acc ----
  __syncthreads();
  float* o_lds = reinterpret_cast<float*>(smem + wave * BW_STAGE_BYTES);
  stage_o(o_lds, dq, p.scale);
  __syncthreads();
  AlphaView none;
  none.p = nullptr; none.scalar = 0.f; none.sb = none.ss = none.sh = none.sd = 0; none.dtype = ICSA_DT_F32;
  store_rows(o_lds, p.dq, b, h, qtok0, 32, nullptr, none);
}

// ------------------------------------------------------------------------------------------
// dk / dv: kInterval = true -> interval partials per (chunk, query range);
//          kInterval = false -> exact part per key block + the summed partials
// ------------------------------------------------------------------------------------------
#define BWKV_TILES_BYTES (4 * K_TILE_BYTES)
#define BWKV_LDS_BYTES (BWKV_TILES_BYTES + 2 * 64 * 4 + 2 * ICSA_D * 4 + BW_MAX_NQ * 2 + 16)

template <bool kInterval>
__global__ void __launch_bounds__(BW_THREADS) icsa_sparse_bwd_dkv_kernel(SparseBwdParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_dyn[];
  bf16* qs = reinterpret_cast<bf16*>(smem_dyn);
  bf16* dos = reinterpret_cast<bf16*>(smem_dyn + K_TILE_BYTES);
  bf16* qts = reinterpret_cast<bf16*>(smem_dyn + 2 * K_TILE_BYTES);
  bf16* dots = reinterpret_cast<bf16*>(smem_dyn + 3 * K_TILE_BYTES);
  float* lse_l = reinterpret_cast<float*>(smem_dyn + BWKV_TILES_BYTES);
  float* dd_l = lse_l + 64;
  float* ivec = dd_l + 64;                             // [2][128] interval sums (exact kernel)
  unsigned short* qlist = reinterpret_cast<unsigned short*>(ivec + 2 * ICSA_D);
  int* qcount = reinterpret_cast<int*>(qlist + BW_MAX_NQ);

  const int n_work = kInterval ? p.B * p.H * p.nc * p.nsplit : p.B * p.H * p.NKV;
  const int work = xcd_remap(blockIdx.x, n_work);
  if (work < 0) return;
  int bh, blk, split = 0;
  if (kInterval) {
    bh = work / (p.nc * p.nsplit);
    const int rem = work % (p.nc * p.nsplit);
    blk = rem / p.nsplit;                              // chunk of 64 compressed blocks
    split = rem % p.nsplit;
  } else {
    bh = work / p.NKV;
    blk = work % p.NKV;                                // key block
  }
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 31;
  const int key0 = blk * ICSA_BLOCK + 32 * wave;       // this wave's first key (or compressed block)

  bf16x8 kf[8], vf[8];
  if (kInterval) {
    load_q_frags(kf, p.kcb + ((int64_t)bh * p.NKVp + key0) * ICSA_D, ICSA_D, 32);
    load_q_frags(vf, p.vcb + ((int64_t)bh * p.NKVp + key0) * ICSA_D, ICSA_D, 32);
  } else {
    load_q_frags(kf, p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh + (int64_t)key0 * p.k_st, p.k_st, 32);
    load_q_frags(vf, p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + (int64_t)key0 * p.v_st, p.v_st, 32);
  }

  // query blocks to visit, ascending
  int i_begin = 0, i_count;
  if (kInterval) {
    i_begin = split * p.qb_per_split;
    i_count = max(0, min(p.NQ, i_begin + p.qb_per_split) - i_begin);
  } else {
    if (wave == 0) {
      const int w = blk >> 6;
      const unsigned long long bit = 1ull << (blk & 63);
      int cnt = 0;
      for (int base = 0; base < p.NQ; base += 64) {
        const int i = base + lane;
        const bool on = i < p.NQ && (p.selbits[((int64_t)bh * p.NQ + i) * p.nc + w] & bit) != 0ull;
        const unsigned long long bal = __ballot(on);
        if (on) qlist[cnt + __popcll(bal & ((1ull << lane) - 1ull))] = (unsigned short)i;
        cnt += __popcll(bal);
      }
      if (lane == 0) *qcount = cnt;
    }
    __syncthreads();
    i_count = *qcount;
  }

  const int ckey = key0 + li;                          // interval: this lane's compressed block
  const bool key_valid = !kInterval || ckey < p.NKV;
  const float cexp = kInterval ? p.scale_log2 * (1.0f / 64.0f) : p.scale_log2;
  const float dmul = kInterval ? 64.0f : 1.0f;
  const float dsmul = kInterval ? (1.0f / 64.0f) : 1.0f;

  const bf16* qb0 = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const bf16* dob0 = p.dout + (int64_t)b * p.do_sb + (int64_t)h * p.do_sh;
  const bf16* qtb = p.qt + (int64_t)bh * ICSA_D * p.TQ;
  const bf16* dotb = p.dot + (int64_t)bh * ICSA_D * p.TQ;
  floatx16 dk[4] = {}, dv[4] = {};
  floatx16 s[2], dp[2];
  bf16x8 pf[4], dsf[4];

  for (int n = 0; n < i_count; ++n) {
    const int i = kInterval ? i_begin + n : (int)qlist[n];
    __syncthreads();                                   // previous tiles consumed
    bw_row_tile(qs, qb0 + (int64_t)i * ICSA_BLOCK * p.q_st, p.q_st);
    bw_row_tile(dos, dob0 + (int64_t)i * ICSA_BLOCK * p.do_st, p.do_st);
    bw_t_tile(qts, qtb + (int64_t)i * ICSA_BLOCK, p.TQ);
    bw_t_tile(dots, dotb + (int64_t)i * ICSA_BLOCK, p.TQ);
    if (tid < 64) {
      lse_l[tid] = p.lse[(int64_t)bh * p.TQ + i * ICSA_BLOCK + tid];
      dd_l[tid] = p.dvec[(int64_t)bh * p.TQ + i * ICSA_BLOCK + tid];
    }
    bool on = key_valid;
    if (kInterval) on = on && ((p.selbits[((int64_t)bh * p.NQ + i) * p.nc + blk] >> (32 * wave + li)) & 1ull) == 0ull;
    __syncthreads();
    qk_tile(s, qs, kf);                                // S[q][key]: lane = key, elements = queries
    qk_tile(dp, dos, vf);
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r0 = 32 * sub + 8 * g + 4 * (lane >> 5);    // acc_row(4 g + x, lane) = r0 + x
        const floatx4 l4 = *reinterpret_cast<const floatx4*>(lse_l + r0);
        const floatx4 d4 = *reinterpret_cast<const floatx4*>(dd_l + r0);
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          const int e = 4 * g + x;
          const float pr = on ? __builtin_amdgcn_exp2f(fmaf(s[sub][e], cexp, -l4[x])) : 0.f;
          pf[2 * sub + (e >> 3)][e & 7] = (bf16)pr;
          dsf[2 * sub + (e >> 3)][e & 7] = (bf16)(pr * (dp[sub][e] - dmul * d4[x]) * dsmul);
        }
      }
    pv_tile(dv, dots, pf);                             // dV^T[d][key] += dO^T P
    pv_tile(dk, qts, dsf);                             // dK^T[d][key] += Q^T dS
  }

  __syncthreads();
  float* o_lds = reinterpret_cast<float*>(smem_dyn + wave * BW_STAGE_BYTES);
  AlphaView one;
  one.p = nullptr; one.scalar = 1.f; one.sb = one.ss = one.sh = one.sd = 0; one.dtype = ICSA_DT_F32;
  if (kInterval) {
    // partials [split][bh][NKVp][D] (dk part without the scale; dS already carries 1/64)
    const int64_t base = (((int64_t)split * p.B * p.H + bh) * p.NKVp) * ICSA_D;
    stage_o(o_lds, dk, 1.f);
    __syncthreads();
    store_rows(o_lds, OutView{p.dkc_part + base, 0, ICSA_D, 0, ICSA_DT_F32}, 0, 0, key0, 32, nullptr, one);
    __syncthreads();
    stage_o(o_lds, dv, 1.f);
    __syncthreads();
    store_rows(o_lds, OutView{p.dvc_part + base, 0, ICSA_D, 0, ICSA_DT_F32}, 0, 0, key0, 32, nullptr, one);
  } else {
    // interval contributions of this block, summed over the splits in order
    {
      const int d = tid;                               // 128 threads = 128 dims
      float sk = 0.f, sv = 0.f;
      for (int sp = 0; sp < p.nsplit; ++sp) {
        const int64_t off = ((((int64_t)sp * p.B * p.H + bh) * p.NKVp) + blk) * ICSA_D + d;
        sk += p.dkc_part[off];
        sv += p.dvc_part[off];
      }
      ivec[d] = sk * p.scale;
      ivec[ICSA_D + d] = sv;
    }
    stage_o(o_lds, dk, p.scale);
    __syncthreads();
    store_rows(o_lds, p.dk, b, h, key0, 32, ivec, one);
    __syncthreads();
    stage_o(o_lds, dv, 1.f);
    __syncthreads();
    store_rows(o_lds, p.dv, b, h, key0, 32, ivec + ICSA_D, one);
  }
}

hipError_t launch_sparse_bwd_prep(const SparseBwdParams& p, hipStream_t stream) {
  const int BH = p.B * p.H;
  if (BH == 0 || p.NQ == 0) return hipSuccess;
  if (p.nc > BW_MAX_CHUNKS || p.NKVp != p.nc * ICSA_BLOCK) return hipErrorInvalidValue;
  hipLaunchKernelGGL(icsa_sparse_bwd_rows_kernel, dim3(p.NQ, BH), dim3(256), 0, stream, p);
  hipLaunchKernelGGL(icsa_sparse_bwd_sums_kernel, dim3(p.nc, BH), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_sparse_bwd(const SparseBwdParams& p, hipStream_t stream) {
  const int BH = p.B * p.H;
  if (BH == 0 || p.NQ == 0) return hipSuccess;
  if (p.top_k < 1 || p.top_k > BW_MAX_TOPK || p.NKV < 1 || p.nc > BW_MAX_CHUNKS ||
      p.NKVp != p.nc * ICSA_BLOCK || p.NQ > BW_MAX_NQ || p.nsplit < 1 ||
      (int64_t)p.nsplit * p.qb_per_split < p.NQ)
    return hipErrorInvalidValue;
  static const hipError_t attr_i = hipFuncSetAttribute(
      reinterpret_cast<const void*>(icsa_sparse_bwd_dkv_kernel<true>),
      hipFuncAttributeMaxDynamicSharedMemorySize, BWKV_LDS_BYTES);
  static const hipError_t attr_e = hipFuncSetAttribute(
      reinterpret_cast<const void*>(icsa_sparse_bwd_dkv_kernel<false>),
      hipFuncAttributeMaxDynamicSharedMemorySize, BWKV_LDS_BYTES);
  if (attr_i != hipSuccess) return attr_i;
  if (attr_e != hipSuccess) return attr_e;
  hipLaunchKernelGGL(icsa_sparse_bwd_dq_kernel, dim3(xcd_grid(BH * p.NQ)), dim3(BW_THREADS), 0, stream, p);
  hipLaunchKernelGGL(icsa_sparse_bwd_dkv_kernel<true>, dim3(xcd_grid(BH * p.nc * p.nsplit)), dim3(BW_THREADS),
                     BWKV_LDS_BYTES, stream, p);
  hipLaunchKernelGGL(icsa_sparse_bwd_dkv_kernel<false>, dim3(xcd_grid(BH * p.NKV)), dim3(BW_THREADS),
                     BWKV_LDS_BYTES, stream, p);
  return hipGetLastError();
}
