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
// Ragged lengths (the Triton host): NQ = cdiv(TQ, 64), NKV = cdiv(TKV, 64).  Rows past TQ
// and TKV read as zero (q, dO, lse, D, k, v: the tensor descriptors' zero fill), keys past
// TKV are masked out of the exact part (triton_kernels.py:348), and gradient rows past TQ /
// TKV are not stored.
// P and dS are rounded to bf16 for the MFMA (the reference rounds P for dv and uses fp32
// dots for dq / dk).  Workgroup = 2 waves; wave w owns queries (or keys) 32 w .. 32 w + 31.
#include "attn_tile.h"
#include "icsa_kernels.h"

#define BW_THREADS 128
#define BW_MAX_TOPK 512
#define BW_MAX_CHUNKS 32                 // NKV <= 2048
#define BW_MAX_NQ 4096
#define BW_STAGE_BYTES (32 * O_LDS_STRIDE * 4)   // one wave's fp32 staging rows

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
  float acc = 0.f;
  if (tok < p.TQ) {                               // rows past TQ: D = 0
  const bf16* dor = p.dout + (int64_t)b * p.do_sb + (int64_t)h * p.do_sh + (int64_t)tok * p.do_st + 32 * qq;
  const bf16* orr = p.out + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)tok * p.o_st + 32 * qq;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(dor + 8 * c);
    const bf16x8 o = *reinterpret_cast<const bf16x8*>(orr + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf((float)a[e], (float)o[e], acc);
  }
  }
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  if (qq == 0) p.dvec[(int64_t)bh * p.NQ * ICSA_BLOCK + tok] = acc;   // D rows padded to NQ * 64
  __syncthreads();
  if (t < p.nc) p.selbits[((int64_t)bh * p.NQ + i) * p.nc + t] = sel[t];
}

// prep: bf16 block sums from the f32 sums (rows >= NKV zero)
__global__ void __launch_bounds__(256) icsa_sparse_bwd_sums_kernel(SparseBwdParams p) {
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
      *reinterpret_cast<bf16x8*>(dst + 8 * g) = pack8_bf16(v);
    }
  }
}

// ------------------------------------------------------------------------------------------
// Tile DMA.  A 16 KB row tile (64 rows x 128 dims, swizzled by rt_swz) is 16
// LDS-DMA instructions, 8 per wave; each lands 1 KB at consecutive LDS addresses (lane l
// at +16 l), so the XOR swizzle is applied on the global side.  A step's tiles are the only
// loads in flight when a kernel waits for them (vmcnt(0)): the next step's tiles are issued
// after the workgroup barrier that follows, which also tells that both waves are done with
// the buffer they overwrite (two buffers, one barrier per step).
// ------------------------------------------------------------------------------------------
#define BW_WAIT(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")

// Row tiles use the shared layout of attn_tile.h (rt_swz / rt_off).
#define BW_PF 3                 // MFMA operand read-ahead (steps)

// S^T (or S) for the 64 rows of a backward row tile: s[sub] covers rows 32 sub .. 32 sub + 31.
// Step t uses sub = t % 2 and dims 16 (t / 2) .. + 15; operands are read BW_PF steps ahead
// (with one wave per SIMD nothing else hides the LDS latency).
__device__ __forceinline__ void qk_tile_bw(floatx16 s[2], const bf16* tile, const bf16x8 bf[8]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, hl = lane >> 5;
  auto ld = [&](int t) -> bf16x8 {
    return *reinterpret_cast<const bf16x8*>(tile + rt_off(32 * (t & 1) + li, 2 * (t >> 1) + hl));
  };
  bf16x8 a[16];
#pragma unroll
  for (int t = 0; t < BW_PF; ++t) a[t] = ld(t);
  __builtin_amdgcn_sched_barrier(0);
  floatx16 acc0 = {}, acc1 = {};
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    if (t + BW_PF < 16) a[t + BW_PF] = ld(t + BW_PF);
    if (t & 1) acc1 = mfma32x32x16(a[t], bf[t >> 1], acc1);
    else acc0 = mfma32x32x16(a[t], bf[t >> 1], acc0);
    __builtin_amdgcn_sched_barrier(0);
  }
  s[0] = acc0;
  s[1] = acc1;
}

// Rows >= valid lie outside the buffer range and land nothing: bw_fill_rows zeroes them once
// the tile's loads have completed.
__device__ __forceinline__ void bw_dma_rows(unsigned char* tile, const bf16* base, int64_t rs, int wave,
                                            int lane, int valid = ICSA_BLOCK) {
  const __amdgpu_buffer_rsrc_t rsrc =
      make_rsrc(base, valid > 0 ? ((int64_t)(valid - 1) * rs + ICSA_D) * 2 : 0);
  unsigned char* dst = tile + wave * 8192;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 32 * wave + 4 * i + (lane >> 4);
    const int off = (int)(r * rs * 2) + (((lane & 15) ^ rt_swz(r)) << 4);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr)(dst + 1024 * i), 16, off, 0, 0, 0);
  }
}

// Zero this wave's rows >= valid of a row tile (the bytes its DMA lanes would have landed).
__device__ __forceinline__ void bw_fill_rows(unsigned char* tile, int valid, int wave, int lane) {
  if (valid >= ICSA_BLOCK) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 32 * wave + 4 * i + (lane >> 4);
    if (r >= valid) *reinterpret_cast<u32x4*>(tile + r * ICSA_D * 2 + (lane & 15) * 16) = u32x4{0u, 0u, 0u, 0u};
  }
}


// ------------------------------------------------------------------------------------------
// dq: one workgroup per query block.  Steps t = 0 .. n_ex + nc - 1: the valid selected
// blocks, then the interval chunks.  Per step the K and V rows (16 DMA per wave) land in
// one of two buffers while the other step's S^T = K Q^T, dP^T = V dO^T and
// dQ^T += K^T dS^T (K^T read transposed from the K rows) run.
// ------------------------------------------------------------------------------------------
#define BWQ_LDS_BYTES (4 * K_TILE_BYTES + BW_MAX_TOPK * 4 + BW_MAX_CHUNKS * 8 + 16)

__global__ void __launch_bounds__(BW_THREADS) icsa_sparse_bwd_dq_kernel(SparseBwdParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_q[];
  int* src_l = reinterpret_cast<int*>(smem_q + 4 * K_TILE_BYTES);
  unsigned long long* sel_l = reinterpret_cast<unsigned long long*>(src_l + BW_MAX_TOPK);
  int* n_ex_l = reinterpret_cast<int*>(sel_l + BW_MAX_CHUNKS);

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
  if (wave == 0) {                                     // valid selected blocks, list order kept
    const int* row = p.idx + ((int64_t)bh * p.NQ + qb) * p.top_k;
    int cnt = 0;
    for (int base = 0; base < p.top_k; base += 64) {
      const int u = base + lane;
      const int j = u < p.top_k ? row[u] : -1;
      const bool on = j >= 0 && j < p.NKV;            // out-of-range entries: zero blocks, no gradient
      const unsigned long long bal = __ballot(on);
      if (on) src_l[cnt + __popcll(bal & ((1ull << lane) - 1ull))] = j;
      cnt += __popcll(bal);
    }
    if (lane == 0) *n_ex_l = cnt;
  }
  const int q_valid = max(0, min(32, p.TQ - qtok0));  // this wave's real query rows
  bf16x8 qf[8], dof[8];
  load_q_frags(qf, p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh + (int64_t)qtok0 * p.q_st, p.q_st, q_valid);
  load_q_frags(dof, p.dout + (int64_t)b * p.do_sb + (int64_t)h * p.do_sh + (int64_t)qtok0 * p.do_st, p.do_st,
               q_valid);
  const float lse = li < q_valid ? p.lse[(int64_t)bh * p.TQ + qtok0 + li] : 0.f;
  const float dd = p.dvec[(int64_t)bh * p.NQ * ICSA_BLOCK + qtok0 + li];
  int tro[4];
  rt_tr_offsets<false>(tro, lane);
  __syncthreads();
  const int n_ex = *n_ex_l;
  const int T = n_ex + p.nc;

  const bf16* kb = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16* vb = p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  const bf16* kcb = p.kcb + (int64_t)bh * p.NKVp * ICSA_D;
  const bf16* vcb = p.vcb + (int64_t)bh * p.NKVp * ICSA_D;
  // real key rows of exact step t (the last block of a ragged TKV is partial)
  auto key_rows = [&](int t) -> int {
    return min(ICSA_BLOCK, p.TKV - __builtin_amdgcn_readfirstlane(src_l[t]) * ICSA_BLOCK);
  };
  // buffer u: K rows at 2 u tiles, V rows at 2 u + 1
  auto issue = [&](int t) {
    unsigned char* kt = smem_q + (t & 1) * 2 * K_TILE_BYTES;
    if (t < n_ex) {
      const int j = __builtin_amdgcn_readfirstlane(src_l[t]);
      const int valid = key_rows(t);
      bw_dma_rows(kt, kb + (int64_t)j * ICSA_BLOCK * p.k_st, p.k_st, wave, lane, valid);
      bw_dma_rows(kt + K_TILE_BYTES, vb + (int64_t)j * ICSA_BLOCK * p.v_st, p.v_st, wave, lane, valid);
    } else {
      const int ch = t - n_ex;
      bw_dma_rows(kt, kcb + (int64_t)ch * ICSA_BLOCK * ICSA_D, ICSA_D, wave, lane);
      bw_dma_rows(kt + K_TILE_BYTES, vcb + (int64_t)ch * ICSA_BLOCK * ICSA_D, ICSA_D, wave, lane);
    }
  };

  floatx16 dq[4] = {};
  floatx16 s[2], dp[2];
  bf16x8 dsf[4];
  const float c64 = p.scale_log2 * (1.0f / 64.0f);
  issue(0);                                            // T >= nc >= 1
  for (int t = 0; t < T; ++t) {
    const int kvalid = t < n_ex ? key_rows(t) : ICSA_BLOCK;
    BW_WAIT(0);                                        // step t's tiles, the only loads in flight
    if (kvalid < ICSA_BLOCK) {                         // zero key / value rows past TKV
      bw_fill_rows(smem_q + (t & 1) * 2 * K_TILE_BYTES, kvalid, wave, lane);
      bw_fill_rows(smem_q + (t & 1) * 2 * K_TILE_BYTES + K_TILE_BYTES, kvalid, wave, lane);
    }
    ATT_BARRIER();                                     // step t complete; step t - 1's buffer read by both waves
    if (t + 1 < T) issue(t + 1);                       // into that buffer
    const unsigned char* ks = smem_q + (t & 1) * 2 * K_TILE_BYTES;
    qk_tile_bw(s, reinterpret_cast<const bf16*>(ks), qf);                  // S^T[key][query]
    qk_tile_bw(dp, reinterpret_cast<const bf16*>(ks + K_TILE_BYTES), dof); // dP^T
    if (t < n_ex) {
      const int thr = mask_threshold(kvalid, lane);
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const bool masked = acc_row_const(sub, e) >= thr;           // keys past TKV
          const float pr = masked ? 0.f : __builtin_amdgcn_exp2f(fmaf(s[sub][e], p.scale_log2, -lse));
          dsf[2 * sub + (e >> 3)][e & 7] = (bf16)(pr * (dp[sub][e] - dd));
        }
    } else {                                           // unselected block sums: score / 64, dS / 64
      const int ch = t - n_ex;
      // masked blocks of the chunk (selected, or >= NKV) as one word; element e of sub-tile
      // sub is bit 8 (e / 4) + e % 4 of word sub of that word >> 4 hl
      unsigned long long mb = sel_l[ch];
      const int n_real = p.NKV - ch * ICSA_BLOCK;
      if (n_real < ICSA_BLOCK) mb |= ~0ull << n_real;
      const unsigned long long ml = mb >> (4 * (lane >> 5));
      const unsigned wd[2] = {(unsigned)ml, (unsigned)(ml >> 32)};
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const bool masked = (wd[sub] >> (8 * (e >> 2) + (e & 3))) & 1u;
          const float pr = masked ? 0.f : __builtin_amdgcn_exp2f(fmaf(s[sub][e], c64, -lse));
          dsf[2 * sub + (e >> 3)][e & 7] = (bf16)(pr * (dp[sub][e] - 64.0f * dd) * (1.0f / 64.0f));
        }
    }
    pv_tile_tr<BW_PF, false>(dq, ks, tro, dsf);                      // dQ^T += K^T dS^T
  }

  // ---- epilogue: dq = scale * acc ----
  __syncthreads();
  float* o_lds = reinterpret_cast<float*>(smem_q + wave * BW_STAGE_BYTES);
  stage_o(o_lds, dq, p.scale);
  __syncthreads();
  AlphaView none;
  none.p = nullptr; none.scalar = 0.f; none.sb = none.ss = none.sh = none.sd = 0; none.dtype = ICSA_DT_F32;
  store_rows(o_lds, p.dq, b, h, qtok0, q_valid, nullptr, none);
}

// ------------------------------------------------------------------------------------------
// dk / dv: kInterval = true -> interval partials per (chunk, query range);
//          kInterval = false -> exact part per key block + the summed partials.
// Per visited query block: its Q and dO rows plus lse (wave 0) / D (wave 1), 17 DMA per
// wave, land in one of two buffers while the previous block's S = Q K^T, dP = dO V^T,
// dV^T += dO^T P and dK^T += Q^T dS run (Q^T, dO^T read transposed from the rows).
// ------------------------------------------------------------------------------------------
#define BWKV_BUF_BYTES (2 * K_TILE_BYTES + 2 * 64 * 4)      // Q rows, dO rows, lse, D
#define BWKV_LIST_BYTES 8192                 // exact: u16 query list; interval: u64 selection words
#define BWKV_LDS_BYTES (2 * BWKV_BUF_BYTES + 2 * ICSA_D * 4 + BWKV_LIST_BYTES + 16)

template <bool kInterval>
__global__ void __launch_bounds__(BW_THREADS) icsa_sparse_bwd_dkv_kernel(SparseBwdParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_dyn[];
  float* ivec = reinterpret_cast<float*>(smem_dyn + 2 * BWKV_BUF_BYTES);   // [2][128] interval sums
  unsigned char* list = reinterpret_cast<unsigned char*>(ivec + 2 * ICSA_D);
  unsigned short* qlist = reinterpret_cast<unsigned short*>(list);
  unsigned long long* wlist = reinterpret_cast<unsigned long long*>(list);
  int* qcount = reinterpret_cast<int*>(list + BWKV_LIST_BYTES);

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
  } else {                                             // keys past TKV read as zero
    const int kv = max(0, min(32, p.TKV - key0));
    load_q_frags(kf, p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh + (int64_t)key0 * p.k_st, p.k_st, kv);
    load_q_frags(vf, p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh + (int64_t)key0 * p.v_st, p.v_st, kv);
  }
  int tro[4];
  rt_tr_offsets<false>(tro, lane);

  // query blocks to visit, ascending
  int i_begin = 0, i_count;
  if (kInterval) {
    i_begin = split * p.qb_per_split;
    i_count = max(0, min(p.NQ, i_begin + p.qb_per_split) - i_begin);
    for (int u = tid; u < i_count; u += BW_THREADS)
      wlist[u] = p.selbits[((int64_t)bh * p.NQ + i_begin + u) * p.nc + blk];
    __syncthreads();
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

  const int ckey = key0 + li;                          // this lane's key (interval: compressed block)
  const bool key_valid = ckey < (kInterval ? p.NKV : p.TKV);
  const float cexp = kInterval ? p.scale_log2 * (1.0f / 64.0f) : p.scale_log2;
  const float dmul = kInterval ? 64.0f : 1.0f;
  const float dsmul = kInterval ? (1.0f / 64.0f) : 1.0f;

  const bf16* qb0 = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const bf16* dob0 = p.dout + (int64_t)b * p.do_sb + (int64_t)h * p.do_sh;
  const float* rowvec = wave == 0 ? p.lse + (int64_t)bh * p.TQ : p.dvec + (int64_t)bh * p.NQ * ICSA_BLOCK;
  auto qblock = [&](int n) -> int {
    return kInterval ? i_begin + n : __builtin_amdgcn_readfirstlane((int)qlist[n]);
  };
  // real query rows of block qblock(n) (the last block of a ragged TQ is partial)
  auto q_rows = [&](int n) -> int { return min(ICSA_BLOCK, p.TQ - qblock(n) * ICSA_BLOCK); };
  auto issue = [&](int n) {
    const int i = qblock(n), valid = q_rows(n);
    unsigned char* buf = smem_dyn + (n & 1) * BWKV_BUF_BYTES;
    bw_dma_rows(buf, qb0 + (int64_t)i * ICSA_BLOCK * p.q_st, p.q_st, wave, lane, valid);
    bw_dma_rows(buf + K_TILE_BYTES, dob0 + (int64_t)i * ICSA_BLOCK * p.do_st, p.do_st, wave, lane, valid);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(rowvec + (int64_t)i * ICSA_BLOCK, valid * 4);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_ptr)(buf + 2 * K_TILE_BYTES + wave * 256), 4,
                                             lane * 4, 0, 0, 0);
  };

  floatx16 dk[4] = {}, dv[4] = {};
  floatx16 s[2], dp[2];
  bf16x8 pf[4], dsf[4];
  if (i_count > 0) issue(0);
  for (int n = 0; n < i_count; ++n) {
    bool on = key_valid;
    if (kInterval) on = on && ((wlist[n] >> (32 * wave + li)) & 1ull) == 0ull;
    BW_WAIT(0);                                        // block n's tiles, the only loads in flight
    const int qvalid = q_rows(n);
    if (qvalid < ICSA_BLOCK) {                         // zero Q / dO rows and lse / D past TQ
      unsigned char* buf = smem_dyn + (n & 1) * BWKV_BUF_BYTES;
      bw_fill_rows(buf, qvalid, wave, lane);
      bw_fill_rows(buf + K_TILE_BYTES, qvalid, wave, lane);
      if (lane >= qvalid) reinterpret_cast<float*>(buf + 2 * K_TILE_BYTES + wave * 256)[lane] = 0.f;
    }
    ATT_BARRIER();                                     // block n complete; block n - 1's buffer read by both waves
    if (n + 1 < i_count) issue(n + 1);                 // into that buffer
    const unsigned char* qs = smem_dyn + (n & 1) * BWKV_BUF_BYTES;
    const unsigned char* dos = qs + K_TILE_BYTES;
    const float* lse_l = reinterpret_cast<const float*>(qs + 2 * K_TILE_BYTES);
    const float* dd_l = lse_l + 64;
    // One stream of 64 MFMAs, operands read BW_PF steps ahead, with the elementwise work
    // slotted between MFMAs that do not depend on it (one wave per SIMD: nothing else
    // fills the matrix pipe while this wave runs VALU code):
    //   t  0..15  S and dP of query rows 0-31   (t even: S = Q K^T, odd: dP = dO V^T; kk = t / 2 % 8)
    //   t 16..31  S and dP of rows 32-63        + P, dS of rows 0-31 (one element per MFMA)
    //   t 32..63  u = t - 32: m = u / 8, ds = u / 2 % 4; u even: dV^T += dO^T P, odd:
    //             dK^T += Q^T dS                + P, dS of rows 32-63 during u < 16
    const bf16* qsb = reinterpret_cast<const bf16*>(qs);
    const bf16* dosb = reinterpret_cast<const bf16*>(dos);
    const int hl = lane >> 5;
    auto ld = [&](int t) -> bf16x8 {
      if (t < 32) {
        const int sub = t >> 4, kk = (t & 15) >> 1;
        return *reinterpret_cast<const bf16x8*>(((t & 1) ? dosb : qsb) + rt_off(32 * sub + li, 2 * kk + hl));
      }
      const int u = t - 32, m = u >> 3, ds = (u >> 1) & 3;
      const unsigned char* tile = (u & 1) ? qs : dos;
      const rt_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((rt_lds_v4s)(tile + tro[ds] + m * 16 * ICSA_D * 2));
      const rt_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((rt_lds_v4s)(tile + rt_tr_hi<false>(tro[ds]) + m * 16 * ICSA_D * 2));
      const short __attribute__((ext_vector_type(8))) a8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      return __builtin_bit_cast(bf16x8, a8);
    };
    floatx4 l4[2][4], d4[2][4];                        // lse / D of the rows each lane holds
    auto ld_rows = [&](int sub) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int r0 = 32 * sub + 8 * g + 4 * (lane >> 5);  // acc_row(4 g + x, lane) = r0 + x
        l4[sub][g] = *reinterpret_cast<const floatx4*>(lse_l + r0);
        d4[sub][g] = *reinterpret_cast<const floatx4*>(dd_l + r0);
      }
    };
    auto elem = [&](int sub, int e) {
      const float pr = on ? __builtin_amdgcn_exp2f(fmaf(s[sub][e], cexp, -l4[sub][e >> 2][e & 3])) : 0.f;
      pf[2 * sub + (e >> 3)][e & 7] = (bf16)pr;
      dsf[2 * sub + (e >> 3)][e & 7] = (bf16)(pr * (dp[sub][e] - dmul * d4[sub][e >> 2][e & 3]) * dsmul);
    };
    bf16x8 a[64];
    ld_rows(0);
#pragma unroll
    for (int t = 0; t < BW_PF; ++t) a[t] = ld(t);
    s[0] = s[1] = dp[0] = dp[1] = floatx16{};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 64; ++t) {
      if (t + BW_PF < 64) a[t + BW_PF] = ld(t + BW_PF);
      if (t < 32) {
        const int sub = t >> 4, kk = (t & 15) >> 1;
        if (t & 1) dp[sub] = mfma32x32x16(a[t], vf[kk], dp[sub]);
        else s[sub] = mfma32x32x16(a[t], kf[kk], s[sub]);
      } else {
        const int u = t - 32, m = u >> 3, ds = (u >> 1) & 3;
        if (u & 1) dk[ds] = mfma32x32x16(a[t], dsf[m], dk[ds]);
        else dv[ds] = mfma32x32x16(a[t], pf[m], dv[ds]);
      }
      if (t == 16) ld_rows(1);
      if (t >= 16 && t < 32) elem(0, t - 16);
      if (t >= 32 && t < 48) elem(1, t - 32);
      __builtin_amdgcn_sched_barrier(0);
    }
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
    const int kv = max(0, min(32, p.TKV - key0));     // rows past TKV are not stored
    stage_o(o_lds, dk, p.scale);
    __syncthreads();
    store_rows(o_lds, p.dk, b, h, key0, kv, ivec, one);
    __syncthreads();
    stage_o(o_lds, dv, 1.f);
    __syncthreads();
    store_rows(o_lds, p.dv, b, h, key0, kv, ivec + ICSA_D, one);
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
      p.NKVp != p.nc * ICSA_BLOCK || p.NQ > BW_MAX_NQ || p.nsplit < 1 || p.qb_per_split > 1024 ||
      (int64_t)p.nsplit * p.qb_per_split < p.NQ)
    return hipErrorInvalidValue;
  static std::atomic<unsigned> set_q{0u}, set_i{0u}, set_e{0u};
  hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(icsa_sparse_bwd_dq_kernel), BWQ_LDS_BYTES, &set_q);
  if (attr != hipSuccess) return attr;
  attr = ensure_lds_limit(reinterpret_cast<const void*>(icsa_sparse_bwd_dkv_kernel<true>), BWKV_LDS_BYTES, &set_i);
  if (attr != hipSuccess) return attr;
  attr = ensure_lds_limit(reinterpret_cast<const void*>(icsa_sparse_bwd_dkv_kernel<false>), BWKV_LDS_BYTES, &set_e);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(icsa_sparse_bwd_dq_kernel, dim3(xcd_grid(BH * p.NQ)), dim3(BW_THREADS), BWQ_LDS_BYTES,
                     stream, p);
  hipLaunchKernelGGL(icsa_sparse_bwd_dkv_kernel<true>, dim3(xcd_grid(BH * p.nc * p.nsplit)), dim3(BW_THREADS),
                     BWKV_LDS_BYTES, stream, p);
  hipLaunchKernelGGL(icsa_sparse_bwd_dkv_kernel<false>, dim3(xcd_grid(BH * p.NKV)), dim3(BW_THREADS),
                     BWKV_LDS_BYTES, stream, p);
  return hipGetLastError();
}
