// Stage 4: sparse piecewise attention with the first-order interval approximation, for the
// diffuse query blocks.
//
// Reference: sparse_piecewise_attn_1st_intervals_tilelang (tilelang_host.py:229-274) ->
// sparse_piecewise_attn_tilelang_hosttopk fast path (:121-206) -> fused kernel
// tilelang_kernels.py:681-997; Triton forward triton_kernels.py:122-263 is the same
// algorithm.  Per 64-row query block:
//   1. exact online softmax over the top_k selected new-KV blocks (:863-868);
//   2. interval pass over chunks of 64 compressed blocks in ascending order (:886-978):
//      z = q . KCsum_j * scale / 64, -inf for selected blocks and blocks >= NKV; the
//      running max and acc/l are rescaled, but g_acc (+= p VCsum) and g_l (+= 64 sum p)
//      are never rescaled afterwards -- the reference's behaviour, kept on purpose;
//   3. out = (acc + g_acc) / (l + g_l), 0 when the denominator is 0 (:980-992).
//
// The new KV is read in place: new-KV block j lives at source block kvmap[j] of the
// (k, vt) buffers -- target blocks and the selected source blocks of the original
// sequence -- or is an all-zero block (kvmap -1, the reference's TKV zero padding, which
// is attended with logit 0).  KC / VC^T are the bf16 block sums of the new KV.
//
// Workgroup = 2 waves = one query block (wave w: rows 32*w..+31).  Epilogue fuses the
// residual and the scatter to [B, S, H, D] like the flash-attention kernel.
#include "attn_tile.h"
#include "icsa_kernels.h"

#define SP_THREADS 128
#define SP_MAX_TOPK 512
// K tile + V^T tile (32 KB), or the epilogue's 2 x 32 x O_LDS_STRIDE fp32 staging rows
#define SP_LDS_BYTES (2 * 32 * O_LDS_STRIDE * 4 > K_TILE_BYTES + V_TILE_BYTES \
                          ? 2 * 32 * O_LDS_STRIDE * 4 : K_TILE_BYTES + V_TILE_BYTES)

__global__ void __launch_bounds__(SP_THREADS) icsa_sparse_kernel(SparseParams p) {
  // K tile | V^T tile, reused as the fp32 output staging area in the epilogue
  __shared__ __attribute__((aligned(16))) unsigned char smem[SP_LDS_BYTES];
  __shared__ int idx_l[SP_MAX_TOPK];
  bf16* ks = reinterpret_cast<bf16*>(smem);
  bf16* vs = reinterpret_cast<bf16*>(smem + K_TILE_BYTES);

  const int n_work = p.B * p.H * p.n_qblk;
  const int work = xcd_remap(blockIdx.x, n_work);
  if (work < 0) return;
  const int bh = work / p.n_qblk, slot = work % p.n_qblk;
  const int b = bh / p.H, h = bh % p.H;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int qblk = p.qblocks ? p.qblocks[(int64_t)bh * p.qb_stride + p.qb_offset + slot] : slot;
  const int qtok0 = qblk * ICSA_BLOCK + 32 * wave;
  const int q_valid = max(0, min(32, p.Sq - qtok0));

  const int top_k = p.top_k;
  const int* idx_g = p.idx + ((int64_t)bh * p.n_qblk + slot) * top_k;
  for (int t = threadIdx.x; t < top_k; t += SP_THREADS) idx_l[t] = idx_g[t];

  bf16x8 qf[8];
  load_q_frags(qf, p.q + (int64_t)b * p.q_sb + (int64_t)qtok0 * p.q_ss + (int64_t)h * p.q_sh, p.q_ss,
               q_valid);
  __syncthreads();

  floatx16 o[4] = {};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;
  const int* kvmap = p.kvmap + (int64_t)bh * p.NKV;
  const bf16* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16* vtbase = p.vt + (int64_t)b * p.vt_sb + (int64_t)h * p.vt_sh;
  TileRegs<SP_THREADS> regs;

  // ---- 1. exact blocks ----
  for (int t = 0; t < top_k; ++t) {
    const int j = idx_l[t];
    // out-of-range entries of a caller-provided list read as an all-zero block
    const int src = (j < 0 || j >= p.NKV) ? -1 : (p.kvmap_identity ? j : kvmap[j]);
    if (src >= 0) {
      const int tok0 = src * ATT_BN;
      tile_load_regs(regs, kbase + (int64_t)tok0 * p.k_st, p.k_st, min(ATT_BN, p.Sk - tok0),
                     vtbase + tok0, p.vt_sd, false);
    } else {
      tile_load_regs(regs, kbase, p.k_st, 0, vtbase, p.vt_sd, true);
    }
    if (t > 0) __syncthreads();                 // previous tile fully consumed
    tile_store_lds(regs, ks, vs);
    __syncthreads();
    floatx16 s[2];
    qk_tile(s, ks, qf);
    float mx = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sub][i]);
    mx = xhalf_max(mx);
    const float m_new = fmaxf(m_run, mx * c);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float rs = 0.f;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(s[sub][i], c, -m_new));
        s[sub][i] = e;
        rs += e;
      }
    l_run = fmaf(l_run, alpha, rs);
    if (__ballot(m_new != m_run) != 0ull) {
#pragma unroll
      for (int ds = 0; ds < 4; ++ds)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[ds][i] *= alpha;
    }
    m_run = m_new;
    bf16x8 pf[4];
    pack_p(pf, s);
    pv_tile(o, vs, pf);
  }

  // ---- 2. interval approximation over chunks of 64 compressed blocks ----
  floatx16 g[4] = {};
  float gl_run = 0.f;
  const float c64 = c * (1.0f / 64.0f);
  const bf16* kcb = p.kc + (int64_t)bh * p.NKVp * ICSA_D;
  const bf16* vcb = p.vct + (int64_t)bh * ICSA_D * p.NKVp;
  const int n_chunks = (p.NKV + ATT_BN - 1) / ATT_BN;
  int tptr = 0;                                    // first idx_l entry >= chunk start
  for (int ch = 0; ch < n_chunks; ++ch) {
    const int j0 = ch * ATT_BN;
    tile_load_regs(regs, kcb + (int64_t)j0 * ICSA_D, ICSA_D, ATT_BN, vcb + j0, p.NKVp, false);
    // selection mask of this chunk (idx_l ascending)
    unsigned long long selm = 0ull;
    while (tptr < top_k && idx_l[tptr] < j0 + ATT_BN) {
      if (idx_l[tptr] >= j0) selm |= 1ull << (idx_l[tptr] - j0);
      ++tptr;
    }
    __syncthreads();
    tile_store_lds(regs, ks, vs);
    __syncthreads();
    floatx16 s[2];
    qk_tile(s, ks, qf);
    float mx = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int jj = 32 * sub + acc_row(i, lane);
        const bool masked = (j0 + jj >= p.NKV) || ((selm >> jj) & 1ull);
        const float z = masked ? -INFINITY : s[sub][i] * c64;
        s[sub][i] = z;
        mx = fmaxf(mx, z);
      }
    mx = xhalf_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    l_run *= alpha;
    if (__ballot(m_new != m_run) != 0ull) {
#pragma unroll
      for (int ds = 0; ds < 4; ++ds)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[ds][i] *= alpha;
    }
    m_run = m_new;
    float rs = 0.f;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = __builtin_amdgcn_exp2f(s[sub][i] - m_new);
        s[sub][i] = e;
        rs += e;
      }
    gl_run += rs;
    bf16x8 pf[4];
    pack_p(pf, s);
    pv_tile(g, vs, pf);
  }

  // ---- 3. combine + epilogue ----
  const float den = xhalf_sum(l_run) + 64.0f * xhalf_sum(gl_run);
  const float inv = den == 0.f ? 0.f : 1.f / den;
#pragma unroll
  for (int ds = 0; ds < 4; ++ds)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[ds][i] += g[ds][i];
  __syncthreads();
  float* o_lds = reinterpret_cast<float*>(smem) + wave * 32 * O_LDS_STRIDE;
  stage_o(o_lds, o, inv);
  __syncthreads();
  if (q_valid > 0) {
    const float* oc = p.out_c ? p.out_c + ((int64_t)bh * p.nb_q + qblk) * ICSA_D : nullptr;
    store_rows(o_lds, p.out, b, h, qtok0, q_valid, oc, p.alpha);
  }
}

hipError_t launch_sparse(const SparseParams& p, hipStream_t stream) {
  const int n_work = p.B * p.H * p.n_qblk;
  if (n_work == 0) return hipSuccess;
  if (p.top_k < 1 || p.top_k > SP_MAX_TOPK || p.top_k > p.NKV) return hipErrorInvalidValue;
  if (p.NKVp % ATT_BN != 0 || p.NKVp < p.NKV) return hipErrorInvalidValue;
  hipLaunchKernelGGL(icsa_sparse_kernel, dim3(xcd_grid(n_work)), dim3(SP_THREADS), 0, stream, p);
  return hipGetLastError();
}
