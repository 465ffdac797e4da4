// Stage 3: bf16 MFMA flash attention for the peaked query blocks (and the dense baseline).
//
// Reference: flash_attn_func(q_flat, new_k, new_v) at editing_sparse_attention.py:209-215 --
// dense non-causal softmax(q k^T / sqrt(D)) v of every peaked 64-row query block over the
// whole new KV, followed by the scatter and residual of :217-232.
//
// The new KV is never materialised: key tile j < n_tgt_tiles is target tile j of the
// original sequence (keys >= t_limit masked: the partial last target tile), tile
// n_tgt_tiles + r is source block sel_base + sel[r] (tokens >= Sk are zero keys with
// logit 0, exactly like the reference's zero padding of k_padded).
//
// Workgroup = 4 waves = two 64-row query blocks taken from the per-head block list
// (wave w: block w/2, rows 32*(w%2)..+31).  K / V^T tiles are double buffered in LDS
// through registers; one barrier per tile.  Epilogue fuses 1/l, the residual
// alpha * out_c[block] and the scatter back to [B, S, H, D].
#include "attn_tile.h"
#include "icsa_kernels.h"

#define FA_QBLK_PER_WG 2
#define FA_LDS_BYTES (2 * (K_TILE_BYTES + V_TILE_BYTES) + 4096)

__device__ __forceinline__ void fa_tile_src(const FlashParams& p, int b, int h, int bh, int j,
                                            const bf16*& krow0, int& k_valid, const bf16*& vcol0,
                                            int& mask_from) {
  int tok0;
  if (j < p.n_tgt_tiles) {
    tok0 = j * ATT_BN;
    mask_from = p.t_limit - tok0;          // keys at or past t_limit are masked
  } else {
    tok0 = (p.sel_base + p.sel[(int64_t)bh * p.sel_stride + (j - p.n_tgt_tiles)]) * ATT_BN;
    mask_from = ATT_BN;                    // appended source blocks are never masked
  }
  k_valid = min(ATT_BN, p.Sk - tok0);
  krow0 = p.k + (int64_t)b * p.k_sb + (int64_t)tok0 * p.k_ss + (int64_t)h * p.k_sh;
  vcol0 = p.vt + (int64_t)b * p.vt_sb + (int64_t)h * p.vt_sh + tok0;
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
icsa_flash_kernel(FlashParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  // buffer i: K tile at smem + i * K_TILE_BYTES, V^T tile at smem + 2*K_TILE_BYTES + i*V_TILE_BYTES
#define FA_KS(i) reinterpret_cast<bf16*>(smem + (i) * K_TILE_BYTES)
#define FA_VS(i) reinterpret_cast<bf16*>(smem + 2 * K_TILE_BYTES + (i) * V_TILE_BYTES)

  const int npairs = (p.n_qblk + FA_QBLK_PER_WG - 1) / FA_QBLK_PER_WG;
  const int work = xcd_remap(blockIdx.x, p.B * p.H * npairs);
  if (work < 0) return;
  const int bh = work / npairs, pair = work % npairs;
  const int b = bh / p.H, h = bh % p.H;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int slot = pair * FA_QBLK_PER_WG + (wave >> 1);
  const bool active = slot < p.n_qblk;
  int qblk = 0;
  if (active) qblk = p.qblocks ? p.qblocks[(int64_t)bh * p.qb_stride + p.qb_offset + slot] : slot;
  const int qtok0 = qblk * ICSA_BLOCK + 32 * (wave & 1);
  const int q_valid = active ? max(0, min(32, p.Sq - qtok0)) : 0;

  bf16x8 qf[8];
  load_q_frags(qf, p.q + (int64_t)b * p.q_sb + (int64_t)qtok0 * p.q_ss + (int64_t)h * p.q_sh, p.q_ss,
               q_valid);

  floatx16 o[4] = {};
  float m_run = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;
  const int n_tiles = p.n_tgt_tiles + p.n_sel;

  TileRegs<256> regs;
  const bf16 *krow0, *vcol0;
  int k_valid, mask_from;
  fa_tile_src(p, b, h, bh, 0, krow0, k_valid, vcol0, mask_from);
  tile_load_regs(regs, krow0, p.k_ss, k_valid, vcol0, p.vt_sd, false);
  tile_store_lds(regs, FA_KS(0), FA_VS(0));
  __syncthreads();

  for (int j = 0; j < n_tiles; ++j) {
    const int buf = j & 1;
    const int cur_mask = mask_from;
    const bool has_next = j + 1 < n_tiles;
    if (has_next) {
      fa_tile_src(p, b, h, bh, j + 1, krow0, k_valid, vcol0, mask_from);
      tile_load_regs(regs, krow0, p.k_ss, k_valid, vcol0, p.vt_sd, false);
    }
    if (q_valid > 0) {
      floatx16 s[2];
      qk_tile(s, FA_KS(buf), qf);
      if (cur_mask < ATT_BN) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (32 * sub + acc_row(i, lane) >= cur_mask) s[sub][i] = -INFINITY;
      }
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
      pv_tile(o, FA_VS(buf), pf);
    }
    if (has_next) tile_store_lds(regs, FA_KS(buf ^ 1), FA_VS(buf ^ 1));
    __syncthreads();
  }

  // epilogue: stage O through LDS (K/V buffers are free after the last barrier)
  float* o_lds = reinterpret_cast<float*>(smem) + wave * 32 * O_LDS_STRIDE;
  const float l_tot = xhalf_sum(l_run);
  const float inv_l = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (q_valid > 0) stage_o(o_lds, o, inv_l);
  __syncthreads();
  if (q_valid > 0) {
    const float* oc = p.out_c ? p.out_c + ((int64_t)bh * p.nb_q + qblk) * ICSA_D : nullptr;
    store_rows(o_lds, p.out, b, h, qtok0, q_valid, oc, p.alpha);
  }
}

hipError_t launch_flash(const FlashParams& p, hipStream_t stream) {
  const int npairs = (p.n_qblk + FA_QBLK_PER_WG - 1) / FA_QBLK_PER_WG;
  const int n_work = p.B * p.H * npairs;
  if (n_work == 0) return hipSuccess;
  if (p.n_tgt_tiles + p.n_sel <= 0) return hipErrorInvalidValue;
  static bool attr_set = false;
  if (!attr_set) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(icsa_flash_kernel),
                        hipFuncAttributeMaxDynamicSharedMemorySize, FA_LDS_BYTES);
    attr_set = true;
  }
  hipLaunchKernelGGL(icsa_flash_kernel, dim3(xcd_grid(n_work)), dim3(256), FA_LDS_BYTES, stream, p);
  return hipGetLastError();
}
