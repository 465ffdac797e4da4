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
// Workgroup = 4 waves = two 64-row query blocks from the per-head block list (wave w:
// block w/2, rows 32*(w%2)..+31); two workgroups share a CU so the MFMA work of one wave
// overlaps the softmax VALU work of another.  K / V^T tiles are double buffered in LDS and
// arrive by direct global->LDS buffer loads (LDS DMA: lane l of a load lands at M0 + 16 l)
// issued one tile ahead, so no vector registers stage them; one barrier per tile.  The LDS
// XOR swizzle is applied on the global side: each lane fetches the chunk that belongs in
// its LDS slot.  Per-lane global offsets are computed once, the tile start is the scalar
// base of a buffer resource whose range covers only key rows below Sk, and every LDS
// offset is hoisted out of the tile loop, so the loop's vector ALU work is the softmax.
//
// Lazy rescale: probabilities are taken relative to a reference max m_ref that is raised
// only when a row max exceeds it by more than FA_RESCALE_LOG2 (so p <= 2^8), so the O / l
// rescale runs on a few tiles per row.  Exact in real arithmetic.
#include "attn_tile.h"
#include "icsa_kernels.h"

#define FA_QBLK_PER_WG 2
#define FA_LDS_BYTES (2 * (K_TILE_BYTES + V_TILE_BYTES) + 4096)
#define FA_RESCALE_LOG2 8.0f

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
icsa_flash_kernel(FlashParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int npairs = (p.n_qblk + FA_QBLK_PER_WG - 1) / FA_QBLK_PER_WG;
  const int work = xcd_remap(blockIdx.x, p.B * p.H * npairs);
  if (work < 0) return;
  const int bh = work / npairs, pair = work % npairs;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 31, hl = lane >> 5;
  const int slot = pair * FA_QBLK_PER_WG + (wave >> 1);
  const bool active = slot < p.n_qblk;
  int qblk = 0;
  if (active) qblk = p.qblocks ? p.qblocks[(int64_t)bh * p.qb_stride + p.qb_offset + slot] : slot;
  const int qtok0 = qblk * ICSA_BLOCK + 32 * (wave & 1);
  const int q_valid = active ? max(0, min(32, p.Sq - qtok0)) : 0;

  bf16x8 qf[8];
  load_q_frags(qf, p.q + (int64_t)b * p.q_sb + (int64_t)qtok0 * p.q_ss + (int64_t)h * p.q_sh, p.q_ss,
               q_valid);

  // ---- per-lane offsets, hoisted out of the tile loop ----
  const bf16* kb = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16* vb = p.vt + (int64_t)b * p.vt_sb + (int64_t)h * p.vt_sh;
  // DMA segment s = 4 * wave + i (1 KB each): K rows 4s..4s+3, V^T rows 8s..8s+7.
  int kvo[4], vvo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = 4 * wave + i;
    const int kr = 4 * s + (lane >> 4), kp = lane & 15;          // LDS row / physical chunk
    const int kc = kp ^ (kr & 15);                               // logical chunk in that slot
    kvo[i] = (int)(((int64_t)kr * p.k_ss + 8 * kc) * 2);
    const int vd = 8 * s + (lane >> 3), vp = lane & 7;
    const int vc = vp ^ ((vd >> 1) & 7);
    vvo[i] = (int)(((int64_t)vd * p.vt_sd + 8 * vc) * 2);
  }
  int kro[8], vro[4];                                 // MFMA operand read offsets (bytes)
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) kro[kk] = k_lds_off(li, 2 * kk + hl) * 2;   // + 32 rows per sub-tile
#pragma unroll
  for (int m = 0; m < 4; ++m) vro[m] = v_lds_off(li, 2 * m + hl) * 2;        // + 32 d rows per sub-tile

  auto tile_tok0 = [&](int j) -> int {
    return j < p.n_tgt_tiles ? j * ATT_BN
                             : (p.sel_base + p.sel[(int64_t)bh * p.sel_stride + (j - p.n_tgt_tiles)]) * ATT_BN;
  };
  typedef __attribute__((address_space(3))) void* lds_ptr;
  // Issues the DMA of tile j into LDS buffer buf.  Each tile gets scalar buffer resources
  // based at its first row; the K range covers key rows below Sk only.  Returns the
  // number of valid key rows (rows past it are zero-filled by fill_tail after the wait).
  auto issue_tile = [&](int j, int buf) -> int {
    const int tok0 = tile_tok0(j);
    const int k_valid = min(ATT_BN, p.Sk - tok0);
    const int64_t k_bytes = k_valid > 0 ? ((int64_t)(k_valid - 1) * p.k_ss + ICSA_D) * 2 : 0;
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kb + (int64_t)tok0 * p.k_ss, k_bytes);
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc(vb + tok0, ((int64_t)(ICSA_D - 1) * p.vt_sd + ATT_BN) * 2);
    unsigned char* kdst = smem + buf * K_TILE_BYTES + wave * 4096;
    unsigned char* vdst = smem + 2 * K_TILE_BYTES + buf * V_TILE_BYTES + wave * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_ptr)(kdst + 1024 * i), 16, kvo[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_ptr)(vdst + 1024 * i), 16, vvo[i], 0, 0, 0);
    return k_valid;
  };
  // Zero the key rows >= k_valid of this wave's own DMA segments (rows 16 w .. 16 w + 15)
  // after its DMA completed, so padding keys are exact zeros.
  auto fill_tail = [&](int buf, int k_valid) {
    if (k_valid >= ATT_BN) return;
    const int row = 16 * wave + (lane >> 2);
    if (row >= k_valid) {
      unsigned char* dst = smem + buf * K_TILE_BYTES + row * ICSA_D * 2 + (lane & 3) * 64;
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(dst + 16 * i) = u32x4{0u, 0u, 0u, 0u};
    }
  };

  floatx16 o[4] = {};
  float m_ref = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;
  const int n_tiles = p.n_tgt_tiles + p.n_sel;

  {
    const int kv0 = issue_tile(0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    fill_tail(0, kv0);
  }
  __syncthreads();

  for (int j = 0; j < n_tiles; ++j) {
    const int buf = j & 1;
    const bool has_next = j + 1 < n_tiles;
    int kv_next = ATT_BN;
    if (has_next) kv_next = issue_tile(j + 1, buf ^ 1);
    if (q_valid > 0) {
      const unsigned char* ks = smem + buf * K_TILE_BYTES;
      const unsigned char* vs = smem + 2 * K_TILE_BYTES + buf * V_TILE_BYTES;
      floatx16 s[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        floatx16 acc = {};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(ks + kro[kk] + sub * 32 * ICSA_D * 2);
          acc = mfma32x32x16(a, qf[kk], acc);
        }
        s[sub] = acc;
      }
      const int mask_from = j < p.n_tgt_tiles ? p.t_limit - j * ATT_BN : ATT_BN;
      if (mask_from < ATT_BN) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (32 * sub + acc_row(i, lane) >= mask_from) s[sub][i] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sub][i]);
      mx = xhalf_max(mx) * c;
      const bool need = mx > m_ref + FA_RESCALE_LOG2;
      if (__ballot(need) != 0ull) {
        const float mn = need ? mx : m_ref;
        const float a = __builtin_amdgcn_exp2f(m_ref - mn);
#pragma unroll
        for (int ds = 0; ds < 4; ++ds)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[ds][i] *= a;
        l_run *= a;
        m_ref = mn;
      }
      float rs = 0.f;
      bf16x8 pf[4];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = __builtin_amdgcn_exp2f(fmaf(s[sub][i], c, -m_ref));
          rs += e;
          pf[2 * sub + (i >> 3)][i & 7] = (bf16)e;
        }
      l_run += rs;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(vs + vro[m] + ds * 32 * ATT_BN * 2);
          o[ds] = mfma32x32x16(a, pf[m], o[ds]);
        }
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (has_next) fill_tail(buf ^ 1, kv_next);
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
  // per-(b, h) slices must be addressable with 32-bit buffer offsets
  if ((int64_t)p.Sk * p.k_ss * 2 > 0x7fffffffLL || (int64_t)ICSA_D * p.vt_sd * 2 > 0x7fffffffLL)
    return hipErrorInvalidValue;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(icsa_flash_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
      FA_LDS_BYTES);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(icsa_flash_kernel, dim3(xcd_grid(n_work)), dim3(256), FA_LDS_BYTES, stream, p);
  return hipGetLastError();
}
