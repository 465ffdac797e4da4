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
// Workgroup = 8 waves = four 64-row query blocks (wave w: block w/2, rows 32*(w%2)..+31),
// all sharing each K / V^T tile.  The waves form two groups, G0 = waves 0-3 and G1 = waves
// 4-7, so every SIMD holds one wave of each.  The groups run the same sequence of phases
//     GEMM(k) = { S(k) = K(k) Q^T ;  O += V(k-1)^T P(k-1) }      (32 MFMAs)
//     SOFT(k) = { row max, lazy rescale, P(k) = exp2(S(k) c - m) } (~1000 VALU cycles)
// G1 one slot behind G0, with a workgroup barrier between slots: in every slot one wave per
// SIMD feeds the matrix pipe while the other keeps the vector ALU busy ("ping-pong").
//
// Tiles arrive by direct global->LDS buffer loads (LDS DMA: lane l of a load lands at
// M0 + 16 l): K(k+1) and V(k) are issued in slot 2k and waited for at the end of slot
// 2k+1, double buffered.  The LDS XOR swizzle is applied on the global side: each lane
// fetches the chunk that belongs in its LDS slot.  Per-lane global offsets are computed
// once, the tile start is the scalar base of a buffer resource whose range covers only key
// rows below Sk, and every LDS offset is hoisted out of the loop.
//
// Softmax state: probabilities are taken relative to a reference max m_ref that is raised
// only when a row max exceeds it by more than FA_RESCALE_LOG2 (so p <= 2^8); the O / l
// rescale then runs on a few tiles per row.  Exact in real arithmetic.
#include "attn_tile.h"
#include "icsa_kernels.h"

#define FA_WAVES 8
#define FA_THREADS (FA_WAVES * 64)
#define FA_QBLK_PER_WG (FA_WAVES / 2)
#define FA_STAGE_BYTES (FA_WAVES * 32 * O_LDS_STRIDE * 4)    // epilogue staging, all waves
#define FA_TILE_BYTES (2 * (K_TILE_BYTES + V_TILE_BYTES))
#define FA_MAX_SEL 4096                                      // extra tiles (LDS list)
#define FA_LDS_BYTES (FA_TILE_BYTES + 4 * FA_MAX_SEL > FA_STAGE_BYTES ? FA_TILE_BYTES + 4 * FA_MAX_SEL \
                                                                    : FA_STAGE_BYTES)
#define FA_RESCALE_LOG2 8.0f
#ifndef FA_PF
#define FA_PF 3             // operand prefetch depth (MFMA steps)
#endif

__global__ void __launch_bounds__(FA_THREADS) __attribute__((amdgpu_waves_per_eu(2)))
icsa_flash_kernel(FlashParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int ngrp = (p.n_qblk + FA_QBLK_PER_WG - 1) / FA_QBLK_PER_WG;
  const int work = xcd_remap(blockIdx.x, p.B * p.H * ngrp);
  if (work < 0) return;
  const int bh = work / ngrp, grp = work % ngrp;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x;
  // wave index made provably wave-uniform (a scalar), so per-group branches stay uniform
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 31, hl = lane >> 5;
  const int group = wave >> 2;                        // 0: leads, 1: one slot behind
  const int slot = grp * FA_QBLK_PER_WG + (wave >> 1);
  const bool active = slot < p.n_qblk;
  int qblk = 0;
  if (active) qblk = p.qblocks ? p.qblocks[(int64_t)bh * p.qb_stride + p.qb_offset + slot] : slot;
  const int qtok0 = qblk * ICSA_BLOCK + 32 * (wave & 1);
  const int q_valid = active ? max(0, min(32, p.Sq - qtok0)) : 0;

  // token start of every extra (selected source) tile, kept in LDS past the tile buffers
  int* sel_l = reinterpret_cast<int*>(smem + FA_TILE_BYTES);
  for (int r = tid; r < p.n_sel; r += FA_THREADS)
    sel_l[r] = (p.sel_base + p.sel[(int64_t)bh * p.sel_stride + r]) * ATT_BN;

  bf16x8 qf[8];
  load_q_frags(qf, p.q + (int64_t)b * p.q_sb + (int64_t)qtok0 * p.q_ss + (int64_t)h * p.q_sh, p.q_ss,
               q_valid);
  __syncthreads();                                    // sel_l ready

  // ---- per-lane offsets, hoisted out of the loop ----
  const bf16* kb = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16* vb = p.vt + (int64_t)b * p.vt_sb + (int64_t)h * p.vt_sh;
  // DMA segment s = 2 * wave + i (1 KB each): K rows 4s..4s+3, V^T rows 8s..8s+7.
  int kvo[2], vvo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int s = 2 * wave + i;
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
    return j < p.n_tgt_tiles ? j * ATT_BN : __builtin_amdgcn_readfirstlane(sel_l[j - p.n_tgt_tiles]);
  };
  auto kbuf = [&](int i) -> unsigned char* { return smem + i * K_TILE_BYTES; };
  auto vbuf = [&](int i) -> unsigned char* { return smem + 2 * K_TILE_BYTES + i * V_TILE_BYTES; };
  // DMA of K tile j into K buffer j & 1; the range covers only key rows below Sk.
  // Returns the number of valid key rows (rows past it are zeroed by fill_tail).
  auto issue_k = [&](int j) -> int {
    const int tok0 = tile_tok0(j);
    const int k_valid = min(ATT_BN, p.Sk - tok0);
    const int64_t k_bytes = k_valid > 0 ? ((int64_t)(k_valid - 1) * p.k_ss + ICSA_D) * 2 : 0;
    const __amdgpu_buffer_rsrc_t krs = make_rsrc(kb + (int64_t)tok0 * p.k_ss, k_bytes);
    unsigned char* dst = kbuf(j & 1) + wave * 2048;
#pragma unroll
    for (int s = 0; s < 2; ++s)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (lds_ptr)(dst + 1024 * s), 16, kvo[s], 0, 0, 0);
    return k_valid;
  };
  auto issue_v = [&](int j) {
    const int tok0 = tile_tok0(j);
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc(vb + tok0, ((int64_t)(ICSA_D - 1) * p.vt_sd + ATT_BN) * 2);
    unsigned char* dst = vbuf(j & 1) + wave * 2048;
#pragma unroll
    for (int s = 0; s < 2; ++s)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (lds_ptr)(dst + 1024 * s), 16, vvo[s], 0, 0, 0);
  };
  // Zero key rows >= k_valid of this wave's own DMA segments (rows 8 w .. 8 w + 7), after
  // its DMA completed, so padding keys are exact zeros.
  auto fill_tail = [&](int j, int k_valid) {
    if (k_valid >= ATT_BN) return;
    const int row = 8 * wave + (lane >> 3);
    if (row >= k_valid) {
      unsigned char* dst = kbuf(j & 1) + row * ICSA_D * 2 + (lane & 7) * 32;
      *reinterpret_cast<u32x4*>(dst) = u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(dst + 16) = u32x4{0u, 0u, 0u, 0u};
    }
  };

  floatx16 o[4] = {};
  floatx16 s[2];
  bf16x8 pf[4];
  float m_ref = -INFINITY, l_run = 0.f;
  const float c = p.scale_log2;
  const int n_tiles = p.n_tgt_tiles + p.n_sel;

  // GEMM(k): O += V(k-1)^T P(k-1) (k >= 1) and S(k) = K(k) Q^T (k < n).  Operands are read
  // from LDS into registers FA_PF MFMA steps ahead of their use (explicit software
  // pipeline), so the matrix pipe does not wait on LDS latency.
  auto gemm = [&](int k) {
    __builtin_amdgcn_s_setprio(1);              // the matrix-feeding wave wins issue ties
    if (k >= 1) {
      const unsigned char* vs = vbuf((k - 1) & 1);
      bf16x8 va[16];
#pragma unroll
      for (int t = 0; t < FA_PF; ++t)
        va[t] = *reinterpret_cast<const bf16x8*>(vs + vro[t >> 2] + (t & 3) * 32 * ATT_BN * 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        if (t + FA_PF < 16) {
          const int u = t + FA_PF;
          va[u] = *reinterpret_cast<const bf16x8*>(vs + vro[u >> 2] + (u & 3) * 32 * ATT_BN * 2);
        }
        o[t & 3] = mfma32x32x16(va[t], pf[t >> 2], o[t & 3]);
        __builtin_amdgcn_sched_barrier(0);    // keep the read-ahead order
      }
    }
    if (k < n_tiles) {
      const unsigned char* ks = kbuf(k & 1);
      bf16x8 ka[16];
      floatx16 acc0 = {}, acc1 = {};
#pragma unroll
      for (int t = 0; t < FA_PF; ++t)
        ka[t] = *reinterpret_cast<const bf16x8*>(ks + kro[t >> 1] + (t & 1) * 32 * ICSA_D * 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        if (t + FA_PF < 16) {
          const int u = t + FA_PF;
          ka[u] = *reinterpret_cast<const bf16x8*>(ks + kro[u >> 1] + (u & 1) * 32 * ICSA_D * 2);
        }
        if (t & 1) acc1 = mfma32x32x16(ka[t], qf[t >> 1], acc1);
        else acc0 = mfma32x32x16(ka[t], qf[t >> 1], acc0);
        __builtin_amdgcn_sched_barrier(0);
      }
      s[0] = acc0;
      s[1] = acc1;
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // SOFT(k): mask, row max, lazy rescale, P(k)
  auto soft = [&](int k) {
    const int mask_from = k < p.n_tgt_tiles ? p.t_limit - k * ATT_BN : ATT_BN;
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
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = __builtin_amdgcn_exp2f(fmaf(s[sub][i], c, -m_ref));
        rs += e;
        pf[2 * sub + (i >> 3)][i & 7] = (bf16)e;
      }
    l_run += rs;
  };

  // Slot schedule.  Slot t ends with a workgroup barrier.  issue(k) = DMA of K(k+1) and
  // V(k), started at the beginning of slot 2k and waited for at the end of slot 2k+1.
  // Both groups run the same loop body  [GEMM(k) | barrier | SOFT(k) | barrier]:  group 0
  // in slots (2k, 2k+1), group 1 one slot later (2k+1, 2k+2) -- it enters with one extra
  // barrier and group 0 leaves with one, so the barrier counts match.  Only the DMA
  // issue / wait points differ between the groups.
  const bool compute = q_valid > 0;
  const bool lag = group == 1;
  auto issue = [&](int k) -> int {
    int kv_next = ATT_BN;
    if (k + 1 < n_tiles) kv_next = issue_k(k + 1);
    if (k < n_tiles) issue_v(k);
    return kv_next;
  };
  auto wait_fill = [&](int k, int kv_next) {       // completes issue(k)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (k + 1 < n_tiles) fill_tail(k + 1, kv_next);
  };

  {
    const int kv0 = issue_k(0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    fill_tail(0, kv0);
  }
  __syncthreads();
  int kv_pending = ATT_BN;
  if (lag) {                       // slot 0 for group 1: issue(0), then its first barrier
    kv_pending = issue(0);
    ATT_BARRIER();
  }
  for (int k = 0; k <= n_tiles; ++k) {
    if (!lag) kv_pending = issue(k);            // slot 2k starts
    if (compute) gemm(k);
    if (lag) wait_fill(k, kv_pending);          // end of slot 2k+1 (group 1 view)
    ATT_BARRIER();
    if (lag) kv_pending = issue(k + 1);         // slot 2k+2 starts (group 1 view)
    if (compute && k < n_tiles) soft(k);
    if (!lag) wait_fill(k, kv_pending);         // end of slot 2k+1 (group 0 view)
    ATT_BARRIER();
  }
  if (!lag) ATT_BARRIER();       // group 0's extra slot

  // ---- epilogue: 1/l, residual, scatter (the workgroup owns the CU's LDS: one round) ----
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
  const int ngrp = (p.n_qblk + FA_QBLK_PER_WG - 1) / FA_QBLK_PER_WG;
  const int n_work = p.B * p.H * ngrp;
  if (n_work == 0) return hipSuccess;
  if (p.n_tgt_tiles + p.n_sel <= 0 || p.n_sel > FA_MAX_SEL) return hipErrorInvalidValue;
  // per-(b, h) slices must be addressable with 32-bit buffer offsets
  if ((int64_t)p.Sk * p.k_ss * 2 > 0x7fffffffLL || (int64_t)ICSA_D * p.vt_sd * 2 > 0x7fffffffLL)
    return hipErrorInvalidValue;
  static std::atomic<unsigned> lds_set{0u};
  const hipError_t attr = ensure_lds_limit(reinterpret_cast<const void*>(icsa_flash_kernel), FA_LDS_BYTES, &lds_set);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(icsa_flash_kernel, dim3(xcd_grid(n_work)), dim3(FA_THREADS), FA_LDS_BYTES, stream, p);
  return hipGetLastError();
}
