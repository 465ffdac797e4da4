// Stage 3: bf16 MFMA flash attention for the peaked query blocks (and the dense baseline).
//
// Reference: flash_attn_func(q_flat, new_k, new_v) at editing_sparse_attention.py:209-215 --
// dense non-causal softmax(q k^T / sqrt(D)) v of every peaked 64-row query block over the
// whole new KV, followed by the scatter and residual of :217-232.
//
// The new KV is never materialised: key tile j < n_tgt_tiles is target tile j of the
// original sequence (keys >= t_limit masked: the partial last target tile), tile
// n_tgt_tiles + r is source block sel_base + sel[r] (tokens >= Sk are zero keys with
// logit 0, exactly like the reference's zero padding of k_padded).  K is read in place;
// V^T holds tile j at columns 64 j .. 64 j + 63 (the pipeline writes it in that order).
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
// M0 + 16 l), four buffers deep.  Issuing LDS DMA blocks the issuing wave while the CU's
// vector-memory path takes earlier requests, so only waves in their SOFT phase issue it,
// one 1-KB segment between every 8 exponentials (group 1: K tiles, group 0: V^T tiles; the
// slot schedule below).  The LDS XOR swizzle is applied on the global side: each lane
// fetches the chunk that belongs in its LDS slot.  Per-lane global offsets are computed
// once, the tile start is the scalar base of a buffer resource whose range covers only key
// rows below Sk, and every LDS offset is hoisted out of the loop.
//
// Softmax state: probabilities are taken relative to a reference max m_ref, computed first
// and checked afterwards: only when a lane's partial sum of the tile exceeds 2^64 (or is NaN,
// as against the initial m_ref = -inf) is the row max of the tile taken, the reference
// raised, O / l rescaled and the tile recomputed.  In the common case no per-tile max
// reduction precedes the exponentials.  Exact in real arithmetic.
#include "attn_tile.h"
#include "icsa_kernels.h"

#define FA_WAVES 8
#define FA_THREADS (FA_WAVES * 64)
#define FA_QBLK_PER_WG (FA_WAVES / 2)
#define FA_STAGE_BYTES (FA_WAVES * 32 * O_LDS_STRIDE * 4)    // epilogue staging, all waves
#define FA_NBUF 4                                            // K and V^T tile buffers
#define FA_TILE_BYTES (FA_NBUF * (K_TILE_BYTES + V_TILE_BYTES))
#define FA_MAX_SEL 4096                                      // extra tiles (LDS list)
#define FA_JUNK_OFF (FA_TILE_BYTES + 4 * FA_MAX_SEL)         // landing area of disabled DMA
#define FA_LOOP_BYTES (FA_JUNK_OFF + 4096)
#define FA_LDS_BYTES (FA_LOOP_BYTES > FA_STAGE_BYTES ? FA_LOOP_BYTES : FA_STAGE_BYTES)
// A lane's 32 probabilities of a tile sum to at most 2^64 relative to the row's reference
// max before the reference is raised: O and l then stay below 2^64 * keys * |v|, far inside
// the fp32 range, and bf16(p) keeps its relative precision at any magnitude.
#define FA_PSUM_MAX 18446744073709551616.0f
#ifndef FA_PF
#define FA_PF 5             // operand prefetch depth (MFMA steps); 3, 4, 6 and 8 measured slower
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
  int kro[8], vro[4];                                 // MFMA operand read offsets (bytes)
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) kro[kk] = k_lds_off(li, 2 * kk + hl) * 2;   // + 32 rows per sub-tile
#pragma unroll
  for (int m = 0; m < 4; ++m) vro[m] = v_lds_off(li, 2 * m + hl) * 2;        // + 32 d rows per sub-tile

  auto tile_tok0 = [&](int j) -> int {
    return j < p.n_tgt_tiles ? j * ATT_BN : __builtin_amdgcn_readfirstlane(sel_l[j - p.n_tgt_tiles]);
  };
  // buffer of tile j
  auto kbuf = [&](int j) -> unsigned char* { return smem + (j % FA_NBUF) * K_TILE_BYTES; };
  auto vbuf = [&](int j) -> unsigned char* {
    return smem + FA_NBUF * K_TILE_BYTES + (j % FA_NBUF) * V_TILE_BYTES;
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
      const unsigned char* vs = vbuf(k - 1);
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
      const unsigned char* ks = kbuf(k);
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
  // This wave's share (4 one-KB segments) of one tile's DMA, issued one segment at a time
  // from inside the SOFT phase (see the slot schedule below).
  const bool lag_w = group == 1;
  const int dw = wave & 3;
  int dofs[4];                            // segment offsets: K rows (group 1) / V^T rows (group 0)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int sg = 4 * dw + i;
    if (lag_w) {
      const int kr = 4 * sg + (lane >> 4), kc = (lane & 15) ^ (kr & 15);
      dofs[i] = (int)(((int64_t)kr * p.k_ss + 8 * kc) * 2);
    } else {
      const int vd = 8 * sg + (lane >> 3), vc = (lane & 7) ^ ((vd >> 1) & 7);
      dofs[i] = (int)(((int64_t)vd * p.vt_sd + 8 * vc) * 2);
    }
  }
  __amdgpu_buffer_rsrc_t dma_rs = make_rsrc(kb, 0);
  unsigned char* dma_dst = smem;
  bool dma_on = false;
  // sets up this wave's part of tile j: K(j) for group 1, V^T(j) for group 0
  // Byte ranges fit 32 bits (checked at launch), so only the base addresses take 64-bit
  // arithmetic: the setup runs in the SOFT phase, where its scalar work competes with the
  // exponentials.  Past the last tile the issue stays branch-free: an empty range into a
  // junk LDS area.
  const int k_row_bytes = (int)p.k_ss * 2;
  const int v_rec = (ICSA_D - 1) * (int)p.vt_sd * 2 + ATT_BN * 2;
  auto dma_setup = [&](int j) {
    dma_on = j < n_tiles;
    const int tok0 = dma_on ? tile_tok0(j) : 0;
    if (lag_w) {
      const int k_valid = dma_on ? min(ATT_BN, p.Sk - tok0) : 0;
      const int k_rec = k_valid > 0 ? (k_valid - 1) * k_row_bytes + ICSA_D * 2 : 0;
      dma_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(kb + (int64_t)tok0 * p.k_ss), (short)0, k_rec,
                                                 0x00020000);
    } else {
      dma_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(vb + (int64_t)(dma_on ? j : 0) * ATT_BN),
                                                 (short)0, dma_on ? v_rec : 0, 0x00020000);
    }
    dma_dst = !dma_on ? smem + FA_JUNK_OFF : (lag_w ? kbuf(j) : vbuf(j)) + dw * 4096;
  };
  auto dma_seg = [&](int i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(dma_rs, (lds_ptr)(dma_dst + 1024 * i), 16, dofs[i], 0, 0, 0);
  };
  // SOFT(k): mask, P(k) against the reference max, and -- only when some probability of the
  // tile left the allowed range -- a rescale to the tile's row max and a second pass.  The
  // wave's DMA segments go out one at a time between the exponentials of the first pass.
  auto soft = [&](int k) {
    const int mask_from = k < p.n_tgt_tiles ? p.t_limit - k * ATT_BN : ATT_BN;
    if (mask_from < ATT_BN) {
      // keys >= mask_from as one 64-bit word; element i of sub-tile sub is key
      // 32 sub + 8 (i / 4) + 4 hl + i % 4, bit 8 (i / 4) + i % 4 of word sub of the word
      // shifted by 4 hl.  Integer selects: per-element compares would hold 32 lane masks in
      // scalar registers, which spill into vector lanes and slow every SOFT phase.
      const unsigned long long mw = (~0ull << max(mask_from, 0)) >> (4 * hl);
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const unsigned wd = (unsigned)(mw >> (32 * sub));
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int kb = 8 * (i >> 2) + (i & 3);
          const unsigned all = (unsigned)((int)(wd << (31 - kb)) >> 31);
          s[sub][i] = __uint_as_float((all & 0xff800000u) | (__float_as_uint(s[sub][i]) & ~all));
        }
      }
    }
    // four partial sums: a single chain of 32 dependent adds measured 0.4 % slower
    float rsv[4];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if ((i & 7) == 0) {                // DMA segment 2 sb + i / 8 before every 8th exponential
          __builtin_amdgcn_sched_barrier(0);
          dma_seg(2 * sb + (i >> 3));
          __builtin_amdgcn_sched_barrier(0);
        }
        const float e = __builtin_amdgcn_exp2f(fmaf(s[sb][i], c, -m_ref));
        if (sb == 0 && i < 4) rsv[i] = e;      // no adds of 0.f (not foldable: signed zeros)
        else rsv[i & 3] += e;
        pf[2 * sb + (i >> 3)][i & 7] = (bf16)e;
      }
    float rs = (rsv[0] + rsv[1]) + (rsv[2] + rsv[3]);
    // The partial sum exceeds FA_PSUM_MAX (or is NaN: the first tile, against m_ref = -inf)
    // only when a score rose far above the reference: then raise the reference of every row
    // whose tile max exceeds it, rescale O and l, and recompute the tile's probabilities.
    if (__ballot(!(rs <= FA_PSUM_MAX)) != 0ull) {
      float mx = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sub][i]);
      mx = xhalf_max(mx) * c;
      const float mn = mx > m_ref ? mx : m_ref;
      const float a = __builtin_amdgcn_exp2f(m_ref - mn);
#pragma unroll
      for (int ds = 0; ds < 4; ++ds)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[ds][i] *= a;
      l_run *= a;
      m_ref = mn;
      rs = 0.f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = __builtin_amdgcn_exp2f(fmaf(s[sb][i], c, -m_ref));
          rs += e;
          pf[2 * sb + (i >> 3)][i & 7] = (bf16)e;
        }
    }
    l_run += rs;
  };

  // Slot schedule.  Every slot ends with a workgroup barrier; group 0 runs GEMM(k) in slot
  // 2k and SOFT(k) in slot 2k + 1, group 1 one slot later.  Issuing LDS-DMA blocks the
  // issuing wave while the CU's vector-memory path drains earlier requests (about 22
  // s_memtime ticks per 1-KB instruction), so the tile DMA is issued only by waves in their
  // SOFT phase, one segment between every 8 exponentials, never by a GEMM wave:
  //   K(j): group 1 during SOFT(j - 4), slot 2j - 6; waited for by group 1 at the end of its
  //         GEMM(j - 1), slot 2j - 1; read in slots 2j (group 0) and 2j + 1 (group 1);
  //   V(j): group 0 during SOFT(j - 2), slot 2j - 3; waited for by group 0 at the end of its
  //         SOFT(j), slot 2j + 1; read (as PV(j)) in slots 2j + 2 and 2j + 3.
  // Four buffers per kind: K(j) overwrites K(j - 4), last read in slot 2j - 7; V(j)
  // overwrites V(j - 4), last read (PV(j - 4)) in slot 2j - 5.  Loads complete in issue
  // order, so vmcnt(8) waits for all but this wave's two newest tiles.  Slots past the last
  // tile issue empty-range loads into a junk LDS area (the issue stays branch-free).
  const bool compute = q_valid > 0;
  const bool lag = group == 1;
  // zero key rows >= k_valid of a group-1 wave's K segments (rows 16 dw .. 16 dw + 15)
  auto fill_tail4 = [&](int j, int k_valid) {
    if (k_valid >= ATT_BN) return;
    const int row = 16 * dw + (lane >> 2);
    if (row >= k_valid) {
      unsigned char* dst = kbuf(j) + row * ICSA_D * 2 + (lane & 3) * 64;
#pragma unroll
      for (int e = 0; e < 4; ++e) *reinterpret_cast<u32x4*>(dst + 16 * e) = u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto issue_all = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_seg(i);
  };
  // wait for a tile, leaving the `newer` (at most two) tiles issued after it in flight
  auto wait_n = [&](int newer) {
    if (newer >= 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (newer == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  auto kvalid_of = [&](int j) -> int { return min(ATT_BN, p.Sk - tile_tok0(j)); };
  if (lag) {
    for (int j = 0; j < 3; ++j) { dma_setup(j); issue_all(); }
    wait_n(min(2, n_tiles - 1));          // K(0): K(1), K(2) are newer when they exist
    fill_tail4(0, kvalid_of(0));
  } else {
    dma_setup(0); issue_all();
    dma_setup(1); issue_all();
  }
  ATT_BARRIER();
  if (lag) {                               // slot 0 for group 1: K(3)
    dma_setup(3);
    issue_all();
    ATT_BARRIER();
  }
  for (int k = 0; k <= n_tiles; ++k) {
    if (compute) gemm(k);
    if (lag && k + 1 < n_tiles) {          // K(k + 1); K(k + 2), K(k + 3) are newer
      wait_n(min(2, n_tiles - (k + 2)));
      fill_tail4(k + 1, kvalid_of(k + 1));
    }
    ATT_BARRIER();
    dma_setup(lag ? k + 4 : k + 2);
    if (compute && k < n_tiles) soft(k);
    else issue_all();
    if (!lag && k < n_tiles) wait_n(min(2, n_tiles - (k + 1)));   // V(k); V(k + 1), V(k + 2) newer
    ATT_BARRIER();
  }
  if (!lag) ATT_BARRIER();       // group 0's extra slot
  // empty-range DMA of the last slots may still be in flight towards the junk area, which
  // the output staging below overlaps
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

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
