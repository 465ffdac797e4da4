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
// Equivalent schedule used here.  The rescales of acc / l during the interval compose to
// one factor exp2(m_exact - m_final), so the interval runs twice over the compressed
// chunks: pass 1 computes only the running max (-> m_final), acc / l are rescaled once,
// and pass 2 recomputes the same running max chunk by chunk and accumulates the
// non-rescaled g terms straight into the output accumulator.  That costs one extra
// Q.KC product per chunk and frees the separate g accumulator (64 registers), which is
// what lets two waves share each SIMD.  Pass 1 is skipped when a Cauchy-Schwarz bound,
// |q| max_j |KC_j| c / 64 (max_j |KC_j| per head from icsa_kc_bound_kernel), lies below the
// exact max of every row of the workgroup: then the running max cannot rise and
// m_final = m_exact, bit for bit.
//
// The new KV is read in place: new-KV block j lives at source block kvmap[j] of the
// K / V buffers -- target blocks and the selected source blocks of the original
// sequence -- or is an all-zero block (kvmap -1 / an out-of-range caller index, the
// reference's TKV zero padding, attended with logit 0).  When t % 64 != 0 the new-KV
// blocks from n_t on straddle two of those (the reference concatenates t target tokens
// with whole 64-token source blocks, editing_sparse_attention.py:138-159): the first
// t % 64 rows come from the tail of the block before, the rest from the head of
// kvmap[j], and each lane's DMA row picks its segment (SparseParams::seg_a).  KC and VC (or VC^T) are the bf16
// block sums of the new KV.  With mask_tail (the Triton host's ragged TKV)
// the keys of an exact block at or past Sk get no weight instead (triton_kernels.py:185);
// the interval part is the same in both modes.
//
// Workgroup = 2 waves = one query block (wave w: rows 32 w .. 32 w + 31); four workgroups
// share a CU.  One K buffer and one V buffer per workgroup, filled by direct
// global->LDS loads (lane l lands at M0 + 16 l; the XOR swizzle is applied on the global
// side).  V comes in one of two layouts (template parameter VROW; SEG adds the straddling
// new-KV blocks, row-major V only):
//   * VROW: 64 rows of the caller's row-major V, a row tile (attn_tile.h) whose PV
//     operands are formed by transposing LDS reads -- no transposed copy of V is needed
//     (the sparse host entry points, and the materialised new KV of t % 64 != 0);
//   * !VROW: a V^T tile (128 d rows of 64 keys in kv_slot order) from the pipeline's
//     transposed copy of the new KV (new-KV block j at columns 64 j ..; written for the
//     flash kernel by the pooling pass and after the selection); PV operands are plain
//     16-byte reads, which the LDS delivers at a higher rate than transposing ones.
// K(t+1) is issued as soon as both waves finished reading K(t) and lands while the softmax
// and PV of tile t run; V(t) is issued at the workgroup barrier that makes K(t) complete --
// each wave reaches it only after its PV(t - 1) -- and lands during QK and softmax of tile
// t, so a step needs three barriers.  The epilogue fuses the residual and the scatter to
// [B, S, H, D].
// The exact tiles are visited in ascending new-KV order starting at a block that advances
// with the launch index (a rotation of the list), so that the workgroups resident on one
// XCD sweep the new KV together.
#include "attn_tile.h"
#include "icsa_kernels.h"

#define SP_THREADS 128
#define SP_MAX_TOPK 512
#define SP_MAX_CHUNKS 32                 // NKV <= 2048
// one wave's fp32 output staging rows; each tile buffer is at least that large
#define SP_STAGE_BYTES (32 * O_LDS_STRIDE * 4)
#define SP_BUF_BYTES (SP_STAGE_BYTES > K_TILE_BYTES ? SP_STAGE_BYTES : K_TILE_BYTES)
#define SP_RESCALE_LOG2 8.0f
#define SP_PF 2                          // MFMA operand read-ahead (steps); 3 or 4 measured no faster
#define SP_DMA_PER_TILE 8                // LDS-DMA instructions per wave per K or V tile
#ifndef SP_SWEEP_CONC
#define SP_SWEEP_CONC 128                // sweep start advances NKV / SP_SWEEP_CONC per launch
#endif

// vmcnt waits: "all but the newest tile" / "everything".  Loads complete in issue order.
#define SP_WAIT_OLDER() asm volatile("s_waitcnt vmcnt(8)" ::: "memory")
#define SP_WAIT_ALL() asm volatile("s_waitcnt vmcnt(0)" ::: "memory")

// Real rows of a loaded tile: [0, vA) of the first segment [0, a) and [a, a + vB) of the
// second; every other row is zeroed after the load (a = 0: rows [0, vB) real).  The three
// counts (each 0 .. 64) are packed into one word: a tile descriptor is live across a whole
// step, and three of them as separate scalars push the straddling instantiation past its
// scalar registers (spilled to vector lanes and reloaded in the loop).
struct TileRows {
  int w;   // a | vA << 8 | vB << 16
  __device__ __forceinline__ TileRows() : w(0) {}
  __device__ __forceinline__ TileRows(int a, int vA, int vB) : w(a | (vA << 8) | (vB << 16)) {}
  __device__ __forceinline__ int a() const { return w & 0xff; }
  __device__ __forceinline__ int vA() const { return (w >> 8) & 0xff; }
  __device__ __forceinline__ int vB() const { return w >> 16; }
};

template <bool VROW, bool SEG>
__global__ void __launch_bounds__(SP_THREADS) __attribute__((amdgpu_waves_per_eu(2)))
icsa_sparse_kernel(SparseParams p) {
  // K tile and V tile as separate objects, so the compiler can tell a load into one from
  // reads of the other; in the epilogue they hold the fp32 output rows of wave 0 / wave 1.
  __shared__ __attribute__((aligned(16))) unsigned char kbuf[SP_BUF_BYTES];
  __shared__ __attribute__((aligned(16))) unsigned char vbuf[SP_BUF_BYTES];
  __shared__ int src_l[SP_MAX_TOPK];                  // source block of exact tile t (-1: zeros)
  __shared__ int tokA_l[SP_MAX_TOPK];                 // straddling tile: token of row 0 (-1: none)
  __shared__ int nkv_l[SP_MAX_TOPK];                  // its new-KV block (V^T column block; -1: zeros)
  __shared__ unsigned long long sel_l[SP_MAX_CHUNKS];  // selected new-KV blocks per chunk
  __shared__ int rot_l;                               // exact tiles visited from list entry rot_l
  __shared__ int skip_l[2];                           // per wave: the interval max pass is not needed

  const int n_work = p.B * p.H * p.n_qblk;
  const int work = xcd_remap(blockIdx.x, n_work);
  if (work < 0) return;
  const int bh = work / p.n_qblk, slot = work % p.n_qblk;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 31, hl = lane >> 5;
  const int qblk = p.qblocks ? p.qblocks[(int64_t)bh * p.qb_stride + p.qb_offset + slot] : slot;
  const int qtok0 = qblk * ICSA_BLOCK + 32 * wave;
  const int q_valid = max(0, min(32, p.Sq - qtok0));

  const int top_k = p.top_k;
  const int nc = (p.NKV + ATT_BN - 1) / ATT_BN;      // interval chunks
  const int T1 = top_k, T2 = top_k + nc, T = top_k + 2 * nc;

  // ---- block lists: source blocks of the exact tiles, selection bitmask per chunk ----
  for (int c = tid; c < nc; c += SP_THREADS) sel_l[c] = 0ull;
  if (tid == 0) rot_l = 0;
  // Sweep start: the workgroups of one XCD (blockIdx.x % 8) launch in order and run at about
  // the same pace, so starting the ascending list of launch w = blockIdx.x / 8 at new-KV
  // block w * NKV / SP_SWEEP_CONC keeps the resident workgroups reading nearby blocks at the
  // same time, shared in that XCD's L2.  Only the order of the online softmax changes.
  const int sweep0 = (int)(((int64_t)(blockIdx.x / 8) * p.NKV / SP_SWEEP_CONC) % p.NKV);
  __syncthreads();
  {
    const int* idx_g = p.idx + ((int64_t)bh * p.n_qblk + slot) * top_k;
    const int* kvmap = p.kvmap + (int64_t)bh * p.NKV;
    for (int t = tid; t < top_k; t += SP_THREADS) {
      const int j = idx_g[t];
      int src = -1;                 // out-of-range entries of a caller list: a zero block
      int tok_a = -1;
      if (j >= 0 && j < p.NKV) {
        src = p.kvmap_identity ? j : kvmap[j];
        if (SEG && j >= p.seg_from) {
          const int prev = j == p.seg_from ? -2 : (p.kvmap_identity ? j - 1 : kvmap[j - 1]);
          tok_a = prev == -2 ? ATT_BN * p.seg_from
                             : (prev >= 0 ? ATT_BN * prev + ATT_BN - p.seg_a : 0x3fffffff);  // past Sk: zeros
        }
        atomicOr(&sel_l[j >> 6], 1ull << (j & 63));
        if (j < sweep0) atomicAdd(&rot_l, 1);
      }
      src_l[t] = src;
      tokA_l[t] = tok_a;
      nkv_l[t] = src >= 0 ? j : -1;
    }
  }

  bf16x8 qf[8];
  load_q_frags(qf, p.q + (int64_t)b * p.q_sb + (int64_t)qtok0 * p.q_ss + (int64_t)h * p.q_sh, p.q_ss,
               q_valid);
  // max_j |KC_j| of the head (used after the exact loop; loaded now so the exact loop hides
  // the load)
  float kc_max = INFINITY;
  if (p.kc_bound != nullptr) {
    kc_max = 0.f;
    for (int g = 0; g < p.kc_bound_n; ++g) kc_max = fmaxf(kc_max, p.kc_bound[(int64_t)bh * p.kc_bound_n + g]);
  }

  // ---- DMA segments ----
  // K tiles and V row tiles: this wave's rows 32 w .. 32 w + 31 in 8 one-KB segments of 4
  // rows (segment i: rows 32 w + 4 i + lane / 16, lane % 16 = physical 16-byte chunk; K
  // chunks swizzled by row % 16, V chunks by rv_swz).
  // V^T tiles: d rows 64 w .. 64 w + 63 in 8 segments of 8 rows (d = 64 w + 8 i + lane / 8).
  const bf16* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const bf16* vbase = VROW ? p.v + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh
                           : p.vt + (int64_t)b * p.vt_sb + (int64_t)h * p.vt_sh;
  const bf16* kcb = p.kc + (int64_t)bh * p.NKVp * ICSA_D;
  const bf16* vcb = (VROW ? p.vc : p.vct) + (int64_t)bh * p.NKVp * ICSA_D;
  const int k_row0 = 32 * wave + (lane >> 4);        // tile row of segment 0
  const int v_row0 = 64 * wave + (lane >> 3);        // d row of V^T segment 0
  int kro[8], vro[4];                                 // MFMA operand read offsets (bytes)
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) kro[kk] = k_lds_off(li, 2 * kk + hl) * 2;
  if constexpr (VROW) {
    rt_tr_offsets<true>(vro, lane);                   // transposing reads of the row tile
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m) vro[m] = v_lds_off(li, 2 * m + hl) * 2;
  }

  __syncthreads();                                    // src_l / sel_l / rot_l ready
  const int rot = __builtin_amdgcn_readfirstlane(rot_l);
  // list entry of exact tile g (the ascending list rotated to start at entry rot)
  auto ex_entry = [&](int g) -> int { return g + rot < top_k ? g + rot : g + rot - top_k; };

  // Buffer resources with 32-bit byte ranges (every per-(b, h) slice fits: checked at
  // launch), so only the base addresses take 64-bit arithmetic: the scalar setup of a tile
  // runs once per step beside the softmax, and spilled scalar registers cost vector lanes.
  auto rsrc32 = [](const void* base, int bytes) -> __amdgpu_buffer_rsrc_t {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
  };
  // element strides as 32-bit values: launch_sparse rejects slices with Sk * stride * 2 at or
  // above 2^31, so every token offset tok * stride inside a (b, h) slice fits 32 bits
  const int k_st32 = (int)p.k_st, v_st32 = (int)p.v_st;

  // A straddling exact tile (tokA_l >= 0): rows r < seg_a from token tok_a + r, rows
  // r >= seg_a from token 64 src + r - seg_a.  One buffer resource over the head's rows,
  // per-lane row offsets; rows past Sk (or of a zero block) read token 0 and are zeroed
  // after the wait.  Returns the rows that are real: [0, vA) and [seg_a, seg_a + vB).
  const int seg_a = p.seg_a;
  auto issue_straddle = [&](unsigned char* dst, const bf16* head, int rs_el, int tok_a, int src,
                            bool vrow) -> TileRows {
    const int tok_b = src < 0 ? -1 : ATT_BN * src;
    const int vA = max(0, min(seg_a, p.Sk - tok_a));
    const int vB = tok_b < 0 ? 0 : max(0, min(ATT_BN - seg_a, p.Sk - tok_b));
    const int rs2 = (int)rs_el * 2;
    const __amdgpu_buffer_rsrc_t rs = rsrc32(head, (p.Sk - 1) * rs2 + ICSA_D * 2);
#pragma unroll
    for (int i = 0; i < SP_DMA_PER_TILE; ++i) {
      const int r = k_row0 + 4 * i;
      const bool lo = r < seg_a;
      const bool ok = lo ? r < vA : r - seg_a < vB;
      const int tok = ok ? (lo ? tok_a + r : tok_b + r - seg_a) : 0;
      const int swz = vrow ? rv_swz(r) : (r & 15);
      const int off = tok * rs2 + (((lane & 15) ^ swz) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(dst + 1024 * i), 16, off, 0, 0, 0);
    }
    return TileRows(seg_a, vA, vB);
  };

  // Tile g: g < T1 exact block src_l[g]; T1 <= g < T2 pass-1 chunk g - T1 (K only);
  // g >= T2 pass-2 chunk g - T2.  issue_k / issue_v return the rows that are real (the
  // rest are zeroed after the wait; a V^T tile is either all real -- the copy is zero
  // padded -- or a zero block).
  auto issue_k = [&](int g) -> TileRows {
    const bf16* base;
    int bytes;
    int valid, rs2;                        // rs2: key row stride in bytes
    const bool ex = g < T1;
    if (ex) {
      const int tok_a = __builtin_amdgcn_readfirstlane(tokA_l[ex_entry(g)]);
      const int src = __builtin_amdgcn_readfirstlane(src_l[ex_entry(g)]);
      if constexpr (SEG)
        if (tok_a >= 0) return issue_straddle(kbuf + wave * 8192, kbase, k_st32, tok_a, src, false);
      const int tok0 = src * ATT_BN;
      valid = src < 0 ? 0 : min(ATT_BN, p.Sk - tok0);
      base = kbase + (src < 0 ? 0 : tok0 * k_st32);
      rs2 = k_st32 * 2;
      bytes = valid > 0 ? (valid - 1) * rs2 + ICSA_D * 2 : 0;
    } else {
      const int c = g < T2 ? g - T1 : g - T2;
      valid = ATT_BN;
      base = kcb + (int64_t)c * ATT_BN * ICSA_D;
      bytes = ATT_BN * ICSA_D * 2;
      rs2 = ICSA_D * 2;
    }
    const __amdgpu_buffer_rsrc_t rs = rsrc32(base, bytes);
    unsigned char* dst = kbuf + wave * 8192;
#pragma unroll
    for (int i = 0; i < SP_DMA_PER_TILE; ++i) {
      const int r = k_row0 + 4 * i;
      const int off = r * rs2 + (((lane & 15) ^ (r & 15)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(dst + 1024 * i), 16, off, 0, 0, 0);
    }
    return TileRows(0, 0, valid);
  };
  auto issue_v = [&](int g) -> TileRows {
    const bf16* base;
    int bytes;
    int valid, rs2;                        // rs2: row stride in bytes (V rows / V^T d rows)
    const bool ex = g < T1;
    if (ex) {
      const int src = __builtin_amdgcn_readfirstlane(src_l[ex_entry(g)]);
      const int tok0 = src * ATT_BN;
      if constexpr (VROW) {
        const int tok_a = __builtin_amdgcn_readfirstlane(tokA_l[ex_entry(g)]);
        if constexpr (SEG)
          if (tok_a >= 0) return issue_straddle(vbuf + wave * 8192, vbase, v_st32, tok_a, src, true);
        valid = src < 0 ? 0 : min(ATT_BN, p.Sk - tok0);
        base = vbase + (src < 0 ? 0 : tok0 * v_st32);
        rs2 = v_st32 * 2;
        bytes = valid > 0 ? (valid - 1) * rs2 + ICSA_D * 2 : 0;
      } else {                           // V^T holds new-KV block j at columns 64 j ..
        const int jn = __builtin_amdgcn_readfirstlane(nkv_l[ex_entry(g)]);
        valid = jn < 0 ? 0 : ATT_BN;
        base = vbase + (jn < 0 ? 0 : (int64_t)jn * ATT_BN);
        rs2 = (int)p.vt_sd * 2;
        bytes = jn < 0 ? 0 : (ICSA_D - 1) * rs2 + ATT_BN * 2;
      }
    } else {
      const int c = g - T2;
      valid = ATT_BN;
      base = vcb + (int64_t)c * ATT_BN * (VROW ? ICSA_D : 1);
      rs2 = VROW ? ICSA_D * 2 : p.NKVp * 2;
      bytes = VROW ? ATT_BN * ICSA_D * 2 : (ICSA_D - 1) * rs2 + ATT_BN * 2;
    }
    const __amdgpu_buffer_rsrc_t rs = rsrc32(base, bytes);
    unsigned char* dst = vbuf + wave * 8192;
#pragma unroll
    for (int i = 0; i < SP_DMA_PER_TILE; ++i) {
      int off;
      if constexpr (VROW) {
        const int r = k_row0 + 4 * i;
        off = r * rs2 + (((lane & 15) ^ rv_swz(r)) << 4);
      } else {
        const int d = v_row0 + 8 * i;
        off = d * rs2 + (((lane & 7) ^ ((d >> 1) & 7)) << 4);
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(dst + 1024 * i), 16, off, 0, 0, 0);
    }
    return TileRows(0, 0, valid);
  };
  // After the wait: zero this wave's key rows that are not real in the K buffer / a V row
  // tile (rows past the sequence and zero blocks are zero keys and values).
  auto fill_rows = [&](unsigned char* buf, TileRows v) {
    const int va = v.a(), vA = v.vA(), vB = v.vB();
    if (vA >= va && vB >= ATT_BN - va) return;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 32 * wave + 4 * i + (lane >> 4);
      if (r < va ? r >= vA : r - va >= vB)         // 4-byte stores: one zero register
        for (int e = 0; e < 4; ++e) *reinterpret_cast<unsigned*>(buf + r * ICSA_D * 2 + (lane & 15) * 16 + 4 * e) = 0u;
    }
  };
  // ... and this wave's half of a V^T tile of a zero block
  auto fill_v = [&](TileRows v) {
    if constexpr (VROW) {
      fill_rows(vbuf, v);
    } else {
      if (v.vB() > 0) return;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int d = 64 * wave + 8 * i + (lane >> 3);
        *reinterpret_cast<u32x4*>(vbuf + d * ATT_BN * 2 + (lane & 7) * 16) = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  floatx16 o[4] = {};
  floatx16 s[2];
  bf16x8 pf[4];

  // S^T = K Q^T for the K buffer; operands read SP_PF steps ahead of their MFMA.
  auto qk = [&]() {
    bf16x8 ka[16];
    floatx16 acc0 = {}, acc1 = {};
#pragma unroll
    for (int t = 0; t < SP_PF; ++t)
      ka[t] = *reinterpret_cast<const bf16x8*>(kbuf + kro[t >> 1] + (t & 1) * 32 * ICSA_D * 2);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      if (t + SP_PF < 16) {
        const int u = t + SP_PF;
        ka[u] = *reinterpret_cast<const bf16x8*>(kbuf + kro[u >> 1] + (u & 1) * 32 * ICSA_D * 2);
      }
      if (t & 1) acc1 = mfma32x32x16(ka[t], qf[t >> 1], acc1);
      else acc0 = mfma32x32x16(ka[t], qf[t >> 1], acc0);
      __builtin_amdgcn_sched_barrier(0);
    }
    s[0] = acc0;
    s[1] = acc1;
  };
  // O^T += V^T P^T for the V buffer
  auto pv = [&]() {
    if constexpr (VROW) {
      pv_tile_tr<SP_PF, true>(o, vbuf, vro, pf);       // transposing reads of the row tile
    } else {
      bf16x8 va[16];
#pragma unroll
      for (int t = 0; t < SP_PF; ++t)
        va[t] = *reinterpret_cast<const bf16x8*>(vbuf + vro[t >> 2] + (t & 3) * 32 * ATT_BN * 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        if (t + SP_PF < 16) {
          const int u = t + SP_PF;
          va[u] = *reinterpret_cast<const bf16x8*>(vbuf + vro[u >> 2] + (u & 3) * 32 * ATT_BN * 2);
        }
        o[t & 3] = mfma32x32x16(va[t], pf[t >> 2], o[t & 3]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  auto rescale_o = [&](float a) {
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[ds][i] *= a;
  };
  // interval chunk: raw scores of selected blocks and blocks >= NKV set to -inf; returns the
  // chunk max in log2 units (q . KC c / 64)
  const float c64 = p.scale_log2 * (1.0f / 64.0f);
  auto interval_z = [&](int c) -> float {
    // masked blocks of the chunk as one uniform 64-bit word (selected, or >= NKV)
    unsigned long long mb = sel_l[c];
    const int n_real = p.NKV - c * ATT_BN;
    if (n_real < ATT_BN) mb |= ~0ull << n_real;
    // accumulator element i of sub-tile sub is block 32 sub + 8 (i / 4) + 4 hl + i % 4: bit
    // 8 (i / 4) + i % 4 of word sub of mb >> 4 hl, spread to a full mask that selects -inf
    const unsigned long long ml = mb >> (4 * hl);
    const unsigned wd[2] = {(unsigned)ml, (unsigned)(ml >> 32)};
    float mx = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int k = 8 * (i >> 2) + (i & 3);
        const unsigned all = (unsigned)((int)(wd[sub] << (31 - k)) >> 31);
        const float z = __uint_as_float((all & 0xff800000u) | (__float_as_uint(s[sub][i]) & ~all));
        s[sub][i] = z;
        mx = fmaxf(mx, z);
      }
    // the scale is positive, so the max of the scaled scores is the scaled max (the same
    // rounded value): the exponentials take s * c64 - m in one fma
    return xhalf_max(mx) * c64;
  };

  const float c = p.scale_log2;
  float m_ref = -INFINITY;      // reference max of the exact part (raised lazily)
  float m_true = -INFINITY;     // exact running max (the reference's m after the exact loop)
  float l_run = 0.f;

  TileRows kv_pending = issue_k(0);
  TileRows vv_pending;

  // ---- 1. exact blocks ----
  // Three barriers per block: V(t) is issued right after the first one, which every wave
  // passes only after its PV(t - 1), so no barrier is needed after PV.
  for (int t = 0; t < T1; ++t) {
    SP_WAIT_ALL();                         // K(t), the only load in flight
    fill_rows(kbuf, kv_pending);
    ATT_BARRIER();                         // K(t) complete; V buffer free
    vv_pending = issue_v(t);
    qk();
    ATT_BARRIER();                       // K buffer free
    const TileRows kv_next = issue_k(t + 1);   // T > T1: always a next K tile
    // keys past Sk take no part (the Triton host; its new KV never straddles)
    if (!SEG && p.mask_tail && kv_pending.vB() < ATT_BN) {
      // keys >= vB as one 64-bit word; element i of sub-tile sub is key 32 sub + 8 (i / 4) +
      // 4 hl + i % 4: integer selects, no per-element compare masks in scalar registers
      const unsigned long long mw = (~0ull << kv_pending.vB()) >> (4 * hl);
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
    float mx = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[sub][i]);
    mx = xhalf_max(mx) * c;
    m_true = fmaxf(m_true, mx);
    const bool need = mx > m_ref + SP_RESCALE_LOG2;
    if (__ballot(need) != 0ull) {
      const float mn = need ? mx : m_ref;
      const float a = __builtin_amdgcn_exp2f(m_ref - mn);
      rescale_o(a);
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
    SP_WAIT_OLDER();                       // V(t); K(t+1) is the newer tile in flight
    fill_v(vv_pending);
    ATT_BARRIER();
    pv();
    kv_pending = kv_next;
  }
  // Pass 1 only finds the final running max.  Every interval score satisfies
  // |q . KC_j| <= |q| |KC_j| (Cauchy-Schwarz; the fp32 sums stay within 2^-10 of it), so
  // when |q| max_j |KC_j| c / 64 < m_true for every row of the workgroup, the running max
  // never leaves m_true and pass 1 is skipped (bit-identical result).  Rows past the query
  // end take no part.
  if (p.kc_bound != nullptr) {
    float qn2 = 0.f;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = bf2f(qf[kk][e]);
        qn2 = fmaf(x, x, qn2);
      }
    const float bound = sqrtf(xhalf_sum(qn2)) * kc_max * c64 * (1.0f + 0x1p-10f);
    const bool safe = bound < m_true || li >= q_valid;
    if (lane == 0) skip_l[wave] = __ballot(!safe) == 0ull ? 1 : 0;
  } else if (lane == 0) {
    skip_l[wave] = 0;
  }
  ATT_BARRIER();                           // V buffer free; skip_l ready
  issue_v(T2);                             // pass 2's first V tile, after K(T1)
  const bool skip1 = (skip_l[0] & skip_l[1]) != 0;

  // ---- 2a. interval pass 1: running max over the chunks ----
  // (K(T1) is chunk 0 of KC, the same tile as pass 2's first K(T2): a skipped pass 1
  // leaves it in flight for pass 2)
  float m_run = m_true;
  for (int ch = 0; ch < (skip1 ? 0 : nc); ++ch) {
    if (ch == 0) SP_WAIT_OLDER();          // V(T2) was issued after K(T1)
    else SP_WAIT_ALL();
    ATT_BARRIER();
    qk();
    ATT_BARRIER();
    issue_k(T1 + ch + 1);                  // the last one is pass 2's first K tile
    m_run = fmaxf(m_run, interval_z(ch));
  }
  // acc / l as the reference holds them after every interval rescale
  {
    const float a = __builtin_amdgcn_exp2f(m_ref - m_run);
    rescale_o(a);
    l_run *= a;
  }

  // ---- 2b. interval pass 2: non-rescaled g terms, accumulated into o ----
  float m_c = m_true, gl_run = 0.f;
  // Three barriers per chunk, as in the exact loop: V(g) is issued after the first one
  // (V(T2) has been in its buffer since before pass 1).
  for (int ch = 0; ch < nc; ++ch) {
    const int g = T2 + ch;
    SP_WAIT_ALL();                         // K(g); V(g - 1) was waited for before its PV
    ATT_BARRIER();                         // K(g) complete; V buffer free
    if (ch > 0) issue_v(g);
    qk();
    ATT_BARRIER();
    const bool more = g + 1 < T;
    if (more) issue_k(g + 1);
    float rs = 0.f;
    if (!VROW || SEG || p.interval_bn == ATT_BN) {
      m_c = fmaxf(m_c, interval_z(ch));
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = __builtin_amdgcn_exp2f(fmaf(s[sub][i], c64, -m_c));
          rs += e;
          pf[2 * sub + (i >> 3)][i & 7] = (bf16)e;
        }
    } else {
      // reference chunks of BN = 16 or 32 blocks (tilelang_kernels.py:886-978 with a
      // smaller BN): the running max takes each sub-chunk's max in turn, in block order.
      // Quarter u (16 blocks) of the tile: sub-tile u / 2, accumulator elements
      // 8 (u % 2) .. + 7 (blocks 8 (i / 4) + 4 hl + i % 4 of the sub-tile).
      interval_z(ch);                    // masks selected blocks and blocks >= NKV
      const int per = p.interval_bn >> 4;  // quarters per reference chunk: 1 or 2
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if ((u & (per - 1)) == 0) {
          float mx = -INFINITY;
#pragma unroll
          for (int x = 0; x < 2; ++x)
            if (x < per) {
              const int uu = u + x;
#pragma unroll
              for (int i = 0; i < 8; ++i) mx = fmaxf(mx, s[uu >> 1][8 * (uu & 1) + i]);
            }
          m_c = fmaxf(m_c, xhalf_max(mx) * c64);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float e = __builtin_amdgcn_exp2f(fmaf(s[u >> 1][8 * (u & 1) + i], c64, -m_c));
          rs += e;
          pf[u][i] = (bf16)e;
        }
      }
    }
    gl_run += rs;
    if (more) SP_WAIT_OLDER();             // V(g); K(g + 1) is the newer tile in flight
    else SP_WAIT_ALL();
    ATT_BARRIER();
    pv();
  }
  ATT_BARRIER();                           // both waves' PV done before the staging below

  // ---- 3. combine + epilogue ----
  const float den = xhalf_sum(l_run) + 64.0f * xhalf_sum(gl_run);
  const float inv = den == 0.f ? 0.f : 1.f / den;
  float* o_lds = reinterpret_cast<float*>(wave == 0 ? kbuf : vbuf);
  stage_o(o_lds, o, inv);
  // the log-sum-exp the Triton forward saves for its backward (triton_kernels.py:249-252):
  // final running max + log2 of the combined denominator, in log2-scaled score units
  if (p.lse != nullptr && hl == 0 && li < q_valid)
    p.lse[(int64_t)bh * p.Sq + qtok0 + li] = m_run + log2f(den);
  __syncthreads();
  if (q_valid > 0) {
    const float* oc = p.out_c ? p.out_c + ((int64_t)bh * p.nb_q + qblk) * ICSA_D : nullptr;
    store_rows(o_lds, p.out, b, h, qtok0, q_valid, oc, p.alpha);
  }
}

// Workgroup (b, h, y) takes the rows j = 16 (y + G i) + r, r = 0 .. 15 (i = 0, 1, ...): 16
// lanes per row, one 16-byte chunk each, the squared norm summed over the 16 lanes with
// lane shuffles; the workgroup maximum goes through an LDS atomic (non-negative floats
// order like their bit patterns).
__global__ void __launch_bounds__(256) icsa_kc_bound_kernel(const bf16* kc, int NKV, int NKVp, float* out) {
  __shared__ unsigned mx;
  const int bh = blockIdx.x, y = blockIdx.y, G = gridDim.y;
  const int r = threadIdx.x >> 4, ch = threadIdx.x & 15;
  if (threadIdx.x == 0) mx = 0u;
  __syncthreads();
  float best = 0.f;
  for (int j0 = 16 * y; j0 < NKV; j0 += 16 * G) {
    const int j = j0 + r;
    float n2 = 0.f;
    if (j < NKV) {
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(kc + ((int64_t)bh * NKVp + j) * ICSA_D + 8 * ch);
#pragma unroll
      for (int e = 0; e < 8; ++e) n2 = fmaf(bf2f(v[e]), bf2f(v[e]), n2);
    }
#pragma unroll
    for (int w = 1; w < 16; w <<= 1) n2 += __shfl_xor(n2, w);
    best = fmaxf(best, n2);
  }
  atomicMax(&mx, __float_as_uint(best));
  __syncthreads();
  if (threadIdx.x == 0) out[(int64_t)bh * G + y] = sqrtf(__uint_as_float(mx));
}

hipError_t launch_kc_bound(const bf16* kc, int BH, int NKV, int NKVp, float* out, int* G,
                           hipStream_t stream) {
  const int groups = (NKV + 15) / 16;                 // 16-row groups
  *G = groups < 8 ? groups : 8;
  if (BH <= 0 || NKV <= 0) return hipSuccess;
  hipLaunchKernelGGL(icsa_kc_bound_kernel, dim3(BH, *G), dim3(256), 0, stream, kc, NKV, NKVp, out);
  return hipGetLastError();
}

hipError_t launch_sparse(const SparseParams& p, hipStream_t stream) {
  const int n_work = p.B * p.H * p.n_qblk;
  if (n_work == 0) return hipSuccess;
  if (p.top_k < 1 || p.top_k > SP_MAX_TOPK || p.top_k > p.NKV) return hipErrorInvalidValue;
  if (p.NKV < 1 || p.NKV > SP_MAX_CHUNKS * ATT_BN) return hipErrorInvalidValue;
  if (p.NKVp % ATT_BN != 0 || p.NKVp < p.NKV) return hipErrorInvalidValue;
  // per-(b, h) slices must be addressable with 32-bit buffer offsets
  if ((int64_t)p.Sk * p.k_st * 2 > 0x7fffffffLL || 64LL * p.k_st * 2 > 0x7fffffffLL)
    return hipErrorInvalidValue;
  if (p.v_rows ? ((int64_t)p.Sk * p.v_st * 2 > 0x7fffffffLL || 64LL * p.v_st * 2 > 0x7fffffffLL || !p.vc)
               : ((int64_t)ICSA_D * p.vt_sd * 2 > 0x7fffffffLL || !p.vct))
    return hipErrorInvalidValue;
  // reference interval chunks of 16 or 32 blocks: the host entry points (row-major V)
  if (!(p.interval_bn == ATT_BN || ((p.interval_bn == 16 || p.interval_bn == 32) && p.v_rows && p.seg_a == 0)))
    return hipErrorInvalidValue;
  // straddling blocks: row-major V, seg_a in [0, 64), no Triton-style tail mask
  if (p.seg_a < 0 || p.seg_a >= ATT_BN || (p.seg_a > 0 && (!p.v_rows || p.mask_tail || p.seg_from < 0)))
    return hipErrorInvalidValue;
  const dim3 grid(xcd_grid(n_work));
  if (p.seg_a > 0)
    hipLaunchKernelGGL((icsa_sparse_kernel<true, true>), grid, dim3(SP_THREADS), 0, stream, p);
  else if (p.v_rows)
    hipLaunchKernelGGL((icsa_sparse_kernel<true, false>), grid, dim3(SP_THREADS), 0, stream, p);
  else
    hipLaunchKernelGGL((icsa_sparse_kernel<false, false>), grid, dim3(SP_THREADS), 0, stream, p);
  return hipGetLastError();
}
