// Parameter blocks and host launchers of every ICSA kernel (internal interface between
// the kernel translation units and the C ABI in api.hip).
#pragma once

#include "icsa_common.h"

// ---------------------------------------------------------------- stage 1 (pool.hip)
struct PoolParams {
  TokTensor x[3];       // inputs (p == nullptr -> skipped)
  float* sums[3];       // [B, H, NB, D] fp32 block sums (nullptr -> skipped)
  bf16* xb[3];          // bf16 copies, strides xb_* (nullptr -> skipped)
  int64_t xb_sb, xb_ss, xb_sh;
  bf16* vt;             // transposed copy of x[vt_src] (nullptr -> skipped)
  int64_t vt_sb, vt_sh, vt_sd;
  int vt_src;
  int vt_limit, vt_nblk;  // vt_limit: only blocks n < vt_nblk are transposed
  int B, S, H, NB;      // S tokens, NB = ceil(S / 64) blocks
};
hipError_t launch_pool(const PoolParams& p, hipStream_t stream);
// V^T of a list of blocks only: block base + list[bh * stride + r], r < n, of x[vt_src],
// stored as V^T block dst0 + r (the selected source blocks, transposed after the selection
// into the columns that follow the target blocks)
hipError_t launch_vt_blocks(const PoolParams& p, const int* list, int base, int stride, int n,
                            int dst0, hipStream_t stream);

// ---------------------------------------------------------------- stage 2 (compressed.hip)
struct CompressedParams {
  const float* qsum;    // [BH, NB, D]
  const float* ksum;
  const float* vsum;
  float* L;             // [BH, NB, NB] logits (P = exp(L - m) / z is formed where it is used)
  float* out_c;         // [BH, NB, D]
  float* sharp;         // [BH, NB]
  float* colpart;       // [BH, ceil(n_t/64), n_s] source-column sums per 64-row target strip
  float* rstat;         // [BH, NB, 2] row max, 1 / row sum of exp
  bf16* vmt;            // [BH, 2, D, compressed_nbp(NB)] scratch: the value means transposed,
                        // split in two bf16 parts (written and read by the compressed stage)
  int BH, NB, S;        // S: tokens (last block size = S - (NB-1)*64)
  int n_t, n_s, k_sparsity;
};
inline int compressed_nbp(int NB) { return (NB + 63) / 64 * 64; }
inline int64_t compressed_vmt_bytes(int BH, int NB) { return (int64_t)BH * 2 * ICSA_D * compressed_nbp(NB) * 2; }
hipError_t launch_compressed(const CompressedParams& p, hipStream_t stream);

struct SelectParams {
  const float* colpart; // [BH, ceil(n_t/64), n_s] (CompressedParams::colpart)
  const float* sharp;   // [BH, NB]
  float* src_score;     // [BH, n_s]
  int* sel;             // [BH, topK]   (ranked order)
  int* order;           // [BH, NB]     (first n_peaked peaked, rest diffuse)
  int* kvmap;           // [BH, NKV]    start block in the K/Vt source of new-KV block j, -1 zero
  int BH, NB, n_t, n_s, topK, NKV;
  int inject_sel, inject_order;   // 1: sel / order already hold caller decisions
};
hipError_t launch_select(const SelectParams& p, hipStream_t stream);

struct NewKvSumsParams {
  const float* ksum;    // [BH, Nsrc, D] source block sums
  const float* vsum;
  const int* kvmap;     // [BH, NKV]  source block index (token start / 64) or -1
  int map_identity;     // 1: kvmap ignored, block j -> j
  float* kc32;          // [BH, NKV, D]   fp32 sums of new-KV blocks
  bf16* kc;             // [BH, NKVp, D]  bf16 sums (rows >= NKV zero)
  bf16* vct;            // [BH, D, NKVp]  bf16 sums of v transposed, kv_slot() order (nullptr: none)
  bf16* vc;             // [BH, NKVp, D]  bf16 sums of v, row-major (nullptr: none)
  int BH, Nsrc, NKV, NKVp;
  // straddling blocks j in [seg_from, NKV) (seg_a > 0; see SparseParams) are summed from the
  // token rows of k / v (dtype as given, rows >= S zero) instead of copied from ksum / vsum
  TokTensor k, v;
  int seg_a, seg_from, S, H;
};
hipError_t launch_newkv_sums(const NewKvSumsParams& p, hipStream_t stream);

struct Level3Params {
  const float* qsum;    // [BH, NQsrc, D]
  const int* rows;      // [BH, rows_stride] q-block list (nullptr -> identity)
  int rows_offset, rows_stride;
  const float* kc32;    // [BH, NKV, D]
  int* idx;             // [BH, n_rows, top_k]  ascending block indices
  float* scores;        // [BH, n_rows, NKV]  scratch
  int BH, NQsrc, n_rows, NKV, top_k;
};
hipError_t launch_level3(const Level3Params& p, hipStream_t stream);

// ---------------------------------------------------------------- new-KV gather (gather.hip)
struct GatherParams {
  TokTensor k, v;       // [B, S, H, D]
  const int* sel;       // [BH, topK]
  bf16* kn;             // [BH, Tp, D]  row-major new K
  bf16* vn;             // [BH, Tp, D]  row-major new V
  int B, H, S, t, topK, Tkv, Tp;
};
hipError_t launch_gather(const GatherParams& p, hipStream_t stream);

// ---------------------------------------------------------------- stage 3 (flash_attn.hip)
struct FlashParams {
  const bf16* q; int64_t q_sb, q_ss, q_sh;      // [B, Sq, H, D]
  const bf16* k; int64_t k_sb, k_ss, k_sh;      // [B, Sk, H, D]
  const bf16* vt; int64_t vt_sb, vt_sh, vt_sd;  // [B, H, D, 64 n_tiles]: tile j at columns 64 j ..
  int B, H, Sq, Sk;
  const int* qblocks; int qb_offset, qb_stride; int n_qblk;   // per-bh q-block list
  int t_limit, n_tgt_tiles;        // KV tiles [0, n_tgt_tiles) of 64 keys, keys >= t_limit masked
  const int* sel; int sel_stride; int n_sel; int sel_base;    // extra tiles at (sel_base + sel[r]) * 64
  const float* out_c;              // [BH, NBq, D] residual (nullptr -> none)
  int nb_q;
  AlphaView alpha;
  OutView out;
  float scale_log2;                // log2(e) / sqrt(D)
};
hipError_t launch_flash(const FlashParams& p, hipStream_t stream);

// ---------------------------------------------------------------- Wan q/k producer (wan_qk.hip)
#define ICSA_WAN_MAX_B 16
struct WanRmsParams {
  TokTensor y[2];       // q / k projections [B, S, H*D] (sb, ss; rows contiguous)
  float* rinv[2];       // [B, S] 1 / rms of each row
  TokTensor alpha_logit;   // [B, S] alpha_1(x) (p == nullptr -> no gate)
  float* gate;          // [B, S] (sigmoid(a) - 0.5) * 0.5 in the reference's bf16 steps
  int B, S, H;
  float eps;
};
struct WanQkParams {
  TokTensor y[2];       // as WanRmsParams::y (same dtype)
  const float* w[2];    // RMSNorm weights [H*D]
  const float* rinv[2]; // WanRmsParams::rinv
  const float* rope_cos;   // [rope_rows, D/2]  cos / sin of the model's freqs table
  const float* rope_sin;
  int grids[6 * ICSA_WAN_MAX_B];   // per batch: target f, h, w; source f, h, w
  int tag;              // 1: source tokens rotated on their own grid after the target
  OutView out[2];       // bf16 [B, S, H, D]
  float* sums[2];       // [B, H, NB, D] fp32 block sums of the rotated fp32 values
  int B, S, H, NB;
};
hipError_t launch_wan_qk(const WanRmsParams& rp, const WanQkParams& qp, hipStream_t stream);

// ---------------------------------------------------------------- Wan block glue (wan_block.hip)
struct LnModParams {
  const void* x; int x_dtype; int64_t x_sb, x_ss;      // residual stream [B, S, dim]
  const bf16* y; int64_t y_sb, y_ss;                    // optional update x += y * gate
  const float* gate; int64_t g_sb;                      // [B, dim]
  float* x_out; int64_t xo_sb, xo_ss;                   // updated x (f32; may alias x)
  const float* lw; const float* lb;                     // optional LayerNorm affine [dim]
  const float* shift; const float* scale; int64_t mod_sb;   // optional [B, dim] modulation
  bf16* out; int64_t o_sb, o_ss;                        // bf16 [B, S, dim] (nullptr: update only)
  int B, S, dim;
  float eps;
};
hipError_t launch_ln_mod(const LnModParams& p, hipStream_t stream);

// ---------------------------------------------------------------- stage 4 (sparse_attn.hip)
struct SparseParams {
  const bf16* q; int64_t q_sb, q_ss, q_sh;      // [B, Sq, H, D]
  const bf16* k; int64_t k_sb, k_st, k_sh;      // keys: b, token, h strides
  // values in one of two layouts (the kernel is instantiated for each):
  int v_rows;                        // 1: row-major v (b, token, h strides, like k) with
                                     //    row-major block sums vc; 0: transposed vt
                                     //    [B, H, D, Tp] (b, h, d strides) with vct
  const bf16* v; int64_t v_sb, v_st, v_sh;
  const bf16* vt; int64_t vt_sb, vt_sh, vt_sd;
  int B, H, Sq, Sk;                  // Sk: tokens available in k / v (rows >= Sk read as 0)
  int mask_tail;                     // 1: exact-part keys >= Sk take no part (the Triton
                                     // host, triton_kernels.py:185); 0: they are zero keys
                                     // attended with logit 0 (TileLang's zero padding)
  const int* qblocks; int qb_offset, qb_stride; int n_qblk;
  const int* kvmap; int kvmap_identity;         // [BH, NKV] source block of new-KV block
  // Straddling new-KV blocks (the pipeline's in-place new KV when t % 64 != 0): block
  // j >= seg_from takes rows r < seg_a from tokens segA(j) + r and rows r >= seg_a from
  // 64 kvmap[j] + r - seg_a, with segA(seg_from) = 64 seg_from (the target tail) and
  // segA(j) = 64 kvmap[j - 1] + 64 - seg_a otherwise (the tail of the previous selected
  // block).  seg_a = 0: every block is the 64 rows from 64 kvmap[j].  Row-major V only.
  int seg_a, seg_from;
  const int* idx;                    // [BH, n_qblk, top_k] ascending
  int top_k, NKV, NKVp;
  const bf16* kc;                    // [BH, NKVp, D]
  const bf16* vc;                    // [BH, NKVp, D]  (v_rows)
  const bf16* vct;                   // [BH, D, NKVp]  (!v_rows)
  const float* out_c; int nb_q;
  AlphaView alpha;
  OutView out;
  float scale_log2;
  float* lse;                        // optional [BH, Sq]: m + log2(l + g_l) per query (log2 units)
  // optional [BH, kc_bound_n] partial maxima of |KC_j| (launch_kc_bound): a workgroup whose
  // rows all satisfy |q| max |KC_j| c / 64 < exact max skips the interval max pass
  const float* kc_bound; int kc_bound_n;
  // blocks per interval chunk of the reference (BN): the running max of the non-rescaled
  // interval terms is taken per chunk of that many blocks; 64, or 16 / 32 (row-major V)
  int interval_bn;
};
hipError_t launch_sparse(const SparseParams& p, hipStream_t stream);
// out[bh * G + y] = max over the new-KV blocks j < NKV with (j / 16) % G == y of the L2
// norm of the bf16 row kc[bh, j, :] (fp32 arithmetic); G = min(8, cdiv(NKV, 16)) is
// returned in *G (at most NKV, so BH * G floats fit wherever BH * NKV do)
hipError_t launch_kc_bound(const bf16* kc, int BH, int NKV, int NKVp, float* out, int* G,
                           hipStream_t stream);

// ---------------------------------------------------------------- backward (sparse_bwd.hip)
// Gradients of the sparse piecewise attention (triton_kernels.py:265-486, 541-598) without
// atomics: dq query-major, dk / dv key-major over fixed-order query lists.
struct SparseBwdParams {
  const bf16* q;    int64_t q_sb, q_sh, q_st;     // [B, H, TQ, D] element strides
  const bf16* k;    int64_t k_sb, k_sh, k_st;     // [B, H, TKV, D]
  const bf16* v;    int64_t v_sb, v_sh, v_st;
  const bf16* dout; int64_t do_sb, do_sh, do_st;  // [B, H, TQ, D]
  const bf16* out;  int64_t o_sb, o_sh, o_st;
  const float* lse;                  // [BH, TQ] log2 units
  const int* idx;                    // [BH, NQ, top_k]
  int B, H, TQ, TKV, NQ, NKV, NKVp, nc, top_k, nsplit, qb_per_split;
  float scale, scale_log2;
  // workspace
  const float* ksum; const float* vsum;   // [BH, NKV, D] f32 block sums
  float* dvec;                       // [BH, TQ] rowsum(dO * O)
  unsigned long long* selbits;       // [BH, NQ, nc] selected key blocks per query block
  bf16* kcb; bf16* vcb;              // [BH, NKVp, D] bf16 block sums, rows >= NKV zero
  float* dkc_part; float* dvc_part;  // [nsplit, BH, NKVp, D] interval partials
  OutView dq, dk, dv;                // (sb, token stride, sh, dtype)
};
hipError_t launch_sparse_bwd_prep(const SparseBwdParams& p, hipStream_t stream);
hipError_t launch_sparse_bwd(const SparseBwdParams& p, hipStream_t stream);
