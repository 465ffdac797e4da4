/*
 * icsa.h -- C ABI of the MI355X (gfx950) in-context sparse attention library (libicsa.so).
 *
 * Every entry point takes raw device pointers, explicit sizes and element strides, and a
 * HIP stream (passed as void*, 0 = the null stream).  Work is enqueued on that stream and
 * the call returns without synchronising.  Nothing here allocates device memory: scratch
 * comes from a caller-provided workspace whose size the matching *_workspace_size()
 * function returns.  Results are deterministic (fixed reduction orders, no float atomics).
 *
 * Status codes: ICSA_OK (0) or a negative ICSA_E*; icsa_last_error() returns a
 * thread-local message describing the last failure on the calling thread.
 *
 * Tensors: dtype codes ICSA_BF16 / ICSA_F32.  Token tensors are [B, S, H, D] (or the
 * reference's [B, H, T, D] for the sparse host function) with the innermost dimension
 * contiguous; strides are in elements.  Only D = 128 is supported.  Base pointers and
 * strides must keep 16-byte alignment of every row.
 *
 * Reference interfaces replaced (paths relative to the reference repository root):
 *   icsa_editing_sparse_attention   <- editing_sparse_attention(q, k, v, t_seq_len, s_seq_len,
 *                                        alpha_2, alpha_3, SPARSITY_RATIO, backend)
 *                                        in_context_sparse_attention/editing_sparse_attention.py:67-232
 *   icsa_sparse_piecewise_attn      <- sparse_piecewise_attn_1st_intervals_tilelang(q, k, v,
 *                                        sparsity, block_size)
 *                                        in_context_sparse_attention/tilelang_host.py:229-274
 *                                        (same contract as triton_host.py:11-30)
 *   icsa_flash_attn                 <- flash_attn_func(q, k, v) used at
 *                                        editing_sparse_attention.py:211-215 (third-party
 *                                        flash-attn >= 2.7; dense non-causal attention)
 *   icsa_pool                       <- block compression, editing_sparse_attention.py:96-111
 *                                        and compress_seq :37-55 (sums; means = sums / size)
 *   icsa_gather_kv                  <- new_k / new_v construction,
 *                                        editing_sparse_attention.py:138-159
 *   icsa_wan_qk_prologue            <- the q / k producer of WanSelfAttention.forward,
 *                                        model.py:156-171: WanRMSNorm (model.py:103-114),
 *                                        rope_apply (model.py:69-95), alpha_1 gate (:162),
 *                                        plus stage 1's q / k pooling (esa.py:107-111)
 *   icsa_wan_ln_modulate            <- the residual / LayerNorm / adaLN steps of
 *                                        WanAttentionBlock.forward, model.py:249-270
 *                                        (WanLayerNorm, model.py:117-122)
 *   icsa_editing_sparse_attention_presummed
 *                                   <- editing_sparse_attention (esa.py:67-232) fed by that
 *                                        producer (q / k block sums already computed)
 *   icsa_sparse_piecewise_attn_fwd  <- SparsePiecewiseAttn1stIntervalsFunction.forward,
 *                                        triton_kernels.py:489-539 (output, lse, indices
 *                                        saved for the backward)
 *   icsa_sparse_piecewise_attn_bwd  <- SparsePiecewiseAttn1stIntervalsFunction.backward,
 *                                        triton_kernels.py:541-598, and its kernel
 *                                        sparse_piecewise_attn_1st_intervals_bwd_kernel
 *                                        :265-486
 */
#ifndef ICSA_H_
#define ICSA_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ICSA_BF16 0
#define ICSA_F32 1

#define ICSA_OK 0
#define ICSA_EINVAL (-1)       /* invalid argument (null pointer, bad shape/stride/dtype) */
#define ICSA_EUNSUPPORTED (-2) /* valid but unsupported here (D != 128, sizes over limits) */
#define ICSA_EWORKSPACE (-3)   /* workspace too small */
#define ICSA_EHIP (-4)         /* HIP runtime / launch error */

/* Workspace sub-buffers of icsa_editing_sparse_attention, in layout order. */
enum icsa_ws_slot {
  ICSA_WS_QSUM = 0,   /* f32 [B*H, NB, D]   block sums of q                       */
  ICSA_WS_KSUM,       /* f32 [B*H, NB, D]                                          */
  ICSA_WS_VSUM,       /* f32 [B*H, NB, D]                                          */
  ICSA_WS_VT,         /* bf16 [B*H, D, (ceil(t/64) + topK)*64] V^T of the new KV
                         (kv_slot order): target blocks, then the selected ones    */
  ICSA_WS_QB,         /* bf16 [B, S, H, D] copy of q (only when q is f32)           */
  ICSA_WS_KB,         /* bf16 [B, S, H, D] copy of k (only when k is f32)           */
  ICSA_WS_VB,         /* bf16 [B, S, H, D] copy of v (only when v is f32 and
                         t % 64 != 0: the sparse kernel's row-major values)         */
  ICSA_WS_LOGITS,     /* f32 [B*H, NB, NB]  compressed logits L; the softmax P =
                         exp(L - m) / z with ICSA_WS_RSTAT (P is not stored)        */
  ICSA_WS_OUTC,       /* f32 [B*H, NB, D]   compressed attention output             */
  ICSA_WS_SHARP,      /* f32 [B*H, NB]      sharpness                               */
  ICSA_WS_SRCSCORE,   /* f32 [B*H, n_s]     source-block column mass                */
  ICSA_WS_SEL,        /* i32 [B*H, topK]    selected source blocks (ranked)         */
  ICSA_WS_ORDER,      /* i32 [B*H, NB]      peaked blocks then diffuse blocks        */
  ICSA_WS_KVMAP,      /* i32 [B*H, NKV]     new-KV block -> source block (-1 zero)   */
  ICSA_WS_KC32,       /* f32 [B*H, NKV, D]  new-KV block sums of k                   */
  ICSA_WS_KC,         /* bf16 [B*H, NKVp, D]                                        */
  ICSA_WS_VCT,        /* bf16 [B*H, D, NKVp] new-KV block sums of v, transposed (t % 64 == 0 only) */
  ICSA_WS_L3,         /* i32 [B*H, n_diffuse, top_k] per-block exact lists (ascending) */
  ICSA_WS_VC,         /* bf16 [B*H, NKVp, D] new-KV block sums of v (t % 64 != 0 only) */
  ICSA_WS_COLP,       /* f32 [B*H, ceil(n_t/64), n_s] source-column mass per target strip */
  ICSA_WS_L3S,        /* f32 [B*H, n_diffuse, NKV] level-3 block scores (scratch;    */
                      /* afterwards its first B*H*8 floats hold the interval bound;  */
                      /* before them, the compressed stage's split value means,      */
                      /* bf16 [B*H, 2, D, ceil(NB/64)*64]; sized for the larger)     */
  ICSA_WS_RSTAT,      /* f32 [B*H, NB, 2]   row max and 1 / row sum of the compressed softmax */
  ICSA_WS_COUNT
};

/* Derived sizes of one editing call (editing_sparse_attention.py:89-172,
 * tilelang_host.py:151-171).  sizes_out[]: NB, n_t, n_s, topK, Tkv, k_sparsity,
 * n_peaked, n_diffuse, TKV_pad, NKV, top_k, NKVp (12 entries). */
int icsa_editing_sizes(int B, int S, int H, int D, int t_seq_len, double sparsity, double srr,
                       double flat_ratio, int32_t* sizes_out);

/* Workspace bytes of icsa_editing_sparse_attention for these shapes / dtypes. */
int64_t icsa_editing_workspace_size(int B, int S, int H, int D, int t_seq_len, double sparsity,
                                    double srr, double flat_ratio, int q_dtype, int k_dtype,
                                    int v_dtype);

/* Byte offsets of every ICSA_WS_* sub-buffer (offsets_out[ICSA_WS_COUNT]; size-0 slots
 * repeat the next offset).  Returns the total size like *_workspace_size. */
int64_t icsa_editing_workspace_layout(int B, int S, int H, int D, int t_seq_len, double sparsity,
                                      double srr, double flat_ratio, int q_dtype, int k_dtype,
                                      int v_dtype, int64_t* offsets_out);

/* The whole in-context sparse attention path for q, k, v [B, S, H, D] (target tokens
 * first, t_seq_len of them): pooling, compressed attention, per-head source retrieval
 * (SRR = srr), peaked/diffuse split (flat_ratio peaked), exact flash attention for the
 * peaked blocks, sparse piecewise attention for the diffuse blocks, residual
 * out = attn + alpha_2 * out_c.  q/k/v: bf16 or f32 each.  alpha: NULL -> alpha_scalar,
 * else a tensor broadcast to [B, S, H, D] through strides (a_sd may be 0).  out: bf16 or
 * f32 [B, S, H, D].  inject_sel [B*H, topK], inject_order [B*H, NB] and inject_l3
 * [B*H, n_diffuse, top_k] (ascending) optionally replace the path's own decisions (NULL:
 * computed).  s_seq_len is not needed (unused by the reference as well). */
int icsa_editing_sparse_attention(
    const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
    const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    int B, int S, int H, int D, int t_seq_len, double sparsity, double srr, double flat_ratio,
    const void* alpha, int alpha_dtype, int64_t a_sb, int64_t a_ss, int64_t a_sh, int64_t a_sd,
    float alpha_scalar,
    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    const int32_t* inject_sel, const int32_t* inject_order, const int32_t* inject_l3,
    void* workspace, int64_t workspace_bytes, void* stream);

/* Stage boundaries recorded by icsa_editing_sparse_attention_ev (event index). */
#define ICSA_STAGE_START 0      /* before stage 1                                   */
#define ICSA_STAGE_POOL 1       /* after pooling (+ V transpose)                      */
#define ICSA_STAGE_COMPRESSED 2 /* after compressed attention (logits, softmax, out_c) */
#define ICSA_STAGE_SELECT 3     /* after retrieval, split, new-KV sums, level-3 top-k */
#define ICSA_STAGE_SPARSE 4     /* after the sparse piecewise kernel (diffuse blocks)  */
#define ICSA_STAGE_FLASH 5      /* after the flash-attention kernel (peaked blocks)    */
#define ICSA_STAGE_COUNT 6

/* Same as icsa_editing_sparse_attention, and records hipEvent_t stage_events[i]
 * (ICSA_STAGE_COUNT created events) on the stream at each stage boundary, for profiling
 * on the stream the kernels run on.  No synchronisation is added.  (No counterpart in the
 * reference, which publishes no per-stage timing.) */
int icsa_editing_sparse_attention_ev(
    const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
    const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    int B, int S, int H, int D, int t_seq_len, double sparsity, double srr, double flat_ratio,
    const void* alpha, int alpha_dtype, int64_t a_sb, int64_t a_ss, int64_t a_sh, int64_t a_sd,
    float alpha_scalar,
    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    const int32_t* inject_sel, const int32_t* inject_order, const int32_t* inject_l3,
    void* workspace, int64_t workspace_bytes, void* stream, void* const* stage_events);

/* Bytes of the static device scratch of icsa_editing_sparse_attention_noalloc (256 MiB). */
#define ICSA_NOALLOC_SCRATCH_BYTES (256LL << 20)

/* icsa_editing_sparse_attention without a workspace argument and without any allocation:
 * its scratch is a file-scope __device__ array of ICSA_NOALLOC_SCRATCH_BYTES, one per
 * device, which the device holds from this entry's first call on it until the process
 * ends (the array's code object loads at that call).  Same arguments (minus
 * workspace / workspace_bytes), semantics and results as icsa_editing_sparse_attention.
 * Calls whose workspace (icsa_editing_workspace_size) exceeds the scratch return
 * ICSA_EUNSUPPORTED before any device work; 256 MiB covers, e.g., B = 1, S = 65,536,
 * H <= 8 (one GPU's share of the 40 heads on 8 GPUs).  Nothing in the scratch needs to
 * start at zero, and every call overwrites what it reads.  All calls on one device share
 * that device's scratch: calls that overlap in time on one device (different streams or
 * host threads without ordering) race and give undefined results.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). */
int icsa_editing_sparse_attention_noalloc(
    const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
    const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    int B, int S, int H, int D, int t_seq_len, double sparsity, double srr, double flat_ratio,
    const void* alpha, int alpha_dtype, int64_t a_sb, int64_t a_ss, int64_t a_sh, int64_t a_sd,
    float alpha_scalar,
    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    const int32_t* inject_sel, const int32_t* inject_order, const int32_t* inject_l3,
    void* stream);

/* Workspace bytes of icsa_sparse_piecewise_attn and icsa_sparse_piecewise_attn_fwd (ragged
 * TQ / TKV are sized in whole 64-token blocks). */
int64_t icsa_sparse_piecewise_workspace_size(int B, int H, int TQ, int TKV, int D, double sparsity);

/* Sparse piecewise attention (first-order intervals) on q [B, H, TQ, D], k/v [B, H, TKV, D]
 * bf16 (strides sb, sh, st), TQ and TKV multiples of 64: block sums, top_k =
 * max(1, int(sparsity * TKV/64)) blocks per query block (inject_idx [B*H, TQ/64, top_k]
 * ascending replaces them; idx_out receives the lists used, either may be NULL), exact
 * attention over those blocks plus the interval approximation elsewhere.  out: bf16
 * [B, H, TQ, D]. */
int icsa_sparse_piecewise_attn(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int B, int H, int TQ, int TKV, int D, double sparsity,
    const int32_t* inject_idx, int32_t* idx_out,
    void* out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    void* workspace, int64_t workspace_bytes, void* stream);

/* sparse_piecewise_attn_tilelang_hosttopk (tilelang_host.py:121-226): the same function as
 * icsa_sparse_piecewise_attn with the interval taken over chunks of interval_bn (= BN: 16,
 * 32 or 64) compressed blocks, which decides where the non-rescaled interval terms take
 * their running max (tilelang_kernels.py:886-978).  interval_bn = 64 equals
 * icsa_sparse_piecewise_attn.  Workspace: icsa_sparse_piecewise_workspace_size. */
int icsa_sparse_piecewise_attn_hosttopk(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int B, int H, int TQ, int TKV, int D, double sparsity, int interval_bn,
    const int32_t* inject_idx, int32_t* idx_out,
    void* out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    void* workspace, int64_t workspace_bytes, void* stream);

/* The Triton host's forward (workspace: icsa_sparse_piecewise_workspace_size) with the state
 * its backward needs.  Contract of triton_host.py:11-30 / triton_kernels.py:489-539: TQ and
 * TKV need not be multiples of 64 (rows past them read as zeros in the block sums); the
 * top_k = max(1, int(sparsity * (TKV / 64))) exact blocks (integer division: the floor) are
 * chosen among cdiv(TKV, 64) candidates; keys at or past TKV take no part in the exact
 * attention (triton_kernels.py:185); the interval covers all cdiv(TKV, 64) blocks.  For
 * TQ, TKV multiples of 64 the result equals icsa_sparse_piecewise_attn's.
 * idx_out [B*H, cdiv(TQ, 64), top_k] (required) and lse_out [B*H, TQ] f32 (required), the
 * log-sum-exp in log2 units as the Triton forward stores it: the final running max of the
 * log2-scaled scores plus log2(l + g_l). */
int icsa_sparse_piecewise_attn_fwd(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int B, int H, int TQ, int TKV, int D, double sparsity,
    const int32_t* inject_idx, int32_t* idx_out,
    void* out, int64_t o_sb, int64_t o_sh, int64_t o_st, float* lse_out,
    void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of icsa_sparse_piecewise_attn_bwd. */
int64_t icsa_sparse_piecewise_attn_bwd_workspace_size(int B, int H, int TQ, int TKV, int D);

/* Gradients of icsa_sparse_piecewise_attn_fwd: dout, q, out [B, H, TQ, D] and k, v
 * [B, H, TKV, D] bf16 (strides sb, sh, st), lse [B*H, TQ] and idx [B*H, cdiv(TQ, 64),
 * top_k] from the forward (distinct block indices per row; entries outside
 * [0, cdiv(TKV, 64)) are skipped).  dq / dk / dv are written (not accumulated) as bf16 or
 * f32 (dtype codes).  Deterministic: every gradient is a fixed-order sum, no atomics.
 * Ragged TQ / TKV as the Triton backward (triton_kernels.py:265-486, :541-598): rows past
 * the lengths read as zero, keys past TKV take no part in the exact blocks, the last
 * block's sums cover its real rows. */
int icsa_sparse_piecewise_attn_bwd(
    const void* dout, int64_t do_sb, int64_t do_sh, int64_t do_st,
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void* out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    const float* lse, const int32_t* idx,
    int B, int H, int TQ, int TKV, int D, int top_k,
    void* dq, int dq_dtype, int64_t dq_sb, int64_t dq_sh, int64_t dq_st,
    void* dk, int dk_dtype, int64_t dk_sb, int64_t dk_sh, int64_t dk_st,
    void* dv, int dv_dtype, int64_t dv_sb, int64_t dv_sh, int64_t dv_st,
    void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of icsa_flash_attn. */
int64_t icsa_flash_attn_workspace_size(int B, int Sk, int H, int D);

/* Dense non-causal attention softmax(q k^T / sqrt(D)) v: q [B, Sq, H, D], k/v [B, Sk, H, D]
 * bf16, out [B, Sq, H, D] bf16 or f32.  Also this library's dense baseline. */
int icsa_flash_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                    const void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                    const void* v, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                    int B, int Sq, int Sk, int H, int D,
                    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* Stage 1 alone: f32 block sums [B*H, NB, D] of q, k, v [B, S, H, D] (any may be NULL)
 * and, if vt != NULL, V transposed to bf16 [B*H, D, NB*64] (kv_slot order, zero padded). */
int icsa_pool(const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,
              const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
              const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
              int B, int S, int H, int D, float* qsum, float* ksum, float* vsum, void* vt,
              void* stream);

/* New-KV gather: kn, vn bf16 [B*H, Tp, D] with Tp = ceil((t + 64*topK)/64)*64 from
 * k, v [B, S, H, D] and sel [B*H, topK] (rows past t + 64*topK are zero). */
int icsa_gather_kv(const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                   const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                   int B, int S, int H, int D, int t_seq_len, const int32_t* sel, int topK,
                   void* kn, void* vn, void* stream);

/* Largest batch of icsa_wan_qk_prologue (per-batch RoPE grids travel as kernel arguments). */
#define ICSA_WAN_MAX_BATCH 16

/* Workspace bytes of icsa_wan_qk_prologue (two f32 [B, S] arrays of 1 / rms). */
int64_t icsa_wan_qk_workspace_size(int B, int S);

/* Producer of the attention inputs in the Wan DiT self-attention (model.py:156-171).
 * yq, yk: the q / k projections [B, S, H*D] (bf16 or f32, both y_dtype; element strides
 * y_sb, y_ss; each row contiguous).  For each token row: r = rsqrt(mean(y^2) + eps),
 * n = bf16(y * r), m = n * w (wq / wk: f32 [H*D] RMSNorm weights), then the 3D RoPE of
 * rope_apply: pair j of a head is rotated by rope_cos/sin[pos, j] (f32 [rope_rows, D/2],
 * the model's freqs table), pos being the token's frame index for the first
 * D/2 - 2*floor(D/6) pairs, its row and column index for floor(D/6) pairs each.  grids: host
 * array int32 [B, 6] = target (f, h, w), source (f, h, w); target tokens come first, and
 * with tag == 1 the source tokens follow on their own grid; later tokens are not rotated.
 * Outputs: q_out / k_out bf16 [B, S, H, D] (strides o_*), qsum / ksum f32 [B*H, NB, D]
 * 64-token block sums of the rotated f32 values (NB = ceil(S/64)), and, if alpha_logit
 * is not NULL ([B, S] via al_sb, al_ss, the alpha_1(x) projection), gate_out f32 [B, S]
 * = (sigmoid(a) - 0.5) * 0.5 computed with the reference's bf16 roundings.  B <= 16.
 * Single-tensor mode: yk == NULL processes q only (wk, k_out, ksum ignored); qsum == NULL
 * (with ksum NULL) skips the block sums.  With every grid extent 0 nothing is rotated:
 * the q / k RMSNorm of the cross attention (model.py:180-188). */
int icsa_wan_qk_prologue(
    const void* yq, const void* yk, int y_dtype, int64_t y_sb, int64_t y_ss,
    const float* wq, const float* wk, float eps,
    const float* rope_cos, const float* rope_sin, int rope_rows,
    const int32_t* grids, int tag,
    const void* alpha_logit, int alpha_dtype, int64_t al_sb, int64_t al_ss,
    int B, int S, int H, int D,
    void* q_out, void* k_out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    float* qsum, float* ksum, float* gate_out,
    void* workspace, int64_t workspace_bytes, void* stream);

/* icsa_editing_sparse_attention for q / k produced by icsa_wan_qk_prologue: q and k must
 * be bf16, qsum / ksum are their f32 block sums [B*H, NB, D]; stage 1 then pools only v.
 * Workspace: icsa_editing_workspace_size(..., ICSA_BF16, ICSA_BF16, v_dtype).  stage_events as in
 * icsa_editing_sparse_attention_ev (NULL: none). */
int icsa_editing_sparse_attention_presummed(
    const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
    const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    int B, int S, int H, int D, int t_seq_len, double sparsity, double srr, double flat_ratio,
    const void* alpha, int alpha_dtype, int64_t a_sb, int64_t a_ss, int64_t a_sh, int64_t a_sd,
    float alpha_scalar,
    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    const int32_t* inject_sel, const int32_t* inject_order, const int32_t* inject_l3,
    void* workspace, int64_t workspace_bytes, void* stream, void* const* stage_events,
    const float* qsum, const float* ksum);

/* One pass of the Wan DiT block glue per token row (model.py:249-270):
 *   x' = x + y * gate             if y != NULL (y bf16 [B, S, dim], gate f32 [B, dim] by g_sb;
 *                                  x' written to x_out f32 [B, S, dim], which may alias x)
 *   out = bf16( LN(x') [* lw + lb] [* (1 + scale) + shift] )   if out != NULL
 * LN: LayerNorm over dim without affine (WanLayerNorm), eps; lw / lb: optional f32 [dim]
 * affine (norm3); shift / scale: optional f32 [B, dim] by mod_sb (adaLN e[0] / e[1] and
 * e[3] / e[4]).  x: bf16 or f32 [B, S, dim] (strides x_sb, x_ss); for bf16 x the LayerNorm
 * result is rounded to bf16 first (.type_as(x)).  dim % 4 == 0, dim <= 6144; rows 16-byte
 * aligned. */
int icsa_wan_ln_modulate(const void* x, int x_dtype, int64_t x_sb, int64_t x_ss,
                         const void* y, int64_t y_sb, int64_t y_ss, const float* gate, int64_t g_sb,
                         float* x_out, int64_t xo_sb, int64_t xo_ss,
                         const float* lw, const float* lb,
                         const float* shift, const float* scale, int64_t mod_sb, float eps,
                         int B, int S, int dim, void* out, int64_t o_sb, int64_t o_ss, void* stream);

/* Last error message of the calling thread ("" if none). */
const char* icsa_last_error(void);

/* Library version, major * 10000 + minor * 100 + patch. */
int icsa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ICSA_H_ */
