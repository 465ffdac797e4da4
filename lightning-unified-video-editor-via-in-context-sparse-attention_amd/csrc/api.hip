// C ABI of libicsa.so: argument validation, derived sizes, workspace layout and the launch
// sequence of each entry point.  Declarations and contracts: include/icsa.h.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "icsa_kernels.h"
#include "../../include/icsa.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(ICSA_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define ICSA_HIP_TRY(expr, what)                 \
  do {                                           \
    hipError_t e_ = (expr);                      \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }
int ceil_div(int a, int b) { return (a + b - 1) / b; }
int elsize(int dtype) { return dtype == ICSA_F32 ? 4 : 2; }

struct Sizes {
  int NB, n_t, n_s, topK, Tkv, k_sparsity, n_peaked, n_diffuse, TKV_pad, NKV, top_k, NKVp;
};

// editing_sparse_attention.py:89-94, 126-129, 139, 164, 169-172, 189-198;
// tilelang_host.py:151-152, 171.  Ratios are applied as int(n * ratio) in double precision,
// which equals the reference's integer divisions for dyadic ratios.
Sizes derive(int S, int t, double sparsity, double srr, double flat_ratio) {
  Sizes z;
  z.NB = ceil_div(S, ICSA_BLOCK);
  z.n_t = t / ICSA_BLOCK;
  z.n_s = z.NB - z.n_t;
  z.topK = (int)((double)z.n_s * srr);
  z.Tkv = t + z.topK * ICSA_BLOCK;
  z.k_sparsity = std::max(1, (int)((double)z.n_t * sparsity));
  z.n_peaked = (int)((double)z.NB * flat_ratio);
  z.n_diffuse = z.NB - z.n_peaked;
  z.TKV_pad = ceil_div(z.Tkv, ICSA_BLOCK) * ICSA_BLOCK;
  z.NKV = z.TKV_pad / ICSA_BLOCK;
  z.top_k = std::max(1, (int)(sparsity * (double)z.NKV));
  z.NKVp = ceil_div(z.NKV, 64) * 64;
  return z;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool row_ok(const void* p, int dtype, int64_t s0, int64_t s1, int64_t s2) {
  const int64_t m = 16 / elsize(dtype);
  return aligned16(p) && s0 % m == 0 && s1 % m == 0 && s2 % m == 0;
}

int check_dtype(int dt, const char* name) {
  if (dt != ICSA_BF16 && dt != ICSA_F32) return fail(ICSA_EINVAL, "%s: dtype %d is not bf16 (0) or f32 (1)", name, dt);
  return ICSA_OK;
}

struct Layout {
  int64_t off[ICSA_WS_COUNT];
  int64_t total;
};

// Columns of the pipeline's V^T: the new KV's tiles in order, the ceil(t / 64) target tiles
// then the topK selected source blocks (tile j at columns 64 j .. 64 j + 63)
int64_t vt_columns(const Sizes& z, int t) { return ((int64_t)ceil_div(t, ICSA_BLOCK) + z.topK) * ICSA_BLOCK; }

Layout editing_layout(int B, int S, int H, const Sizes& z, int t, int q_dtype, int k_dtype, int v_dtype) {
  const int64_t BH = (int64_t)B * H;
  const int64_t D = ICSA_D;
  const bool unaligned = (t % ICSA_BLOCK) != 0;
  int64_t sz[ICSA_WS_COUNT];
  sz[ICSA_WS_QSUM] = BH * z.NB * D * 4;
  sz[ICSA_WS_KSUM] = BH * z.NB * D * 4;
  sz[ICSA_WS_VSUM] = BH * z.NB * D * 4;
  sz[ICSA_WS_VT] = BH * D * vt_columns(z, t) * 2;
  sz[ICSA_WS_QB] = q_dtype == ICSA_F32 ? (int64_t)B * S * H * D * 2 : 0;
  sz[ICSA_WS_KB] = k_dtype == ICSA_F32 ? (int64_t)B * S * H * D * 2 : 0;
  sz[ICSA_WS_VB] = (unaligned && v_dtype == ICSA_F32) ? (int64_t)B * S * H * D * 2 : 0;
  sz[ICSA_WS_LOGITS] = BH * z.NB * z.NB * 4;
  sz[ICSA_WS_OUTC] = BH * z.NB * D * 4;
  sz[ICSA_WS_SHARP] = BH * z.NB * 4;
  sz[ICSA_WS_SRCSCORE] = BH * std::max(z.n_s, 1) * 4;
  sz[ICSA_WS_SEL] = BH * std::max(z.topK, 1) * 4;
  sz[ICSA_WS_ORDER] = BH * z.NB * 4;
  sz[ICSA_WS_KVMAP] = BH * z.NKV * 4;
  sz[ICSA_WS_KC32] = BH * z.NKV * D * 4;
  sz[ICSA_WS_KC] = BH * z.NKVp * D * 2;
  sz[ICSA_WS_VCT] = unaligned ? 0 : BH * D * z.NKVp * 2;
  sz[ICSA_WS_L3] = BH * std::max(z.n_diffuse, 1) * z.top_k * 4;
  sz[ICSA_WS_VC] = unaligned ? BH * z.NKVp * D * 2 : 0;
  sz[ICSA_WS_COLP] = BH * ceil_div(z.n_t, ICSA_BLOCK) * std::max(z.n_s, 1) * 4;
  // the level-3 scores, and before them the compressed stage's split value means
  sz[ICSA_WS_L3S] = std::max(BH * std::max(z.n_diffuse, 1) * z.NKV * 4, compressed_vmt_bytes((int)BH, z.NB));
  sz[ICSA_WS_RSTAT] = BH * z.NB * 2 * 4;
  Layout L;
  int64_t o = 0;
  for (int i = 0; i < ICSA_WS_COUNT; ++i) {
    L.off[i] = o;
    o += align256(sz[i]);
  }
  L.total = o;
  return L;
}

int validate_common(int B, int S, int H, int D) {
  if (B <= 0 || S <= 0 || H <= 0) return fail(ICSA_EINVAL, "B, S, H must be positive (got %d, %d, %d)", B, S, H);
  if (D != ICSA_D) return fail(ICSA_EUNSUPPORTED, "head dim D=%d unsupported (only 128)", D);
  return ICSA_OK;
}

AlphaView make_alpha(const void* alpha, int alpha_dtype, int64_t a_sb, int64_t a_ss, int64_t a_sh,
                     int64_t a_sd, float scalar) {
  AlphaView a;
  a.p = alpha;
  a.sb = a_sb; a.ss = a_ss; a.sh = a_sh; a.sd = a_sd;
  a.dtype = alpha_dtype;
  a.scalar = scalar;
  return a;
}

const float kLog2e = 1.4426950408889634f;

// Test hook: ICSA_DEBUG_NO_INTERVAL_SKIP=1 in the environment turns the sparse kernel's
// interval-bound skip off (interval pass 1 always runs), so that tests can compare the two
// schedules bit for bit.  Read at every call; no other behaviour depends on the environment.
bool interval_skip_enabled() {
  const char* e = std::getenv("ICSA_DEBUG_NO_INTERVAL_SKIP");
  return !(e != nullptr && e[0] == '1');
}

}  // namespace

extern "C" {

const char* icsa_last_error(void) { return g_last_error.c_str(); }

int icsa_version(void) { return 100; }

int icsa_editing_sizes(int B, int S, int H, int D, int t_seq_len, double sparsity, double srr,
                       double flat_ratio, int32_t* sizes_out) {
  int rc = validate_common(B, S, H, D);
  if (rc) return rc;
  if (t_seq_len < 0 || t_seq_len > S) return fail(ICSA_EINVAL, "t_seq_len %d outside [0, S=%d]", t_seq_len, S);
  if (!sizes_out) return fail(ICSA_EINVAL, "sizes_out is NULL");
  Sizes z = derive(S, t_seq_len, sparsity, srr, flat_ratio);
  const int v[12] = {z.NB, z.n_t, z.n_s, z.topK, z.Tkv, z.k_sparsity, z.n_peaked, z.n_diffuse,
                     z.TKV_pad, z.NKV, z.top_k, z.NKVp};
  std::memcpy(sizes_out, v, sizeof(v));
  return ICSA_OK;
}

int64_t icsa_editing_workspace_layout(int B, int S, int H, int D, int t_seq_len, double sparsity,
                                      double srr, double flat_ratio, int q_dtype, int k_dtype,
                                      int v_dtype, int64_t* offsets_out) {
  if (validate_common(B, S, H, D)) return -1;
  if (t_seq_len < 0 || t_seq_len > S) return -1;
  Sizes z = derive(S, t_seq_len, sparsity, srr, flat_ratio);
  Layout L = editing_layout(B, S, H, z, t_seq_len, q_dtype, k_dtype, v_dtype);
  if (offsets_out) std::memcpy(offsets_out, L.off, sizeof(L.off));
  return L.total;
}

int64_t icsa_editing_workspace_size(int B, int S, int H, int D, int t_seq_len, double sparsity,
                                    double srr, double flat_ratio, int q_dtype, int k_dtype,
                                    int v_dtype) {
  return icsa_editing_workspace_layout(B, S, H, D, t_seq_len, sparsity, srr, flat_ratio, q_dtype,
                                       k_dtype, v_dtype, nullptr);
}

}  // extern "C"

namespace {

#define ICSA_EDITING_ARGS                                                                    \
    const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,                   \
    const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,                   \
    const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,                   \
    int B, int S, int H, int D, int t_seq_len, double sparsity, double srr, double flat_ratio, \
    const void* alpha, int alpha_dtype, int64_t a_sb, int64_t a_ss, int64_t a_sh, int64_t a_sd, \
    float alpha_scalar,                                                                      \
    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,                     \
    const int32_t* inject_sel, const int32_t* inject_order, const int32_t* inject_l3,        \
    void* workspace, int64_t workspace_bytes, void* stream_
#define ICSA_EDITING_PASS                                                                    \
    q, q_dtype, q_sb, q_ss, q_sh, k, k_dtype, k_sb, k_ss, k_sh, v, v_dtype, v_sb, v_ss, v_sh, \
    B, S, H, D, t_seq_len, sparsity, srr, flat_ratio, alpha, alpha_dtype, a_sb, a_ss, a_sh,  \
    a_sd, alpha_scalar, out, out_dtype, o_sb, o_ss, o_sh, inject_sel, inject_order,          \
    inject_l3, workspace, workspace_bytes, stream_

int editing_impl(ICSA_EDITING_ARGS, void* const* stage_events, const float* qsum_in,
                 const float* ksum_in) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  auto mark = [&](int i) -> hipError_t {
    return stage_events ? hipEventRecord(reinterpret_cast<hipEvent_t>(stage_events[i]), stream)
                        : hipSuccess;
  };
  int rc = validate_common(B, S, H, D);
  if (rc) return rc;
  if ((rc = check_dtype(q_dtype, "q")) || (rc = check_dtype(k_dtype, "k")) ||
      (rc = check_dtype(v_dtype, "v")) || (rc = check_dtype(out_dtype, "out")))
    return rc;
  if (alpha && (rc = check_dtype(alpha_dtype, "alpha"))) return rc;
  const bool presummed = qsum_in != nullptr || ksum_in != nullptr;
  if (presummed && (!qsum_in || !ksum_in || q_dtype != ICSA_BF16 || k_dtype != ICSA_BF16))
    return fail(ICSA_EINVAL, "presummed q/k: both qsum and ksum are required and q, k must be bf16");
  if (!q || !k || !v || !out || !workspace) return fail(ICSA_EINVAL, "null q/k/v/out/workspace pointer");
  if (!row_ok(q, q_dtype, q_sb, q_ss, q_sh) || !row_ok(k, k_dtype, k_sb, k_ss, k_sh) ||
      !row_ok(v, v_dtype, v_sb, v_ss, v_sh) || !row_ok(out, out_dtype, o_sb, o_ss, o_sh))
    return fail(ICSA_EINVAL, "q/k/v/out rows must be 16-byte aligned (pointer and strides)");
  if (t_seq_len < 0 || t_seq_len > S) return fail(ICSA_EINVAL, "t_seq_len %d outside [0, S=%d]", t_seq_len, S);
  if (!(sparsity > 0.0) || !(srr >= 0.0) || !(flat_ratio >= 0.0 && flat_ratio <= 1.0))
    return fail(ICSA_EINVAL, "sparsity must be > 0, srr >= 0, flat_ratio in [0, 1]");
  const Sizes z = derive(S, t_seq_len, sparsity, srr, flat_ratio);
  if (z.Tkv <= 0) return fail(ICSA_EINVAL, "empty new KV (t_seq_len + 64 * topK == 0)");
  if (z.n_t > 4096 || z.n_s > 4096 || z.NB > 4096)
    return fail(ICSA_EUNSUPPORTED, "NB=%d blocks exceeds the 4096-block limit", z.NB);
  if (z.NKV > 2048 || z.top_k > 512)
    return fail(ICSA_EUNSUPPORTED, "NKV=%d / top_k=%d exceed limits (2048 / 512)", z.NKV, z.top_k);
  const Layout L = editing_layout(B, S, H, z, t_seq_len, q_dtype, k_dtype, v_dtype);
  if (workspace_bytes < L.total)
    return fail(ICSA_EWORKSPACE, "workspace %lld bytes < required %lld", (long long)workspace_bytes,
                (long long)L.total);
  char* ws = reinterpret_cast<char*>(workspace);
  auto WS = [&](int slot) { return ws + L.off[slot]; };
  const int BH = B * H;
  const int64_t Tvt = vt_columns(z, t_seq_len);
  const bool unaligned = (t_seq_len % ICSA_BLOCK) != 0;

  // ---- stage 1: pooling (+ V transposed, + bf16 copies of f32 q/k) ----
  PoolParams pp;
  std::memset(&pp, 0, sizeof(pp));
  if (!presummed) {                 // q / k sums from their producer otherwise
    pp.x[0] = TokTensor{q, q_sb, q_ss, q_sh, q_dtype};
    pp.x[1] = TokTensor{k, k_sb, k_ss, k_sh, k_dtype};
    pp.sums[0] = reinterpret_cast<float*>(WS(ICSA_WS_QSUM));
    pp.sums[1] = reinterpret_cast<float*>(WS(ICSA_WS_KSUM));
  }
  pp.x[2] = TokTensor{v, v_sb, v_ss, v_sh, v_dtype};
  pp.sums[2] = reinterpret_cast<float*>(WS(ICSA_WS_VSUM));
  pp.xb[0] = q_dtype == ICSA_F32 ? reinterpret_cast<bf16*>(WS(ICSA_WS_QB)) : nullptr;
  pp.xb[1] = k_dtype == ICSA_F32 ? reinterpret_cast<bf16*>(WS(ICSA_WS_KB)) : nullptr;
  // row-major bf16 values for the sparse kernel's straddling tiles (t % 64 != 0)
  pp.xb[2] = (unaligned && v_dtype == ICSA_F32) ? reinterpret_cast<bf16*>(WS(ICSA_WS_VB)) : nullptr;
  pp.xb_sb = (int64_t)S * H * ICSA_D; pp.xb_ss = (int64_t)H * ICSA_D; pp.xb_sh = ICSA_D;
  pp.vt = reinterpret_cast<bf16*>(WS(ICSA_WS_VT));
  pp.vt_sb = (int64_t)H * ICSA_D * Tvt; pp.vt_sh = ICSA_D * Tvt; pp.vt_sd = Tvt;
  pp.vt_src = 2;
  // V^T holds the new KV's tiles only: the pooling pass transposes the target blocks (block
  // n at columns 64 n ..), the selected source blocks follow after the selection
  pp.vt_limit = 1; pp.vt_nblk = ceil_div(t_seq_len, ICSA_BLOCK);
  pp.B = B; pp.S = S; pp.H = H; pp.NB = z.NB;
  ICSA_HIP_TRY(mark(ICSA_STAGE_START), "event");
  ICSA_HIP_TRY(launch_pool(pp, stream), "pool");
  ICSA_HIP_TRY(mark(ICSA_STAGE_POOL), "event");
  const float* qsum = presummed ? qsum_in : pp.sums[0];
  const float* ksum = presummed ? ksum_in : pp.sums[1];

  // bf16 views of q / k used by the attention kernels
  const bf16* qb = q_dtype == ICSA_BF16 ? reinterpret_cast<const bf16*>(q) : pp.xb[0];
  const int64_t qb_sb = q_dtype == ICSA_BF16 ? q_sb : pp.xb_sb;
  const int64_t qb_ss = q_dtype == ICSA_BF16 ? q_ss : pp.xb_ss;
  const int64_t qb_sh = q_dtype == ICSA_BF16 ? q_sh : pp.xb_sh;
  const bf16* kb = k_dtype == ICSA_BF16 ? reinterpret_cast<const bf16*>(k) : pp.xb[1];
  const int64_t kb_sb = k_dtype == ICSA_BF16 ? k_sb : pp.xb_sb;
  const int64_t kb_ss = k_dtype == ICSA_BF16 ? k_ss : pp.xb_ss;
  const int64_t kb_sh = k_dtype == ICSA_BF16 ? k_sh : pp.xb_sh;

  // ---- stage 2: compressed attention, retrieval, split ----
  CompressedParams cp;
  cp.qsum = qsum; cp.ksum = ksum; cp.vsum = pp.sums[2];
  cp.L = reinterpret_cast<float*>(WS(ICSA_WS_LOGITS));
  cp.out_c = reinterpret_cast<float*>(WS(ICSA_WS_OUTC));
  cp.sharp = reinterpret_cast<float*>(WS(ICSA_WS_SHARP));
  cp.colpart = reinterpret_cast<float*>(WS(ICSA_WS_COLP));
  cp.rstat = reinterpret_cast<float*>(WS(ICSA_WS_RSTAT));
  cp.vmt = reinterpret_cast<bf16*>(WS(ICSA_WS_L3S));    // free until the level-3 scores
  cp.BH = BH; cp.NB = z.NB; cp.S = S; cp.n_t = z.n_t; cp.n_s = z.n_s; cp.k_sparsity = z.k_sparsity;
  ICSA_HIP_TRY(launch_compressed(cp, stream), "compressed attention");
  ICSA_HIP_TRY(mark(ICSA_STAGE_COMPRESSED), "event");

  int32_t* sel = reinterpret_cast<int32_t*>(WS(ICSA_WS_SEL));
  int32_t* order = reinterpret_cast<int32_t*>(WS(ICSA_WS_ORDER));
  if (inject_sel && z.topK > 0)
    ICSA_HIP_TRY(hipMemcpyAsync(sel, inject_sel, (size_t)BH * z.topK * 4, hipMemcpyDeviceToDevice, stream),
                 "inject sel");
  if (inject_order)
    ICSA_HIP_TRY(hipMemcpyAsync(order, inject_order, (size_t)BH * z.NB * 4, hipMemcpyDeviceToDevice, stream),
                 "inject order");
  SelectParams sp;
  sp.colpart = cp.colpart; sp.sharp = cp.sharp;
  sp.src_score = reinterpret_cast<float*>(WS(ICSA_WS_SRCSCORE));
  sp.sel = sel; sp.order = order;
  sp.kvmap = reinterpret_cast<int*>(WS(ICSA_WS_KVMAP));
  sp.BH = BH; sp.NB = z.NB; sp.n_t = z.n_t; sp.n_s = z.n_s; sp.topK = z.topK; sp.NKV = z.NKV;
  sp.inject_sel = inject_sel ? 1 : 0;
  sp.inject_order = inject_order ? 1 : 0;
  ICSA_HIP_TRY(launch_select(sp, stream), "select");
  ICSA_HIP_TRY(launch_vt_blocks(pp, sel, z.n_t, std::max(z.topK, 1), z.topK, pp.vt_nblk, stream),
               "V^T of the selected blocks");

  // ---- new-KV block sums ----
  // The new KV is read in place.  For t % 64 != 0 its blocks from n_t on straddle two
  // blocks of the sequence (the t % 64 target-tail tokens, or the tail of the previous
  // selected block, then the head of the next one); their sums come from the token rows.
  const int seg_a = t_seq_len % ICSA_BLOCK;
  NewKvSumsParams np;
  std::memset(&np, 0, sizeof(np));
  np.kc32 = reinterpret_cast<float*>(WS(ICSA_WS_KC32));
  np.kc = reinterpret_cast<bf16*>(WS(ICSA_WS_KC));
  np.vct = unaligned ? nullptr : reinterpret_cast<bf16*>(WS(ICSA_WS_VCT));
  np.vc = unaligned ? reinterpret_cast<bf16*>(WS(ICSA_WS_VC)) : nullptr;
  np.BH = BH; np.NKV = z.NKV; np.NKVp = z.NKVp;
  np.ksum = ksum; np.vsum = pp.sums[2];
  np.kvmap = sp.kvmap; np.map_identity = 0; np.Nsrc = z.NB;
  np.k = TokTensor{k, k_sb, k_ss, k_sh, k_dtype};
  np.v = TokTensor{v, v_sb, v_ss, v_sh, v_dtype};
  np.seg_a = seg_a; np.seg_from = z.n_t; np.S = S; np.H = H;
  // values of the sparse kernel: V^T tiles (aligned t) or row-major bf16 rows (straddling tiles)
  const bf16* vrow = v_dtype == ICSA_BF16 ? reinterpret_cast<const bf16*>(v) : pp.xb[2];
  const int64_t vr_sb = v_dtype == ICSA_BF16 ? v_sb : pp.xb_sb;
  const int64_t vr_ss = v_dtype == ICSA_BF16 ? v_ss : pp.xb_ss;
  const int64_t vr_sh = v_dtype == ICSA_BF16 ? v_sh : pp.xb_sh;
  if (z.n_diffuse > 0) ICSA_HIP_TRY(launch_newkv_sums(np, stream), "new-KV sums");

  // ---- level-3 selection for the diffuse blocks ----
  int32_t* l3 = reinterpret_cast<int32_t*>(WS(ICSA_WS_L3));
  if (z.n_diffuse > 0) {
    if (inject_l3) {
      ICSA_HIP_TRY(hipMemcpyAsync(l3, inject_l3, (size_t)BH * z.n_diffuse * z.top_k * 4,
                                  hipMemcpyDeviceToDevice, stream), "inject l3");
    } else {
      Level3Params lp;
      lp.qsum = qsum; lp.rows = order; lp.rows_offset = z.n_peaked; lp.rows_stride = z.NB;
      lp.kc32 = np.kc32; lp.idx = l3; lp.scores = reinterpret_cast<float*>(WS(ICSA_WS_L3S));
      lp.BH = BH; lp.NQsrc = z.NB; lp.n_rows = z.n_diffuse; lp.NKV = z.NKV; lp.top_k = z.top_k;
      ICSA_HIP_TRY(launch_level3(lp, stream), "level-3 top-k");
    }
  }

  ICSA_HIP_TRY(mark(ICSA_STAGE_SELECT), "event");
  const AlphaView av = make_alpha(alpha, alpha_dtype, a_sb, a_ss, a_sh, a_sd, alpha_scalar);
  OutView ov{out, o_sb, o_ss, o_sh, out_dtype};
  const float scale_log2 = kLog2e / std::sqrt((float)ICSA_D);

  // ---- stage 4: sparse piecewise attention on the diffuse blocks ----
  if (z.n_diffuse > 0) {
    SparseParams s;
    std::memset(&s, 0, sizeof(s));
    s.q = qb; s.q_sb = qb_sb; s.q_ss = qb_ss; s.q_sh = qb_sh;
    s.k = kb; s.k_sb = kb_sb; s.k_st = kb_ss; s.k_sh = kb_sh;
    s.v_rows = unaligned ? 1 : 0;
    if (unaligned) {
      s.v = vrow; s.v_sb = vr_sb; s.v_st = vr_ss; s.v_sh = vr_sh;
    } else {
      s.vt = pp.vt; s.vt_sb = pp.vt_sb; s.vt_sh = pp.vt_sh; s.vt_sd = pp.vt_sd;
    }
    s.B = B; s.H = H; s.Sq = S; s.Sk = S;
    s.qblocks = order; s.qb_offset = z.n_peaked; s.qb_stride = z.NB; s.n_qblk = z.n_diffuse;
    s.kvmap = sp.kvmap; s.kvmap_identity = 0;
    s.seg_a = seg_a; s.seg_from = z.n_t;
    s.interval_bn = ICSA_BLOCK;        // the TileLang pipeline's BN (tilelang_host.py:127)
    s.idx = l3; s.top_k = z.top_k; s.NKV = z.NKV; s.NKVp = z.NKVp;
    s.kc = np.kc; s.vct = np.vct; s.vc = np.vc;
    s.out_c = cp.out_c; s.nb_q = z.NB;
    s.alpha = av; s.out = ov; s.scale_log2 = scale_log2; s.lse = nullptr;
    s.mask_tail = 0;                   // zero-padded new KV attended with logit 0 (TileLang)
    // the level-3 score rows are free again: BH * min(8, cdiv(NKV, 16)) floats of them hold the |KC_j|
    // bound of the interval pass
    if (interval_skip_enabled()) {
      s.kc_bound = reinterpret_cast<float*>(WS(ICSA_WS_L3S));
      ICSA_HIP_TRY(launch_kc_bound(np.kc, BH, z.NKV, z.NKVp, reinterpret_cast<float*>(WS(ICSA_WS_L3S)),
                                   &s.kc_bound_n, stream), "interval bound");
    }
    ICSA_HIP_TRY(launch_sparse(s, stream), "sparse attention");
  }
  ICSA_HIP_TRY(mark(ICSA_STAGE_SPARSE), "event");

  // ---- stage 3: flash attention on the peaked blocks ----
  if (z.n_peaked > 0) {
    FlashParams f;
    f.q = qb; f.q_sb = qb_sb; f.q_ss = qb_ss; f.q_sh = qb_sh;
    f.k = kb; f.k_sb = kb_sb; f.k_ss = kb_ss; f.k_sh = kb_sh;
    f.vt = pp.vt; f.vt_sb = pp.vt_sb; f.vt_sh = pp.vt_sh; f.vt_sd = pp.vt_sd;
    f.B = B; f.H = H; f.Sq = S; f.Sk = S;
    f.qblocks = order; f.qb_offset = 0; f.qb_stride = z.NB; f.n_qblk = z.n_peaked;
    f.t_limit = t_seq_len; f.n_tgt_tiles = ceil_div(t_seq_len, ICSA_BLOCK);
    f.sel = sel; f.sel_stride = std::max(z.topK, 1); f.n_sel = z.topK; f.sel_base = z.n_t;
    f.out_c = cp.out_c; f.nb_q = z.NB;
    f.alpha = av; f.out = ov; f.scale_log2 = scale_log2;
    ICSA_HIP_TRY(launch_flash(f, stream), "flash attention");
  }
  ICSA_HIP_TRY(mark(ICSA_STAGE_FLASH), "event");
  return ICSA_OK;
}

}  // namespace

extern "C" {

int icsa_editing_sparse_attention(ICSA_EDITING_ARGS) {
  return editing_impl(ICSA_EDITING_PASS, nullptr, nullptr, nullptr);
}

int icsa_editing_sparse_attention_ev(ICSA_EDITING_ARGS, void* const* stage_events) {
  return editing_impl(ICSA_EDITING_PASS, stage_events, nullptr, nullptr);
}

int icsa_editing_sparse_attention_presummed(ICSA_EDITING_ARGS, void* const* stage_events,
                                            const float* qsum, const float* ksum) {
  if (!qsum || !ksum) return fail(ICSA_EINVAL, "qsum / ksum are NULL");
  return editing_impl(ICSA_EDITING_PASS, stage_events, qsum, ksum);
}

}  // extern "C"

// ---------------------------------------------------------------------------------------
// No-allocation variant of icsa_editing_sparse_attention: its workspace is this file-scope
// device array (each device on which the entry runs holds its own copy until the process
// ends).  This file defines no kernel, so the array's code object is loaded onto a device
// only by the hipGetSymbolAddress of the entry's first call there; keep kernels out of this
// file, or every process that launches them would hold the array.  In host code `scratch`
// names a host-side stand-in, never the device memory, so the host only ever uses the
// per-device address returned by hipGetSymbolAddress.
// ---------------------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[ICSA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on the device that runs `stream`, looked up on the first
// call for that device and kept for later calls.  The lookup needs that device current,
// and the launches that follow set per-device kernel attributes on the current device,
// so a stream of any other device is refused.
int scratch_for_stream_device(hipStream_t stream, void** out) {
  int dev = 0, sdev = 0;
  ICSA_HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  if (stream != nullptr) {
    ICSA_HIP_TRY(hipStreamGetDevice(stream, &sdev), "hipStreamGetDevice");
    if (sdev != dev)
      return fail(ICSA_EINVAL, "stream belongs to device %d but device %d is current; make the "
                  "stream's device current before the call", sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ICSA_EUNSUPPORTED, "device %d outside the %d devices the scratch table covers", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    ICSA_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(ICSA_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return ICSA_OK;
}

}  // namespace

extern "C" {

int icsa_editing_sparse_attention_noalloc(
    const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,
    const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
    const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
    int B, int S, int H, int D, int t_seq_len, double sparsity, double srr, double flat_ratio,
    const void* alpha, int alpha_dtype, int64_t a_sb, int64_t a_ss, int64_t a_sh, int64_t a_sd,
    float alpha_scalar,
    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    const int32_t* inject_sel, const int32_t* inject_order, const int32_t* inject_l3,
    void* stream_) {
  // sizes first: an oversized request fails before any HIP call
  int rc = validate_common(B, S, H, D);
  if (rc) return rc;
  if ((rc = check_dtype(q_dtype, "q")) || (rc = check_dtype(k_dtype, "k")) || (rc = check_dtype(v_dtype, "v")))
    return rc;
  if (t_seq_len < 0 || t_seq_len > S) return fail(ICSA_EINVAL, "t_seq_len %d outside [0, S=%d]", t_seq_len, S);
  const Sizes z = derive(S, t_seq_len, sparsity, srr, flat_ratio);
  const int64_t need = editing_layout(B, S, H, z, t_seq_len, q_dtype, k_dtype, v_dtype).total;
  if (need > (int64_t)ICSA_NOALLOC_SCRATCH_BYTES)
    return fail(ICSA_EUNSUPPORTED,
                "this call needs %lld bytes of scratch, more than the %lld-byte static scratch of "
                "icsa_editing_sparse_attention_noalloc; call icsa_editing_sparse_attention with a "
                "workspace instead", (long long)need, (long long)ICSA_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = scratch_for_stream_device(reinterpret_cast<hipStream_t>(stream_), &ws))) return rc;
  void* workspace = ws;
  const int64_t workspace_bytes = ICSA_NOALLOC_SCRATCH_BYTES;
  return editing_impl(ICSA_EDITING_PASS, nullptr, nullptr, nullptr);
}

int icsa_wan_ln_modulate(const void* x, int x_dtype, int64_t x_sb, int64_t x_ss,
                         const void* y, int64_t y_sb, int64_t y_ss, const float* gate, int64_t g_sb,
                         float* x_out, int64_t xo_sb, int64_t xo_ss,
                         const float* lw, const float* lb,
                         const float* shift, const float* scale, int64_t mod_sb, float eps,
                         int B, int S, int dim, void* out, int64_t o_sb, int64_t o_ss, void* stream_) {
  int rc = check_dtype(x_dtype, "x");
  if (rc) return rc;
  if (B <= 0 || S <= 0 || dim <= 0) return fail(ICSA_EINVAL, "B, S, dim must be positive");
  if (dim % 4 != 0 || dim > 6144) return fail(ICSA_EUNSUPPORTED, "dim=%d: need dim %% 4 == 0 and <= 6144", dim);
  if (!x) return fail(ICSA_EINVAL, "x is NULL");
  if (y && (!gate || !x_out)) return fail(ICSA_EINVAL, "y given without gate / x_out");
  if (!y && !out) return fail(ICSA_EINVAL, "nothing to do (y and out are NULL)");
  if (!lw != !lb) return fail(ICSA_EINVAL, "lw and lb must be both given or both NULL");
  if (!shift != !scale) return fail(ICSA_EINVAL, "shift and scale must be both given or both NULL");
  auto al = [&](const void* p, int64_t s0, int64_t s1, int es) {
    return p == nullptr || (aligned16(p) && (s0 * es) % 16 == 0 && (s1 * es) % 16 == 0);
  };
  if (!al(x, x_sb, x_ss, elsize(x_dtype)) || !al(y, y_sb, y_ss, 2) || !al(gate, g_sb, 0, 4) ||
      !al(x_out, xo_sb, xo_ss, 4) || !al(lw, 0, 0, 4) || !al(lb, 0, 0, 4) || !al(shift, mod_sb, 0, 4) ||
      !al(scale, mod_sb, 0, 4) || !al(out, o_sb, o_ss, 2) || (dim * 2) % 16 != 0)
    return fail(ICSA_EINVAL, "rows must be 16-byte aligned (pointers and strides)");
  LnModParams p;
  std::memset(&p, 0, sizeof(p));
  p.x = x; p.x_dtype = x_dtype; p.x_sb = x_sb; p.x_ss = x_ss;
  p.y = reinterpret_cast<const bf16*>(y); p.y_sb = y_sb; p.y_ss = y_ss;
  p.gate = gate; p.g_sb = g_sb;
  p.x_out = x_out; p.xo_sb = xo_sb; p.xo_ss = xo_ss;
  p.lw = lw; p.lb = lb; p.shift = shift; p.scale = scale; p.mod_sb = mod_sb;
  p.out = reinterpret_cast<bf16*>(out); p.o_sb = o_sb; p.o_ss = o_ss;
  p.B = B; p.S = S; p.dim = dim; p.eps = eps;
  ICSA_HIP_TRY(launch_ln_mod(p, reinterpret_cast<hipStream_t>(stream_)), "layer norm / modulate");
  return ICSA_OK;
}

int64_t icsa_wan_qk_workspace_size(int B, int S) {
  if (B <= 0 || S <= 0) return -1;
  return align256((int64_t)B * S * 4) * 2;
}

int icsa_wan_qk_prologue(
    const void* yq, const void* yk, int y_dtype, int64_t y_sb, int64_t y_ss,
    const float* wq, const float* wk, float eps,
    const float* rope_cos, const float* rope_sin, int rope_rows,
    const int32_t* grids, int tag,
    const void* alpha_logit, int alpha_dtype, int64_t al_sb, int64_t al_ss,
    int B, int S, int H, int D,
    void* q_out, void* k_out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
    float* qsum, float* ksum, float* gate_out,
    void* workspace, int64_t workspace_bytes, void* stream_) {
  int rc = validate_common(B, S, H, D);
  if (rc) return rc;
  if ((rc = check_dtype(y_dtype, "y"))) return rc;
  if (alpha_logit && (rc = check_dtype(alpha_dtype, "alpha_logit"))) return rc;
  if (B > ICSA_WAN_MAX_BATCH) return fail(ICSA_EUNSUPPORTED, "B=%d exceeds %d", B, ICSA_WAN_MAX_BATCH);
  if (!yq || !wq || !rope_cos || !rope_sin || !grids || !q_out || !workspace)
    return fail(ICSA_EINVAL, "null pointer argument");
  if (yk && (!wk || !k_out)) return fail(ICSA_EINVAL, "yk given without wk / k_out");
  if (!qsum != !(yk ? ksum : qsum)) return fail(ICSA_EINVAL, "qsum and ksum must be both given or both NULL");
  if (alpha_logit && !gate_out) return fail(ICSA_EINVAL, "alpha_logit given without gate_out");
  if (!row_ok(yq, y_dtype, y_sb, y_ss, D) || (yk && !row_ok(yk, y_dtype, y_sb, y_ss, D)) ||
      !row_ok(q_out, ICSA_BF16, o_sb, o_ss, o_sh) || (yk && !row_ok(k_out, ICSA_BF16, o_sb, o_ss, o_sh)))
    return fail(ICSA_EINVAL, "y / q_out / k_out rows must be 16-byte aligned (pointer and strides)");
  if (!aligned16(wq) || (yk && !aligned16(wk)) || !aligned16(rope_cos) || !aligned16(rope_sin))
    return fail(ICSA_EINVAL, "norm weights and RoPE tables must be 16-byte aligned");
  if (!(eps >= 0.f)) return fail(ICSA_EINVAL, "eps must be >= 0");
  if (tag != 0 && tag != 1) return fail(ICSA_EINVAL, "tag must be 0 or 1");
  for (int b = 0; b < B; ++b)
    for (int a = 0; a < 6; ++a) {
      const int g = grids[6 * b + a];
      if (g < 0 || (g > 0 && g > rope_rows))
        return fail(ICSA_EINVAL, "grid size %d of batch %d outside [0, rope_rows=%d]", g, b, rope_rows);
    }
  const int64_t need = icsa_wan_qk_workspace_size(B, S);
  if (workspace_bytes < need)
    return fail(ICSA_EWORKSPACE, "workspace %lld bytes < required %lld", (long long)workspace_bytes,
                (long long)need);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  char* ws = reinterpret_cast<char*>(workspace);
  WanRmsParams rp;
  std::memset(&rp, 0, sizeof(rp));
  rp.y[0] = TokTensor{yq, y_sb, y_ss, D, y_dtype};
  rp.y[1] = TokTensor{yk, y_sb, y_ss, D, y_dtype};      // p == nullptr: q only
  rp.rinv[0] = reinterpret_cast<float*>(ws);
  rp.rinv[1] = reinterpret_cast<float*>(ws + align256((int64_t)B * S * 4));
  rp.alpha_logit = TokTensor{alpha_logit, al_sb, al_ss, 0, alpha_dtype};
  rp.gate = gate_out;
  rp.B = B; rp.S = S; rp.H = H; rp.eps = eps;
  WanQkParams qp;
  std::memset(&qp, 0, sizeof(qp));
  qp.y[0] = rp.y[0]; qp.y[1] = rp.y[1];
  qp.w[0] = wq; qp.w[1] = wk;
  qp.rinv[0] = rp.rinv[0]; qp.rinv[1] = rp.rinv[1];
  qp.rope_cos = rope_cos; qp.rope_sin = rope_sin;
  std::memcpy(qp.grids, grids, sizeof(int) * 6 * B);
  qp.tag = tag;
  qp.out[0] = OutView{q_out, o_sb, o_ss, o_sh, ICSA_DT_BF16};
  qp.out[1] = OutView{k_out, o_sb, o_ss, o_sh, ICSA_DT_BF16};
  qp.sums[0] = qsum; qp.sums[1] = ksum;
  qp.B = B; qp.S = S; qp.H = H; qp.NB = ceil_div(S, ICSA_BLOCK);
  ICSA_HIP_TRY(launch_wan_qk(rp, qp, stream), "wan q/k producer");
  return ICSA_OK;
}

// ---------------------------------------------------------------------------------------

}  // extern "C"

namespace {
struct SpLayout {
  int64_t qsum, ksum, vsum, kc32, kc, vc, idx, scores, total;
};
// Sizes for TQ / TKV rounded up to whole blocks (the Triton host's ragged lengths); the
// index buffer holds max(1, int(sparsity * NKV)) entries per query block, which is at
// least the Triton host's floor top_k.
SpLayout sparse_layout(int B, int H, int TQ, int TKV, double sparsity) {
  const int64_t BH = (int64_t)B * H;
  const int NQ = ceil_div(TQ, ICSA_BLOCK), NKV = ceil_div(TKV, ICSA_BLOCK);
  const int NKVp = ceil_div(NKV, 64) * 64;
  const int top_k = std::max(1, (int)(sparsity * (double)NKV));
  SpLayout L;
  int64_t o = 0;
  L.qsum = o; o += align256(BH * NQ * ICSA_D * 4);
  L.ksum = o; o += align256(BH * NKV * ICSA_D * 4);
  L.vsum = o; o += align256(BH * NKV * ICSA_D * 4);
  L.kc32 = o; o += align256(BH * NKV * ICSA_D * 4);
  L.kc = o; o += align256(BH * NKVp * ICSA_D * 2);
  L.vc = o; o += align256(BH * NKVp * ICSA_D * 2);
  L.idx = o; o += align256(BH * NQ * top_k * 4);
  L.scores = o; o += align256(BH * NQ * (int64_t)NKV * 4);
  L.total = o;
  return L;
}
}  // namespace

extern "C" {

int64_t icsa_sparse_piecewise_workspace_size(int B, int H, int TQ, int TKV, int D, double sparsity) {
  if (B <= 0 || H <= 0 || TQ <= 0 || TKV <= 0 || D != ICSA_D) return ICSA_EINVAL;
  if (!(sparsity > 0.0)) return ICSA_EINVAL;
  return sparse_layout(B, H, TQ, TKV, sparsity).total;
}

// triton == 0: the TileLang host (tilelang_host.py:229-274): TQ, TKV multiples of 64,
//   top_k = max(1, int(sparsity * NKV)).
// triton == 1: the Triton host (triton_host.py:11-30 -> triton_kernels.py:489-539): ragged
//   TQ / TKV, NKV = cdiv(TKV, 64) candidate blocks, top_k = max(1, int(sparsity *
//   (TKV // 64))), keys >= TKV masked out of the exact part.
static int sparse_piecewise_impl(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int B, int H, int TQ, int TKV, int D, double sparsity,
    const int32_t* inject_idx, int32_t* idx_out,
    void* out, int64_t o_sb, int64_t o_sh, int64_t o_st, float* lse_out,
    void* workspace, int64_t workspace_bytes, void* stream_, int triton, int interval_bn) {
  int rc = validate_common(B, TQ, H, D);
  if (rc) return rc;
  if (interval_bn != 16 && interval_bn != 32 && interval_bn != 64)
    return fail(ICSA_EUNSUPPORTED, "interval chunk BN=%d unsupported (16, 32 or 64)", interval_bn);
  if (TKV <= 0) return fail(ICSA_EINVAL, "TKV must be positive");
  if (!triton && (TQ % ICSA_BLOCK || TKV % ICSA_BLOCK))
    return fail(ICSA_EINVAL, "TQ/TKV must be divisible by the block size 64 (got %d, %d)", TQ, TKV);
  if (!q || !k || !v || !out || !workspace) return fail(ICSA_EINVAL, "null q/k/v/out/workspace pointer");
  if (!row_ok(q, ICSA_BF16, q_sb, q_sh, q_st) || !row_ok(k, ICSA_BF16, k_sb, k_sh, k_st) ||
      !row_ok(v, ICSA_BF16, v_sb, v_sh, v_st) || !row_ok(out, ICSA_BF16, o_sb, o_sh, o_st))
    return fail(ICSA_EINVAL, "q/k/v/out rows must be 16-byte aligned (pointer and strides)");
  if (!(sparsity > 0.0)) return fail(ICSA_EINVAL, "sparsity must be > 0");
  const int NQ = ceil_div(TQ, ICSA_BLOCK), NKV = ceil_div(TKV, ICSA_BLOCK);
  const int NKVp = ceil_div(NKV, 64) * 64;
  const int top_k = std::max(1, (int)(sparsity * (double)(triton ? TKV / ICSA_BLOCK : NKV)));
  if (NKV > 2048 || top_k > 512 || top_k > NKV)
    return fail(ICSA_EUNSUPPORTED, "NKV=%d / top_k=%d exceed limits (2048 / 512)", NKV, top_k);
  const SpLayout L = sparse_layout(B, H, TQ, TKV, sparsity);
  if (workspace_bytes < L.total)
    return fail(ICSA_EWORKSPACE, "workspace %lld bytes < required %lld", (long long)workspace_bytes,
                (long long)L.total);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  char* ws = reinterpret_cast<char*>(workspace);
  const int BH = B * H;

  PoolParams pq;
  std::memset(&pq, 0, sizeof(pq));
  pq.x[0] = TokTensor{q, q_sb, q_st, q_sh, ICSA_BF16};
  pq.sums[0] = reinterpret_cast<float*>(ws + L.qsum);
  pq.B = B; pq.S = TQ; pq.H = H; pq.NB = NQ;
  ICSA_HIP_TRY(launch_pool(pq, stream), "pool q");
  PoolParams pk;
  std::memset(&pk, 0, sizeof(pk));
  pk.x[1] = TokTensor{k, k_sb, k_st, k_sh, ICSA_BF16};
  pk.x[2] = TokTensor{v, v_sb, v_st, v_sh, ICSA_BF16};
  pk.sums[1] = reinterpret_cast<float*>(ws + L.ksum);
  pk.sums[2] = reinterpret_cast<float*>(ws + L.vsum);
  pk.B = B; pk.S = TKV; pk.H = H; pk.NB = NKV;
  ICSA_HIP_TRY(launch_pool(pk, stream), "pool k/v");

  NewKvSumsParams np;
  std::memset(&np, 0, sizeof(np));  // seg_a = 0: no straddling blocks
  np.ksum = pk.sums[1]; np.vsum = pk.sums[2]; np.kvmap = nullptr; np.map_identity = 1;
  np.kc32 = reinterpret_cast<float*>(ws + L.kc32);
  np.kc = reinterpret_cast<bf16*>(ws + L.kc);
  np.vct = nullptr;
  np.vc = reinterpret_cast<bf16*>(ws + L.vc);
  np.BH = BH; np.Nsrc = NKV; np.NKV = NKV; np.NKVp = NKVp;
  ICSA_HIP_TRY(launch_newkv_sums(np, stream), "block sums");

  int32_t* idx = reinterpret_cast<int32_t*>(ws + L.idx);
  if (inject_idx) {
    ICSA_HIP_TRY(hipMemcpyAsync(idx, inject_idx, (size_t)BH * NQ * top_k * 4, hipMemcpyDeviceToDevice,
                                stream), "inject idx");
  } else {
    Level3Params lp;
    lp.qsum = pq.sums[0]; lp.rows = nullptr; lp.rows_offset = 0; lp.rows_stride = 0;
    lp.kc32 = np.kc32; lp.idx = idx; lp.scores = reinterpret_cast<float*>(ws + L.scores);
    lp.BH = BH; lp.NQsrc = NQ; lp.n_rows = NQ; lp.NKV = NKV; lp.top_k = top_k;
    ICSA_HIP_TRY(launch_level3(lp, stream), "block top-k");
  }
  if (idx_out)
    ICSA_HIP_TRY(hipMemcpyAsync(idx_out, idx, (size_t)BH * NQ * top_k * 4, hipMemcpyDeviceToDevice, stream),
                 "copy idx");

  SparseParams s;
  std::memset(&s, 0, sizeof(s));   // seg_a = 0: the caller's new KV is contiguous
  s.q = reinterpret_cast<const bf16*>(q); s.q_sb = q_sb; s.q_ss = q_st; s.q_sh = q_sh;
  s.k = reinterpret_cast<const bf16*>(k); s.k_sb = k_sb; s.k_st = k_st; s.k_sh = k_sh;
  s.v_rows = 1;                      // v read in place, row tiles
  s.v = reinterpret_cast<const bf16*>(v); s.v_sb = v_sb; s.v_st = v_st; s.v_sh = v_sh;
  s.vt = nullptr; s.vt_sb = s.vt_sh = s.vt_sd = 0;
  s.B = B; s.H = H; s.Sq = TQ; s.Sk = TKV;
  s.qblocks = nullptr; s.qb_offset = 0; s.qb_stride = 0; s.n_qblk = NQ;
  s.kvmap = nullptr; s.kvmap_identity = 1;
  s.idx = idx; s.top_k = top_k; s.NKV = NKV; s.NKVp = NKVp;
  s.kc = np.kc; s.vct = nullptr; s.vc = np.vc;
  s.out_c = nullptr; s.nb_q = NQ;
  s.alpha = make_alpha(nullptr, ICSA_F32, 0, 0, 0, 0, 0.f);
  s.out = OutView{out, o_sb, o_st, o_sh, ICSA_BF16};
  s.scale_log2 = kLog2e / std::sqrt((float)ICSA_D);
  s.lse = lse_out;
  s.mask_tail = triton;
  s.interval_bn = interval_bn;
  // the block top-k score rows are free again: BH * min(8, cdiv(NKV, 16)) floats of them hold the
  // |KC_j| bound of the interval pass
  if (interval_skip_enabled()) {
    s.kc_bound = reinterpret_cast<float*>(ws + L.scores);
    ICSA_HIP_TRY(launch_kc_bound(np.kc, BH, NKV, NKVp, reinterpret_cast<float*>(ws + L.scores),
                                 &s.kc_bound_n, stream), "interval bound");
  }
  ICSA_HIP_TRY(launch_sparse(s, stream), "sparse attention");
  return ICSA_OK;
}

int icsa_sparse_piecewise_attn(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int B, int H, int TQ, int TKV, int D, double sparsity,
    const int32_t* inject_idx, int32_t* idx_out,
    void* out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    void* workspace, int64_t workspace_bytes, void* stream) {
  return sparse_piecewise_impl(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st, B, H,
                               TQ, TKV, D, sparsity, inject_idx, idx_out, out, o_sb, o_sh, o_st,
                               nullptr, workspace, workspace_bytes, stream, 0, ICSA_BLOCK);
}

int icsa_sparse_piecewise_attn_hosttopk(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int B, int H, int TQ, int TKV, int D, double sparsity, int interval_bn,
    const int32_t* inject_idx, int32_t* idx_out,
    void* out, int64_t o_sb, int64_t o_sh, int64_t o_st,
    void* workspace, int64_t workspace_bytes, void* stream) {
  return sparse_piecewise_impl(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st, B, H,
                               TQ, TKV, D, sparsity, inject_idx, idx_out, out, o_sb, o_sh, o_st,
                               nullptr, workspace, workspace_bytes, stream, 0, interval_bn);
}

int icsa_sparse_piecewise_attn_fwd(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    int B, int H, int TQ, int TKV, int D, double sparsity,
    const int32_t* inject_idx, int32_t* idx_out,
    void* out, int64_t o_sb, int64_t o_sh, int64_t o_st, float* lse_out,
    void* workspace, int64_t workspace_bytes, void* stream) {
  if (!idx_out || !lse_out) return fail(ICSA_EINVAL, "idx_out and lse_out are required (saved for the backward)");
  return sparse_piecewise_impl(q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb, v_sh, v_st, B, H,
                               TQ, TKV, D, sparsity, inject_idx, idx_out, out, o_sb, o_sh, o_st,
                               lse_out, workspace, workspace_bytes, stream, 1, ICSA_BLOCK);
}

// ---------------------------------------------------------------------------------------

}  // extern "C"

namespace {
struct BwLayout {
  int64_t ksum, vsum, dvec, selbits, kcb, vcb, dkc, dvc, total;
  int nsplit, qb_per_split;
};
// Interval partials: enough (chunk, query-range) workgroups to fill the GPU, each range at
// least 8 and at most 1024 query blocks long (the kernel stages a range's selection words
// in LDS).
BwLayout bwd_layout(int B, int H, int TQ, int TKV) {
  const int64_t BH = (int64_t)B * H;
  const int NQ = ceil_div(TQ, ICSA_BLOCK), NKV = ceil_div(TKV, ICSA_BLOCK);
  const int nc = ceil_div(NKV, 64), NKVp = nc * 64;
  BwLayout L;
  // interval workgroups: about five rounds of the 512 that fit on the GPU (two per CU), so
  // the last round's tail is small (1,080 workgroups, 2.1 rounds, measured 2 % slower)
  const int want = std::max(1, ceil_div(2560, (int)std::max<int64_t>(1, BH * nc)));
  int qbps = std::max(8, ceil_div(NQ, want));
  qbps = std::min(qbps, std::min(NQ, 1024));
  L.qb_per_split = qbps;
  L.nsplit = ceil_div(NQ, qbps);
  int64_t o = 0;
  L.ksum = o; o += align256(BH * NKV * ICSA_D * 4);
  L.vsum = o; o += align256(BH * NKV * ICSA_D * 4);
  L.dvec = o; o += align256(BH * (int64_t)NQ * ICSA_BLOCK * 4);   // D rows padded to whole blocks
  L.selbits = o; o += align256(BH * NQ * (int64_t)nc * 8);
  L.kcb = o; o += align256(BH * NKVp * ICSA_D * 2);
  L.vcb = o; o += align256(BH * NKVp * ICSA_D * 2);
  L.dkc = o; o += align256((int64_t)L.nsplit * BH * NKVp * ICSA_D * 4);
  L.dvc = o; o += align256((int64_t)L.nsplit * BH * NKVp * ICSA_D * 4);
  L.total = o;
  return L;
}
}  // namespace

extern "C" {

int64_t icsa_sparse_piecewise_attn_bwd_workspace_size(int B, int H, int TQ, int TKV, int D) {
  if (B <= 0 || H <= 0 || TQ <= 0 || TKV <= 0 || D != ICSA_D) return ICSA_EINVAL;
  return bwd_layout(B, H, TQ, TKV).total;
}

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
    void* workspace, int64_t workspace_bytes, void* stream_) {
  int rc = validate_common(B, TQ, H, D);
  if (rc) return rc;
  if ((rc = check_dtype(dq_dtype, "dq")) || (rc = check_dtype(dk_dtype, "dk")) || (rc = check_dtype(dv_dtype, "dv")))
    return rc;
  if (TKV <= 0) return fail(ICSA_EINVAL, "TKV must be positive");
  if (!dout || !q || !k || !v || !out || !lse || !idx || !dq || !dk || !dv || !workspace)
    return fail(ICSA_EINVAL, "null pointer argument");
  if (!row_ok(dout, ICSA_BF16, do_sb, do_sh, do_st) || !row_ok(q, ICSA_BF16, q_sb, q_sh, q_st) ||
      !row_ok(k, ICSA_BF16, k_sb, k_sh, k_st) || !row_ok(v, ICSA_BF16, v_sb, v_sh, v_st) ||
      !row_ok(out, ICSA_BF16, o_sb, o_sh, o_st) || !row_ok(dq, dq_dtype, dq_sb, dq_sh, dq_st) ||
      !row_ok(dk, dk_dtype, dk_sb, dk_sh, dk_st) || !row_ok(dv, dv_dtype, dv_sb, dv_sh, dv_st))
    return fail(ICSA_EINVAL, "rows must be 16-byte aligned (pointer and strides)");
  const int NQ = ceil_div(TQ, ICSA_BLOCK), NKV = ceil_div(TKV, ICSA_BLOCK);   // ragged: last block partial
  if (NQ > 4096 || NKV > 2048)
    return fail(ICSA_EUNSUPPORTED, "NQ=%d / NKV=%d exceed limits (4096 / 2048)", NQ, NKV);
  if (top_k < 1 || top_k > 512 || top_k > NKV)
    return fail(ICSA_EINVAL, "top_k=%d must be in [1, min(512, NKV=%d)]", top_k, NKV);
  const BwLayout L = bwd_layout(B, H, TQ, TKV);
  if (workspace_bytes < L.total)
    return fail(ICSA_EWORKSPACE, "workspace %lld bytes < required %lld", (long long)workspace_bytes,
                (long long)L.total);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  char* ws = reinterpret_cast<char*>(workspace);
  const int nc = ceil_div(NKV, 64);

  PoolParams pk;                                   // f32 block sums of k / v (the forward's)
  std::memset(&pk, 0, sizeof(pk));
  pk.x[1] = TokTensor{k, k_sb, k_st, k_sh, ICSA_BF16};
  pk.x[2] = TokTensor{v, v_sb, v_st, v_sh, ICSA_BF16};
  pk.sums[1] = reinterpret_cast<float*>(ws + L.ksum);
  pk.sums[2] = reinterpret_cast<float*>(ws + L.vsum);
  pk.B = B; pk.S = TKV; pk.H = H; pk.NB = NKV;
  ICSA_HIP_TRY(launch_pool(pk, stream), "pool k/v");

  SparseBwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = reinterpret_cast<const bf16*>(q); p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.k = reinterpret_cast<const bf16*>(k); p.k_sb = k_sb; p.k_sh = k_sh; p.k_st = k_st;
  p.v = reinterpret_cast<const bf16*>(v); p.v_sb = v_sb; p.v_sh = v_sh; p.v_st = v_st;
  p.dout = reinterpret_cast<const bf16*>(dout); p.do_sb = do_sb; p.do_sh = do_sh; p.do_st = do_st;
  p.out = reinterpret_cast<const bf16*>(out); p.o_sb = o_sb; p.o_sh = o_sh; p.o_st = o_st;
  p.lse = lse; p.idx = idx;
  p.B = B; p.H = H; p.TQ = TQ; p.TKV = TKV; p.NQ = NQ; p.NKV = NKV; p.nc = nc; p.NKVp = nc * 64;
  p.top_k = top_k; p.nsplit = L.nsplit; p.qb_per_split = L.qb_per_split;
  p.scale = 1.0f / std::sqrt((float)ICSA_D);
  p.scale_log2 = kLog2e / std::sqrt((float)ICSA_D);
  p.ksum = pk.sums[1]; p.vsum = pk.sums[2];
  p.dvec = reinterpret_cast<float*>(ws + L.dvec);
  p.selbits = reinterpret_cast<unsigned long long*>(ws + L.selbits);
  p.kcb = reinterpret_cast<bf16*>(ws + L.kcb);
  p.vcb = reinterpret_cast<bf16*>(ws + L.vcb);
  p.dkc_part = reinterpret_cast<float*>(ws + L.dkc);
  p.dvc_part = reinterpret_cast<float*>(ws + L.dvc);
  p.dq = OutView{dq, dq_sb, dq_st, dq_sh, dq_dtype == ICSA_F32 ? ICSA_DT_F32 : ICSA_DT_BF16};
  p.dk = OutView{dk, dk_sb, dk_st, dk_sh, dk_dtype == ICSA_F32 ? ICSA_DT_F32 : ICSA_DT_BF16};
  p.dv = OutView{dv, dv_sb, dv_st, dv_sh, dv_dtype == ICSA_F32 ? ICSA_DT_F32 : ICSA_DT_BF16};
  ICSA_HIP_TRY(launch_sparse_bwd_prep(p, stream), "backward prep");
  ICSA_HIP_TRY(launch_sparse_bwd(p, stream), "backward");
  return ICSA_OK;
}

int64_t icsa_flash_attn_workspace_size(int B, int Sk, int H, int D) {
  if (B <= 0 || Sk <= 0 || H <= 0 || D != ICSA_D) return -1;
  return align256((int64_t)B * H * ICSA_D * ceil_div(Sk, ICSA_BLOCK) * ICSA_BLOCK * 2);
}

int icsa_flash_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                    const void* k, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                    const void* v, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                    int B, int Sq, int Sk, int H, int D,
                    void* out, int out_dtype, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                    void* workspace, int64_t workspace_bytes, void* stream_) {
  int rc = validate_common(B, Sq, H, D);
  if (rc) return rc;
  if (Sk <= 0) return fail(ICSA_EINVAL, "Sk must be positive");
  if ((rc = check_dtype(out_dtype, "out"))) return rc;
  if (!q || !k || !v || !out || !workspace) return fail(ICSA_EINVAL, "null q/k/v/out/workspace pointer");
  if (!row_ok(q, ICSA_BF16, q_sb, q_ss, q_sh) || !row_ok(k, ICSA_BF16, k_sb, k_ss, k_sh) ||
      !row_ok(v, ICSA_BF16, v_sb, v_ss, v_sh) || !row_ok(out, out_dtype, o_sb, o_ss, o_sh))
    return fail(ICSA_EINVAL, "q/k/v/out rows must be 16-byte aligned (pointer and strides)");
  const int64_t need = icsa_flash_attn_workspace_size(B, Sk, H, D);
  if (workspace_bytes < need)
    return fail(ICSA_EWORKSPACE, "workspace %lld bytes < required %lld", (long long)workspace_bytes,
                (long long)need);
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const int NBk = ceil_div(Sk, ICSA_BLOCK);
  const int64_t Skp = (int64_t)NBk * ICSA_BLOCK;
  PoolParams pv;
  std::memset(&pv, 0, sizeof(pv));
  pv.x[2] = TokTensor{v, v_sb, v_ss, v_sh, ICSA_BF16};
  pv.vt = reinterpret_cast<bf16*>(workspace);
  pv.vt_sb = (int64_t)H * ICSA_D * Skp; pv.vt_sh = ICSA_D * Skp; pv.vt_sd = Skp;
  pv.vt_src = 2;
  pv.B = B; pv.S = Sk; pv.H = H; pv.NB = NBk;
  ICSA_HIP_TRY(launch_pool(pv, stream), "transpose v");
  FlashParams f;
  f.q = reinterpret_cast<const bf16*>(q); f.q_sb = q_sb; f.q_ss = q_ss; f.q_sh = q_sh;
  f.k = reinterpret_cast<const bf16*>(k); f.k_sb = k_sb; f.k_ss = k_ss; f.k_sh = k_sh;
  f.vt = pv.vt; f.vt_sb = pv.vt_sb; f.vt_sh = pv.vt_sh; f.vt_sd = pv.vt_sd;
  f.B = B; f.H = H; f.Sq = Sq; f.Sk = Sk;
  f.qblocks = nullptr; f.qb_offset = 0; f.qb_stride = 0; f.n_qblk = ceil_div(Sq, ICSA_BLOCK);
  f.t_limit = Sk; f.n_tgt_tiles = NBk;
  f.sel = nullptr; f.sel_stride = 0; f.n_sel = 0; f.sel_base = 0;
  f.out_c = nullptr; f.nb_q = 0;
  f.alpha = make_alpha(nullptr, ICSA_F32, 0, 0, 0, 0, 0.f);
  f.out = OutView{out, o_sb, o_ss, o_sh, out_dtype};
  f.scale_log2 = kLog2e / std::sqrt((float)ICSA_D);
  ICSA_HIP_TRY(launch_flash(f, stream), "flash attention");
  return ICSA_OK;
}

int icsa_pool(const void* q, int q_dtype, int64_t q_sb, int64_t q_ss, int64_t q_sh,
              const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
              const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
              int B, int S, int H, int D, float* qsum, float* ksum, float* vsum, void* vt,
              void* stream_) {
  int rc = validate_common(B, S, H, D);
  if (rc) return rc;
  PoolParams pp;
  std::memset(&pp, 0, sizeof(pp));
  const void* src[3] = {q, k, v};
  const int dt[3] = {q_dtype, k_dtype, v_dtype};
  const int64_t st[3][3] = {{q_sb, q_ss, q_sh}, {k_sb, k_ss, k_sh}, {v_sb, v_ss, v_sh}};
  float* sums[3] = {qsum, ksum, vsum};
  for (int i = 0; i < 3; ++i) {
    if (!src[i]) continue;
    if ((rc = check_dtype(dt[i], "input"))) return rc;
    if (!row_ok(src[i], dt[i], st[i][0], st[i][1], st[i][2]))
      return fail(ICSA_EINVAL, "input %d rows must be 16-byte aligned", i);
    pp.x[i] = TokTensor{src[i], st[i][0], st[i][1], st[i][2], dt[i]};
    pp.sums[i] = sums[i];
  }
  if (vt && !v) return fail(ICSA_EINVAL, "vt requested without v");
  const int NB = ceil_div(S, ICSA_BLOCK);
  const int64_t Sp = (int64_t)NB * ICSA_BLOCK;
  pp.vt = reinterpret_cast<bf16*>(vt);
  pp.vt_sb = (int64_t)H * ICSA_D * Sp; pp.vt_sh = ICSA_D * Sp; pp.vt_sd = Sp;
  pp.vt_src = 2;
  pp.B = B; pp.S = S; pp.H = H; pp.NB = NB;
  ICSA_HIP_TRY(launch_pool(pp, reinterpret_cast<hipStream_t>(stream_)), "pool");
  return ICSA_OK;
}

int icsa_gather_kv(const void* k, int k_dtype, int64_t k_sb, int64_t k_ss, int64_t k_sh,
                   const void* v, int v_dtype, int64_t v_sb, int64_t v_ss, int64_t v_sh,
                   int B, int S, int H, int D, int t_seq_len, const int32_t* sel, int topK,
                   void* kn, void* vn, void* stream_) {
  int rc = validate_common(B, S, H, D);
  if (rc) return rc;
  if ((rc = check_dtype(k_dtype, "k")) || (rc = check_dtype(v_dtype, "v"))) return rc;
  if (!k || !v || !kn || !vn || (topK > 0 && !sel)) return fail(ICSA_EINVAL, "null pointer");
  if (t_seq_len < 0 || t_seq_len > S || topK < 0) return fail(ICSA_EINVAL, "bad t_seq_len / topK");
  if (!row_ok(k, k_dtype, k_sb, k_ss, k_sh) || !row_ok(v, v_dtype, v_sb, v_ss, v_sh))
    return fail(ICSA_EINVAL, "k/v rows must be 16-byte aligned");
  GatherParams gp;
  gp.k = TokTensor{k, k_sb, k_ss, k_sh, k_dtype};
  gp.v = TokTensor{v, v_sb, v_ss, v_sh, v_dtype};
  gp.sel = sel;
  gp.kn = reinterpret_cast<bf16*>(kn);
  gp.vn = reinterpret_cast<bf16*>(vn);
  gp.B = B; gp.H = H; gp.S = S; gp.t = t_seq_len; gp.topK = topK;
  gp.Tkv = t_seq_len + topK * ICSA_BLOCK;
  gp.Tp = ceil_div(gp.Tkv, ICSA_BLOCK) * ICSA_BLOCK;
  if (gp.Tp == 0) return ICSA_OK;
  ICSA_HIP_TRY(launch_gather(gp, reinterpret_cast<hipStream_t>(stream_)), "gather");
  return ICSA_OK;
}

}  // extern "C"
