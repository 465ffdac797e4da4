// Caller-side producer of the attention inputs in the Wan DiT self-attention.
//
// Reference: WanSelfAttention.forward, model.py:152-171:
//   q = norm_q(self.q(x)) ; k = norm_k(self.k(x))           WanRMSNorm, model.py:103-114
//   alpha_1 = (sigmoid(self.alpha_1(x)) - 0.5) * 0.5           model.py:162
//   q = rope_apply(q, ...) ; k = rope_apply(k, ...)            model.py:69-95 (float64 complex)
// after which editing_sparse_attention pools q / k (editing_sparse_attention.py:107-111).
// The Linear projections stay with the caller (library GEMMs); these kernels take their
// outputs y = x W^T + b and produce, in one read of y and one write:
//   * bf16 q / k in [B, S, H, D]  (what the attention kernels read),
//   * fp32 64-token block sums of the fp32 rotated q / k (what stage 1 would have computed),
//   * the alpha_1 gate.
//
// Arithmetic follows the reference step by step:
//   r      = rsqrt(mean_{H*D}(y^2) + eps)          fp32 (x.float() in _norm)
//   n      = y * r, rounded to bf16 for bf16 y     .type_as(x)
//   m      = float(n) * w                          bf16 * fp32 weight -> fp32
//   (m0 + i m1) * (cos + i sin)                    the complex product of rope_apply, in fp32
//                                                  here (float64 there; both round to fp32)
// RoPE positions: token p < t_len sits at (f, h, w) of the target grid; with TAG == 1 the
// next s_len tokens restart at (0, 0, 0) on the source grid; every later token is not
// rotated (pad_freqs pads with ones).  Pair j of a head uses the f axis for j < D/2 - 2*(D/2/3),
// then the h axis and the w axis for D/2/3 pairs each (rope_apply's freqs.split).
#include "icsa_kernels.h"

// ---- per-token RMS factors (+ alpha gate): one wave per token ----
__global__ void __launch_bounds__(256) icsa_wan_rms_kernel(WanRmsParams p) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t tok_all = (int64_t)blockIdx.x * 4 + wave;          // b * S + s
  if (tok_all >= (int64_t)p.B * p.S) return;
  const int b = (int)(tok_all / p.S), s = (int)(tok_all % p.S);
  const int dim = p.H * ICSA_D;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const TokTensor& y = p.y[i];
    if (y.p == nullptr) continue;           // single-tensor mode (k absent)
    float ss = 0.f;
    for (int c = lane; c < dim / 8; c += 64) {
      float v[8];
      if (y.dtype == ICSA_DT_F32)
        load8_f32<float>(reinterpret_cast<const float*>(y.p) + (int64_t)b * y.sb + (int64_t)s * y.ss + 8 * c, v);
      else
        load8_f32<bf16>(reinterpret_cast<const bf16*>(y.p) + (int64_t)b * y.sb + (int64_t)s * y.ss + 8 * c, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) p.rinv[i][tok_all] = 1.f / sqrtf(ss / (float)dim + p.eps);
  }
  if (p.alpha_logit.p != nullptr && lane == 0) {
    const int64_t off = (int64_t)b * p.alpha_logit.sb + (int64_t)s * p.alpha_logit.ss;
    const float a = p.alpha_logit.dtype == ICSA_DT_F32 ? reinterpret_cast<const float*>(p.alpha_logit.p)[off]
                                                       : (float)reinterpret_cast<const bf16*>(p.alpha_logit.p)[off];
    // bf16 arithmetic of the reference: sigmoid, - 0.5 and * 0.5 each round to bf16
    const float sg = (float)(bf16)(1.f / (1.f + expf(-a)));
    const float g = (float)(bf16)(sg - 0.5f) * 0.5f;
    p.gate[tok_all] = g;
  }
}

// RoPE position of token tok on axis a (0: frames, 1: height, 2: width); -1: not rotated
__device__ __forceinline__ void rope_pos(const WanQkParams& p, int b, int tok, int pos[3]) {
  const int* g = p.grids + 6 * b;   // kernel-argument array
  const int t_len = g[0] * g[1] * g[2];
  const int s_len = g[3] * g[4] * g[5];
  int local = -1;
  const int* gr = g;
  if (tok < t_len) {
    local = tok;
  } else if (p.tag == 1 && tok < t_len + s_len) {
    local = tok - t_len;
    gr = g + 3;
  }
  if (local < 0) {
    pos[0] = pos[1] = pos[2] = -1;
    return;
  }
  const int hw = gr[1] * gr[2];
  pos[0] = local / hw;
  pos[1] = (local / gr[2]) % gr[1];
  pos[2] = local % gr[2];
}

// ---- normalise, rotate, cast, block sums: one workgroup per (head, 64-token block, b) ----
// q and k are processed in the same pass: they share the token positions and the cos / sin
// of every pair, and their row loads are in flight together.
template <typename T>
__global__ void __launch_bounds__(256) icsa_wan_qk_kernel(WanQkParams p) {
  constexpr bool kBf16In = sizeof(T) == 2;
  __shared__ float red[2][16][ICSA_D + 4];
  __shared__ int pos_s[ICSA_BLOCK][4];
  __shared__ float r_s[2][ICSA_BLOCK];
  // head fastest: neighbouring workgroups cover one token row's heads, so the rows stream
  const int h = blockIdx.x, n = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x;
  if (t < ICSA_BLOCK) {                     // RoPE positions of the block's tokens, once
    int pos[3];
    rope_pos(p, b, n * ICSA_BLOCK + t, pos);
    pos_s[t][0] = pos[0];
    pos_s[t][1] = pos[1];
    pos_s[t][2] = pos[2];
  } else if (t < 3 * ICSA_BLOCK) {          // 1 / rms of the block's q and k rows
    const int i = (t - ICSA_BLOCK) / ICSA_BLOCK, r = t % ICSA_BLOCK;
    const int tok = n * ICSA_BLOCK + r;
    r_s[i][r] = (tok < p.S && p.y[i].p != nullptr) ? p.rinv[i][(int64_t)b * p.S + tok] : 0.f;
  }
  __syncthreads();
  const int c = t & 15;          // chunk of 8 dims: pairs 4c .. 4c + 3
  const int g = t >> 4;          // 16 token groups of 4 tokens
  const int nt = p.y[1].p != nullptr ? 2 : 1;     // single-tensor mode: q only
  const T* ybase[2];
  float w[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (i >= nt) break;
    ybase[i] = reinterpret_cast<const T*>(p.y[i].p) + (int64_t)b * p.y[i].sb + (int64_t)h * ICSA_D + 8 * c;
    load8_f32<float>(p.w[i] + h * ICSA_D + 8 * c, w[i]);
  }
  const int npair = ICSA_D / 2;
  const int n_hw = npair / 3, n_f = npair - 2 * n_hw;
  int axis[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int j = 4 * c + e;
    axis[e] = j < n_f ? 0 : (j < n_f + n_hw ? 1 : 2);
  }
  const bool one_axis = axis[0] == axis[3];
  float acc[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int r = g + 16 * jj;
    const int tok = n * ICSA_BLOCK + r;
    if (tok >= p.S) continue;
    float v[2][8];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if (i < nt) load8_f32<T>(ybase[i] + (int64_t)tok * p.y[i].ss, v[i]);
    const int* pos = pos_s[r];
    float cs[4], sn[4];
    if (one_axis) {                        // the chunk's 4 pairs use one axis: one row segment
      const int ps = pos[axis[0]];
      if (ps >= 0) {
        const floatx4 c4 = *reinterpret_cast<const floatx4*>(p.rope_cos + (int64_t)ps * npair + 4 * c);
        const floatx4 s4 = *reinterpret_cast<const floatx4*>(p.rope_sin + (int64_t)ps * npair + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) { cs[e] = c4[e]; sn[e] = s4[e]; }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) { cs[e] = 1.f; sn[e] = 0.f; }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ps = pos[axis[e]];
        cs[e] = ps >= 0 ? p.rope_cos[(int64_t)ps * npair + 4 * c + e] : 1.f;
        sn[e] = ps >= 0 ? p.rope_sin[(int64_t)ps * npair + 4 * c + e] : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i >= nt) break;
      const float rr = r_s[i][r];
      float m[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // .type_as(x): the normalised row returns to the projection dtype before the weight
        const float nrm = v[i][e] * rr;
        m[e] = (kBf16In ? (float)(bf16)nrm : nrm) * w[i][e];
      }
      float o[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float m0 = m[2 * e], m1 = m[2 * e + 1];
        o[2 * e] = fmaf(m0, cs[e], -m1 * sn[e]);
        o[2 * e + 1] = fmaf(m0, sn[e], m1 * cs[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[i][e] += o[e];
      const OutView& ov = p.out[i];
      bf16* dst = reinterpret_cast<bf16*>(ov.p) + (int64_t)b * ov.sb + (int64_t)tok * ov.ss +
                  (int64_t)h * ov.sh + 8 * c;
      *reinterpret_cast<bf16x8*>(dst) = pack8_bf16(o);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[i][g][8 * c + e] = acc[i][e];
  __syncthreads();
  {
    const int i = t >> 7, d = t & 127;     // 256 threads: (tensor, dim)
    if (i < nt && p.sums[i] != nullptr) {
      float s = 0.f;
#pragma unroll
      for (int gg = 0; gg < 16; ++gg) s += red[i][gg][d];    // fixed order, as the pool kernel
      p.sums[i][(((int64_t)b * p.H + h) * p.NB + n) * ICSA_D + d] = s;
    }
  }
}

hipError_t launch_wan_qk(const WanRmsParams& rp, const WanQkParams& qp, hipStream_t stream) {
  const int64_t ntok = (int64_t)rp.B * rp.S;
  hipLaunchKernelGGL(icsa_wan_rms_kernel, dim3((unsigned)((ntok + 3) / 4)), dim3(256), 0, stream, rp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 grid(qp.H, qp.NB, qp.B);
  if (qp.y[0].dtype == ICSA_DT_F32)
    hipLaunchKernelGGL(icsa_wan_qk_kernel<float>, grid, dim3(256), 0, stream, qp);
  else
    hipLaunchKernelGGL(icsa_wan_qk_kernel<bf16>, grid, dim3(256), 0, stream, qp);
  return hipGetLastError();
}
