// New-KV gather: materialise new_k / new_v = [K[:t] | K_pad[n_t*64 + 64*sel[r] + i]]
// as [B, H, Tp, D] bf16 (rows >= Tkv zero).
//
// Reference: editing_sparse_attention.py:138-159 (new_k / new_v construction; K_pad is K
// zero-padded to a multiple of 64 tokens) and :189-198 (zero padding of TKV to a multiple
// of 64 for the sparse call).  The fused pipeline reads the new KV in place when t is a
// multiple of 64; this kernel serves an unaligned t (new-KV blocks then straddle source
// blocks) and the materialised-KV entry point.
#include "icsa_kernels.h"

template <typename TK, typename TV>
__global__ void __launch_bounds__(256) icsa_gather_kernel(GatherParams p) {
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int ch = threadIdx.x & 15;
  if (row >= p.Tp) return;
  const int n_t = p.t / ICSA_BLOCK;
  int src = -1;
  if (row < p.t) {
    src = row;
  } else if (row < p.Tkv) {
    const int r = (row - p.t) / ICSA_BLOCK, i = (row - p.t) % ICSA_BLOCK;
    src = (n_t + p.sel[(int64_t)bh * p.topK + r]) * ICSA_BLOCK + i;
    if (src >= p.S) src = -1;
  }
  float kv[8], vv[8];
  if (src >= 0) {
    load8_f32<TK>(reinterpret_cast<const TK*>(p.k.p) + (int64_t)b * p.k.sb + (int64_t)src * p.k.ss +
                      (int64_t)h * p.k.sh + 8 * ch, kv);
    load8_f32<TV>(reinterpret_cast<const TV*>(p.v.p) + (int64_t)b * p.v.sb + (int64_t)src * p.v.ss +
                      (int64_t)h * p.v.sh + 8 * ch, vv);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) { kv[e] = 0.f; vv[e] = 0.f; }
  }
  const int64_t off = ((int64_t)bh * p.Tp + row) * ICSA_D + 8 * ch;
  *reinterpret_cast<bf16x8*>(p.kn + off) = pack8_bf16(kv);
  *reinterpret_cast<bf16x8*>(p.vn + off) = pack8_bf16(vv);
}

hipError_t launch_gather(const GatherParams& p, hipStream_t stream) {
  dim3 grid((p.Tp + 15) / 16, p.B * p.H);
  const int code = p.k.dtype * 2 + p.v.dtype;
  switch (code) {
    case 0: hipLaunchKernelGGL((icsa_gather_kernel<bf16, bf16>), grid, dim3(256), 0, stream, p); break;
    case 1: hipLaunchKernelGGL((icsa_gather_kernel<bf16, float>), grid, dim3(256), 0, stream, p); break;
    case 2: hipLaunchKernelGGL((icsa_gather_kernel<float, bf16>), grid, dim3(256), 0, stream, p); break;
    case 3: hipLaunchKernelGGL((icsa_gather_kernel<float, float>), grid, dim3(256), 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
