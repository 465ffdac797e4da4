// Tile toolkit shared by the flash-attention (stage 3) and sparse piecewise (stage 4)
// kernels.  One wave owns 32 queries; a key tile is 64 keys x 128 dims.
//
// Orientation: the score tile is computed transposed, S^T[key][query] = K Q^T, with
// v_mfma_f32_32x32x16_bf16 (A = K rows from LDS, B = Q^T held in registers).  The result
// layout puts one query per lane (lane % 32) and 16 of the 32 keys of a sub-tile in each
// lane; the other 16 keys of that query sit in lane ^ 32.  Row max / row sum therefore
// need one v_permlane32_swap per tile instead of a 32-lane reduction.
//
// PV: O^T[d][query] += V^T[d][key] P^T[key][query] with A = V^T from LDS and B = P^T
// straight from the score registers.  The keys one lane holds for a 16-key MFMA step are
// {0-3, 8-11} (lanes 0-31) and {4-7, 12-15} (lanes 32-63); V^T is stored with bits 2 and
// 3 of the token index swapped (kv_slot) so those 8 keys are one contiguous 16-byte read.
//
// LDS tiles are XOR-swizzled in 16-byte chunks so the MFMA operand reads are free of bank
// conflicts: K tile row r chunk c at c ^ (r & 15); V^T tile row d chunk c at c ^ ((d>>1)&7).
#pragma once

#include <atomic>

#include "icsa_common.h"

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once per device
// (the attribute belongs to the device's copy of the kernel).  `done`: one bit per device.
inline hipError_t ensure_lds_limit(const void* func, int bytes, std::atomic<unsigned>* done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const unsigned bit = dev >= 0 && dev < 32 ? (1u << dev) : 0u;
  if (bit != 0u && (done->load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(func, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit != 0u) done->fetch_or(bit, std::memory_order_release);
  return e;
}

#define ATT_BN 64                         // keys per tile
#define K_TILE_BYTES (ATT_BN * ICSA_D * 2)    // 16 KB
#define V_TILE_BYTES (ICSA_D * ATT_BN * 2)    // 16 KB

// Raw buffer resource over [base, base + bytes): loads past the range return no data,
// which keeps a tile's DMA inside the rows that exist.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffffLL ? 0x7fffffff : (int)(bytes < 0 ? 0 : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// Workgroup barrier without a memory fence.  __syncthreads() also waits for every
// outstanding LDS-DMA load (vmcnt(0)), which would cut a tile prefetch short; kernels
// using this wait for their tile DMA explicitly.  LDS reads and writes issued before the
// barrier are complete when it is passed (lgkmcnt(0)).
#define ATT_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// Register staging of one K + V^T tile for a workgroup of NT threads (NT = 256 or 128).
template <int NT>
struct TileRegs {
  static constexpr int N = (ATT_BN * ICSA_D / 8) / NT;   // 16-byte chunks per thread per tile
  u32x4 k[N];
  u32x4 v[N];
};

__device__ __forceinline__ int k_lds_off(int row, int chunk) {     // in bf16 elements
  return row * ICSA_D + ((chunk ^ (row & 15)) << 3);
}
__device__ __forceinline__ int v_lds_off(int d, int chunk) {
  return d * ATT_BN + ((chunk ^ ((d >> 1) & 7)) << 3);
}

// Global -> registers for one tile.  krow0: pointer to key row 0 of the tile, k_rs: key row
// stride (elements), k_valid: rows < k_valid are real (others read as 0).  vcol0: pointer
// to V^T row d = 0 at the tile's first slot, v_rs: V^T row stride; v_zero: zero V^T tile.
template <int NT>
__device__ __forceinline__ void tile_load_regs(TileRegs<NT>& r, const bf16* krow0, int64_t k_rs,
                                               int k_valid, const bf16* vcol0, int64_t v_rs,
                                               bool v_zero) {
  constexpr int N = TileRegs<NT>::N;
  constexpr int KR = NT / 16;          // key rows covered per pass
  constexpr int VR = NT / 8;           // V^T rows covered per pass
  const int t = threadIdx.x;
  const int kr = t >> 4, kc = t & 15;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int row = kr + KR * i;
    if (row < k_valid)
      r.k[i] = *reinterpret_cast<const u32x4*>(krow0 + (int64_t)row * k_rs + 8 * kc);
    else
      r.k[i] = u32x4{0u, 0u, 0u, 0u};
  }
  const int vd = t >> 3, vc = t & 7;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int d = vd + VR * i;
    if (!v_zero)
      r.v[i] = *reinterpret_cast<const u32x4*>(vcol0 + (int64_t)d * v_rs + 8 * vc);
    else
      r.v[i] = u32x4{0u, 0u, 0u, 0u};
  }
}

template <int NT>
__device__ __forceinline__ void tile_store_lds(const TileRegs<NT>& r, bf16* ks, bf16* vs) {
  constexpr int N = TileRegs<NT>::N;
  constexpr int KR = NT / 16;
  constexpr int VR = NT / 8;
  const int t = threadIdx.x;
  const int kr = t >> 4, kc = t & 15;
#pragma unroll
  for (int i = 0; i < N; ++i)
    *reinterpret_cast<u32x4*>(ks + k_lds_off(kr + KR * i, kc)) = r.k[i];
  const int vd = t >> 3, vc = t & 7;
#pragma unroll
  for (int i = 0; i < N; ++i)
    *reinterpret_cast<u32x4*>(vs + v_lds_off(vd + VR * i, vc)) = r.v[i];
}

// Q^T operand of one wave: 32 queries (rows qrow0 + lane%32, rows >= q_valid are zero).
__device__ __forceinline__ void load_q_frags(bf16x8 qf[8], const bf16* qrow0, int64_t q_rs,
                                             int q_valid) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, hl = lane >> 5;
  if (li < q_valid) {
    const bf16* src = qrow0 + (int64_t)li * q_rs + 8 * hl;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) qf[kk] = *reinterpret_cast<const bf16x8*>(src + 16 * kk);
  } else {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      bf16x8 z;
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] = (bf16)0.f;
      qf[kk] = z;
    }
  }
}

// S^T for the 64 keys of an LDS K tile: s[ks] covers keys 32*ks .. 32*ks + 31.
__device__ __forceinline__ void qk_tile(floatx16 s[2], const bf16* ks, const bf16x8 qf[8]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, hl = lane >> 5;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    floatx16 acc = {};
    const int row = 32 * sub + li;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(ks + k_lds_off(row, 2 * kk + hl));
      acc = mfma32x32x16(a, qf[kk], acc);
    }
    s[sub] = acc;
  }
}

// O^T[4 d-subtiles] += V^T P^T for one tile; p[m] holds the bf16 probabilities of 16-key
// step m (m = 0..3).
__device__ __forceinline__ void pv_tile(floatx16 o[4], const bf16* vs, const bf16x8 p[4]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, hl = lane >> 5;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(vs + v_lds_off(32 * ds + li, 2 * m + hl));
      o[ds] = mfma32x32x16(a, p[m], o[ds]);
    }
  }
}

// ---------------------------------------------------------------------------------------
// Row tiles: 64 rows x 128 dims bf16, row-major as in the caller's tensors, for operands
// that are needed transposed (V in PV, and K / Q / dO in the backward).  16-byte chunk c of
// row r sits at slot c ^ swz(r).
//  * rt_swz (backward tiles, also read untransposed): a bijection of r % 16, so 16-byte
//    operand reads of 16 consecutive rows (one chunk) hit 16 distinct slots;
//  * rv_swz (the forward kernels' V tiles, only ever read transposed): r % 4 alone, so rows
//    8 apart share a slot pattern.
// Both move rows 4 a + x (x = 0..3) to different slot quadrants, so a transposing read
// (4 rows x 4 chunk positions x 2 halves per half-wave) touches 32 distinct 8-byte bank
// pairs.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ int rt_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int rv_swz(int r) { return (r & 3) << 2; }
template <bool RV>
__device__ __forceinline__ int tile_swz(int r) { return RV ? rv_swz(r) : rt_swz(r); }
__device__ __forceinline__ int rt_off(int row, int chunk) {        // in bf16 elements
  return row * ICSA_D + ((chunk ^ rt_swz(row)) << 3);
}

typedef short rt_v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) rt_v4s* rt_lds_v4s;

// Transposed MFMA operands straight from a row tile (ds_read_b64_tr_b16).  Within each
// group of 16 lanes, lane j of the transposing read receives element j % 4 of the 4-element
// vectors read by lanes j / 4 + 4 e (e = 0..3).  For the A operand of
// O^T[d][key] += X^T[d][row] P[row][key] (X a 64 x 128 row tile, lane l = 16 g + s holding
// A[d = 32 ds + l % 32][k = 8 (l / 32) + e]) with the row order of the score accumulators
// (k -> row 16 m + 8 (e / 4) + 4 (l / 32) + e % 4), lane 16 g + s reads the 4 dims
// 32 ds + 16 (g % 2) + 4 (s % 4) .. + 3 of row 16 m + 4 (g / 2) + s / 4 (+ 8 for e >= 4).
// tro[ds]: those byte offsets (rows 0..7, e < 4) for m = 0; step m adds 16 rows.  The
// rows 8 further on (e >= 4) are derived, not stored: rv_swz(r + 8) = rv_swz(r), a constant
// 8-row offset; rt_swz(r + 8) = rt_swz(r) ^ 2 for r < 8, slot bit 1 (byte bit 5) flipped.
template <bool RV>
__device__ __forceinline__ void rt_tr_offsets(int tro[4], int lane) {
  const int g = lane >> 4, s = lane & 15;
  const int row = 4 * (g >> 1) + (s >> 2);
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
    const int col = 32 * ds + 16 * (g & 1) + 4 * (s & 3);
    tro[ds] = row * (ICSA_D * 2) + (((col >> 3) ^ tile_swz<RV>(row)) << 4) + (col & 7) * 2;
  }
}
template <bool RV>
__device__ __forceinline__ int rt_tr_hi(int off) { return (RV ? off : (off ^ 32)) + 8 * ICSA_D * 2; }

// The transposed A operand of PV step t = 4 m + ds (two transposing reads).
template <bool RV>
__device__ __forceinline__ bf16x8 rt_tr_operand(const unsigned char* tile, const int tro[4], int t) {
  const int m = t >> 2, ds = t & 3;
  const rt_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((rt_lds_v4s)(tile + tro[ds] + m * 16 * ICSA_D * 2));
  const rt_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (rt_lds_v4s)(tile + rt_tr_hi<RV>(tro[ds]) + m * 16 * ICSA_D * 2));
  const short __attribute__((ext_vector_type(8))) a8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, a8);
}

// o[4 d-subtiles] += X^T P for a row tile X (bytes at `tile`); p[m]: bf16 B operand of
// 16-row step m, straight from the score accumulators.  Each operand is read PF steps ahead.
template <int PF, bool RV>
__device__ __forceinline__ void pv_tile_tr(floatx16 o[4], const unsigned char* tile, const int tro[4],
                                           const bf16x8 p[4]) {
  bf16x8 a[16];
#pragma unroll
  for (int t = 0; t < PF; ++t) a[t] = rt_tr_operand<RV>(tile, tro, t);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    if (t + PF < 16) a[t + PF] = rt_tr_operand<RV>(tile, tro, t + PF);
    o[t & 3] = mfma32x32x16(a[t], p[t >> 2], o[t & 3]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// bf16 B operand of PV step m from the score registers (keys of sub-tile m/2, half m%2).
__device__ __forceinline__ void pack_p(bf16x8 p[4], const floatx16 s[2]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int e = 0; e < 8; ++e) p[m][e] = (bf16)s[m >> 1][8 * (m & 1) + e];
  }
}

// Residual epilogue: out[tok, d] = o[query][d] * inv_l + alpha(b,tok,h,d) * out_c[blk][d].
// o_lds: this wave's [32][O_LDS_STRIDE] fp32 staging area.  Rows >= rows_valid skipped.
#define O_LDS_STRIDE (ICSA_D + 1)

__device__ __forceinline__ void stage_o(float* o_lds, const floatx16 o[4], float inv_l) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 31;
#pragma unroll
  for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
    for (int i = 0; i < 16; ++i) o_lds[li * O_LDS_STRIDE + 32 * ds + acc_row(i, lane)] = o[ds][i] * inv_l;
  }
}

__device__ __forceinline__ float alpha_at(const AlphaView& a, int b, int tok, int h, int d) {
  if (a.p == nullptr) return a.scalar;
  const int64_t off = (int64_t)b * a.sb + (int64_t)tok * a.ss + (int64_t)h * a.sh + (int64_t)d * a.sd;
  if (a.dtype == ICSA_DT_F32) return reinterpret_cast<const float*>(a.p)[off];
  return (float)reinterpret_cast<const bf16*>(a.p)[off];
}

// Stores the wave's 32 staged rows starting at token tok0 (rows tok0 + r for r < rows_valid).
__device__ __forceinline__ void store_rows(const float* o_lds, const OutView& out, int b, int h,
                                           int tok0, int rows_valid, const float* oc_row,
                                           const AlphaView& alpha) {
  const int lane = threadIdx.x & 63;
  const int ch = lane & 15;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = (lane >> 4) + 4 * j;
    if (r >= rows_valid) continue;
    const int tok = tok0 + r;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = o_lds[r * O_LDS_STRIDE + 8 * ch + e];
    if (oc_row != nullptr) {
      const floatx4 c0 = *reinterpret_cast<const floatx4*>(oc_row + 8 * ch);
      const floatx4 c1 = *reinterpret_cast<const floatx4*>(oc_row + 8 * ch + 4);
      if (alpha.p == nullptr || alpha.sd == 0) {
        const float a = alpha_at(alpha, b, tok, h, 8 * ch);
#pragma unroll
        for (int e = 0; e < 4; ++e) { v[e] = fmaf(a, c0[e], v[e]); v[4 + e] = fmaf(a, c1[e], v[4 + e]); }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = fmaf(alpha_at(alpha, b, tok, h, 8 * ch + e), c0[e], v[e]);
          v[4 + e] = fmaf(alpha_at(alpha, b, tok, h, 8 * ch + 4 + e), c1[e], v[4 + e]);
        }
      }
    }
    const int64_t off = (int64_t)b * out.sb + (int64_t)tok * out.ss + (int64_t)h * out.sh + 8 * ch;
    if (out.dtype == ICSA_DT_BF16) {
      *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(out.p) + off) = pack8_bf16(v);
    } else {
      float* dst = reinterpret_cast<float*>(out.p) + off;
      *reinterpret_cast<floatx4*>(dst) = floatx4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<floatx4*>(dst + 4) = floatx4{v[4], v[5], v[6], v[7]};
    }
  }
}
