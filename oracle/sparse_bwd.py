"""CPU oracle of the sparse piecewise attention backward (test infrastructure only).

TEST INFRASTRUCTURE ONLY -- imported by tests/, never by the HIP product path.

Restated from the reference (paths relative to the reference repository root):

* ``triton_kernels.py:265-486``  ``sparse_piecewise_attn_1st_intervals_bwd_kernel``: per
  64-row query block, with ``D = rowsum(dO * O)`` and ``P = exp2(s - lse)`` (scores in log2
  units, ``lse`` saved by the forward):
    - exact part, every selected block: ``dS = P (dO V^T - D)``; ``dq += dS K scale``;
      ``dk += dS^T q scale``; ``dv += P^T dO`` (:330-377);
    - interval part, every unselected block ``c < NKV`` (block sums KC / VC):
      ``s = q KC^T scale / 64``; ``dS = P (dO VC^T - 64 D)``; ``dq += dS KC scale / 64``;
      ``dKC = dS^T q scale``, ``dVC = P^T dO``; every key row of block c receives
      ``dKC_c / 64`` and ``dVC_c`` (:379-475).
* ``triton_kernels.py:541-598``  ``SparsePiecewiseAttn1stIntervalsFunction.backward``: fp32
  gradients, cast to the inputs' dtype at the end.

Ragged lengths (the Triton host passes any TQ / TKV): ``NQ = cdiv(TQ, 64)``,
``NKV = cdiv(TKV, 64)``; q / dO / o rows past TQ and k / v rows past TKV are zero (the
reference's tensor descriptors read zeros there, lse included, :284-313), keys at
positions >= TKV are masked out of the exact part (``-inf``, :348), the interval takes
every unselected block ``c < NKV`` with the block sums over the real rows and the same
``/ 64`` and weight 64 (:400-412), and only rows < TQ / < TKV of the gradients exist.

The reference's fp32 atomics become plain sums here (the order of a float64 sum does not
matter at the tolerance).  The lse passed in is used as given: the forward's
non-rescaled interval accumulators make it differ from the true log-sum-exp when the
running max grows inside the interval loop, and the backward reproduces the reference
with that lse.

Pinning (tests/test_sparse_bwd_oracle.py): (i) when o and lse are those of softmax
attention over the "virtual keys" (the selected blocks' rows plus one key KC_c / 64 of
multiplicity 64 per unselected block) the result equals torch.autograd's gradient of that
attention, built independently from gathers and block sums; (ii) top_k = NKV reduces to
the gradient of float64 scaled_dot_product_attention; (iii) shifting lse by delta scales
every gradient by 2^-delta (lse is in log2 units); (iv) brute-force scalar loops.
"""
from __future__ import annotations

import math

import torch

from .icsa_oracle import BLOCK_M

LOG2E = 1.0 / math.log(2.0)


def sparse_piecewise_attn_bwd(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                              v: torch.Tensor, o: torch.Tensor, lse: torch.Tensor,
                              indices: torch.Tensor, dtype=torch.float64):
    """Gradients ``(dq, dk, dv)`` (``dtype``) of the sparse piecewise attention.

    q, do, o ``[B,H,TQ,D]``; k, v ``[B,H,TKV,D]`` (any lengths); lse ``[B,H,TQ]``
    in log2 units; indices ``[B,H,NQ,top_k]`` (selected key blocks per query block, in any
    order, distinct)."""
    B, H, TQ0, D = q.shape
    TKV0 = k.shape[2]
    NQ, NKV = -(-TQ0 // BLOCK_M), -(-TKV0 // BLOCK_M)
    TQ, TKV = NQ * BLOCK_M, NKV * BLOCK_M
    top_k = indices.shape[-1]
    scale = 1.0 / math.sqrt(D)
    pad_q = lambda t: torch.nn.functional.pad(t.to(dtype), (0, 0, 0, TQ - TQ0))
    pad_k = lambda t: torch.nn.functional.pad(t.to(dtype), (0, 0, 0, TKV - TKV0))
    qd, dod, od = pad_q(q), pad_q(do), pad_q(o)
    kd, vd = pad_k(k), pad_k(v)
    lse_n = torch.nn.functional.pad(lse.to(dtype), (0, TQ - TQ0)) / LOG2E   # natural-log units
    key_real = (torch.arange(TKV) < TKV0).view(NKV, BLOCK_M)              # exact-part key mask
    Dv = (dod * od).sum(-1)                                # [B,H,TQ]
    KC = kd.view(B, H, NKV, BLOCK_M, D).sum(3)
    VC = vd.view(B, H, NKV, BLOCK_M, D).sum(3)
    idx = indices.long()

    # exact part: per query block, its top_k blocks as one key set of top_k * 64 rows
    kb = kd.view(B, H, NKV, BLOCK_M, D)
    vb = vd.view(B, H, NKV, BLOCK_M, D)
    bi = torch.arange(B).view(B, 1, 1, 1)
    hi = torch.arange(H).view(1, H, 1, 1)
    kx = kb[bi, hi, idx].reshape(B, H, NQ, top_k * BLOCK_M, D)
    vx = vb[bi, hi, idx].reshape(B, H, NQ, top_k * BLOCK_M, D)
    qb = qd.view(B, H, NQ, BLOCK_M, D)
    dob = dod.view(B, H, NQ, BLOCK_M, D)
    lb = lse_n.view(B, H, NQ, BLOCK_M, 1)
    Db = Dv.view(B, H, NQ, BLOCK_M, 1)
    p = torch.exp(torch.matmul(qb, kx.transpose(-2, -1)) * scale - lb)
    p = p * key_real[idx].reshape(B, H, NQ, 1, top_k * BLOCK_M)
    ds = p * (torch.matmul(dob, vx.transpose(-2, -1)) - Db)
    dq = torch.matmul(ds, kx) * scale
    dkx = (torch.matmul(ds.transpose(-2, -1), qb) * scale).view(B, H, NQ, top_k, BLOCK_M, D)
    dvx = torch.matmul(p.transpose(-2, -1), dob).view(B, H, NQ, top_k, BLOCK_M, D)
    dk = torch.zeros(B, H, NKV, BLOCK_M, D, dtype=dtype)
    dv = torch.zeros_like(dk)
    flat = idx.reshape(B, H, NQ * top_k)
    for b in range(B):
        for h in range(H):
            dk[b, h].index_add_(0, flat[b, h], dkx[b, h].reshape(NQ * top_k, BLOCK_M, D))
            dv[b, h].index_add_(0, flat[b, h], dvx[b, h].reshape(NQ * top_k, BLOCK_M, D))

    # interval part: every unselected block of every query block
    selected = torch.zeros(B, H, NQ, NKV, dtype=torch.bool)
    selected.scatter_(-1, idx, True)
    sel_rows = selected.repeat_interleave(BLOCK_M, dim=2)            # [B,H,TQ,NKV]
    s = torch.matmul(qd, KC.transpose(-2, -1)) * (scale / BLOCK_M)
    pc = torch.exp(s - lse_n[..., None]).masked_fill(sel_rows, 0.0)
    dsc = pc * (torch.matmul(dod, VC.transpose(-2, -1)) - BLOCK_M * Dv[..., None])
    dq = dq.reshape(B, H, TQ, D) + torch.matmul(dsc, KC) * (scale / BLOCK_M)
    dKC = torch.matmul(dsc.transpose(-2, -1), qd) * scale             # [B,H,NKV,D]
    dVC = torch.matmul(pc.transpose(-2, -1), dod)
    dk = dk + (dKC / BLOCK_M)[:, :, :, None, :]
    dv = dv + dVC[:, :, :, None, :]
    return (dq[:, :, :TQ0], dk.reshape(B, H, TKV, D)[:, :, :TKV0],
            dv.reshape(B, H, TKV, D)[:, :, :TKV0])
