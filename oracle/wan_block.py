"""CPU oracle of one Wan DiT block around the attention path (test infrastructure only).

TEST INFRASTRUCTURE ONLY -- imported by tests/, never by the HIP product path.

Restated from the reference (paths relative to the reference repository root):

* ``model.py:224-270``  ``WanAttentionBlock.forward``: adaLN chunks of modulation + e,
                        norm1 / modulate -> self attention -> gated residual, norm3 ->
                        cross attention -> residual, norm2 / modulate -> FFN -> gated residual.
* ``model.py:117-122``  ``WanLayerNorm`` (LayerNorm over dim, optional affine).
* ``model.py:152-177``  ``WanSelfAttention.forward`` (via oracle.wan_glue and the path oracle).
* ``model.py:180-188``  ``WanT2VCrossAttention.forward`` with ``wanx/attention.py:18-83``
                        (dense attention on bf16 q / k / v, bf16 result).
* ``model.py:243-245``  the FFN: Linear, GELU(tanh), Linear.

Precision: float64 between the rounding points of the model under bf16 autocast -- every
Linear takes bf16 inputs, bf16 weights and bias and returns bf16; LayerNorm, RMSNorm,
modulation and the residual stream are fp32-or-better.  The self attention's ranked
decisions may be injected (the GPU's own, so that a near-tie cannot cascade).

Pinning: the block is a composition of pinned parts (oracle.wan_glue, the path oracle, the
textbook LayerNorm / SDPA / GELU of PyTorch in float64); tests/test_wan_block_oracle.py
additionally checks the composition against closed forms (zero modulation gates make the
block the identity; a zero FFN / cross-attention output projection removes that branch).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import icsa_oracle as O
from . import wan_glue as W


def bf(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 and return float64 (a rounding point of the bf16 model)."""
    return t.to(torch.bfloat16).to(torch.float64)


def linear(x, w, b=None):
    """nn.Linear under bf16 autocast: bf16 input, weight and bias; bf16 result."""
    y = bf(x) @ bf(w).T
    if b is not None:
        y = y + bf(b)
    return bf(y)


def layer_norm(x, eps, w=None, b=None):
    x = x.to(torch.float64)
    mean = x.mean(-1, keepdim=True)
    var = (x - mean).pow(2).mean(-1, keepdim=True)
    y = (x - mean) / torch.sqrt(var + eps)
    if w is not None:
        y = y * w.double() + b.double()
    return y


def wan_block_forward(P: dict, x, e, context, grid, src_grid, tag, freqs, num_heads, eps=1e-6,
                      decisions=None, sparsity=0.0625, x_is_bf16=False, device="cpu"):
    """One block on float64 tensors.  P: the block's state dict (reference parameter names).
    x [B, S, dim], e [B, 6, dim], context [B, L, dim].  ``x_is_bf16``: the block input is the
    bf16 patch embedding (the model's first block), so norm1's ``.type_as(x)`` rounds the
    LayerNorm to bf16.  ``device``: where the float64 arithmetic runs (the same operations
    on either device).  Returns (x, path-oracle info)."""
    B, S, dim = x.shape
    H = num_heads
    D = dim // H
    p = {k: v.detach().to(device).double() for k, v in P.items()}
    x = x.detach().to(device).double()
    context = context.detach().to(device).double()
    em = (p["modulation"] + e.detach().to(device).double()).chunk(6, dim=1)

    # self attention on norm1(x) * (1 + e1) + e0 (model.py:255-257)
    n1 = layer_norm(x, eps)
    h = (bf(n1) if x_is_bf16 else n1) * (1 + em[1]) + em[0]
    yq = linear(h, p["self_attn.q.weight"], p["self_attn.q.bias"])
    yk = linear(h, p["self_attn.k.weight"], p["self_attn.k.bias"])
    yv = linear(h, p["self_attn.v.weight"], p["self_attn.v.bias"])
    al = linear(h, p["self_attn.alpha_1.weight"])
    q, k = W.wan_qk(yq.to(torch.bfloat16), yk.to(torch.bfloat16), p["self_attn.norm_q.weight"],
                    p["self_attn.norm_k.weight"], eps, [grid] * B, [src_grid] * B, tag, freqs, H)
    gate = W.alpha_gate(al.view(B, S).float()).view(B, S, 1, 1)
    t = grid[0] * grid[1] * grid[2]
    xa, info = O.editing_sparse_attention(q, k, yv.view(B, S, H, D), t, S - t, alpha_2=gate,
                                          SPARSITY_RATIO=sparsity, decisions=decisions)
    y = linear(xa.reshape(B, S, dim), p["self_attn.o.weight"], p["self_attn.o.bias"])
    x = x + y * em[2]

    # cross attention on norm3(x) (model.py:264, 180-188)
    if "norm3.weight" in p:
        h = layer_norm(x, eps, p["norm3.weight"], p["norm3.bias"])
    else:
        h = x
    cq = W.rms_norm(linear(h, p["cross_attn.q.weight"], p["cross_attn.q.bias"]),
                    p["cross_attn.norm_q.weight"], eps)
    ck = W.rms_norm(linear(context, p["cross_attn.k.weight"], p["cross_attn.k.bias"]),
                    p["cross_attn.norm_k.weight"], eps)
    cv = linear(context, p["cross_attn.v.weight"], p["cross_attn.v.bias"])
    L = context.shape[1]
    qh = bf(cq).view(B, S, H, D).transpose(1, 2)
    kh = bf(ck).view(B, L, H, D).transpose(1, 2)
    vh = cv.view(B, L, H, D).transpose(1, 2).contiguous()
    # softmax(q k^T / sqrt(D)) v, the textbook attention (what SDPA computes), with contiguous
    # operands and queries in chunks to bound the [S, L] score memory
    kt = kh.transpose(-2, -1).contiguous()
    att = torch.cat([torch.matmul(torch.softmax(torch.matmul(qh[:, :, i:i + 8192], kt) / math.sqrt(D), -1), vh)
                     for i in range(0, S, 8192)], dim=2).transpose(1, 2).reshape(B, S, dim)
    y = linear(bf(att), p["cross_attn.o.weight"], p["cross_attn.o.bias"])
    x = x + y

    # FFN on norm2(x) * (1 + e4) + e3 (model.py:265-268)
    h = layer_norm(x, eps) * (1 + em[4]) + em[3]
    f1 = linear(h, p["ffn.0.weight"], p["ffn.0.bias"])
    g = bf(F.gelu(f1, approximate="tanh"))
    y = linear(g, p["ffn.2.weight"], p["ffn.2.bias"])
    x = x + y * em[5]
    return x, info
