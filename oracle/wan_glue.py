"""CPU oracle of the Wan DiT glue that produces the attention inputs (test infrastructure only).

TEST INFRASTRUCTURE ONLY -- imported by tests/ and bench.py's reference-glue leg, never by
the HIP product path.

Restated from the reference (paths relative to the reference repository root):

* ``model.py:57-62``    ``rope_params``: complex128 table exp(i * pos * theta^(-2j/dim)).
* ``model.py:380-385``  the model's ``freqs``: three tables of widths D - 4*(D//6), 2*(D//6),
                        2*(D//6) concatenated along the pair axis.
* ``model.py:69-95``    ``rope_apply``: per batch element, target tokens rotated on the
                        target grid (frame, row, column), with TAG == 1 the source tokens
                        on their own grid after them, later tokens by 1 (``pad_freqs``);
                        the product runs in float64 and the result is cast to float32.
* ``model.py:103-114``  ``WanRMSNorm``: ``_norm(x.float()).type_as(x) * weight`` over the
                        model dim H*D.
* ``model.py:162``      the ``alpha_1`` gate ``(sigmoid(a) - 0.5) * 0.5``, evaluated in the
                        dtype of the projection (bf16 under the model's autocast).

Pinning (tests/test_wan_glue.py):

===================  ================================================================
function             pinned by
===================  ================================================================
``rope_params``      closed form at chosen (pos, j): angle = pos * theta^(-2j/dim);
                     unit modulus; position 0 is 1
``wan_freqs``        column split widths 22 / 21 / 21 for D = 128 (model.py:383-385,
                     rope_apply's split); each part equals its own rope_params table
``rope_apply``       brute-force scalar loop (math.cos / math.sin per element) at toy
                     grids; rotation preserves every pair's modulus; the relative-
                     position property (<rope(q, p1), rope(k, p2)> depends only on
                     p1 - p2 on each axis); token (0, 0, 0) and padding tokens are not
                     rotated; TAG == 1 source tokens restart at position (0, 0, 0)
``rms_norm``         unit RMS (before the bf16 rounding) for weight 1; invariance under
                     positive scaling of the row; outputs are bf16 values times weight
``alpha_gate``       gate(0) = 0; closed form at chosen logits with bf16 rounding
===================  ================================================================
"""
from __future__ import annotations

import math
from typing import Sequence

import torch


def rope_params(max_seq_len: int, dim: int, theta: float = 10000.0) -> torch.Tensor:
    """complex128 [max_seq_len, dim // 2]: exp(i * pos / theta^(2j / dim)) (model.py:57-62)."""
    assert dim % 2 == 0
    pos = torch.arange(max_seq_len, dtype=torch.float64)
    inv = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                          torch.arange(0, dim, 2, dtype=torch.float64) / dim)
    ang = torch.outer(pos, inv)
    return torch.polar(torch.ones_like(ang), ang)


def wan_freqs(head_dim: int = 128, max_seq_len: int = 1024) -> torch.Tensor:
    """The model's RoPE table (model.py:380-385): complex128 [max_seq_len, head_dim // 2]."""
    d = head_dim
    return torch.cat([rope_params(max_seq_len, d - 4 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6))], dim=1)


def rope_split(head_dim: int) -> tuple[int, int, int]:
    """Pair counts of the frame / row / column axes (rope_apply's freqs.split, model.py:71)."""
    c = head_dim // 2
    return (c - 2 * (c // 3), c // 3, c // 3)


def token_positions(S: int, grid: Sequence[int], src_grid: Sequence[int], tag: int):
    """int64 [S, 3] (frame, row, column) per token, -1 for tokens that are not rotated."""
    pos = torch.full((S, 3), -1, dtype=torch.int64)
    f, h, w = grid
    n_t = f * h * w
    idx = torch.arange(min(n_t, S))
    pos[:len(idx), 0] = idx // (h * w)
    pos[:len(idx), 1] = (idx // w) % h
    pos[:len(idx), 2] = idx % w
    if tag == 1:
        sf, sh, sw = src_grid
        n_s = sf * sh * sw
        lo, hi = n_t, min(S, n_t + n_s)
        if hi > lo:
            idx = torch.arange(hi - lo)
            pos[lo:hi, 0] = idx // (sh * sw)
            pos[lo:hi, 1] = (idx // sw) % sh
            pos[lo:hi, 2] = idx % sw
    return pos


def rope_apply(x: torch.Tensor, grid_sizes, source_grid_sizes, tag: int,
               freqs: torch.Tensor) -> torch.Tensor:
    """model.py:69-95 on x [B, S, H, D]: float64 complex product, returned as float32."""
    B, S, H, D = x.shape
    nf, nh, nw = rope_split(D)
    out = torch.empty(B, S, H, D, dtype=torch.float32, device=x.device)
    for b in range(B):
        pos = token_positions(S, [int(v) for v in grid_sizes[b]],
                              [int(v) for v in source_grid_sizes[b]], tag)
        rot = torch.ones(S, D // 2, dtype=torch.complex128)
        ok = pos[:, 0] >= 0
        parts = torch.split(freqs, [nf, nh, nw], dim=1)
        for a in range(3):
            cols = slice(sum((nf, nh, nw)[:a]), sum((nf, nh, nw)[:a + 1]))
            rot[ok, cols] = parts[a][pos[ok, a]]
        xc = torch.view_as_complex(x[b].to(torch.float64).reshape(S, H, D // 2, 2).contiguous())
        out[b] = torch.view_as_real(xc * rot.to(x.device)[:, None, :]).reshape(S, H, D).float()
    return out


def rms_norm(y: torch.Tensor, weight: torch.Tensor, eps: float,
             round_to=torch.bfloat16) -> torch.Tensor:
    """WanRMSNorm (model.py:103-114) on y [..., dim]: r = rsqrt(mean(y^2) + eps) in float64
    here, the normalised row rounded to ``round_to`` (the projection dtype; None keeps
    float64), times the weight.  Returns float64."""
    y64 = y.to(torch.float64)
    n = y64 * torch.rsqrt(y64.pow(2).mean(dim=-1, keepdim=True) + eps)
    if round_to is not None:
        n = n.to(round_to).to(torch.float64)
    return n * weight.to(torch.float64)


def alpha_gate(logit: torch.Tensor) -> torch.Tensor:
    """(sigmoid(a) - 0.5) * 0.5 with every step rounded to bf16 (model.py:162 under the
    model's bf16 autocast).  Returns float32 values."""
    s = torch.sigmoid(logit.to(torch.float64)).to(torch.bfloat16)
    g = (s.float() - 0.5).to(torch.bfloat16).float() * 0.5
    return g


def wan_qk(yq: torch.Tensor, yk: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, eps: float,
           grid_sizes, source_grid_sizes, tag: int, freqs: torch.Tensor, H: int):
    """The q / k producer of WanSelfAttention.forward (model.py:156-171) on projections
    yq, yk [B, S, H*D] (bf16 or float32): returns float32 q, k [B, S, H, D] as the
    reference hands them to editing_sparse_attention."""
    B, S, dim = yq.shape
    D = dim // H
    out = []
    rnd = torch.bfloat16 if yq.dtype == torch.bfloat16 else None   # .type_as(x)
    for y, w in ((yq, wq), (yk, wk)):
        m = rms_norm(y, w, eps, round_to=rnd).to(torch.float32)     # (bf16 or f32) * w -> f32
        out.append(rope_apply(m.view(B, S, H, D), grid_sizes, source_grid_sizes, tag, freqs))
    return out[0], out[1]
