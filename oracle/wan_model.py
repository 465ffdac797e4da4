"""CPU oracle of the Wan DiT forward around the attention path (test infrastructure only).

TEST INFRASTRUCTURE ONLY -- imported by tests/, never by the HIP product path.

Restated from the reference (paths relative to the reference repository root):

* ``model.py:410-451``  ``WanModel._forward``: patch embeddings of the target and source
                        latents (Conv3d, kernel = stride = patch size), [target | source]
                        concatenation, zero padding to seq_len, sinusoidal time embedding
                        -> time_embedding -> time_projection (float32 region), text
                        embedding of the zero-padded prompts, the blocks, removal of the
                        source tokens, the head and ``unpatchify``.
* ``model.py:25-31``    ``sinusoidal_embedding_1d``.
* ``model.py:272-290``  ``Head`` (float32 region).
* ``model.py:456-466``  ``unpatchify``.

Precision: float64 between the rounding points of the model under bf16 autocast (see
oracle.wan_block); the float32 autocast regions (time embedding, head) are float64 here.
Per-block self-attention decisions may be injected.

Pinning: a composition of pinned parts (oracle.wan_block, float64 textbook ops);
tests/test_wan_model_oracle.py checks the patch embedding against torch's Conv3d, the
unpatchify against an explicit index loop, and that the model with zero-gated blocks
reduces to head(patch embedding).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from .wan_block import bf, linear, layer_norm, wan_block_forward


def sinusoidal_embedding_1d(dim, position):
    half = dim // 2
    position = position.to(torch.float64)
    sinusoid = torch.outer(position, torch.pow(10000, -torch.arange(half, dtype=torch.float64).div(half)))
    return torch.cat([torch.cos(sinusoid), torch.sin(sinusoid)], dim=1)


def patch_embed(u, w, b, patch):
    """Conv3d with kernel = stride = patch on u [C, F, H, W] (bf16 autocast: bf16 result).
    Returns ([L, dim] float64, grid)."""
    C, F_, H_, W_ = u.shape
    pf, ph, pw = patch
    g = (F_ // pf, H_ // ph, W_ // pw)
    p = u.double().reshape(C, g[0], pf, g[1], ph, g[2], pw).permute(1, 3, 5, 0, 2, 4, 6)
    p = p.reshape(-1, C * pf * ph * pw)
    return linear(p, w.reshape(w.shape[0], -1), b), g


def unpatchify(x, grid, patch, c):
    u = x[:math.prod(grid)].reshape(*grid, *patch, c)
    u = torch.einsum('fhwpqrc->cfphqwr', u)
    return u.reshape(c, *[i * j for i, j in zip(grid, patch)])


def wan_model_forward(P: dict, cfg: dict, x_list, t, context_list, seq_len, src_list, freqs,
                      decisions=None):
    """WanModel forward on float64.  P: the model's state dict; cfg: patch_size, dim,
    num_heads, num_layers, freq_dim, text_len, out_dim, eps.  decisions[i]: the ranked
    decisions of block i's self attention (or None).  Returns the list of outputs."""
    p = {k: v.detach().cpu().double() for k, v in P.items()}
    patch = tuple(cfg["patch_size"])
    dim, H, eps = cfg["dim"], cfg["num_heads"], cfg["eps"]
    xs = [patch_embed(u.detach().cpu(), p["patch_embedding.weight"], p["patch_embedding.bias"], patch)
          for u in x_list]
    ss = [patch_embed(u.detach().cpu(), p["source_video_embedding_more_memory.weight"],
                      p["source_video_embedding_more_memory.bias"], patch) for u in src_list]
    rows = [torch.cat([a[0], b[0]]) for a, b in zip(xs, ss)]
    x = torch.stack([torch.cat([r, r.new_zeros(seq_len - r.shape[0], dim)]) for r in rows])
    temb = sinusoidal_embedding_1d(cfg["freq_dim"], t.detach().cpu())
    e = F.linear(F.silu(F.linear(temb, p["time_embedding.0.weight"], p["time_embedding.0.bias"])),
                 p["time_embedding.2.weight"], p["time_embedding.2.bias"])
    e0 = F.linear(F.silu(e), p["time_projection.1.weight"], p["time_projection.1.bias"]).unflatten(1, (6, dim))
    ctx = torch.stack([torch.cat([u.double(), u.new_zeros(cfg["text_len"] - u.shape[0], u.shape[1]).double()])
                       for u in context_list])
    ctx = linear(bf(F.gelu(linear(ctx, p["text_embedding.0.weight"], p["text_embedding.0.bias"]),
                           approximate="tanh")), p["text_embedding.2.weight"], p["text_embedding.2.bias"])
    grid, sgrid = xs[0][1], ss[0][1]
    for i in range(cfg["num_layers"]):
        pre = f"blocks.{i}."
        Pb = {k[len(pre):]: v for k, v in p.items() if k.startswith(pre)}
        x, _ = wan_block_forward(Pb, x, e0, ctx, grid, sgrid, 1, freqs, H, eps,
                                 decisions=decisions[i] if decisions else None, x_is_bf16=(i == 0))
    s_lens = [b[0].shape[0] for b in ss]
    x = torch.stack([u[:u.shape[0] - s_lens[j]] for j, u in enumerate(x)])
    em = (p["head.modulation"] + e.unsqueeze(1)).chunk(2, dim=1)
    out = F.linear(layer_norm(x, eps) * (1 + em[1]) + em[0], p["head.head.weight"], p["head.head.bias"])
    return [unpatchify(u, a[1], patch, cfg["out_dim"]) for u, a in zip(out, xs)]
