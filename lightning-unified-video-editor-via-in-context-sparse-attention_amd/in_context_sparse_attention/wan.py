"""Wan DiT self-attention on the HIP backend: the caller side of the sparse-attention path.

Mirror of ``WanSelfAttention`` (reference ``model.py:125-177``).  The q / k / v / o and
alpha_1 projections stay ``nn.Linear`` layers (library GEMMs).  Everything between the
projections and the output projection runs in libicsa.so:

* ``icsa_wan_qk_prologue`` replaces ``norm_q`` / ``norm_k`` (WanRMSNorm, model.py:103-114),
  the alpha_1 gate (model.py:162), both ``rope_apply`` calls (model.py:69-95, float64 there)
  and stage 1's pooling of q / k.  It writes bf16 q / k and their block sums in one pass
  over the projections.
* ``icsa_editing_sparse_attention_presummed`` runs the attention path on them.

The reference's fp32 q / k intermediates (and its float64 RoPE buffers) are never built.
"""
from __future__ import annotations

import ctypes
import math

import torch
import torch.nn as nn

from . import _lib
from .editing_sparse_attention import Backend, _editing_sparse_attention_hip, derived_sizes
from .hip_host import _require, dtype_code, ptr, stream_ptr

_rope_cache: dict = {}


def rope_params(max_seq_len: int, dim: int, theta: float = 10000.0) -> torch.Tensor:
    """complex128 [max_seq_len, dim // 2] table exp(i * pos / theta^(2j / dim)), the
    reference's ``rope_params`` (model.py:57-62)."""
    assert dim % 2 == 0
    pos = torch.arange(max_seq_len, dtype=torch.float64)
    inv = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64),
                          torch.arange(0, dim, 2, dtype=torch.float64).div(dim))
    ang = torch.outer(pos, inv)
    return torch.polar(torch.ones_like(ang), ang)


def wan_freqs(head_dim: int = 128, max_seq_len: int = 1024) -> torch.Tensor:
    """The model's RoPE table, built as in WanModel.__init__ (model.py:380-385): frame, row
    and column tables of widths D - 4*(D//6), 2*(D//6), 2*(D//6) side by side."""
    d = head_dim
    return torch.cat([rope_params(max_seq_len, d - 4 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6)),
                      rope_params(max_seq_len, 2 * (d // 6))], dim=1)


def rope_tables(freqs: torch.Tensor, device) -> tuple[torch.Tensor, torch.Tensor]:
    """f32 cos / sin [rows, D/2] of the model's complex RoPE table (cached per table)."""
    key = (freqs.data_ptr(), tuple(freqs.shape), str(freqs.device), str(device))
    hit = _rope_cache.get(key)
    if hit is None:
        f = freqs.to(torch.complex128)
        hit = (f.real.to(device=device, dtype=torch.float32).contiguous(),
               f.imag.to(device=device, dtype=torch.float32).contiguous())
        _rope_cache.clear()
        _rope_cache[key] = hit
    return hit


def _grids(grid_sizes, source_video_grid_sizes, B) -> ctypes.Array:
    g = (ctypes.c_int32 * (6 * B))()
    for b in range(B):
        t = [int(x) for x in grid_sizes[b]]
        s = [int(x) for x in source_video_grid_sizes[b]]
        _require(len(t) == 3 and len(s) == 3, "grid sizes are (frames, rows, columns)")
        for a in range(3):
            g[6 * b + a] = t[a]
            g[6 * b + 3 + a] = s[a]
    return g


@torch.no_grad()
def wan_qk_prologue(yq: torch.Tensor, yk: torch.Tensor, norm_q_weight: torch.Tensor,
                    norm_k_weight: torch.Tensor, grid_sizes, source_video_grid_sizes, TAG: int,
                    freqs: torch.Tensor, num_heads: int, alpha_logit: torch.Tensor = None,
                    eps: float = 1e-6):
    """q / k producer of WanSelfAttention.forward on the q / k projections yq, yk [B, S, dim].

    Returns ``(q, k, qsum, ksum, gate)``: bf16 q, k [B, S, H, D]; f32 block sums
    [B, H, NB, D]; f32 gate [B, S] (None without ``alpha_logit``)."""
    _require(yq.is_cuda and yk.is_cuda, "yq, yk must be on the GPU")
    _require(yq.dim() == 3 and yq.shape == yk.shape, "yq, yk must be [B, S, dim]")
    _require(yq.dtype == yk.dtype, "yq and yk must have the same dtype")
    B, S, dim = yq.shape
    H = int(num_heads)
    _require(dim % H == 0, "dim must be a multiple of num_heads")
    D = dim // H
    yq = yq if yq.stride(-1) == 1 else yq.contiguous()
    yk = yk if yk.stride(-1) == 1 else yk.contiguous()
    if yk.stride() != yq.stride():
        yq, yk = yq.contiguous(), yk.contiguous()
    dev = yq.device
    wq = norm_q_weight.detach().to(device=dev, dtype=torch.float32).contiguous()
    wk = norm_k_weight.detach().to(device=dev, dtype=torch.float32).contiguous()
    _require(wq.numel() == dim and wk.numel() == dim, "norm weights must have dim elements")
    cos, sin = rope_tables(freqs, dev)
    _require(cos.shape[1] == D // 2, "freqs must have D/2 columns")
    L = _lib.lib()
    NB = (S + 63) // 64
    q = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=dev)
    k = torch.empty_like(q)
    qsum = torch.empty(B, H, NB, D, dtype=torch.float32, device=dev)
    ksum = torch.empty_like(qsum)
    gate = None
    a_args = [None, _lib.F32, 0, 0]
    if alpha_logit is not None:
        a = alpha_logit.to(dev)
        if a.dtype not in (torch.float32, torch.bfloat16):
            a = a.float()
        a = a.reshape(B, S)
        gate = torch.empty(B, S, dtype=torch.float32, device=dev)
        a_args = [ptr(a), dtype_code(a), a.stride(0), a.stride(1)]
    ws_bytes = L.icsa_wan_qk_workspace_size(B, S)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    rc = L.icsa_wan_qk_prologue(
        ptr(yq), ptr(yk), dtype_code(yq), yq.stride(0), yq.stride(1),
        ptr(wq), ptr(wk), float(eps),
        ptr(cos), ptr(sin), cos.shape[0],
        ctypes.cast(_grids(grid_sizes, source_video_grid_sizes, B), ctypes.c_void_p), int(TAG),
        *a_args,
        B, S, H, D,
        ptr(q), ptr(k), q.stride(0), q.stride(1), q.stride(2),
        ptr(qsum), ptr(ksum), ptr(gate),
        ptr(ws), ws_bytes, stream_ptr(dev))
    _lib.check("icsa_wan_qk_prologue", rc)
    return q, k, qsum, ksum, gate


@torch.no_grad()
def wan_self_attention_core(yq, yk, yv, alpha_logit, norm_q_weight, norm_k_weight, grid_sizes,
                            source_video_grid_sizes, TAG, freqs, num_heads, eps=1e-6,
                            SPARSITY_RATIO=0.0625, srr=0.125, flat_ratio=0.5,
                            out_dtype=torch.float32, stage_events=None):
    """model.py:156-175 between the projections and ``self.o``: returns x [B, S, H, D].

    yq, yk, yv: the q / k / v projections [B, S, dim]; alpha_logit: ``self.alpha_1(x)``
    [B, S, 1] (or None for alpha_2 = 0).  t_seq_len is the target grid of batch 0, as in
    the reference (model.py:164-168).  x is float32 like the reference (q.dtype there)."""
    B, S, dim = yq.shape
    H = int(num_heads)
    D = dim // H
    q, k, qsum, ksum, gate = wan_qk_prologue(yq, yk, norm_q_weight, norm_k_weight, grid_sizes,
                                             source_video_grid_sizes, TAG, freqs, H,
                                             alpha_logit, eps)
    f, h, w = (int(x) for x in grid_sizes[0])
    t_seq_len = f * h * w
    v = yv.reshape(B, S, H, D)
    alpha_2 = gate.view(B, S, 1, 1) if gate is not None else 0.0
    x, _ = _editing_sparse_attention_hip(q, k, v, t_seq_len, alpha_2, SPARSITY_RATIO, srr,
                                         flat_ratio, presummed=(qsum, ksum), out_dtype=out_dtype,
                                         stage_events=stage_events)
    return x


class WanRMSNorm(nn.Module):
    """Parameter holder of the reference's WanRMSNorm (model.py:103-114); the HIP path applies
    it inside ``icsa_wan_qk_prologue``."""

    def __init__(self, dim, eps=1e-5):
        super().__init__()
        self.dim = dim
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))


class WanSelfAttention(nn.Module):
    """WanSelfAttention (model.py:125-177) with the attention core on the HIP backend.

    Same constructor and ``forward(x, seq_lens, grid_sizes, source_video_grid_sizes, TAG,
    freqs)`` as the reference; ``backend`` must be 'hip' here."""

    def __init__(self, dim, num_heads, window_size=(-1, -1), qk_norm=True, eps=1e-6,
                 backend=Backend.HIP):
        assert dim % num_heads == 0
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.window_size = window_size
        self.qk_norm = qk_norm
        self.eps = eps
        self.backend = Backend.validate(backend)
        if self.backend != Backend.HIP:
            raise NotImplementedError("only the 'hip' backend is part of this build")
        _require(qk_norm, "the HIP producer applies the q / k RMSNorm (qk_norm=True)")
        self.q = nn.Linear(dim, dim)
        self.k = nn.Linear(dim, dim)
        self.v = nn.Linear(dim, dim)
        self.o = nn.Linear(dim, dim)
        self.alpha_1 = nn.Linear(dim, 1, bias=False)
        self.alpha_2 = nn.Linear(dim, 1, bias=False)
        nn.init.zeros_(self.alpha_2.weight)
        self.norm_q = WanRMSNorm(dim, eps=eps)
        self.norm_k = WanRMSNorm(dim, eps=eps)

    def forward(self, x, seq_lens, grid_sizes, source_video_grid_sizes, TAG, freqs):
        b, s = x.shape[:2]
        x_att = wan_self_attention_core(
            self.q(x), self.k(x), self.v(x), self.alpha_1(x), self.norm_q.weight,
            self.norm_k.weight, grid_sizes, source_video_grid_sizes, TAG, freqs,
            self.num_heads, self.eps)
        return self.o(x_att.flatten(2).to(x.dtype))


__all__ = ["rope_params", "wan_freqs", "rope_tables", "wan_qk_prologue", "wan_self_attention_core",
           "WanSelfAttention", "WanRMSNorm"]
