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
               f.imag.to(device=device, dtype=torch.float32).contiguous(), freqs)
        if len(_rope_cache) >= 8:                    # a few live tables (model, identity)
            _rope_cache.pop(next(iter(_rope_cache)))
        _rope_cache[key] = hit                       # keeps freqs alive: its address stays unique
    return hit[0], hit[1]


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
def wan_qk_prologue(yq: torch.Tensor, yk, norm_q_weight: torch.Tensor, norm_k_weight,
                    grid_sizes, source_video_grid_sizes, TAG: int, freqs: torch.Tensor,
                    num_heads: int, alpha_logit: torch.Tensor = None, eps: float = 1e-6,
                    want_sums: bool = True):
    """q / k producer of WanSelfAttention.forward on the q / k projections yq, yk [B, S, dim].

    Returns ``(q, k, qsum, ksum, gate)``: bf16 q, k [B, S, H, D]; f32 block sums
    [B, H, NB, D] (None without ``want_sums``); f32 gate [B, S] (None without
    ``alpha_logit``).  ``yk=None`` processes q alone (k, ksum None); all-zero grids rotate
    nothing (the cross attention's RMSNorm)."""
    _require(yq.is_cuda and yq.dim() == 3, "yq must be [B, S, dim] on the GPU")
    if yk is not None:
        _require(yk.is_cuda and yq.shape == yk.shape and yq.dtype == yk.dtype,
                 "yk must match yq in shape and dtype")
    B, S, dim = yq.shape
    H = int(num_heads)
    _require(dim % H == 0, "dim must be a multiple of num_heads")
    D = dim // H
    yq = yq if yq.stride(-1) == 1 else yq.contiguous()
    if yk is not None:
        yk = yk if yk.stride(-1) == 1 else yk.contiguous()
        if yk.stride() != yq.stride():
            yq, yk = yq.contiguous(), yk.contiguous()
    dev = yq.device
    wq = norm_q_weight.detach().to(device=dev, dtype=torch.float32).contiguous()
    _require(wq.numel() == dim, "norm weights must have dim elements")
    wk = None
    if yk is not None:
        wk = norm_k_weight.detach().to(device=dev, dtype=torch.float32).contiguous()
        _require(wk.numel() == dim, "norm weights must have dim elements")
    cos, sin = rope_tables(freqs, dev)
    _require(cos.shape[1] == D // 2, "freqs must have D/2 columns")
    L = _lib.lib()
    NB = (S + 63) // 64
    q = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=dev)
    k = torch.empty_like(q) if yk is not None else None
    qsum = torch.empty(B, H, NB, D, dtype=torch.float32, device=dev) if want_sums else None
    ksum = torch.empty_like(qsum) if (want_sums and yk is not None) else None
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
    with torch.cuda.device(dev):     # the library launches on the current device
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
                            out_dtype=torch.float32, stage_events=None, keep_workspace=False):
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
    x, views = _editing_sparse_attention_hip(q, k, v, t_seq_len, alpha_2, SPARSITY_RATIO, srr,
                                             flat_ratio, presummed=(qsum, ksum), out_dtype=out_dtype,
                                             stage_events=stage_events, keep_workspace=keep_workspace)
    return (x, views) if keep_workspace else x


@torch.no_grad()
def ln_modulate(x: torch.Tensor, shift=None, scale=None, weight=None, bias=None, eps=1e-6,
                y=None, gate=None, out=True, x_out=None):
    """The residual / LayerNorm / adaLN step of WanAttentionBlock.forward (model.py:249-270)
    in one pass (icsa_wan_ln_modulate): with ``y``, x += y * gate (y bf16 [B, S, dim], gate
    f32 [B, dim] or [B, 1, dim]), in place for an f32 x, or into the f32 ``x_out`` (then x
    may be bf16 and is left unchanged); then, unless ``out=False``, returns
    bf16(LN(x) [* weight + bias] [* (1 + scale) + shift]).  A bf16 x without ``y`` rounds
    the LayerNorm to bf16 (WanLayerNorm's ``.type_as(x)``); an updated x is f32 and does not."""
    _require(x.is_cuda and x.dim() == 3 and x.stride(-1) == 1, "x must be [B, S, dim], rows contiguous")
    B, S, dim = x.shape

    def vec(t):
        """[B, dim] f32 view; one [dim] row broadcast over the batch has batch stride 0."""
        if t is None:
            return None
        t = t.detach().to(device=x.device, dtype=torch.float32)
        if t.numel() == B * dim:
            return t.reshape(B, dim).contiguous()
        _require(t.numel() == dim, "modulation / gate vectors must be [B, dim] or [dim]")
        return t.reshape(1, dim).contiguous().expand(B, dim)

    shift, scale, gate = vec(shift), vec(scale), vec(gate)
    wt = weight.detach().to(device=x.device, dtype=torch.float32).contiguous() if weight is not None else None
    bs = bias.detach().to(device=x.device, dtype=torch.float32).contiguous() if bias is not None else None
    if y is not None:
        if x_out is None:
            _require(x.dtype == torch.float32, "the residual stream updated in place must be float32")
            x_out = x
        _require(x_out.dtype == torch.float32 and x_out.shape == x.shape and x_out.stride(-1) == 1,
                 "x_out must be float32 like x, rows contiguous")
        _require(y.shape == x.shape and y.dtype == torch.bfloat16, "y must be bf16 like x")
        y = y if y.stride(-1) == 1 else y.contiguous()
    else:
        _require(x_out is None, "x_out needs y")
    o = torch.empty(B, S, dim, dtype=torch.bfloat16, device=x.device) if out else None
    with torch.cuda.device(x.device):     # the library launches on the current device
        rc = _lib.lib().icsa_wan_ln_modulate(
            ptr(x), dtype_code(x), x.stride(0), x.stride(1),
            ptr(y), y.stride(0) if y is not None else 0, y.stride(1) if y is not None else 0,
            ptr(gate), gate.stride(0) if gate is not None else 0,
            ptr(x_out), x_out.stride(0) if x_out is not None else 0,
            x_out.stride(1) if x_out is not None else 0,
            ptr(wt), ptr(bs),
            ptr(shift), ptr(scale), shift.stride(0) if shift is not None else 0, float(eps),
            B, S, dim, ptr(o), o.stride(0) if o is not None else 0, o.stride(1) if o is not None else 0,
            stream_ptr(x.device))
    _lib.check("icsa_wan_ln_modulate", rc)
    return o


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

    capture = None    # a dict here receives the workspace views (decisions) of the next call

    def forward(self, x, seq_lens, grid_sizes, source_video_grid_sizes, TAG, freqs):
        b, s = x.shape[:2]
        res = wan_self_attention_core(
            self.q(x), self.k(x), self.v(x), self.alpha_1(x), self.norm_q.weight,
            self.norm_k.weight, grid_sizes, source_video_grid_sizes, TAG, freqs,
            self.num_heads, self.eps, out_dtype=x.dtype, keep_workspace=self.capture is not None)
        if self.capture is not None:
            res, self.capture["views"] = res
        # the kernels add the residual in f32 and round once at the store, which equals the
        # reference's f32 result cast to the projection's dtype
        return self.o(res.flatten(2))


class WanLayerNorm(nn.LayerNorm):
    """Parameter holder of the reference's WanLayerNorm (model.py:117-122); applied by
    ``ln_modulate``."""

    def __init__(self, dim, eps=1e-6, elementwise_affine=False):
        super().__init__(dim, elementwise_affine=elementwise_affine, eps=eps)


class WanT2VCrossAttention(nn.Module):
    """WanT2VCrossAttention (model.py:180-188): q / k RMSNorm through the producer in its
    single-tensor, unrotated mode, dense attention over the text tokens through
    ``icsa_flash_attn``.  Same parameters as the reference class."""

    def __init__(self, dim, num_heads, window_size=(-1, -1), qk_norm=True, eps=1e-6):
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.eps = eps
        _require(qk_norm, "the HIP producer applies the q / k RMSNorm (qk_norm=True)")
        self.q = nn.Linear(dim, dim)
        self.k = nn.Linear(dim, dim)
        self.v = nn.Linear(dim, dim)
        self.o = nn.Linear(dim, dim)
        self.alpha_1 = nn.Linear(dim, 1, bias=False)       # unused here, as in the reference
        self.alpha_2 = nn.Linear(dim, 1, bias=False)
        self.norm_q = WanRMSNorm(dim, eps=eps)
        self.norm_k = WanRMSNorm(dim, eps=eps)

    def forward(self, x, context, context_lens=None):
        _require(context_lens is None, "variable text lengths (context_lens) are not supported")
        b = x.shape[0]
        none = [(0, 0, 0)] * b
        no_rope = _identity_freqs(self.head_dim, x.device)
        q = wan_qk_prologue(self.q(x), None, self.norm_q.weight, None, none, none, 0, no_rope,
                            self.num_heads, eps=self.eps, want_sums=False)[0]
        k = wan_qk_prologue(self.k(context), None, self.norm_k.weight, None, none, none, 0,
                            no_rope, self.num_heads, eps=self.eps, want_sums=False)[0]
        v = self.v(context).view(b, -1, self.num_heads, self.head_dim).to(torch.bfloat16)
        from .hip_host import flash_attn_func
        y = flash_attn_func(q, k, v)
        return self.o(y.flatten(2).to(x.dtype))


_id_freqs: dict = {}


def _identity_freqs(head_dim, device):
    key = (head_dim, str(device))
    if key not in _id_freqs:
        _id_freqs[key] = torch.ones(1, head_dim // 2, dtype=torch.complex128)
    return _id_freqs[key]


class WanAttentionBlock(nn.Module):
    """WanAttentionBlock (model.py:224-270) on the HIP backend: same constructor, parameters
    and ``forward(x, e, seq_lens, grid_sizes, freqs, context, context_lens,
    source_video_grid_sizes, TAG)``.  The residual stream is float32 as in the reference;
    every residual update + LayerNorm + adaLN modulation is one ``ln_modulate`` pass, the
    projections and the FFN are library GEMMs, the attentions run in libicsa.so.
    Only the t2v cross attention is part of this build."""

    def __init__(self, cross_attn_type, dim, ffn_dim, num_heads, window_size=(-1, -1),
                 qk_norm=True, cross_attn_norm=False, eps=1e-6, backend=Backend.HIP):
        super().__init__()
        _require(cross_attn_type == 't2v_cross_attn', "only t2v_cross_attn is supported")
        self.dim = dim
        self.ffn_dim = ffn_dim
        self.num_heads = num_heads
        self.window_size = window_size
        self.qk_norm = qk_norm
        self.cross_attn_norm = cross_attn_norm
        self.eps = eps
        self.norm1 = WanLayerNorm(dim, eps)
        self.self_attn = WanSelfAttention(dim, num_heads, window_size, qk_norm, eps, backend=backend)
        self.norm3 = WanLayerNorm(dim, eps, elementwise_affine=True) if cross_attn_norm else nn.Identity()
        self.cross_attn = WanT2VCrossAttention(dim, num_heads, (-1, -1), qk_norm, eps)
        self.norm2 = WanLayerNorm(dim, eps)
        self.ffn = nn.Sequential(nn.Linear(dim, ffn_dim), nn.GELU(approximate='tanh'),
                                 nn.Linear(ffn_dim, dim))
        self.modulation = nn.Parameter(torch.randn(1, 6, dim) / dim ** 0.5)

    def forward(self, x, e, seq_lens, grid_sizes, freqs, context, context_lens,
                source_video_grid_sizes, TAG):
        _require(e.dtype == torch.float32, "e must be float32 (model.py:250)")
        em = (self.modulation.float() + e).chunk(6, dim=1)           # 6 x [B, 1, dim]
        x = x if x.stride(-1) == 1 else x.contiguous()
        # norm1, modulate; a bf16 x (the first block) rounds the LayerNorm to bf16 (.type_as)
        h = ln_modulate(x, shift=em[0], scale=em[1], eps=self.eps)
        y = self.self_attn(h, seq_lens, grid_sizes, source_video_grid_sizes, TAG, freqs)
        xs = torch.empty(x.shape, dtype=torch.float32, device=x.device)  # the f32 residual stream
        if isinstance(self.norm3, nn.Identity):                      # x + y e2 (the input is kept)
            ln_modulate(x, y=y, gate=em[2], out=False, x_out=xs)
            h = xs.to(torch.bfloat16)
        else:                                                        # ... then norm3
            h = ln_modulate(x, y=y, gate=em[2], weight=self.norm3.weight, bias=self.norm3.bias,
                            eps=self.eps, x_out=xs)
        x = xs
        y = self.cross_attn(h, context.to(h.dtype), context_lens)
        ones = torch.ones(x.shape[0], self.dim, device=x.device)
        h = ln_modulate(x, y=y.to(torch.bfloat16), gate=ones, shift=em[3], scale=em[4],
                        eps=self.eps)                                # x += cross, norm2, modulate
        y = self._ffn(h)
        ln_modulate(x, y=y.to(torch.bfloat16), gate=em[5], out=False)   # x += ffn e5
        return x

    def _ffn(self, h):
        """self.ffn(h) (Linear, GELU(tanh), Linear; model.py:243-245) with the bias and the
        GELU applied in the first GEMM's epilogue, on its fp32 accumulator: no separate
        elementwise pass over the [tokens, ffn_dim] hidden.  The reference rounds the first
        Linear's output to bf16 before its GELU; the epilogue rounds once, after it."""
        lin0, lin2 = self.ffn[0], self.ffn[2]
        f = torch._addmm_activation(lin0.bias, h.reshape(-1, h.shape[-1]), lin0.weight.t(), use_gelu=True)
        return torch.nn.functional.linear(f, lin2.weight, lin2.bias).view(*h.shape[:-1], lin2.out_features)


def sinusoidal_embedding_1d(dim, position):
    """model.py:25-31: [len(position), dim] float64 cos / sin embedding."""
    assert dim % 2 == 0
    half = dim // 2
    position = position.type(torch.float64)
    sinusoid = torch.outer(position, torch.pow(10000, -torch.arange(half).to(position).div(half)))
    return torch.cat([torch.cos(sinusoid), torch.sin(sinusoid)], dim=1)


class Head(nn.Module):
    """Head (model.py:272-290): LayerNorm, modulation and the output Linear, in fp32 as the
    reference's autocast(float32) region."""

    def __init__(self, dim, out_dim, patch_size, eps=1e-6):
        super().__init__()
        self.dim = dim
        self.out_dim = out_dim
        self.patch_size = patch_size
        self.eps = eps
        out_dim = math.prod(patch_size) * out_dim
        self.norm = WanLayerNorm(dim, eps)
        self.head = nn.Linear(dim, out_dim)
        self.modulation = nn.Parameter(torch.randn(1, 2, dim) / dim ** 0.5)

    def forward(self, x, e):
        e = (self.modulation.float() + e.float().unsqueeze(1)).chunk(2, dim=1)
        n = nn.functional.layer_norm(x.float(), (self.dim,), eps=self.eps)
        return nn.functional.linear(n * (1 + e[1]) + e[0], self.head.weight.float(),
                                    self.head.bias.float())


class WanModel(nn.Module):
    """WanModel (model.py:308-466), t2v, on the HIP backend: same constructor arguments,
    parameter names and ``forward(x, t, context, seq_len, source_video_latent)``.

    The blocks are ``WanAttentionBlock`` above.  The (1, 2, 2) patch embeddings run as a
    reshape and a library GEMM (kernel = stride), the text / time embeddings and the head
    as in the reference.  Several inputs in the lists (e.g. the conditional and the
    unconditional pass of classifier-free guidance) run as one batch."""

    def __init__(self, model_type='t2v', patch_size=(1, 2, 2), text_len=512, in_dim=16, dim=5120,
                 ffn_dim=13824, freq_dim=256, text_dim=4096, out_dim=16, num_heads=40,
                 num_layers=40, window_size=(-1, -1), qk_norm=True, cross_attn_norm=True,
                 eps=1e-6, use_siglip=False, use_riflex=False, backend=Backend.HIP):
        super().__init__()
        _require(model_type == 't2v', "only the t2v model is part of this build")
        self.model_type = model_type
        self.backend = backend
        self.patch_size = patch_size
        self.source_video_patch_size = patch_size
        self.text_len = text_len
        self.in_dim = in_dim
        self.dim = dim
        self.ffn_dim = ffn_dim
        self.freq_dim = freq_dim
        self.text_dim = text_dim
        self.out_dim = out_dim
        self.num_heads = num_heads
        self.num_layers = num_layers
        self.window_size = window_size
        self.qk_norm = qk_norm
        self.cross_attn_norm = cross_attn_norm
        self.eps = eps
        self.patch_embedding = nn.Conv3d(in_dim, dim, kernel_size=patch_size, stride=patch_size)
        self.source_video_embedding_more_memory = nn.Conv3d(
            in_dim, dim, kernel_size=patch_size, stride=patch_size)
        self.text_embedding = nn.Sequential(
            nn.Linear(text_dim, dim), nn.GELU(approximate='tanh'), nn.Linear(dim, dim))
        self.time_embedding = nn.Sequential(nn.Linear(freq_dim, dim), nn.SiLU(), nn.Linear(dim, dim))
        self.time_projection = nn.Sequential(nn.SiLU(), nn.Linear(dim, dim * 6))
        self.blocks = nn.ModuleList([
            WanAttentionBlock('t2v_cross_attn', dim, ffn_dim, num_heads, window_size, qk_norm,
                              cross_attn_norm, eps, backend=backend)
            for _ in range(num_layers)])
        self.head = Head(dim, out_dim, patch_size, eps)
        d = dim // num_heads
        assert (dim % num_heads) == 0 and d % 2 == 0
        self.freqs = wan_freqs(d)

    def init_weights(self):
        """model.py:395-408."""
        for m in self.modules():
            if isinstance(m, nn.Linear):
                nn.init.xavier_uniform_(m.weight)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
        nn.init.xavier_uniform_(self.patch_embedding.weight.flatten(1))
        for m in self.text_embedding.modules():
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, std=0.02)
        for m in self.time_embedding.modules():
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, std=0.02)
        nn.init.zeros_(self.head.head.weight)

    def _patchify(self, conv, u):
        """Conv3d with kernel = stride as a GEMM: [C, F, H, W] -> [F*(H/ph)*(W/pw), dim]."""
        pf, ph, pw = self.patch_size
        C, F_, H_, W_ = u.shape
        g = (F_ // pf, H_ // ph, W_ // pw)
        p = u.reshape(C, g[0], pf, g[1], ph, g[2], pw).permute(1, 3, 5, 0, 2, 4, 6)
        p = p.reshape(g[0] * g[1] * g[2], C * pf * ph * pw)
        w = conv.weight.reshape(self.dim, -1)
        return nn.functional.linear(p.to(w.dtype), w, conv.bias), g

    def forward(self, x, t, context, seq_len, source_video_latent):
        dev = self.patch_embedding.weight.device
        xs, grids = zip(*[self._patchify(self.patch_embedding, u) for u in x])
        ss, sgrids = zip(*[self._patchify(self.source_video_embedding_more_memory, u)
                           for u in source_video_latent])
        s_lens = [u.shape[0] for u in ss]
        rows = [torch.cat([u, v], dim=0) for u, v in zip(xs, ss)]
        _require(max(r.shape[0] for r in rows) <= seq_len, "seq_len smaller than the token count")
        xb = torch.stack([torch.cat([r, r.new_zeros(seq_len - r.shape[0], self.dim)]) for r in rows])
        def f32_linear(lin, z):                  # the reference's autocast(float32) region
            return nn.functional.linear(z, lin.weight.float(), lin.bias.float())

        temb = sinusoidal_embedding_1d(self.freq_dim, t).float().to(dev)
        e = f32_linear(self.time_embedding[2],
                       nn.functional.silu(f32_linear(self.time_embedding[0], temb)))
        e0 = f32_linear(self.time_projection[1], nn.functional.silu(e)).unflatten(1, (6, self.dim))
        ctx = self.text_embedding(torch.stack([
            torch.cat([u, u.new_zeros(self.text_len - u.size(0), u.size(1))]) for u in context]).to(
                self.text_embedding[0].weight.dtype))
        seq_lens = torch.tensor([r.shape[0] for r in rows], dtype=torch.long)
        h = xb
        for block in self.blocks:
            h = block(h, e0, seq_lens, list(grids), self.freqs, ctx, None, list(sgrids), 1)
        h = torch.stack([u[:u.shape[0] - s_lens[i]] for i, u in enumerate(h)], 0)
        out = self.head(h, e)
        return self.unpatchify(out, grids)

    def unpatchify(self, x, grid_sizes):
        """model.py:456-466."""
        c = self.out_dim
        out = []
        for u, v in zip(x, grid_sizes):
            u = u[:math.prod(v)].view(*v, *self.patch_size, c)
            u = torch.einsum('fhwpqrc->cfphqwr', u)
            u = u.reshape(c, *[i * j for i, j in zip(v, self.patch_size)])
            out.append(u)
        return out


__all__ = ["rope_params", "wan_freqs", "rope_tables", "wan_qk_prologue", "wan_self_attention_core",
           "ln_modulate", "WanSelfAttention", "WanT2VCrossAttention", "WanAttentionBlock",
           "WanRMSNorm", "WanLayerNorm", "Head", "WanModel", "sinusoidal_embedding_1d"]
