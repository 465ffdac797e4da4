"""In-context sparse attention with the MI355X HIP backend.

Mirror of the reference's ``in_context_sparse_attention/editing_sparse_attention.py``:
``Backend`` (:25-34) gains ``HIP = 'hip'``, and ``editing_sparse_attention`` (:67-232) keeps
its signature, including the default ``backend='tilelang'``.  With ``backend='hip'`` the
whole path -- pooling, compressed attention, per-head source retrieval, peaked/diffuse
split, flash attention for the peaked blocks, sparse piecewise attention for the diffuse
blocks, scatter and residual -- runs as one launch sequence of hand-written gfx950 kernels
(libicsa.so) on the current stream; the concatenated new KV, the broadcast out_c and the
gathered query halves are never built.

The TileLang and Triton backends are CUDA-only and are not part of this package: naming
them passes ``Backend.validate`` (they are valid names) but raises ``NotImplementedError``.
The reference's module keeps serving them; it dispatches ``backend='hip'`` here through
the few lines its integration patch adds.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .hip_host import (BLOCK_M, IcsaArgumentError, _require, check_index_lists, dtype_code,
                       inner_contiguous, ptr, stream_ptr)


class Backend:
    """Sparse-attention backend constants (editing_sparse_attention.py:25-34 plus HIP)."""
    TILELANG = 'tilelang'
    TRITON = 'triton'
    HIP = 'hip'

    @classmethod
    def validate(cls, backend: str) -> str:
        if backend not in (cls.TILELANG, cls.TRITON, cls.HIP):
            raise ValueError(
                f"Unknown backend '{backend}'.  Valid: {cls.TILELANG}, {cls.TRITON}, {cls.HIP}")
        return backend


SIZE_NAMES = ["NB", "n_t", "n_s", "topK", "Tkv", "k_sparsity", "n_peaked", "n_diffuse",
              "TKV_pad", "NKV", "top_k", "NKVp"]


def derived_sizes(B, S, H, D, t_seq_len, sparsity=0.0625, srr=0.125, flat_ratio=0.5) -> dict:
    """Derived sizes of one call, computed by the library (icsa_editing_sizes)."""
    out = (ctypes.c_int32 * 12)()
    rc = _lib.lib().icsa_editing_sizes(B, S, H, D, t_seq_len, float(sparsity), float(srr),
                                       float(flat_ratio), ctypes.cast(out, ctypes.c_void_p))
    _lib.check("icsa_editing_sizes", rc)
    return dict(zip(SIZE_NAMES, list(out)))


def _alpha_view(alpha_2, B, S, H, D, device):
    """(tensor or None, scalar, dtype code, strides) of alpha_2 broadcast to [B, S, H, D]."""
    if not isinstance(alpha_2, torch.Tensor):
        return None, float(alpha_2), _lib.F32, (0, 0, 0, 0)
    a = alpha_2
    if a.dtype not in (torch.float32, torch.bfloat16):
        a = a.float()
    a = a.to(device)
    _require(a.dim() <= 4, "alpha_2 must broadcast to [B, S, H, D]")
    a = a.expand(B, S, H, D)
    return a, 0.0, dtype_code(a), tuple(a.stride())


@torch.no_grad()
def _editing_sparse_attention_hip(q, k, v, t_seq_len, alpha_2=1.0, SPARSITY_RATIO=0.0625,
                                  srr=0.125, flat_ratio=0.5, inject=None, keep_workspace=False,
                                  stage_events=None, presummed=None, out_dtype=None, noalloc=False):
    """Runs the fused HIP path; returns ``(x, workspace_views or None)``.

    ``noalloc``: use ``icsa_editing_sparse_attention_noalloc``, whose scratch is the
    library's static device array (no workspace is allocated; the call must fit in
    ``_lib.NOALLOC_SCRATCH_BYTES``); not combinable with ``keep_workspace``,
    ``stage_events`` or ``presummed``.

    ``stage_events``: optional list of ``len(_lib.STAGES)`` recorded ``torch.cuda.Event``s
    (enable_timing=True) that the library re-records at each stage boundary on the stream.
    ``presummed``: optional ``(qsum, ksum)`` f32 [B, H, NB, D] block sums of bf16 q / k from
    their producer (``wan.wan_qk_prologue``); stage 1 then pools only v.
    ``out_dtype``: dtype of x (default q.dtype, as the reference).
    """
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "q, k, v must be on the GPU")
    _require(q.ndim == 4 and q.shape == k.shape == v.shape, "q, k, v must be [B, S, H, D]")
    B, S, H, D = q.shape
    _require(0 <= t_seq_len <= S, f"t_seq_len {t_seq_len} outside [0, {S}]")
    q, k, v = inner_contiguous(q), inner_contiguous(k), inner_contiguous(v)
    for t in (q, k, v):
        dtype_code(t)
    L = _lib.lib()
    sizes = derived_sizes(B, S, H, D, t_seq_len, SPARSITY_RATIO, srr, flat_ratio)
    offs = (ctypes.c_int64 * len(_lib.WS_SLOTS))()
    ws_bytes = L.icsa_editing_workspace_layout(B, S, H, D, t_seq_len, float(SPARSITY_RATIO),
                                               float(srr), float(flat_ratio), dtype_code(q),
                                               dtype_code(k), dtype_code(v),
                                               ctypes.cast(offs, ctypes.c_void_p))
    if ws_bytes < 0:
        raise _lib.IcsaError("icsa_editing_workspace_layout", int(ws_bytes))
    _require(not noalloc or (not keep_workspace and stage_events is None and presummed is None),
             "noalloc cannot be combined with keep_workspace, stage_events or presummed")
    ws = None if noalloc else torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    out = torch.empty(B, S, H, D, dtype=out_dtype or q.dtype, device=q.device)
    sums_args = []
    if presummed is not None:
        qsum, ksum = presummed
        NB = sizes["NB"]
        for name, t in (("qsum", qsum), ("ksum", ksum)):
            _require(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()
                     and tuple(t.shape) == (B, H, NB, D), f"{name} must be contiguous f32 {(B, H, NB, D)}")
        _require(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16,
                 "presummed q / k must be bfloat16")
    a, a_scalar, a_dt, a_st = _alpha_view(alpha_2, B, S, H, D, q.device)
    inject = inject or {}
    inj = {}
    # injected decisions (a testing hook): the kernels index q rows with `order`, source
    # blocks with `sel` and new-KV blocks with `l3`, so their ranges are checked here
    for name, shape, hi in (("sel", (B, H, sizes["topK"]), sizes["n_s"]),
                            ("order", (B, H, sizes["NB"]), sizes["NB"]),
                            ("l3", (B, H, sizes["n_diffuse"], sizes["top_k"]), sizes["NKV"])):
        if inject.get(name) is not None:
            t = inject[name].to(device=q.device, dtype=torch.int32).contiguous()
            _require(tuple(t.shape) == shape, f"inject[{name!r}] must have shape {shape}")
            check_index_lists(t, hi, f"inject[{name!r}]")
            inj[name] = t
    ev_args = []
    fn = L.icsa_editing_sparse_attention
    if stage_events is not None:
        _require(len(stage_events) == len(_lib.STAGES), "one event per stage boundary")
        handles = (ctypes.c_void_p * len(stage_events))(*[e.cuda_event for e in stage_events])
        ev_args = [ctypes.cast(handles, ctypes.c_void_p)]
        fn = L.icsa_editing_sparse_attention_ev
    if presummed is not None:
        fn = L.icsa_editing_sparse_attention_presummed
        ev_args = (ev_args or [None]) + [ptr(presummed[0]), ptr(presummed[1])]
    ws_args = [ptr(ws), ws_bytes]
    if noalloc:
        fn = L.icsa_editing_sparse_attention_noalloc
        ws_args = []
    with torch.cuda.device(q.device):     # the library launches on the current device
        rc = fn(
            ptr(q), dtype_code(q), q.stride(0), q.stride(1), q.stride(2),
            ptr(k), dtype_code(k), k.stride(0), k.stride(1), k.stride(2),
            ptr(v), dtype_code(v), v.stride(0), v.stride(1), v.stride(2),
            B, S, H, D, int(t_seq_len), float(SPARSITY_RATIO), float(srr), float(flat_ratio),
            ptr(a), a_dt, a_st[0], a_st[1], a_st[2], a_st[3], float(a_scalar),
            ptr(out), dtype_code(out), out.stride(0), out.stride(1), out.stride(2),
            ptr(inj.get("sel")), ptr(inj.get("order")), ptr(inj.get("l3")),
            *ws_args, stream_ptr(q.device), *ev_args)
    _lib.check(fn.__name__, rc)
    if not keep_workspace:
        return out, None
    return out, workspace_views(ws, list(offs), sizes, B, H, D)


def workspace_views(ws: torch.Tensor, offs, sizes: dict, B: int, H: int, D: int) -> dict:
    """Typed views of the intermediate buffers (decisions, scores) of one call."""
    z = sizes

    def view(slot, dtype, shape):
        off = offs[_lib.WS_SLOTS.index(slot)]
        n = 1
        for s in shape:
            n *= s
        nbytes = n * torch.empty(0, dtype=dtype).element_size()
        return ws[off:off + nbytes].view(dtype).view(*shape)

    NB = z["NB"]
    logits = view("LOGITS", torch.float32, (B, H, NB, NB))
    row_stats = view("RSTAT", torch.float32, (B, H, NB, 2))      # row max m, 1 / row sum z
    return dict(
        sizes=z,
        q_sums=view("QSUM", torch.float32, (B, H, NB, D)),
        k_sums=view("KSUM", torch.float32, (B, H, NB, D)),
        v_sums=view("VSUM", torch.float32, (B, H, NB, D)),
        logits=logits,
        row_stats=row_stats,
        # the compressed softmax, formed from the stored logits and row statistics as the
        # strip kernel forms it (the library does not store P)
        P=torch.exp(logits - row_stats[..., :1]) * row_stats[..., 1:],
        out_c=view("OUTC", torch.float32, (B, H, NB, D)),
        sharpness=view("SHARP", torch.float32, (B, H, NB)),
        src_score=view("SRCSCORE", torch.float32, (B, H, max(z["n_s"], 1))),
        sel=view("SEL", torch.int32, (B, H, max(z["topK"], 1)))[..., :z["topK"]],
        order=view("ORDER", torch.int32, (B, H, NB)),
        kvmap=view("KVMAP", torch.int32, (B, H, z["NKV"])),
        kc32=view("KC32", torch.float32, (B, H, z["NKV"], D)),
        l3=view("L3", torch.int32, (B, H, max(z["n_diffuse"], 1), z["top_k"]))[:, :, :z["n_diffuse"]],
    )


def editing_sparse_attention(q, k, v, t_seq_len, s_seq_len, alpha_2=1.0, alpha_3=1.0,
                             SPARSITY_RATIO=0.0625, backend=Backend.TILELANG, *, srr=0.125,
                             flat_ratio=0.5):
    """Editing sparse attention (reference: editing_sparse_attention.py:67-232).

    Args:
        q, k, v: [B, S, H, D] (bfloat16 or float32 each; D = 128), target tokens first
        t_seq_len: target-video token count
        s_seq_len: source-video token count (unused, as in the reference)
        alpha_2: residual weight of the compressed-attention shortcut (float or tensor
            broadcastable to [B, S, H, D])
        alpha_3: unused (API compatibility)
        SPARSITY_RATIO: fraction of KV blocks for the exact top-k (also sets k_sparsity)
        backend: 'hip' runs this build; 'tilelang' (the reference's default) and 'triton'
            raise NotImplementedError here
        srr: source retrieval ratio (reference: 1/8, ``n_s // 8``)
        flat_ratio: fraction of query blocks given exact attention (reference: 1/2)

    Returns:
        x: [B, S, H, D] in q.dtype
    """
    backend = Backend.validate(backend)
    if backend != Backend.HIP:
        raise NotImplementedError(
            f"backend '{backend}' is CUDA-only and not part of this MI355X build; use 'hip'")
    x, _ = _editing_sparse_attention_hip(q, k, v, t_seq_len, alpha_2, SPARSITY_RATIO, srr,
                                         flat_ratio)
    return x


# Backward-compatible alias of the reference (editing_sparse_attention.py:235-236): the same
# function with the same default backend.
editing_sparse_attention_tilelang = editing_sparse_attention

__all__ = ["Backend", "editing_sparse_attention", "editing_sparse_attention_tilelang",
           "derived_sizes", "IcsaArgumentError"]
