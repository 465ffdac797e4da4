"""HIP host functions with the reference's kernel-host signatures.

* :func:`sparse_piecewise_attn_1st_intervals_hip` mirrors
  ``sparse_piecewise_attn_1st_intervals_tilelang`` (tilelang_host.py:229-274): same
  arguments, shapes, dtypes, return value and ownership, and the TileLang asserts.
  Argument checks raise :class:`IcsaArgumentError`, an ``AssertionError`` (what the
  reference's asserts raise) that is also a ``ValueError``.
* :func:`sparse_piecewise_attn_1st_intervals` mirrors the Triton host of the same name
  (triton_host.py:11-30), whose contract differs: ragged TQ / TKV, floor top_k over
  TKV // 64, keys past TKV masked out of the exact part (triton_kernels.py:185, 489-539).
* :func:`flash_attn_func` mirrors the call made at editing_sparse_attention.py:211-215
  (flash-attn's ``flash_attn_func(q, k, v)``, dense non-causal, default scale).
* :func:`pool` and :func:`gather_kv` expose stage 1 and the new-KV gather.

Work is enqueued on ``torch.cuda.current_stream()``; scratch memory comes from torch's
caching allocator and is passed to the library as its workspace.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

BLOCK_M = 64


class IcsaArgumentError(AssertionError, ValueError):
    """Invalid argument (the reference raises AssertionError for the same conditions)."""


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise IcsaArgumentError(msg)


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.BF16
    if t.dtype == torch.float32:
        return _lib.F32
    raise TypeError(f"unsupported dtype {t.dtype}: the HIP backend takes bfloat16 or float32")


def inner_contiguous(t: torch.Tensor) -> torch.Tensor:
    """The library needs a unit stride on the last dim and 16-byte aligned rows."""
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(
        (s * es) % 16 == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def check_index_lists(idx: torch.Tensor, hi: int, name: str, allow_neg: bool = False,
                      distinct: bool = True) -> None:
    """Host check of a caller-supplied index list (last dim): entries in ``[0, hi)`` (or -1
    where ``allow_neg``), distinct within each row.  The kernels index device memory with
    these values, so a bad list must be refused before the call, not read out of bounds."""
    if idx.numel() == 0:
        return
    x = idx.long()
    lo_ok = (x >= -1) if allow_neg else (x >= 0)
    _require(bool((lo_ok & (x < hi)).all()), f"{name}: entries must lie in [{'-1' if allow_neg else '0'}, {hi})")
    if distinct and x.shape[-1] > 1:
        srt = torch.sort(x, dim=-1).values
        dup = (srt[..., 1:] == srt[..., :-1]) & (srt[..., 1:] >= 0)
        _require(not bool(dup.any()), f"{name}: entries must be distinct within each list")


def stream_ptr(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


@torch.no_grad()
def sparse_piecewise_attn_1st_intervals_hip(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                            sparsity: float = 0.1, block_size: int = 64, *,
                                            indices: torch.Tensor = None,
                                            return_indices: bool = False, interval_bn: int = 64):
    """Sparse piecewise attention (first-order intervals) on MI355X.

    Args:
        q: [B, H, TQ, D] bfloat16 (TQ multiple of 64)
        k: [B, H, TKV, D] bfloat16 (TKV multiple of 64)
        v: [B, H, TKV, D] bfloat16 (Vdim == D == 128)
        sparsity: fraction of KV blocks attended exactly (top_k = max(1, int(sparsity*NKV)))
        block_size: must be 64
        indices: optional [B, H, TQ/64, top_k] int32 block lists (ascending) to use instead
            of the kernel's own top-k (testing hook; not in the reference signature)
        return_indices: also return the block lists used
        interval_bn: blocks per interval chunk (the TileLang kernel's BN: 16, 32 or 64)

    Returns:
        out: [B, H, TQ, D] bfloat16 (a new tensor owned by the caller)
    """
    _require(q.dtype == k.dtype == v.dtype == torch.bfloat16, "q, k, v must be bfloat16")
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "q, k, v must be on the GPU")
    _require(block_size == 64, "Only block_size=64 supported.")
    _require(q.ndim == 4 and k.ndim == 4 and v.ndim == 4, "q, k, v must be 4-D [B, H, T, D]")
    _require(q.shape[0] == k.shape[0] == v.shape[0], "batch mismatch")
    _require(q.shape[1] == k.shape[1] == v.shape[1], "head mismatch")
    _require(q.shape[3] == k.shape[3], "Kdim must match between q and k")
    _require(k.shape[2] == v.shape[2], "TKV must match between k and v")
    _require(v.shape[3] == q.shape[3], "This entrypoint assumes Vdim == D (so VBlocks==1).")
    B, H, TQ, D = q.shape
    TKV = k.shape[2]
    _require(TQ % BLOCK_M == 0 and TKV % BLOCK_M == 0, "TQ/TKV must be divisible by BT")
    q, k, v = inner_contiguous(q), inner_contiguous(k), inner_contiguous(v)
    L = _lib.lib()
    NQ, NKV = TQ // BLOCK_M, TKV // BLOCK_M
    top_k = max(1, int(sparsity * NKV))
    out = torch.empty(B, H, TQ, D, dtype=torch.bfloat16, device=q.device)
    ws_bytes = L.icsa_sparse_piecewise_workspace_size(B, H, TQ, TKV, D, float(sparsity))
    if ws_bytes < 0:
        raise _lib.IcsaError("icsa_sparse_piecewise_workspace_size", int(ws_bytes))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    inj = None
    if indices is not None:
        inj = indices.to(device=q.device, dtype=torch.int32).contiguous()
        _require(tuple(inj.shape) == (B, H, NQ, top_k), f"indices must be [B, H, {NQ}, {top_k}]")
        check_index_lists(inj, NKV, "indices")
    idx_out = torch.empty(B, H, NQ, top_k, dtype=torch.int32, device=q.device) if return_indices else None
    args = ([ptr(q), q.stride(0), q.stride(1), q.stride(2),
             ptr(k), k.stride(0), k.stride(1), k.stride(2),
             ptr(v), v.stride(0), v.stride(1), v.stride(2),
             B, H, TQ, TKV, D, float(sparsity)],
            [ptr(inj), ptr(idx_out),
             ptr(out), out.stride(0), out.stride(1), out.stride(2),
             ptr(ws), ws_bytes, stream_ptr(q.device)])
    with torch.cuda.device(q.device):     # the library launches on the current device
        if interval_bn == BLOCK_M:
            name = "icsa_sparse_piecewise_attn"
            rc = L.icsa_sparse_piecewise_attn(*args[0], *args[1])
        else:
            name = "icsa_sparse_piecewise_attn_hosttopk"
            rc = L.icsa_sparse_piecewise_attn_hosttopk(*args[0], int(interval_bn), *args[1])
    _lib.check(name, rc)
    return (out, idx_out) if return_indices else out


@torch.no_grad()
def sparse_piecewise_attn_tilelang_hosttopk_hip(q, k, v, sparsity=0.0625, BT=64, BV=32, BN=64,
                                                threads_topk: int = 128, threads_interval: int = 128,
                                                sorted_topk: bool = False, fused_use_wgmma: bool = False):
    """The TileLang pipeline entry ``sparse_piecewise_attn_tilelang_hosttopk``
    (tilelang_host.py:121-226) on MI355X: block sums, ``top_k = max(1, int(sparsity * NKV))``
    blocks per query block by ``QC KC^T``, exact attention over them plus the first-order
    interval over the rest.  The reference's two paths (the fused kernel when ``BV == Vdim``,
    the top-k + interval kernel pair otherwise) compute the same function; here one kernel
    serves both, so ``BV`` only has to divide Vdim.  ``BN`` is the interval chunk size,
    which decides where the non-rescaled interval terms take their running max: 16, 32
    and 64 (the reference's default, which every reference caller passes) run here.
    ``threads_*``, ``sorted_topk`` (the exact loop's visiting order only changes rounding)
    and ``fused_use_wgmma`` select reference launch variants and have no effect here."""
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16
    _require(q.ndim == 4 and k.ndim == 4 and v.ndim == 4, "q, k, v must be 4-D [B, H, T, D]")
    TQ, TKV, Vdim = q.shape[2], k.shape[2], v.shape[3]
    assert TQ % BT == 0 and TKV % BT == 0, "TQ/TKV must be divisible by BT"
    assert Vdim % BV == 0, "Vdim must be divisible by BV"
    _require(BT == BLOCK_M, f"BT={BT} unsupported (the kernels use 64-row blocks)")
    _require(BN in (16, 32, 64), f"BN={BN} unsupported (16, 32 or 64 blocks per interval chunk)")
    return sparse_piecewise_attn_1st_intervals_hip(q, k, v, sparsity, BT, interval_bn=BN)


def _check_sparse_args(q, k, v, block_size, aligned=True):
    """The TileLang host's argument checks (tilelang_host.py:251-259); ``aligned=False``
    drops the multiple-of-64 lengths the Triton host does not need."""
    _require(q.dtype == k.dtype == v.dtype == torch.bfloat16, "q, k, v must be bfloat16")
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "q, k, v must be on the GPU")
    _require(block_size == 64, "Only block_size=64 supported.")
    _require(q.ndim == 4 and k.ndim == 4 and v.ndim == 4, "q, k, v must be 4-D [B, H, T, D]")
    _require(q.shape[0] == k.shape[0] == v.shape[0], "batch mismatch")
    _require(q.shape[1] == k.shape[1] == v.shape[1], "head mismatch")
    _require(q.shape[3] == k.shape[3], "Kdim must match between q and k")
    _require(k.shape[2] == v.shape[2], "TKV must match between k and v")
    _require(v.shape[3] == q.shape[3], "This entrypoint assumes Vdim == D (so VBlocks==1).")
    _require(q.shape[2] > 0 and k.shape[2] > 0, "TQ and TKV must be positive")
    if aligned:
        _require(q.shape[2] % BLOCK_M == 0 and k.shape[2] % BLOCK_M == 0, "TQ/TKV must be divisible by BT")


def triton_top_k(sparsity: float, TKV: int) -> int:
    """Exact blocks per query block of the Triton host: max(1, int(sparsity * (TKV // 64)))
    (triton_kernels.py:501), over cdiv(TKV, 64) candidate blocks."""
    return max(1, int(sparsity * (TKV // BLOCK_M)))


@torch.no_grad()
def sparse_piecewise_attn_1st_intervals_fwd_hip(q, k, v, sparsity: float = 0.1, block_size: int = 64,
                                                indices: torch.Tensor = None):
    """The forward of SparsePiecewiseAttn1stIntervalsFunction (triton_kernels.py:489-539)
    with the state its backward needs, under the Triton host's contract: TQ and TKV need
    not be multiples of 64 (rows past them read as zeros in the block sums), the
    ``top_k = max(1, int(sparsity * (TKV // 64)))`` exact blocks are chosen among
    ``cdiv(TKV, 64)`` candidates, and keys at or past TKV take no part in the exact
    attention (triton_kernels.py:185).  Returns ``(out, lse, indices)``: out bf16
    [B, H, TQ, D]; lse f32 [B, H, TQ] in log2 units (the final running max of the
    log2-scaled scores plus log2 of the combined denominator); indices int32
    [B, H, cdiv(TQ, 64), top_k] (``indices`` given: used instead of the kernel's own top-k)."""
    _check_sparse_args(q, k, v, block_size, aligned=False)
    B, H, TQ, D = q.shape
    TKV = k.shape[2]
    q, k, v = inner_contiguous(q), inner_contiguous(k), inner_contiguous(v)
    L = _lib.lib()
    NQ, NKV = (TQ + BLOCK_M - 1) // BLOCK_M, (TKV + BLOCK_M - 1) // BLOCK_M
    top_k = triton_top_k(sparsity, TKV)
    out = torch.empty(B, H, TQ, D, dtype=torch.bfloat16, device=q.device)
    lse = torch.empty(B, H, TQ, dtype=torch.float32, device=q.device)
    idx = torch.empty(B, H, NQ, top_k, dtype=torch.int32, device=q.device)
    ws_bytes = L.icsa_sparse_piecewise_workspace_size(B, H, TQ, TKV, D, float(sparsity))
    if ws_bytes < 0:
        raise _lib.IcsaError("icsa_sparse_piecewise_workspace_size", int(ws_bytes))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    inj = None
    if indices is not None:
        inj = indices.to(device=q.device, dtype=torch.int32).contiguous()
        _require(tuple(inj.shape) == (B, H, NQ, top_k), f"indices must be [B, H, {NQ}, {top_k}]")
        check_index_lists(inj, NKV, "indices")
    with torch.cuda.device(q.device):     # the library launches on the current device
        rc = L.icsa_sparse_piecewise_attn_fwd(
            ptr(q), q.stride(0), q.stride(1), q.stride(2),
            ptr(k), k.stride(0), k.stride(1), k.stride(2),
            ptr(v), v.stride(0), v.stride(1), v.stride(2),
            B, H, TQ, TKV, D, float(sparsity),
            ptr(inj), ptr(idx),
            ptr(out), out.stride(0), out.stride(1), out.stride(2), ptr(lse),
            ptr(ws), ws_bytes, stream_ptr(q.device))
    _lib.check("icsa_sparse_piecewise_attn_fwd", rc)
    return out, lse, idx


@torch.no_grad()
def sparse_piecewise_attn_1st_intervals(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                        sparsity: float = 0.1, block_size: int = 64) -> torch.Tensor:
    """The Triton host (triton_host.py:11-30) on MI355X: ``SparsePiecewiseAttn1stIntervals
    Function.apply`` under ``no_grad``.  q [B, H, TQ, D], k / v [B, H, TKV, D] bfloat16 with
    any TQ and TKV (the reference's Triton branch passes the unpadded new KV,
    editing_sparse_attention.py:203-207); floor top_k over TKV // 64, keys past TKV masked
    out of the exact part.  Returns a new bf16 [B, H, TQ, D] owned by the caller."""
    out, _, _ = sparse_piecewise_attn_1st_intervals_fwd_hip(q, k, v, sparsity, block_size)
    return out


@torch.no_grad()
def sparse_piecewise_attn_1st_intervals_bwd_hip(do, q, k, v, out, lse, indices, grad_dtype=None,
                                                check_indices=True):
    """Gradients ``(dq, dk, dv)`` of the sparse piecewise attention, as
    SparsePiecewiseAttn1stIntervalsFunction.backward (triton_kernels.py:541-598) computes
    them from the saved (q, k, v, out, lse, indices), without atomics (the same inputs give
    the same bits).  ``grad_dtype``: bf16 (default: q.dtype, as the reference's final cast)
    or float32.  ``indices`` must hold distinct blocks in ``[0, cdiv(TKV, 64))`` per query block
    (the forward's top-k always does; the reference's atomics would count a repeated entry
    twice in every gradient, this build's key-major dk / dv pass once), which
    ``check_indices`` verifies on the host (one device sync).  Ragged TQ / TKV as the
    reference's Triton backward: ``cdiv`` blocks, rows past the lengths read as zero and keys
    past TKV masked out of the exact blocks (triton_kernels.py:348, :404)."""
    _check_sparse_args(q, k, v, 64, aligned=False)
    B, H, TQ, D = q.shape
    TKV = k.shape[2]
    NQ = -(-TQ // BLOCK_M)
    _require(do.shape == q.shape and out.shape == q.shape, "do / out must be [B, H, TQ, D] like q")
    _require(do.dtype == torch.bfloat16 and out.dtype == torch.bfloat16, "do / out must be bfloat16")
    _require(all(t.device == q.device for t in (k, v, do, out, lse, indices)),
             "q, k, v, do, out, lse and indices must be on the same GPU")
    _require(tuple(lse.shape) == (B, H, TQ) and lse.dtype == torch.float32, "lse must be f32 [B, H, TQ]")
    _require(indices.dim() == 4 and tuple(indices.shape[:3]) == (B, H, NQ),
             f"indices must be [B, H, {NQ}, top_k]")
    gd = q.dtype if grad_dtype is None else grad_dtype
    _require(gd in (torch.bfloat16, torch.float32), "grad_dtype must be bfloat16 or float32")
    q, k, v, do, out = (inner_contiguous(t) for t in (q, k, v, do, out))
    lse = lse.contiguous()
    idx = indices.to(dtype=torch.int32).contiguous()
    top_k = idx.shape[-1]
    if check_indices:
        check_index_lists(idx, -(-TKV // BLOCK_M), "indices")
    L = _lib.lib()
    dq = torch.empty(B, H, TQ, D, dtype=gd, device=q.device)
    dk = torch.empty(B, H, TKV, D, dtype=gd, device=q.device)
    dv = torch.empty(B, H, TKV, D, dtype=gd, device=q.device)
    ws_bytes = L.icsa_sparse_piecewise_attn_bwd_workspace_size(B, H, TQ, TKV, D)
    if ws_bytes < 0:
        raise _lib.IcsaError("icsa_sparse_piecewise_attn_bwd_workspace_size", int(ws_bytes))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    g = dtype_code(dq)
    with torch.cuda.device(q.device):     # the library launches on the current device
        rc = L.icsa_sparse_piecewise_attn_bwd(
            ptr(do), do.stride(0), do.stride(1), do.stride(2),
            ptr(q), q.stride(0), q.stride(1), q.stride(2),
            ptr(k), k.stride(0), k.stride(1), k.stride(2),
            ptr(v), v.stride(0), v.stride(1), v.stride(2),
            ptr(out), out.stride(0), out.stride(1), out.stride(2),
            ptr(lse), ptr(idx),
            B, H, TQ, TKV, D, top_k,
            ptr(dq), g, dq.stride(0), dq.stride(1), dq.stride(2),
            ptr(dk), g, dk.stride(0), dk.stride(1), dk.stride(2),
            ptr(dv), g, dv.stride(0), dv.stride(1), dv.stride(2),
            ptr(ws), ws_bytes, stream_ptr(q.device))
    _lib.check("icsa_sparse_piecewise_attn_bwd", rc)
    return dq, dk, dv


class SparsePiecewiseAttn1stIntervalsFunction(torch.autograd.Function):
    """Autograd function of the sparse piecewise attention on MI355X, with the reference
    Function's interface (triton_kernels.py:489-598): ``apply(q, k, v, sparsity,
    block_size)``; the backward returns (dq, dk, dv) in the inputs' dtype and None for
    sparsity and block_size."""

    @staticmethod
    def forward(ctx, q, k, v, sparsity, block_size):
        out, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q, k, v, sparsity, block_size)
        ctx.save_for_backward(q, k, v, out, lse, idx)
        return out

    @staticmethod
    def backward(ctx, do):
        q, k, v, out, lse, idx = ctx.saved_tensors
        dq, dk, dv = sparse_piecewise_attn_1st_intervals_bwd_hip(
            do.to(torch.bfloat16), q, k, v, out, lse, idx, check_indices=False)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None


@torch.no_grad()
def flash_attn_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dropout_p: float = 0.0,
                    softmax_scale=None, causal: bool = False, out_dtype=None) -> torch.Tensor:
    """Dense non-causal attention, ``[B, S, H, D]`` layout (flash-attn's ``flash_attn_func``
    as called at editing_sparse_attention.py:211-215).  bf16 inputs; output bf16 unless
    ``out_dtype=torch.float32``."""
    _require(dropout_p == 0.0 and softmax_scale is None and not causal,
             "only dropout_p=0, default softmax_scale and causal=False are supported")
    _require(q.dtype == k.dtype == v.dtype == torch.bfloat16, "q, k, v must be bfloat16")
    _require(q.is_cuda and k.is_cuda and v.is_cuda, "q, k, v must be on the GPU")
    _require(q.ndim == 4 and k.shape == v.shape and q.shape[0] == k.shape[0] and
             q.shape[2:] == k.shape[2:], "q [B,Sq,H,D], k/v [B,Sk,H,D] expected")
    q, k, v = inner_contiguous(q), inner_contiguous(k), inner_contiguous(v)
    B, Sq, H, D = q.shape
    Sk = k.shape[1]
    out_dtype = out_dtype or torch.bfloat16
    out = torch.empty(B, Sq, H, D, dtype=out_dtype, device=q.device)
    L = _lib.lib()
    ws_bytes = L.icsa_flash_attn_workspace_size(B, Sk, H, D)
    if ws_bytes < 0:
        raise _lib.IcsaError("icsa_flash_attn_workspace_size", int(ws_bytes))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):     # the library launches on the current device
        rc = L.icsa_flash_attn(
            ptr(q), q.stride(0), q.stride(1), q.stride(2),
            ptr(k), k.stride(0), k.stride(1), k.stride(2),
            ptr(v), v.stride(0), v.stride(1), v.stride(2),
            B, Sq, Sk, H, D,
            ptr(out), dtype_code(out), out.stride(0), out.stride(1), out.stride(2),
            ptr(ws), ws_bytes, stream_ptr(q.device))
    _lib.check("icsa_flash_attn", rc)
    return out


@torch.no_grad()
def pool(q=None, k=None, v=None, want_vt: bool = False):
    """Stage 1: fp32 block sums ``[B, H, NB, D]`` of each given ``[B, S, H, D]`` tensor (None
    for absent ones) and, with ``want_vt``, V transposed ``[B, H, D, NB*64]`` bf16."""
    ref = next(t for t in (q, k, v) if t is not None)
    B, S, H, D = ref.shape
    NB = (S + BLOCK_M - 1) // BLOCK_M
    ts = [inner_contiguous(t) if t is not None else None for t in (q, k, v)]
    sums = [torch.empty(B, H, NB, D, dtype=torch.float32, device=ref.device) if t is not None else None
            for t in ts]
    vt = None
    if want_vt:
        _require(v is not None, "want_vt needs v")
        vt = torch.empty(B, H, D, NB * BLOCK_M, dtype=torch.bfloat16, device=ref.device)
    args = []
    for t in ts:
        if t is None:
            args += [ctypes.c_void_p(0), 0, 0, 0, 0]
        else:
            args += [ptr(t), dtype_code(t), t.stride(0), t.stride(1), t.stride(2)]
    with torch.cuda.device(ref.device):     # the library launches on the current device
        rc = _lib.lib().icsa_pool(*args, B, S, H, D, ptr(sums[0]), ptr(sums[1]), ptr(sums[2]), ptr(vt),
                                  stream_ptr(ref.device))
    _lib.check("icsa_pool", rc)
    return sums[0], sums[1], sums[2], vt


@torch.no_grad()
def gather_kv(k: torch.Tensor, v: torch.Tensor, t_seq_len: int, sel: torch.Tensor):
    """Materialised new KV ``[B, H, Tp, D]`` bf16 (editing_sparse_attention.py:138-159, zero
    padded to a multiple of 64 rows)."""
    k, v = inner_contiguous(k), inner_contiguous(v)
    B, S, H, D = k.shape
    topK = sel.shape[-1]
    sel32 = sel.to(device=k.device, dtype=torch.int32).reshape(B * H, topK).contiguous()
    Tkv = t_seq_len + topK * BLOCK_M
    Tp = (Tkv + BLOCK_M - 1) // BLOCK_M * BLOCK_M
    kn = torch.empty(B, H, Tp, D, dtype=torch.bfloat16, device=k.device)
    vn = torch.empty_like(kn)
    with torch.cuda.device(k.device):     # the library launches on the current device
        rc = _lib.lib().icsa_gather_kv(
            ptr(k), dtype_code(k), k.stride(0), k.stride(1), k.stride(2),
            ptr(v), dtype_code(v), v.stride(0), v.stride(1), v.stride(2),
            B, S, H, D, t_seq_len, ptr(sel32), topK, ptr(kn), ptr(vn), stream_ptr(k.device))
    _lib.check("icsa_gather_kv", rc)
    return kn, vn
