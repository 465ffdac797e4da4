"""Vectorised CPU oracle of the reference's in-context sparse attention path.

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the HIP product path.

Restated from the reference (paths relative to the reference repository root):

* ``editing_sparse_attention.py:67-232``  -- the whole algorithm (pad, pool, compressed
  attention, per-head source retrieval, new KV, sharpness split, dispatch, scatter, residual).
* ``tilelang_host.py:121-206, 229-274``   -- sparse host: block sums, ``top_k`` formula,
  KC/VC padding to BN=64.
* ``tilelang_kernels.py:681-997``          -- fused sparse kernel: exact top-k loop and the
  chunked interval approximation with non-rescaled ``g_acc``/``g_l``.
* ``triton_kernels.py:122-263, 489-539``   -- cross-check of the same semantics.

Arithmetic is float64 by default (the "fp32-or-better" reference the parity bar is stated
against) and float32 for the CPU baseline.  The reference's own bf16 rounding points
(bf16 block sums, bf16 level-3 scores, bf16 softmax under autocast) are precision
artefacts, not part of the algorithm, and are not reproduced.

Deterministic tie rule (adopted for every ranked decision): larger value first, and for
equal values the lower index first.  The reference uses ``torch.topk``/``sort``/``argsort``
on CUDA, whose tie order is implementation-defined.

Pinning (which check fixes each function; tests/test_oracle.py):

====================================  =================================================
function                              pinned by
====================================  =================================================
``derive_sizes``                      reference's Appendix-A sizes for every config
                                      (hand-derived constants), closed-form formulas
``pool_blocks``                       constant blocks -> constant; partial last block
                                      divides by its real size; brute-force loops
``compressed_attention``              float64 ``scaled_dot_product_attention``;
                                      brute-force loops
``select_source_blocks``              planted retrieval case with an analytic answer;
                                      brute-force explicit sort
``new_kv_token_map``/``gather_new_kv``  closed-form index identity; brute-force loops
``split_blocks``                      planted peaked blocks with known ranking;
                                      brute-force explicit sort
``sparse_piecewise_attn``             (i) top_k = NKV reduces to dense attention;
                                      (ii) constant-key blocks make the interval exact;
                                      (iii) brute-force scalar online-softmax loops;
                                      (iv) crafted case exposing the non-rescaled
                                      interval accumulators (differs from a rescaled
                                      variant by a known amount)
``dense_attention``                   float64 SDPA; brute-force loops
``editing_sparse_attention``          brute-force end-to-end loops at toy sizes;
                                      output independent of block processing order
====================================  =================================================
"""
from __future__ import annotations

import math
from dataclasses import dataclass, asdict
from typing import Optional

import torch
import torch.nn.functional as F

__all__ = [
    "BLOCK_M", "Sizes", "derive_sizes", "block_sizes", "pool_blocks", "compressed_attention",
    "select_source_blocks", "new_kv_token_map", "gather_new_kv", "split_blocks",
    "sparse_piecewise_attn", "dense_attention", "editing_sparse_attention",
    "ranked_topk", "check_topk_valid", "check_split_valid",
]

BLOCK_M = 64          # editing_sparse_attention.py:22
BN_INTERVAL = 64      # tilelang_host.py:269 (chunk of compressed blocks in the interval loop)


def ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


@dataclass(frozen=True)
class Sizes:
    B: int
    S: int
    H: int
    D: int
    t: int
    NB: int
    n_t: int
    n_s: int
    topK: int
    Tkv: int
    k_sparsity: int
    n_peaked: int
    n_diffuse: int
    TKV_pad: int
    NKV: int
    top_k: int

    def as_dict(self):
        return asdict(self)


def derive_sizes(B: int, S: int, H: int, D: int, t_seq_len: int,
                 sparsity: float = 0.0625, srr: float = 0.125,
                 flat_ratio: float = 0.5) -> Sizes:
    """Every derived size of the path.

    editing_sparse_attention.py:89-94 (NB, partial last block), :126-129 (n_t, n_s,
    topK = n_s // 8), :139 (Tkv), :164 (k_sparsity), :169-172 (NB // 2 peaked blocks),
    :189-198 (TKV padded to a multiple of 64 for the sparse call);
    tilelang_host.py:151-152, 171 (NKV, top_k = max(1, int(sparsity * NKV))).
    ``srr`` and ``flat_ratio`` generalise the reference's integer divisions ``// 8`` and
    ``// 2``; for dyadic ratios ``int(n * r)`` equals the reference's ``n // (1/r)``.
    """
    NB = ceil_div(S, BLOCK_M)
    n_t = t_seq_len // BLOCK_M
    n_s = NB - n_t
    topK = int(n_s * srr)
    Tkv = t_seq_len + topK * BLOCK_M
    k_sparsity = max(1, int(n_t * sparsity))
    n_peaked = int(NB * flat_ratio)
    TKV_pad = ceil_div(Tkv, BLOCK_M) * BLOCK_M
    NKV = TKV_pad // BLOCK_M
    top_k = max(1, int(sparsity * NKV))
    return Sizes(B, S, H, D, t_seq_len, NB, n_t, n_s, topK, Tkv, k_sparsity, n_peaked,
                 NB - n_peaked, TKV_pad, NKV, top_k)


# ---------------------------------------------------------------------------------------
# ranking helpers (deterministic tie rule)
# ---------------------------------------------------------------------------------------

def ranked_order(x: torch.Tensor) -> torch.Tensor:
    """Indices sorting the last dim by value descending, ties by lower index first."""
    return torch.sort(x, dim=-1, descending=True, stable=True).indices


def ranked_topk(x: torch.Tensor, k: int) -> torch.Tensor:
    """First ``k`` indices of :func:`ranked_order` (``torch.topk(sorted=True)`` with the
    deterministic tie rule)."""
    return ranked_order(x)[..., :k]


def check_topk_valid(scores: torch.Tensor, chosen: torch.Tensor, k: int, thr: float,
                     ordered: bool) -> torch.Tensor:
    """Per-row validity of ``chosen`` as a top-``k`` of ``scores`` under tolerance ``thr``.

    A choice is valid when (1) its indices are distinct and in range, (2) no unchosen
    score exceeds the smallest chosen score by more than ``thr`` and, when ``ordered``,
    (3) consecutive chosen scores never increase by more than ``thr``.  Wherever the gap
    between the k-th and (k+1)-th ranked score exceeds ``thr`` a valid choice is
    therefore the exact reference set (and, ordered, the exact reference order wherever
    neighbouring gaps exceed ``thr``).  Returns a bool tensor over the leading dims.
    """
    n = scores.shape[-1]
    chosen = chosen.long()
    in_range = ((chosen >= 0) & (chosen < n)).all(-1)
    c = chosen.clamp(0, n - 1)
    srt = torch.sort(c, dim=-1).values
    distinct = (srt[..., 1:] != srt[..., :-1]).all(-1) if k > 1 else torch.ones_like(in_range)
    sel_scores = torch.gather(scores, -1, c)
    mask = torch.zeros_like(scores, dtype=torch.bool)
    mask.scatter_(-1, c, True)
    unchosen_max = scores.masked_fill(mask, -math.inf).max(-1).values
    ok = in_range & distinct & (unchosen_max <= sel_scores.min(-1).values + thr)
    if ordered and k > 1:
        ok = ok & (sel_scores[..., 1:] <= sel_scores[..., :-1] + thr).all(-1)
    return ok


def check_split_valid(sharpness: torch.Tensor, peaked: torch.Tensor, thr: float) -> torch.Tensor:
    """Set validity of the peaked half (order inside a half does not change outputs)."""
    return check_topk_valid(sharpness, peaked, peaked.shape[-1], thr, ordered=False)


# ---------------------------------------------------------------------------------------
# stage 1: block pooling
# ---------------------------------------------------------------------------------------

def block_sizes(S: int) -> torch.Tensor:
    """``variable_block_sizes`` (editing_sparse_attention.py:92-94)."""
    NB = ceil_div(S, BLOCK_M)
    sizes = torch.full((NB,), BLOCK_M, dtype=torch.int64)
    sizes[-1] = S - (NB - 1) * BLOCK_M
    return sizes


def pool_blocks(x: torch.Tensor, dtype=torch.float64):
    """Block sums and means of ``x [B,S,H,D]`` -> ``[B,H,NB,D]`` each.

    editing_sparse_attention.py:96-111 and ``compress_seq`` :37-55: zero-pad to NB*64,
    sum each 64-token block, divide by the real block size (the last block may be
    partial).  The reference rounds the mean back to the input dtype (:45, :55, :109);
    here it stays in ``dtype``.
    """
    B, S, H, D = x.shape
    NB = ceil_div(S, BLOCK_M)
    xp = F.pad(x.to(dtype), (0, 0, 0, 0, 0, NB * BLOCK_M - S))
    sums = xp.view(B, NB, BLOCK_M, H, D).sum(2).permute(0, 2, 1, 3).contiguous()
    sizes = block_sizes(S).to(device=x.device, dtype=dtype)
    means = sums / sizes.view(1, 1, -1, 1)
    return sums, means


# ---------------------------------------------------------------------------------------
# stage 2: compressed attention, retrieval, split
# ---------------------------------------------------------------------------------------

def compressed_attention(qc: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor):
    """``torch_attention`` on pooled blocks (editing_sparse_attention.py:58-64, 113-118).

    qc, kc, vc: ``[B,H,NB,D]`` means.  Returns ``P [B,H,NB,NB]`` (row softmax of
    ``qc kc^T / sqrt(D)``) and ``out_c [B,H,NB,D] = P vc``.
    """
    D = qc.shape[-1]
    logits = torch.matmul(qc, kc.transpose(-2, -1)) / math.sqrt(D)
    P = torch.softmax(logits, dim=-1)
    return P, torch.matmul(P, vc)


def select_source_blocks(P: torch.Tensor, n_t: int, topK: int):
    """Per-head source-block retrieval (editing_sparse_attention.py:125-136).

    ``score[b,h,j] = sum_{i < n_t} P[b,h,i,n_t+j]``; the first ``topK`` of the ranked
    order (descending score; ``topk(2*topK)[:topK]`` keeps the same first ``topK``).
    The selected list stays in ranked order: it fixes the new-KV block numbering.
    """
    score = P[:, :, :n_t, n_t:].sum(dim=-2)
    return ranked_topk(score, topK), score


def new_kv_token_map(t: int, S: int, sel: torch.Tensor) -> torch.Tensor:
    """Original token index of every new-KV position, or -1 for a zero (padding) token.

    editing_sparse_attention.py:138-159: new KV = ``[K[:t] | K_pad[n_t*64 + 64*sel[r] + i]]``
    where ``K_pad`` is K zero-padded to NB*64 tokens (tokens >= S are zeros).
    """
    B, H, topK = sel.shape
    n_t = t // BLOCK_M
    dev = sel.device
    tgt = torch.arange(t, dtype=torch.int64, device=dev).view(1, 1, t).expand(B, H, t)
    src = (n_t * BLOCK_M + sel.long()[..., None] * BLOCK_M
           + torch.arange(BLOCK_M, dtype=torch.int64, device=dev)).reshape(B, H, topK * BLOCK_M)
    src = torch.where(src < S, src, torch.full_like(src, -1))
    return torch.cat([tgt, src], dim=-1)


def gather_new_kv(x: torch.Tensor, tokmap: torch.Tensor, dtype=torch.float64) -> torch.Tensor:
    """Materialise ``[B,H,Tkv,D]`` from ``x [B,S,H,D]`` through ``tokmap`` (zeros for -1)."""
    B, S, H, D = x.shape
    xh = x.to(dtype).permute(0, 2, 1, 3)
    idx = tokmap.clamp(min=0)
    out = torch.gather(xh, 2, idx[..., None].expand(-1, -1, -1, D))
    return out.masked_fill((tokmap < 0)[..., None], 0.0)


def split_blocks(P: torch.Tensor, n_t: int, k_sparsity: int, n_peaked: int):
    """Sharpness split (editing_sparse_attention.py:161-172).

    ``sharpness[i]`` = sum of the ``k_sparsity`` largest ``P[i, :n_t]`` (every query
    block, target key columns only).  The ``n_peaked`` most peaked blocks (the reference's
    ``flat_indices``) get exact attention; the rest (``sharp_indices``) the sparse kernel.
    """
    top = torch.sort(P[..., :n_t], dim=-1, descending=True).values[..., :k_sparsity]
    sharp = top.sum(dim=-1)
    order = ranked_order(sharp)
    return order[..., :n_peaked], order[..., n_peaked:], sharp


# ---------------------------------------------------------------------------------------
# attention kernels
# ---------------------------------------------------------------------------------------

def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    chunk: Optional[int] = None) -> torch.Tensor:
    """Textbook non-causal softmax attention ``[..., T, D]`` (flash_attn_func at
    editing_sparse_attention.py:211-215), chunked over queries to bound memory (default:
    at most 2^27 score elements per chunk, and at most 4096 queries)."""
    D = q.shape[-1]
    if chunk is None:
        lead = q[..., 0, 0].numel()
        chunk = max(16, min(4096, (1 << 27) // max(1, lead * k.shape[-2])))
    outs = []
    kt = k.transpose(-2, -1).contiguous()
    for s0 in range(0, q.shape[-2], chunk):
        s = torch.matmul(q[..., s0:s0 + chunk, :], kt) / math.sqrt(D)
        outs.append(torch.matmul(torch.softmax(s, dim=-1), v))
    return torch.cat(outs, dim=-2)


def sparse_piecewise_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          sparsity: float = 0.1, indices: Optional[torch.Tensor] = None,
                          dtype=torch.float64, qchunk: int = 64, return_lse: bool = False,
                          mode: str = "tilelang", bn: int = BN_INTERVAL):
    """Sparse piecewise attention with the first-order interval approximation.

    ``mode="triton"`` follows the Triton host instead (triton_host.py:11-30 ->
    SparsePiecewiseAttn1stIntervalsFunction.forward, triton_kernels.py:489-539, kernel
    :122-263), which takes ragged TQ / TKV: block sums over the real rows (zero fill,
    :89-119), ``NKV = cdiv(TKV, 64)`` candidate blocks, ``top_k = max(1, int(sparsity *
    (TKV // 64)))`` (floor, :501), keys at positions >= TKV masked out of the exact part
    (:185), and the interval over all NKV blocks with /64 and weight 64 like TileLang
    (:206-242).  For TQ and TKV multiples of 64 both modes give the same result.

    Semantics of ``sparse_piecewise_attn_1st_intervals_tilelang`` (tilelang_host.py:229-274
    -> :121-206 -> tilelang_kernels.py:681-997).  ``q [B,H,TQ,D]``, ``k``/``v [B,H,TKV,D]``
    with TQ and TKV multiples of 64 (the caller pads TKV with zero tokens,
    editing_sparse_attention.py:189-198).

    * QC/KC/VC: 64-row block sums (tilelang_kernels.py:33-120).
    * ``top_k = max(1, int(sparsity * NKV))`` blocks per query block by ``QC KC^T``
      (tilelang_host.py:171-173).  Default: ranked order; the exact loop visits them in
      ascending block index (the loop order only changes rounding).
    * Exact online softmax over those blocks (tilelang_kernels.py:863-868).
    * Interval over chunks of ``bn`` compressed blocks (the TileLang kernel's BN, 64 by
      default, tilelang_host.py:127) in ascending order
      (tilelang_kernels.py:886-978): score ``q . KC_j / 64`` (-inf for selected blocks and
      blocks >= NKV); the running max and ``acc``/``l`` are rescaled, but ``g_acc`` and
      ``g_l`` (``+= p VC``, ``+= 64 sum p``) are *not* rescaled when the max grows later.
    * ``out = (acc + g_acc) / (l + g_l)``, 0 where the denominator is 0 (:980-992).

    Returns ``(out [B,H,TQ,D], indices [B,H,NQ,top_k] ascending, scores [B,H,NQ,NKV])``,
    and with ``return_lse`` also ``lse [B,H,TQ]`` as the Triton forward stores it for the
    backward (triton_kernels.py:249-252): ``m + log2(l + g_l)`` in log2 units (the final
    running max of the log2-scaled scores; ``-inf`` where the denominator is 0).
    """
    assert mode in ("tilelang", "triton")
    B, H, TQ_real, D = q.shape
    TKV_real = k.shape[2]
    if mode == "tilelang":
        assert TQ_real % BLOCK_M == 0 and TKV_real % BLOCK_M == 0
    dev = q.device              # every intermediate follows the inputs' device
    TQ, TKV = ceil_div(TQ_real, BLOCK_M) * BLOCK_M, ceil_div(TKV_real, BLOCK_M) * BLOCK_M
    NQ, NKV = TQ // BLOCK_M, TKV // BLOCK_M
    scale = 1.0 / math.sqrt(D)
    # rows past the real lengths are zeros (the Triton kernels' boundary fill)
    qd = F.pad(q.to(dtype), (0, 0, 0, TQ - TQ_real))
    kd = F.pad(k.to(dtype), (0, 0, 0, TKV - TKV_real))
    vd = F.pad(v.to(dtype), (0, 0, 0, TKV - TKV_real))
    QC = qd.view(B, H, NQ, BLOCK_M, D).sum(3)
    KC = kd.view(B, H, NKV, BLOCK_M, D).sum(3)
    VC = vd.view(B, H, NKV, BLOCK_M, D).sum(3)
    scores = torch.matmul(QC, KC.transpose(-2, -1).contiguous())
    top_k = max(1, int(sparsity * (NKV if mode == "tilelang" else TKV_real // BLOCK_M)))
    if indices is None:
        indices = ranked_topk(scores, top_k)
    indices = torch.sort(indices.long().to(dev), dim=-1).values
    assert indices.shape == (B, H, NQ, top_k)
    n_chunks = ceil_div(NKV, bn)
    kb = kd.view(B, H, NKV, BLOCK_M, D)
    vb = vd.view(B, H, NKV, BLOCK_M, D)
    out = torch.empty(B, H, TQ, D, dtype=dtype, device=dev)
    lse = torch.empty(B, H, TQ, dtype=dtype, device=dev)
    bi = torch.arange(B, device=dev).view(B, 1, 1, 1)
    hi = torch.arange(H, device=dev).view(1, H, 1, 1)
    for n0 in range(0, NQ, qchunk):
        n1 = min(NQ, n0 + qchunk)
        qb = qd[:, :, n0 * BLOCK_M:n1 * BLOCK_M].view(B, H, n1 - n0, BLOCK_M, D)
        idx = indices[:, :, n0:n1]
        kx = kb[bi, hi, idx].reshape(B, H, n1 - n0, top_k * BLOCK_M, D)
        vx = vb[bi, hi, idx].reshape(B, H, n1 - n0, top_k * BLOCK_M, D)
        s_ex = torch.matmul(qb, kx.transpose(-2, -1).contiguous()) * scale
        if TKV_real < TKV:      # Triton: keys past TKV do not take part (triton_kernels.py:185)
            kpos = (idx[..., None] * BLOCK_M + torch.arange(BLOCK_M, device=dev)).reshape(
                B, H, n1 - n0, 1, top_k * BLOCK_M)
            s_ex = s_ex.masked_fill(kpos >= TKV_real, -math.inf)
        m = s_ex.max(-1).values
        p = torch.exp(s_ex - m[..., None])
        l = p.sum(-1)
        acc = torch.matmul(p, vx)
        s_int = torch.matmul(qb, KC[:, :, None].transpose(-2, -1).contiguous()) * (scale / BLOCK_M)
        selected = torch.zeros(B, H, n1 - n0, NKV, dtype=torch.bool, device=dev)
        selected.scatter_(-1, idx, True)
        s_int = s_int.masked_fill(selected[:, :, :, None, :], -math.inf)
        g_acc = torch.zeros_like(acc)
        g_l = torch.zeros_like(l)
        for c in range(n_chunks):
            j0, j1 = c * bn, min(NKV, (c + 1) * bn)
            s_c = s_int[..., j0:j1]
            m_new = torch.maximum(m, s_c.max(-1).values)
            alpha = torch.exp(m - m_new)
            acc = acc * alpha[..., None]
            l = l * alpha
            pc = torch.exp(s_c - m_new[..., None])
            g_l = g_l + BLOCK_M * pc.sum(-1)
            g_acc = g_acc + torch.matmul(pc, VC[:, :, None, j0:j1])
            m = m_new
        den = l + g_l
        o = (acc + g_acc) / torch.where(den == 0, torch.ones_like(den), den)[..., None]
        o = torch.where((den == 0)[..., None], torch.zeros_like(o), o)
        out[:, :, n0 * BLOCK_M:n1 * BLOCK_M] = o.reshape(B, H, (n1 - n0) * BLOCK_M, D)
        lse[:, :, n0 * BLOCK_M:n1 * BLOCK_M] = ((m + torch.log(den)) / math.log(2.0)).reshape(
            B, H, (n1 - n0) * BLOCK_M)
    out, lse = out[:, :, :TQ_real], lse[:, :, :TQ_real]
    if return_lse:
        return out, indices, scores, lse
    return out, indices, scores


# ---------------------------------------------------------------------------------------
# the whole path
# ---------------------------------------------------------------------------------------

def editing_sparse_attention(q, k, v, t_seq_len: int, s_seq_len: int, alpha_2=1.0,
                             alpha_3=1.0, SPARSITY_RATIO: float = 0.0625,
                             srr: float = 0.125, flat_ratio: float = 0.5,
                             decisions: Optional[dict] = None, dtype=torch.float64):
    """Oracle of ``editing_sparse_attention`` (editing_sparse_attention.py:67-232).

    q, k, v: ``[B,S,H,D]`` (any float dtype; the values are used as given).  ``alpha_2``:
    float or tensor broadcastable to ``[B,S,H,D]``.  ``alpha_3`` and ``s_seq_len`` are
    unused, as in the reference.  ``decisions`` may inject ``sel`` ``[B,H,topK]``,
    ``peaked``/``diffuse`` ``[B,H,n]`` and ``l3`` ``[B,H,n_diffuse,top_k]`` (level-3
    indices per diffuse block, in ``diffuse`` order) -- used to compare downstream stages
    of the GPU path without letting one near-tie cascade.

    Returns ``(x [B,S,H,D] in dtype, info)`` with every intermediate decision and score.
    """
    B, S, H, D = q.shape
    sz = derive_sizes(B, S, H, D, t_seq_len, SPARSITY_RATIO, srr, flat_ratio)
    decisions = {k_: v_.to(q.device) for k_, v_ in (decisions or {}).items() if v_ is not None}
    dev = q.device              # every intermediate follows the inputs' device
    qs, qc = pool_blocks(q, dtype)
    ks, kc = pool_blocks(k, dtype)
    vs, vc = pool_blocks(v, dtype)
    P, out_c = compressed_attention(qc, kc, vc)

    sel_ref, src_score = select_source_blocks(P, sz.n_t, sz.topK)
    sel = decisions.get("sel", sel_ref).long()
    tokmap = new_kv_token_map(t_seq_len, S, sel)
    new_k = gather_new_kv(k, tokmap, dtype)
    new_v = gather_new_kv(v, tokmap, dtype)

    peaked_ref, diffuse_ref, sharp = split_blocks(P, sz.n_t, sz.k_sparsity, sz.n_peaked)
    peaked = decisions.get("peaked", peaked_ref).long()
    diffuse = decisions.get("diffuse", diffuse_ref).long()

    NB = sz.NB
    qpad = F.pad(q.to(dtype), (0, 0, 0, 0, 0, NB * BLOCK_M - S)).permute(0, 2, 1, 3)
    qblk = qpad.reshape(B, H, NB, BLOCK_M, D)
    bi = torch.arange(B, device=dev).view(B, 1, 1)
    hi = torch.arange(H, device=dev).view(1, H, 1)
    out_blk = torch.zeros(B, H, NB, BLOCK_M, D, dtype=dtype, device=dev)

    l3 = None
    l3_scores = None
    if sz.n_diffuse > 0:
        q_diff = qblk[bi, hi, diffuse].reshape(B, H, sz.n_diffuse * BLOCK_M, D)
        pad = sz.TKV_pad - sz.Tkv
        nk = F.pad(new_k, (0, 0, 0, pad))
        nv = F.pad(new_v, (0, 0, 0, pad))
        o_sp, l3, l3_scores = sparse_piecewise_attn(
            q_diff, nk, nv, SPARSITY_RATIO, indices=decisions.get("l3"), dtype=dtype)
        out_blk[bi, hi, diffuse] = o_sp.view(B, H, sz.n_diffuse, BLOCK_M, D)
    if sz.n_peaked > 0:
        q_pk = qblk[bi, hi, peaked].reshape(B, H, sz.n_peaked * BLOCK_M, D)
        o_pk = dense_attention(q_pk, new_k, new_v)
        out_blk[bi, hi, peaked] = o_pk.view(B, H, sz.n_peaked, BLOCK_M, D)

    x = out_blk.view(B, H, NB * BLOCK_M, D).permute(0, 2, 1, 3)[:, :S]
    oc = out_c.repeat_interleave(BLOCK_M, dim=2).permute(0, 2, 1, 3)[:, :S]
    if isinstance(alpha_2, torch.Tensor):
        alpha_2 = alpha_2.to(dtype)
    x = x + oc * alpha_2
    info = dict(sizes=sz, P=P, out_c=out_c, sel=sel, sel_ref=sel_ref, src_score=src_score,
                tokmap=tokmap, sharpness=sharp, peaked=peaked, diffuse=diffuse,
                peaked_ref=peaked_ref, diffuse_ref=diffuse_ref, l3=l3, l3_scores=l3_scores,
                q_sums=qs, k_sums=ks, v_sums=vs)
    return x.contiguous(), info
