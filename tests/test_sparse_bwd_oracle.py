"""CPU pinning of the sparse-attention backward oracle (oracle/sparse_bwd.py) and of the
forward oracle's lse output.

Checks other than the oracle's own formulas:
* virtual-key attention: with one interval chunk (NKV <= 64) the forward is exactly softmax
  attention over the selected blocks' rows plus, per unselected block c, one key KC_c / 64
  of multiplicity 64 (logit bias ln 64) with value VC_c / 64.  That attention is built here
  from masks over the full key set and differentiated by torch.autograd; the oracle's
  forward (out, lse) and backward must match it.  With ragged TQ / TKV (the Triton host) the
  key set holds only the real rows and KC_c / VC_c sum the real rows of block c;
* top_k = NKV: dense attention, gradient of float64 scaled_dot_product_attention;
* lse in log2 units: shifting lse by delta scales every gradient by 2^-delta;
* brute-force scalar loops (D = 4) of the backward formulas.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import icsa_oracle as O
from oracle.sparse_bwd import sparse_piecewise_attn_bwd

pytestmark = pytest.mark.cpu
BM = 64


def _inputs(B, H, TQ, TKV, D, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, TQ, D, generator=g, dtype=torch.float64)
    k = torch.randn(B, H, TKV, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, TKV, D, generator=g, dtype=torch.float64)
    do = torch.randn(B, H, TQ, D, generator=g, dtype=torch.float64)
    return q, k, v, do


def _random_indices(B, H, NQ, NKV, top_k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(NKV, generator=g)[:top_k]
                        for _ in range(B * H * NQ)]).view(B, H, NQ, top_k)


def virtual_attention(q, k, v, idx):
    """Softmax attention over the virtual keys, from masks over [k rows ; KC / 64]."""
    B, H, TQ, D = q.shape
    TKV = k.shape[2]
    NQ, NKV = -(-TQ // BM), -(-TKV // BM)
    pad = (0, 0, 0, NKV * BM - TKV)
    KC = F.pad(k, pad).view(B, H, NKV, BM, D).sum(3)
    VC = F.pad(v, pad).view(B, H, NKV, BM, D).sum(3)
    keys = torch.cat([k, KC / BM], dim=2)
    vals = torch.cat([v, VC / BM], dim=2)
    sel = torch.zeros(B, H, NQ, NKV, dtype=torch.bool)
    sel.scatter_(-1, idx.long(), True)
    sel_q = sel.repeat_interleave(BM, dim=2)[:, :, :TQ]                # [B,H,TQ,NKV]
    allow = torch.cat([sel_q.repeat_interleave(BM, dim=3)[..., :TKV], ~sel_q], dim=3)
    bias = torch.cat([torch.zeros(TKV, dtype=q.dtype), torch.full((NKV,), math.log(BM), dtype=q.dtype)])
    logits = torch.matmul(q, keys.transpose(-2, -1)) / math.sqrt(D) + bias
    logits = logits.masked_fill(~allow, -math.inf)
    o = torch.matmul(torch.softmax(logits, -1), vals)
    lse = torch.logsumexp(logits, -1) / math.log(2.0)
    return o, lse


@pytest.mark.parametrize("NKV,top_k", [(5, 2), (12, 3)])
def test_backward_is_virtual_attention_gradient(NKV, top_k):
    B, H, NQ, D = 1, 2, 3, 16
    q, k, v, do = _inputs(B, H, NQ * BM, NKV * BM, D, seed=NKV)
    idx = _random_indices(B, H, NQ, NKV, top_k, seed=7)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    o, lse = virtual_attention(qr, kr, vr, idx)
    (o * do).sum().backward()
    # the forward oracle (one interval chunk: no late max growth) is the same function
    out_f, _, _, lse_f = O.sparse_piecewise_attn(q, k, v, sparsity=(top_k + 0.5) / NKV,
                                                 indices=idx, return_lse=True)
    assert torch.allclose(out_f, o.detach(), atol=1e-12, rtol=1e-10)
    assert torch.allclose(lse_f, lse.detach(), atol=1e-12, rtol=1e-10)
    dq, dk, dv = sparse_piecewise_attn_bwd(do, q, k, v, o.detach(), lse.detach(), idx)
    for got, ref, name in ((dq, qr.grad, "dq"), (dk, kr.grad, "dk"), (dv, vr.grad, "dv")):
        assert torch.allclose(got, ref, atol=1e-11, rtol=1e-9), (name, (got - ref).abs().max().item())


@pytest.mark.parametrize("TQ,TKV,top_k", [(3 * BM - 17, 5 * BM - 27, 2), (BM + 1, 7 * BM + 1, 3),
                                           (40, 2 * BM, 1)])
def test_ragged_backward_is_virtual_attention_gradient(TQ, TKV, top_k):
    # Triton-host lengths: the last query block and the last key block are partial
    B, H, D = 1, 2, 16
    NQ, NKV = -(-TQ // BM), -(-TKV // BM)
    q, k, v, do = _inputs(B, H, TQ, TKV, D, seed=TQ + TKV)
    idx = _random_indices(B, H, NQ, NKV, top_k, seed=9)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    o, lse = virtual_attention(qr, kr, vr, idx)
    (o * do).sum().backward()
    out_f, _, _, lse_f = O.sparse_piecewise_attn(q, k, v, sparsity=(top_k + 0.5) / (TKV // BM),
                                                 indices=idx, return_lse=True, mode="triton")
    assert torch.allclose(out_f, o.detach(), atol=1e-12, rtol=1e-10)
    assert torch.allclose(lse_f, lse.detach(), atol=1e-12, rtol=1e-10)
    dq, dk, dv = sparse_piecewise_attn_bwd(do, q, k, v, o.detach(), lse.detach(), idx)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    for got, ref, name in ((dq, qr.grad, "dq"), (dk, kr.grad, "dk"), (dv, vr.grad, "dv")):
        assert torch.allclose(got, ref, atol=1e-11, rtol=1e-9), (name, (got - ref).abs().max().item())


def test_ragged_backward_equals_zero_padded_aligned_case():
    # rows past TKV that are zero keys of a selected block still take part in the aligned
    # case, so only a selection without the last block makes the two agree; the aligned
    # gradients of the real rows must then equal the ragged ones
    B, H, D, TQ, TKV = 1, 1, 8, 2 * BM - 5, 3 * BM - 10
    q, k, v, do = _inputs(B, H, TQ, TKV, D, seed=4)
    idx = torch.tensor([[[[0], [1]]]])
    g = torch.Generator().manual_seed(6)
    o = torch.randn(B, H, TQ, D, generator=g, dtype=torch.float64)
    lse = torch.randn(B, H, TQ, generator=g, dtype=torch.float64) + 3.0
    rag = sparse_piecewise_attn_bwd(do, q, k, v, o, lse, idx)
    pq = lambda t: F.pad(t, (0, 0, 0, 2 * BM - TQ))
    pk = lambda t: F.pad(t, (0, 0, 0, 3 * BM - TKV))
    al = sparse_piecewise_attn_bwd(pq(do), pq(q), pk(k), pk(v), pq(o), F.pad(lse, (0, 2 * BM - TQ)), idx)
    for a, r, n in zip(al, rag, (TQ, TKV, TKV)):
        assert torch.allclose(a[:, :, :n], r, atol=1e-12, rtol=1e-10)
    assert torch.count_nonzero(al[0][:, :, TQ:]) == 0      # zero query rows: no gradient


def test_backward_all_selected_is_dense_gradient():
    B, H, NQ, NKV, D = 1, 2, 2, 3, 32
    q, k, v, do = _inputs(B, H, NQ * BM, NKV * BM, D, seed=3)
    idx = torch.arange(NKV).view(1, 1, 1, NKV).expand(B, H, NQ, NKV).contiguous()
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = F.scaled_dot_product_attention(qr, kr, vr)
    (o * do).sum().backward()
    lse = torch.logsumexp(torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(D), -1) / math.log(2.0)
    dq, dk, dv = sparse_piecewise_attn_bwd(do, q, k, v, o.detach(), lse, idx)
    for got, ref in ((dq, qr.grad), (dk, kr.grad), (dv, vr.grad)):
        assert torch.allclose(got, ref, atol=1e-11, rtol=1e-9), (got - ref).abs().max().item()


def test_lse_shift_scales_gradients_by_power_of_two():
    B, H, NQ, NKV, D = 1, 1, 2, 70, 16            # two interval chunks
    q, k, v, do = _inputs(B, H, NQ * BM, NKV * BM, D, seed=5)
    out, idx, _, lse = O.sparse_piecewise_attn(q, k, v, sparsity=0.05, return_lse=True)
    g0 = sparse_piecewise_attn_bwd(do, q, k, v, out, lse, idx)
    g1 = sparse_piecewise_attn_bwd(do, q, k, v, out, lse + 1.5, idx)
    for a, b in zip(g0, g1):
        assert torch.allclose(b, a * 2.0 ** -1.5, atol=1e-12, rtol=1e-10)


def test_backward_bruteforce_loops():
    B, H, NQ, NKV, D, top_k = 1, 1, 2, 3, 4, 1
    TQ, TKV = NQ * BM, NKV * BM
    q, k, v, do = _inputs(B, H, TQ, TKV, D, seed=11)
    idx = torch.tensor([[[[2], [0]]]])
    g = torch.Generator().manual_seed(2)
    o = torch.randn(B, H, TQ, D, generator=g, dtype=torch.float64)       # any saved o / lse
    lse = torch.randn(B, H, TQ, generator=g, dtype=torch.float64) + 3.0
    dq, dk, dv = sparse_piecewise_attn_bwd(do, q, k, v, o, lse, idx)
    sc = 1.0 / math.sqrt(D)
    qq, kk, vv, dd, oo, ll = (t[0, 0].tolist() for t in (q, k, v, do, o, lse))
    KC = [[sum(kk[c * BM + r][d] for r in range(BM)) for d in range(D)] for c in range(NKV)]
    VC = [[sum(vv[c * BM + r][d] for r in range(BM)) for d in range(D)] for c in range(NKV)]
    rdq = [[0.0] * D for _ in range(TQ)]
    rdk = [[0.0] * D for _ in range(TKV)]
    rdv = [[0.0] * D for _ in range(TKV)]
    dot = lambda a, b: sum(x * y for x, y in zip(a, b))
    for i in range(TQ):
        qb = i // BM
        sel = {int(j) for j in idx[0, 0, qb]}
        Di = dot(dd[i], oo[i])
        for c in range(NKV):
            if c in sel:
                for r in range(BM):
                    j = c * BM + r
                    p = 2.0 ** (dot(qq[i], kk[j]) * sc / math.log(2.0) - ll[i])
                    ds = p * (dot(dd[i], vv[j]) - Di)
                    for d in range(D):
                        rdq[i][d] += ds * kk[j][d] * sc
                        rdk[j][d] += ds * qq[i][d] * sc
                        rdv[j][d] += p * dd[i][d]
            else:
                p = 2.0 ** (dot(qq[i], KC[c]) * sc / BM / math.log(2.0) - ll[i])
                ds = p * (dot(dd[i], VC[c]) - BM * Di)
                for d in range(D):
                    rdq[i][d] += ds * KC[c][d] * sc / BM
                for r in range(BM):
                    j = c * BM + r
                    for d in range(D):
                        rdk[j][d] += ds * qq[i][d] * sc / BM
                        rdv[j][d] += p * dd[i][d]
    for got, ref in ((dq, rdq), (dk, rdk), (dv, rdv)):
        ref = torch.tensor(ref, dtype=torch.float64)
        assert torch.allclose(got[0, 0], ref, atol=1e-10, rtol=1e-9), (got[0, 0] - ref).abs().max().item()
