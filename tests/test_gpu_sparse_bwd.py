"""GPU parity of the sparse-attention backward (icsa_sparse_piecewise_attn_fwd / _bwd and the
autograd Function) against oracle.sparse_bwd on the GPU's own forward state.

The backward takes the forward's saved out, lse and block lists, as the reference's
Function does (triton_kernels.py:541-598), so the oracle is evaluated on exactly those:
a near-tie in the forward's top-k cannot change the comparison.

Bar.  The kernels round P and dS to bf16 for the MFMA; the reference rounds P for dv and
uses fp32 dots for dq / dk.  A bf16 rounding moves a term by up to 2^-9 of its size, and a
gradient element sums top_k * 64 + NKV such terms of mixed sign, so the error is judged
against the gradient's own scale: max-abs <= 2e-2 * max|ref| and mean-abs <= 1e-2 *
mean|ref| for each of dq, dk, dv (float32 outputs; float64 oracle).  lse (log2 units,
fp32 sums of fp32 probabilities) must match within 2e-3.
"""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle as O
from oracle.sparse_bwd import sparse_piecewise_attn_bwd
from icsa_hip import (SparsePiecewiseAttn1stIntervalsFunction,
                      sparse_piecewise_attn_1st_intervals_bwd_hip,
                      sparse_piecewise_attn_1st_intervals_fwd_hip)
from parity import compare_out

pytestmark = pytest.mark.gpu


def _bf16(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _check_grad(name, got, ref):
    got = got.double().cpu()
    d = (got - ref).abs()
    mx, mn = d.max().item(), d.mean().item()
    rmax, rmean = ref.abs().max().item(), ref.abs().mean().item()
    print(f"[bwd] {name}: max_abs={mx:.3e} ({mx / rmax:.2e} of max|ref| {rmax:.3e}) "
          f"mean_abs={mn:.3e} ({mn / rmean:.2e} of mean|ref| {rmean:.3e})", flush=True)
    assert torch.isfinite(got).all(), name
    assert mx <= 2e-2 * rmax and mn <= 1e-2 * rmean, (name, mx, rmax, mn, rmean)


def _case(gpu, B, H, TQ, TKV, sparsity, seed):
    q, k, v = _bf16(B, H, TQ, 128, seed=seed), _bf16(B, H, TKV, 128, seed=seed + 1), \
        _bf16(B, H, TKV, 128, seed=seed + 2)
    do = _bf16(B, H, TQ, 128, seed=seed + 3)
    out, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q.to(gpu), k.to(gpu), v.to(gpu), sparsity)
    return q, k, v, do, out, lse, idx


@pytest.mark.parametrize("B,H,TQ,TKV,sparsity", [
    (1, 2, 512, 1024, 0.25), (2, 1, 1024, 4608, 0.0625), (1, 1, 4096, 36864, 0.0625),
    # ragged lengths of the Triton host: partial last query / key blocks
    (1, 2, 1024, 4608 + 37, 0.0625), (2, 1, 1000, 1111, 0.25), (1, 1, 4096 - 27, 36856, 0.0625),
    (1, 1, 40, 65, 1.0),
])
def test_backward_matches_oracle(gpu, B, H, TQ, TKV, sparsity):
    print(f"[case] bwd B={B} H={H} TQ={TQ} TKV={TKV} sparsity={sparsity}", flush=True)
    q, k, v, do, out, lse, idx = _case(gpu, B, H, TQ, TKV, sparsity, seed=20)
    # forward state: output and lse against the oracle on the same block lists
    ref_out, _, _, ref_lse = O.sparse_piecewise_attn(q, k, v, sparsity, indices=idx.long().cpu(),
                                                     return_lse=True, mode="triton")
    compare_out(out, ref_out)
    dl = (lse.double().cpu() - ref_lse).abs().max().item()
    print(f"[bwd] lse max_abs={dl:.3e}", flush=True)
    assert dl <= 2e-3
    dq, dk, dv = sparse_piecewise_attn_1st_intervals_bwd_hip(do.to(gpu), q.to(gpu), k.to(gpu), v.to(gpu),
                                                             out, lse, idx, grad_dtype=torch.float32)
    torch.cuda.synchronize()
    rq, rk, rv = sparse_piecewise_attn_bwd(do, q, k, v, out.cpu(), lse.cpu(), idx.long().cpu())
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    _check_grad("dq", dq, rq)
    _check_grad("dk", dk, rk)
    _check_grad("dv", dv, rv)


def test_autograd_function_ragged_lengths(gpu):
    # the autograd Function at Triton-host lengths: its gradients are those of the
    # backward entry on the forward's saved state, in the inputs' dtype
    q, k, v = (_bf16(1, 2, n, 128, seed=60 + i).to(gpu) for i, n in enumerate((1000, 1111, 1111)))
    do = _bf16(1, 2, 1000, 128, seed=63).to(gpu)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = SparsePiecewiseAttn1stIntervalsFunction.apply(qr, kr, vr, 0.25, 64)
    o.backward(do)
    out, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q, k, v, 0.25)
    assert torch.equal(o.detach(), out)
    want = sparse_piecewise_attn_1st_intervals_bwd_hip(do, q, k, v, out, lse, idx)
    for got, ref in zip((qr.grad, kr.grad, vr.grad), want):
        assert got.dtype == torch.bfloat16 and torch.equal(got, ref)


def test_backward_quirk_case(gpu):
    # a late interval chunk raises the running max: the saved lse is not the true
    # log-sum-exp, and the backward must use it as given
    TQ, TKV = 64, 64 * 192
    q = _bf16(1, 1, TQ, 128, seed=13)
    k = _bf16(1, 1, TKV, 128, seed=14, scale=0.2)
    k[0, 0, 64 * 150:64 * 151] = (20.0 * q[0, 0].float().mean(0)).expand(64, 128).to(torch.bfloat16)
    v = _bf16(1, 1, TKV, 128, seed=15)
    do = _bf16(1, 1, TQ, 128, seed=16)
    inj = torch.arange(12, dtype=torch.int32).view(1, 1, 1, 12)
    out, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q.to(gpu), k.to(gpu), v.to(gpu), 0.0625,
                                                                indices=inj.to(gpu))
    ref_out, _, _, ref_lse = O.sparse_piecewise_attn(q, k, v, 0.0625, indices=inj.long(), return_lse=True)
    compare_out(out, ref_out)
    assert (lse.double().cpu() - ref_lse).abs().max().item() <= 2e-3
    dq, dk, dv = sparse_piecewise_attn_1st_intervals_bwd_hip(do.to(gpu), q.to(gpu), k.to(gpu), v.to(gpu),
                                                             out, lse, idx, grad_dtype=torch.float32)
    rq, rk, rv = sparse_piecewise_attn_bwd(do, q, k, v, out.cpu(), lse.cpu(), idx.long().cpu())
    for name, got, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        _check_grad(name, got, ref)


def test_backward_all_selected_is_dense_gradient(gpu):
    # top_k = NKV: no interval part; the gradient of dense attention (float64 SDPA)
    q, k, v = _bf16(1, 2, 256, 128, seed=40), _bf16(1, 2, 512, 128, seed=41), _bf16(1, 2, 512, 128, seed=42)
    do = _bf16(1, 2, 256, 128, seed=43)
    out, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q.to(gpu), k.to(gpu), v.to(gpu), 1.0)
    assert idx.shape[-1] == 8
    dq, dk, dv = sparse_piecewise_attn_1st_intervals_bwd_hip(do.to(gpu), q.to(gpu), k.to(gpu), v.to(gpu),
                                                             out, lse, idx, grad_dtype=torch.float32)
    qr, kr, vr = (t.double().requires_grad_(True) for t in (q, k, v))
    o = F.scaled_dot_product_attention(qr, kr, vr)
    (o * do.double()).sum().backward()
    _check_grad("dq", dq, qr.grad)
    _check_grad("dk", dk, kr.grad)
    _check_grad("dv", dv, vr.grad)


def test_backward_is_deterministic(gpu):
    q, k, v, do, out, lse, idx = _case(gpu, 1, 4, 1024, 8192, 0.0625, seed=50)
    args = (do.to(gpu), q.to(gpu), k.to(gpu), v.to(gpu), out, lse, idx)
    a = sparse_piecewise_attn_1st_intervals_bwd_hip(*args, grad_dtype=torch.float32)
    b = sparse_piecewise_attn_1st_intervals_bwd_hip(*args, grad_dtype=torch.float32)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_autograd_function(gpu):
    q, k, v = (_bf16(1, 2, 512, 128, seed=60 + i).to(gpu) for i in range(3))
    k = torch.cat([k, _bf16(1, 2, 1536, 128, seed=63).to(gpu)], dim=2)
    v = torch.cat([v, _bf16(1, 2, 1536, 128, seed=64).to(gpu)], dim=2)
    do = _bf16(1, 2, 512, 128, seed=65).to(gpu)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = SparsePiecewiseAttn1stIntervalsFunction.apply(qr, kr, vr, 0.125, 64)
    out.backward(do)
    o2, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q, k, v, 0.125)
    assert torch.equal(out.detach(), o2)
    dq, dk, dv = sparse_piecewise_attn_1st_intervals_bwd_hip(do, q, k, v, o2, lse, idx)
    assert qr.grad.dtype == torch.bfloat16
    assert torch.equal(qr.grad, dq) and torch.equal(kr.grad, dk) and torch.equal(vr.grad, dv)


def test_backward_bad_arguments(gpu):
    from icsa_hip.hip_host import IcsaArgumentError
    q = _bf16(1, 1, 128, 128).to(gpu)
    out, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q, q, q, 0.5)
    with pytest.raises(IcsaArgumentError):
        sparse_piecewise_attn_1st_intervals_bwd_hip(q, q, q, q, out, lse.double(), idx)
    with pytest.raises(IcsaArgumentError):
        sparse_piecewise_attn_1st_intervals_bwd_hip(q, q, q, q, out, lse, idx[:, :, :1])
