"""The Triton host's contract on the GPU (triton_host.py:11-30 -> triton_kernels.py:489-539).

The reference's Triton branch hands the sparse kernel the unpadded new KV
(editing_sparse_attention.py:203-207), ragged whenever t % 64 != 0 -- TKV = 36,856 in the
DiT block of configuration 4.  ``sparse_piecewise_attn_1st_intervals`` takes such lengths:
floor top_k over TKV // 64, cdiv(TKV, 64) candidate blocks, keys past TKV masked out of the
exact part.  Checked against the oracle's ``mode="triton"`` (float64, run on the GPU as the
checker) on the GPU's own block lists, whose validity against the float64 block scores is
checked first.
"""
import pytest
import torch

import oracle as O
from icsa_hip import (sparse_piecewise_attn_1st_intervals, sparse_piecewise_attn_1st_intervals_fwd_hip,
                      sparse_piecewise_attn_1st_intervals_hip)
from icsa_hip.hip_host import triton_top_k
from parity import GAP, compare_out, l3_scale

pytestmark = pytest.mark.gpu


def _inputs(B, H, TQ, TKV, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, H, TQ, 128, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, H, TKV, 128, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, H, TKV, 128, generator=g, device=dev).to(torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("B,H,TQ,TKV,sp", [
    (1, 2, 1024, 4608 + 37, 0.0625),      # partial last candidate block, two interval chunks
    (2, 1, 1000, 1111, 0.25),             # ragged TQ as well
    (1, 40, 32768, 36856, 0.0625),        # the Triton branch at configuration 4 (top_k 35)
])
def test_triton_host_matches_oracle(gpu, B, H, TQ, TKV, sp):
    print(f"[triton] B={B} H={H} TQ={TQ} TKV={TKV} sparsity={sp}", flush=True)
    q, k, v = _inputs(B, H, TQ, TKV, seed=TKV, dev=gpu)
    out, lse, idx = sparse_piecewise_attn_1st_intervals_fwd_hip(q, k, v, sp)
    out2 = sparse_piecewise_attn_1st_intervals(q, k, v, sp)
    torch.cuda.synchronize()
    top_k = triton_top_k(sp, TKV)
    assert idx.shape == (B, H, (TQ + 63) // 64, top_k)
    assert torch.equal(out, out2)
    # the GPU's block lists against the float64 block scores
    _, _, scores = O.sparse_piecewise_attn(q[..., :64, :].double(), k.double(), v.double(), sp, mode="triton")
    qs = torch.nn.functional.pad(q.double(), (0, 0, 0, idx.shape[2] * 64 - TQ))
    qc = qs.view(B, H, -1, 64, 128).sum(3)
    kc = torch.nn.functional.pad(k.double(), (0, 0, 0, (TKV + 63) // 64 * 64 - TKV)).view(B, H, -1, 64, 128).sum(3)
    sc = torch.matmul(qc, kc.transpose(-1, -2).contiguous())
    assert torch.allclose(sc[:, :, :1], scores, rtol=1e-12, atol=1e-9)
    assert O.check_topk_valid(sc / l3_scale(128), idx, top_k, GAP, ordered=False).all()
    ref, _, _, ref_lse = O.sparse_piecewise_attn(q.double(), k.double(), v.double(), sp, indices=idx,
                                                 return_lse=True, mode="triton")
    mx, mn = compare_out(out, ref)
    assert torch.allclose(lse.double(), ref_lse, rtol=0, atol=2e-3)
    print(f"[triton] max_abs={mx:.3e} mean_abs={mn:.3e}", flush=True)


def test_triton_host_equals_tilelang_host_for_aligned_lengths(gpu):
    q, k, v = _inputs(1, 3, 2048, 4608, seed=5, dev=gpu)
    a = sparse_piecewise_attn_1st_intervals(q, k, v, 0.0625)
    b = sparse_piecewise_attn_1st_intervals_hip(q, k, v, 0.0625)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_tilelang_host_keeps_its_asserts(gpu):
    q, k, v = _inputs(1, 1, 128, 4608 + 37, seed=6, dev=gpu)
    with pytest.raises(AssertionError, match="divisible"):
        sparse_piecewise_attn_1st_intervals_hip(q, k, v, 0.0625)
