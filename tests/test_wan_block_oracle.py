"""CPU pinning of the Wan block oracle's composition (oracle/wan_block.py).

The block oracle composes pinned parts (glue oracle, path oracle, float64 textbook ops).
These checks fix the composition itself: with the adaLN gates e[2], e[5] zero and the cross
attention's output projection zero the block is the identity; with only the FFN branch
left, the update equals a direct float64 evaluation through torch.nn.functional."""
import pytest
import torch
import torch.nn.functional as F

from oracle import wan_block as WB
from oracle import wan_glue as W

pytestmark = pytest.mark.cpu


def _params(dim, ffn, seed):
    g = torch.Generator().manual_seed(seed)

    def r(*shape, s=0.05):
        return (torch.randn(*shape, generator=g) * s).to(torch.bfloat16).double()

    P = {"modulation": r(1, 6, dim, s=0.1)}
    for pre in ("self_attn", "cross_attn"):
        for n in ("q", "k", "v", "o"):
            P[f"{pre}.{n}.weight"] = r(dim, dim)
            P[f"{pre}.{n}.bias"] = r(dim, s=0.01)
        P[f"{pre}.alpha_1.weight"] = r(1, dim)
        P[f"{pre}.alpha_2.weight"] = torch.zeros(1, dim, dtype=torch.float64)   # unused, zero-init
        P[f"{pre}.norm_q.weight"] = 1 + r(dim, s=0.1)
        P[f"{pre}.norm_k.weight"] = 1 + r(dim, s=0.1)
    P["norm3.weight"] = 1 + r(dim, s=0.1)
    P["norm3.bias"] = r(dim, s=0.1)
    P["ffn.0.weight"] = r(ffn, dim)
    P["ffn.0.bias"] = r(ffn, s=0.01)
    P["ffn.2.weight"] = r(dim, ffn)
    P["ffn.2.bias"] = r(dim, s=0.01)
    return P


def _case(seed=0):
    dim, ffn, H = 256, 512, 2
    grid = (1, 8, 8)
    S = 128
    g = torch.Generator().manual_seed(seed + 100)
    x = torch.randn(1, S, dim, generator=g).double()
    e = (torch.randn(1, 6, dim, generator=g) * 0.1).double()
    ctx = torch.randn(1, 8, dim, generator=g).to(torch.bfloat16).double()
    return _params(dim, ffn, seed), x, e, ctx, grid, H


def test_block_identity_when_branches_are_gated_off():
    P, x, e, ctx, grid, H = _case(0)
    e[:, 2] = -P["modulation"][:, 2]            # e[2] = 0
    e[:, 5] = -P["modulation"][:, 5]            # e[5] = 0
    P["cross_attn.o.weight"].zero_()
    P["cross_attn.o.bias"].zero_()
    out, _ = WB.wan_block_forward(P, x, e, ctx, grid, grid, 1, W.wan_freqs(128), H)
    assert torch.equal(out, x)


def test_block_ffn_branch_matches_functional_evaluation():
    P, x, e, ctx, grid, H = _case(1)
    e[:, 2] = -P["modulation"][:, 2]
    P["cross_attn.o.weight"].zero_()
    P["cross_attn.o.bias"].zero_()
    out, _ = WB.wan_block_forward(P, x, e, ctx, grid, grid, 1, W.wan_freqs(128), H)
    em = (P["modulation"] + e).chunk(6, dim=1)
    h = F.layer_norm(x, (x.shape[-1],), eps=1e-6) * (1 + em[4]) + em[3]
    bf = lambda t: t.to(torch.bfloat16).double()
    f1 = bf(F.linear(bf(h), P["ffn.0.weight"], P["ffn.0.bias"]))
    y = bf(F.linear(bf(F.gelu(f1, approximate="tanh")), P["ffn.2.weight"], P["ffn.2.bias"]))
    assert torch.allclose(out, x + y * em[5], rtol=0, atol=1e-12)
