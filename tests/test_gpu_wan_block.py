"""GPU parity of the Wan DiT block on the HIP backend (icsa_hip.wan).

* ``ln_modulate`` (icsa_wan_ln_modulate) against float64 LayerNorm / adaLN / residual.
* ``WanAttentionBlock`` end to end against oracle.wan_block on the GPU's own self-attention
  decisions.  Bar: the block output is the float32 residual stream of O(1) values after five
  bf16 GEMM stages; the oracle rounds at the same points but accumulates in float64, so a
  bf16 rounding flip in a GEMM output may propagate.  Tolerance: max-abs 3e-2 and mean-abs
  3e-3 (about 4 and 0.4 bf16 ulps of the typical |x| ~ 1).
"""
import math

import pytest
import torch

from oracle import wan_block as WB
from oracle import wan_glue as W
from icsa_hip import wan
from parity import gpu_decisions
from test_wan_block_oracle import _params

pytestmark = pytest.mark.gpu


def test_ln_modulate_matches_float64(gpu):
    torch.manual_seed(0)
    B, S, dim = 2, 37, 5120
    x = torch.randn(B, S, dim, device=gpu) * 2 + 0.5
    y = torch.randn(B, S, dim, device=gpu).to(torch.bfloat16)
    gate = torch.randn(B, 1, dim, device=gpu) * 0.3
    shift = torch.randn(B, 1, dim, device=gpu) * 0.2
    scale = torch.randn(B, 1, dim, device=gpu) * 0.2
    w = torch.rand(dim, device=gpu) + 0.5
    bb = torch.randn(dim, device=gpu) * 0.1
    x64 = x.double().cpu()
    xu = x64 + y.double().cpu() * gate.double().cpu()
    out = wan.ln_modulate(x, shift=shift, scale=scale, weight=w, bias=bb, y=y, gate=gate)
    torch.cuda.synchronize()
    assert torch.allclose(x.double().cpu(), xu, rtol=1e-6, atol=1e-6), "residual update"
    mean = xu.mean(-1, keepdim=True)
    ln = (xu - mean) / torch.sqrt((xu - mean).pow(2).mean(-1, keepdim=True) + 1e-6)
    ref = (ln * w.double().cpu() + bb.double().cpu()) * (1 + scale.double().cpu()) + shift.double().cpu()
    d = (out.double().cpu() - ref).abs()
    assert (d <= ref.abs() * 2.0 ** -8 + 1e-6).all(), d.max().item()
    # update only, and a plain LayerNorm + modulation of a bf16 x (rounded after the norm)
    xb = torch.randn(B, S, dim, device=gpu).to(torch.bfloat16)
    o2 = wan.ln_modulate(xb, shift=shift, scale=scale)
    xb64 = xb.double().cpu()
    m = xb64.mean(-1, keepdim=True)
    n = ((xb64 - m) / torch.sqrt((xb64 - m).pow(2).mean(-1, keepdim=True) + 1e-6))
    ref2 = n.to(torch.bfloat16).double() * (1 + scale.double().cpu()) + shift.double().cpu()
    d2 = (o2.double().cpu() - ref2).abs()
    # two roundings: a flip of bf16(n) moves the result by one ulp of n times (1 + scale)
    bound = (n.abs() * (1 + scale.double().cpu()).abs() + ref2.abs()) * 2.0 ** -7 + 1e-6
    assert (d2 <= bound).all(), d2.max().item()
    # a bf16 x updated into a separate f32 stream: x is kept, x + y * gate is f32, and the
    # LayerNorm of the updated row is not rounded to bf16 (type promotion in the reference)
    xb_before = xb.clone()
    xs = torch.empty(B, S, dim, device=gpu)
    o3 = wan.ln_modulate(xb, shift=shift, scale=scale, weight=w, bias=bb, y=y, gate=gate, x_out=xs)
    torch.cuda.synchronize()
    assert torch.equal(xb, xb_before), "x must be left unchanged when x_out is given"
    xu3 = xb64 + y.double().cpu() * gate.double().cpu()
    assert torch.allclose(xs.double().cpu(), xu3, rtol=1e-6, atol=1e-6), "update into x_out"
    m3 = xu3.mean(-1, keepdim=True)
    ln3 = (xu3 - m3) / torch.sqrt((xu3 - m3).pow(2).mean(-1, keepdim=True) + 1e-6)
    ref3 = (ln3 * w.double().cpu() + bb.double().cpu()) * (1 + scale.double().cpu()) + shift.double().cpu()
    d3 = (o3.double().cpu() - ref3).abs()
    assert (d3 <= ref3.abs() * 2.0 ** -8 + 1e-6).all(), d3.max().item()


def test_block_matches_oracle(gpu):
    dim, ffn, H = 256, 512, 2
    grid = (2, 16, 16)
    S = 2 * math.prod(grid)
    print(f"[block] dim={dim} ffn={ffn} H={H} S={S}", flush=True)
    P = _params(dim, ffn, 3)
    blk = wan.WanAttentionBlock("t2v_cross_attn", dim, ffn, H, cross_attn_norm=True)
    blk.load_state_dict({k: v.float() for k, v in P.items()}, strict=True)
    blk = blk.to(gpu).to(torch.bfloat16)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, S, dim, generator=g)
    e = torch.randn(1, 6, dim, generator=g) * 0.1
    ctx = torch.randn(1, 24, dim, generator=g).to(torch.bfloat16)
    freqs = W.wan_freqs(128)
    blk.self_attn.capture = {}
    out = blk(x.to(gpu), e.to(gpu), torch.tensor([S]), [grid], freqs, ctx.to(gpu), None, [grid], 1)
    torch.cuda.synchronize()
    dec = gpu_decisions(blk.self_attn.capture["views"])
    blk.self_attn.capture = None
    Pb = {k: v.detach().cpu() for k, v in blk.state_dict().items()}    # the bf16 values used
    ref, _ = WB.wan_block_forward(Pb, x, e, ctx, grid, grid, 1, freqs, H, decisions=dec)
    d = (out.double().cpu() - ref).abs()
    mx, mn = d.max().item(), d.mean().item()
    print(f"[block] max_abs={mx:.3e} mean_abs={mn:.3e} |x|max={ref.abs().max().item():.2f}", flush=True)
    assert torch.isfinite(out).all()
    assert mx <= 3e-2 and mn <= 3e-3, (mx, mn)


def _params_full(dim, ffn, seed, device):
    """Block parameters at full width: xavier-uniform Linear weights (the reference's
    init_weights, model.py:395-408), small random biases, modulation ~ N(0, 1/dim)."""
    g = torch.Generator(device=device).manual_seed(seed)

    def xavier(o, i):
        a = math.sqrt(6.0 / (i + o))
        return ((torch.rand(o, i, generator=g, device=device) * 2 - 1) * a).to(torch.bfloat16)

    def rn(*shape, s):
        return (torch.randn(*shape, generator=g, device=device) * s).to(torch.bfloat16)

    P = {"modulation": (torch.randn(1, 6, dim, generator=g, device=device) / math.sqrt(dim))}
    for pre in ("self_attn", "cross_attn"):
        for n in ("q", "k", "v", "o"):
            P[f"{pre}.{n}.weight"] = xavier(dim, dim)
            P[f"{pre}.{n}.bias"] = rn(dim, s=0.01)
        P[f"{pre}.alpha_1.weight"] = xavier(1, dim)
        P[f"{pre}.alpha_2.weight"] = torch.zeros(1, dim, device=device)
        P[f"{pre}.norm_q.weight"] = 1 + rn(dim, s=0.1).float()
        P[f"{pre}.norm_k.weight"] = 1 + rn(dim, s=0.1).float()
    P["norm3.weight"] = 1 + rn(dim, s=0.1).float()
    P["norm3.bias"] = rn(dim, s=0.1).float()
    P["ffn.0.weight"] = xavier(ffn, dim)
    P["ffn.0.bias"] = rn(ffn, s=0.01)
    P["ffn.2.weight"] = xavier(dim, ffn)
    P["ffn.2.bias"] = rn(dim, s=0.01)
    return P


def test_block_full_width_cfg4(gpu):
    """Configuration 4 at its real width: dim 5120, 40 heads, FFN 13,824, 21x30x52 target and
    source grids (65,520 tokens, t % 64 != 0), 512 text tokens.  The oracle runs the whole
    block in float64 on the GPU on the block's own self-attention decisions."""
    dim, ffn, H = 5120, 13824, 40
    grid = (21, 30, 52)
    S = 2 * math.prod(grid)
    print(f"[block-cfg4] dim={dim} ffn={ffn} H={H} S={S}", flush=True)
    P = _params_full(dim, ffn, 5, gpu)
    blk = wan.WanAttentionBlock("t2v_cross_attn", dim, ffn, H, cross_attn_norm=True)
    blk.load_state_dict({k: v.float().cpu() for k, v in P.items()}, strict=True)
    blk = blk.to(gpu).to(torch.bfloat16)
    g = torch.Generator(device=gpu).manual_seed(12)
    x = torch.randn(1, S, dim, generator=g, device=gpu)
    e = torch.randn(1, 6, dim, generator=g, device=gpu) * 0.1
    ctx = torch.randn(1, 512, dim, generator=g, device=gpu).to(torch.bfloat16)
    freqs = W.wan_freqs(128)
    blk.self_attn.capture = {}
    out = blk(x.clone(), e, torch.tensor([S]), [grid], freqs, ctx, None, [grid], 1)
    torch.cuda.synchronize()
    dec = gpu_decisions(blk.self_attn.capture["views"])
    blk.self_attn.capture = None
    Pb = {k: v.detach() for k, v in blk.state_dict().items()}          # the bf16 values used
    print("[block-cfg4] HIP block done; float64 oracle on the GPU", flush=True)
    ref, info = WB.wan_block_forward(Pb, x, e, ctx, grid, grid, 1, freqs, H, decisions=dec, device=gpu)
    torch.cuda.synchronize()
    d = (out.double() - ref).abs()
    mx, mn = d.max().item(), d.mean().item()
    print(f"[block-cfg4] max_abs={mx:.3e} mean_abs={mn:.3e} |x|max={ref.abs().max().item():.2f}",
          flush=True)
    assert torch.isfinite(out).all()
    assert mx <= 3e-2 and mn <= 3e-3, (mx, mn)


def test_block_full_width_cfg5(gpu):
    """Configuration 5's block at full width for one video of the CFG pair: dim 5120, 40
    heads, FFN 13,824, 21x45x80 target and source grids (151,200 tokens: NB = 2,363,
    NKV = 1,329, top_k = 83), 512 text tokens.  Float64 oracle on the GPU, the block's own
    self-attention decisions."""
    dim, ffn, H = 5120, 13824, 40
    grid = (21, 45, 80)
    S = 2 * math.prod(grid)
    print(f"[block-cfg5] dim={dim} ffn={ffn} H={H} S={S}", flush=True)
    P = _params_full(dim, ffn, 6, gpu)
    blk = wan.WanAttentionBlock("t2v_cross_attn", dim, ffn, H, cross_attn_norm=True)
    blk.load_state_dict({k: v.float().cpu() for k, v in P.items()}, strict=True)
    blk = blk.to(gpu).to(torch.bfloat16)
    del P
    g = torch.Generator(device=gpu).manual_seed(13)
    x = torch.randn(1, S, dim, generator=g, device=gpu)
    e = torch.randn(1, 6, dim, generator=g, device=gpu) * 0.1
    ctx = torch.randn(1, 512, dim, generator=g, device=gpu).to(torch.bfloat16)
    freqs = W.wan_freqs(128)
    blk.self_attn.capture = {}
    out = blk(x.clone(), e, torch.tensor([S]), [grid], freqs, ctx, None, [grid], 1)
    torch.cuda.synchronize()
    dec = gpu_decisions(blk.self_attn.capture["views"])
    blk.self_attn.capture = None
    Pb = {k: v.detach() for k, v in blk.state_dict().items()}
    del blk
    torch.cuda.empty_cache()
    print("[block-cfg5] HIP block done; float64 oracle on the GPU", flush=True)
    ref, info = WB.wan_block_forward(Pb, x, e, ctx, grid, grid, 1, freqs, H, decisions=dec, device=gpu)
    torch.cuda.synchronize()
    d = (out.double() - ref).abs()
    mx, mn = d.max().item(), d.mean().item()
    print(f"[block-cfg5] max_abs={mx:.3e} mean_abs={mn:.3e} |x|max={ref.abs().max().item():.2f}",
          flush=True)
    assert torch.isfinite(out).all()
    assert mx <= 3e-2 and mn <= 3e-3, (mx, mn)
