"""GPU parity of the Wan q/k producer (icsa_wan_qk_prologue) and of the self-attention core
it feeds (icsa_editing_sparse_attention_presummed), both through the C ABI.

Producer: bf16 q / k must equal the oracle's float32 values rounded to bf16, except where
the two float32 computations straddle a bf16 rounding boundary (then within one bf16 ulp of
the rotated pair's modulus, and more than 99 % of the elements bit-equal);
block sums within 1e-4 relative; the gate exact up to one bf16 ulp of the sigmoid.
Attention core: decisions must be valid rankings of the oracle's float64 scores within GAP;
the output is compared with the oracle run on the GPU's own decisions (max-abs 2e-2,
mean-abs 1e-3), the reference's contract being fp32 q / k into editing_sparse_attention.
"""
import math

import pytest
import torch

import oracle as O
from oracle import wan_glue as W
from icsa_hip import wan
from icsa_hip.editing_sparse_attention import _editing_sparse_attention_hip
from parity import GAP, compare_out, gpu_decisions, l3_scale

pytestmark = pytest.mark.gpu


def _projections(B, S, dim, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    yq = (torch.randn(B, S, dim, generator=g) * 1.5 + 0.2).to(dtype)
    yk = (torch.randn(B, S, dim, generator=g) * 0.7 - 0.1).to(dtype)
    yv = torch.randn(B, S, dim, generator=g).to(torch.bfloat16)
    wq = torch.rand(dim, generator=g) + 0.5
    wk = torch.rand(dim, generator=g) + 0.5
    al = (torch.randn(B, S, 1, generator=g) * 2).to(dtype)
    return yq, yk, yv, wq, wk, al


def _check_bf16(gpu_bf16, ref32, name):
    """Rounding-boundary flips of bf16(y * r) move a rotated pair by one bf16 ulp of its
    inputs, so the bound scales with the pair modulus (which the rotation preserves), not
    with the element: a component that nearly cancels may be many of its own ulps off."""
    g = gpu_bf16.float().cpu()
    r = ref32.to(torch.bfloat16).float()
    diff = (g - r).abs()
    pair = ref32.float().view(*ref32.shape[:-1], -1, 2).pow(2).sum(-1).sqrt()
    pair = pair.repeat_interleave(2, dim=-1)
    bad = diff > pair * 2.0 ** -7 + 1e-30
    assert not bad.any(), f"{name}: {bad.sum().item()} elements more than one bf16 ulp off"
    frac = (diff == 0).float().mean().item()
    assert frac > 0.99, f"{name}: only {frac:.4f} of the elements are bit-equal"
    return frac


def _block_sums(x32, NB):
    B, S, H, D = x32.shape
    xp = torch.zeros(B, NB * 64, H, D, dtype=torch.float64)
    xp[:, :S] = x32.double()
    return xp.view(B, NB, 64, H, D).sum(2).permute(0, 2, 1, 3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_producer_matches_oracle(gpu, dtype):
    B, H, D = 2, 4, 128
    grids = [(3, 4, 8), (2, 4, 8)]
    srcs = [(3, 4, 8), (4, 4, 8)]
    S = 3 * 4 * 8 * 2 + 13                                  # 205: padding tokens, partial block
    print(f"[wan] producer B={B} S={S} H={H} dtype={dtype}", flush=True)
    yq, yk, yv, wq, wk, al = _projections(B, S, H * D, 0, dtype)
    freqs = W.wan_freqs(D)
    q, k, qs, ks, gate = wan.wan_qk_prologue(yq.to(gpu), yk.to(gpu), wq, wk, grids, srcs, 1, freqs,
                                             H, alpha_logit=al.to(gpu), eps=1e-6)
    torch.cuda.synchronize()
    qo, ko = W.wan_qk(yq, yk, wq, wk, 1e-6, grids, srcs, 1, freqs, H)
    fq = _check_bf16(q, qo, "q")
    fk = _check_bf16(k, ko, "k")
    NB = (S + 63) // 64
    for got, ref in ((qs, qo), (ks, ko)):
        assert torch.allclose(got.cpu().double(), _block_sums(ref, NB), rtol=1e-4, atol=1e-4)
    g_ref = W.alpha_gate(al.view(B, S).float())
    gd = (gate.cpu() - g_ref).abs()
    assert gd.max().item() <= 2.0 ** -10, gd.max().item()
    print(f"[wan] ok bit-equal q {fq:.4f} k {fk:.4f}", flush=True)


def test_producer_tag0_and_bad_arguments(gpu):
    B, H, D, S = 1, 2, 128, 130
    yq, yk, _, wq, wk, _ = _projections(B, S, H * D, 1)
    freqs = W.wan_freqs(D)
    q, k, _, _, gate = wan.wan_qk_prologue(yq.to(gpu), yk.to(gpu), wq, wk, [(2, 3, 10)], [(1, 2, 20)],
                                           0, freqs, H)
    assert gate is None
    qo, _ = W.wan_qk(yq, yk, wq, wk, 1e-6, [(2, 3, 10)], [(1, 2, 20)], 0, freqs, H)
    _check_bf16(q, qo, "q tag 0")
    from icsa_hip._lib import IcsaError
    with pytest.raises(IcsaError):                          # grid beyond the RoPE table
        wan.wan_qk_prologue(yq.to(gpu), yk.to(gpu), wq, wk, [(2000, 1, 1)], [(1, 1, 1)], 1, freqs, H)


def _attention_case(gpu, B, H, grid, src, pad, seed):
    D = 128
    S = math.prod(grid) + math.prod(src) + pad
    print(f"[wan] core B={B} S={S} H={H} grid={grid} src={src}", flush=True)
    yq, yk, yv, wq, wk, al = _projections(B, S, H * D, seed)
    freqs = W.wan_freqs(D)
    grids, srcs = [grid] * B, [src] * B
    q, k, qs, ks, gate = wan.wan_qk_prologue(yq.to(gpu), yk.to(gpu), wq, wk, grids, srcs, 1, freqs,
                                             H, alpha_logit=al.to(gpu))
    t = math.prod(grid)
    v = yv.to(gpu).view(B, S, H, D)
    x, views = _editing_sparse_attention_hip(q, k, v, t, gate.view(B, S, 1, 1), presummed=(qs, ks),
                                             out_dtype=torch.float32, keep_workspace=True)
    x2 = wan.wan_self_attention_core(yq.to(gpu), yk.to(gpu), yv.to(gpu), al.to(gpu), wq, wk, grids,
                                     srcs, 1, freqs, H)
    torch.cuda.synchronize()
    assert torch.equal(x, x2), "core entry differs from its two steps"
    dec = gpu_decisions(views)
    qo, ko = W.wan_qk(yq, yk, wq, wk, 1e-6, grids, srcs, 1, freqs, H)
    g_ref = W.alpha_gate(al.view(B, S).float()).view(B, S, 1, 1)
    xo, info = O.editing_sparse_attention(qo, ko, yv.view(B, S, H, D).float(), t, S - t,
                                          alpha_2=g_ref, decisions=dec)
    z = info["sizes"]
    if z.topK > 0:
        assert O.check_topk_valid(info["src_score"], dec["sel"], z.topK, GAP, ordered=True).all()
    if 0 < z.n_peaked < z.NB:
        assert O.check_split_valid(info["sharpness"], dec["peaked"], GAP).all()
    if z.n_diffuse > 0:
        ok = O.check_topk_valid(info["l3_scores"] / l3_scale(D), dec["l3"], z.top_k, GAP, ordered=False)
        assert ok.all(), f"{(~ok).sum().item()} exact lists not valid"
    mx, mn = compare_out(x, xo)
    print(f"[wan] ok max_abs={mx:.3e} mean_abs={mn:.3e}", flush=True)


def test_core_aligned(gpu):
    _attention_case(gpu, 1, 2, (2, 32, 32), (2, 32, 32), 0, 3)


def test_core_unaligned_with_padding(gpu):
    # t = 2025 (t % 64 != 0), 14 padding tokens after the source
    _attention_case(gpu, 1, 2, (3, 25, 27), (3, 25, 27), 14, 4)


def test_self_attention_module(gpu):
    torch.manual_seed(5)
    dim, heads = 256, 2
    m = wan.WanSelfAttention(dim, heads).to(gpu).to(torch.bfloat16)
    with torch.no_grad():
        m.alpha_1.weight.normal_(0, 0.05)
    grid = [(2, 16, 16)]
    S = 2 * 512
    x = torch.randn(1, S, dim, device=gpu).to(torch.bfloat16)
    freqs = W.wan_freqs(128)
    y = m(x, torch.tensor([S]), grid, grid, 1, freqs)
    with torch.no_grad():
        core = wan.wan_self_attention_core(m.q(x), m.k(x), m.v(x), m.alpha_1(x), m.norm_q.weight,
                                           m.norm_k.weight, grid, grid, 1, freqs, heads)
        y2 = m.o(core.flatten(2).to(torch.bfloat16))
    torch.cuda.synchronize()
    assert y.shape == (1, S, dim) and torch.isfinite(y.float()).all()
    assert torch.equal(y, y2)


def test_producer_full_size_sampled(gpu):
    """Configuration 4's producer call: 21x30x52 target + source grids, 65,520 tokens, H = 40.
    Sampled rows and blocks against the oracle (the whole oracle is too slow here)."""
    B, H, D = 1, 40, 128
    grid = (21, 30, 52)
    S = 2 * math.prod(grid)
    print(f"[wan] full-size producer S={S} H={H}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(9)
    yq = (torch.randn(B, S, H * D, device=gpu, generator=g) * 1.5).to(torch.bfloat16)
    yk = torch.randn(B, S, H * D, device=gpu, generator=g).to(torch.bfloat16)
    wq = torch.rand(H * D, device=gpu, generator=g) + 0.5
    wk = torch.rand(H * D, device=gpu, generator=g) + 0.5
    freqs = W.wan_freqs(D)
    q, k, qs, ks, _ = wan.wan_qk_prologue(yq, yk, wq, wk, [grid], [grid], 1, freqs, H)
    torch.cuda.synchronize()
    blocks = [0, 1, 255, 511, 512, 700, 1022, 1023]          # includes the target/source seam
    toks = torch.cat([torch.arange(64 * b, min(64 * b + 64, S)) for b in blocks])
    pos = W.token_positions(S, grid, grid, 1)[toks]
    for y, w, out, sums in ((yq, wq, q, qs), (yk, wk, k, ks)):
        rows = y[0, toks].cpu()
        m = W.rms_norm(rows, w.cpu(), 1e-6).to(torch.float32).view(len(toks), H, D)
        # rope for exactly these rows: put each row at its own position
        nf, nh, nw = W.rope_split(D)
        rot = torch.ones(len(toks), D // 2, dtype=torch.complex128)
        parts = torch.split(freqs, [nf, nh, nw], dim=1)
        col = 0
        for a, n_a in enumerate((nf, nh, nw)):
            rot[:, col:col + n_a] = parts[a][pos[:, a]]
            col += n_a
        mc = torch.view_as_complex(m.double().view(len(toks), H, D // 2, 2).contiguous())
        ref = torch.view_as_real(mc * rot[:, None, :]).reshape(len(toks), H, D).float()
        _check_bf16(out[0, toks], ref, "sampled rows")
        starts = [0]
        for b_ in blocks:
            starts.append(starts[-1] + min(64, S - 64 * b_))      # the last block is partial
        ref_sums = torch.stack([ref[starts[i]:starts[i + 1]].double().sum(0)
                                for i in range(len(blocks))], dim=1)        # [H, n_blocks, D]
        got = sums[0][:, blocks].cpu().double()
        assert torch.allclose(got, ref_sums, rtol=1e-4, atol=1e-3)
    print("[wan] ok full-size sampled rows", flush=True)
