"""CPU pinning of the Wan model oracle's own parts (oracle/wan_model.py): the patch embedding
against torch's Conv3d, unpatchify against an explicit index loop, and the whole forward
with every block's output projections zeroed against head(patch embedding)."""
import pytest
import torch
import torch.nn.functional as F

from oracle import wan_glue as W
from oracle import wan_model as WM
from oracle.wan_block import bf, layer_norm

pytestmark = pytest.mark.cpu

CFG = dict(patch_size=(1, 2, 2), dim=256, num_heads=2, num_layers=2, freq_dim=32, text_len=16,
           out_dim=4, eps=1e-6, in_dim=4, ffn_dim=512, text_dim=64)


def model_params(seed, zero_branches=False):
    g = torch.Generator().manual_seed(seed)

    def r(*shape, s=0.05):
        return (torch.randn(*shape, generator=g) * s).to(torch.bfloat16).double()

    d, c = CFG["dim"], CFG["in_dim"]
    P = {"patch_embedding.weight": r(d, c, 1, 2, 2, s=0.2), "patch_embedding.bias": r(d, s=0.02),
         "source_video_embedding_more_memory.weight": r(d, c, 1, 2, 2, s=0.2),
         "source_video_embedding_more_memory.bias": r(d, s=0.02),
         "text_embedding.0.weight": r(d, CFG["text_dim"]), "text_embedding.0.bias": r(d, s=0.01),
         "text_embedding.2.weight": r(d, d), "text_embedding.2.bias": r(d, s=0.01),
         "time_embedding.0.weight": r(d, CFG["freq_dim"]), "time_embedding.0.bias": r(d, s=0.01),
         "time_embedding.2.weight": r(d, d), "time_embedding.2.bias": r(d, s=0.01),
         "time_projection.1.weight": r(6 * d, d), "time_projection.1.bias": r(6 * d, s=0.01),
         "head.modulation": r(1, 2, d, s=0.1), "head.head.weight": r(CFG["out_dim"] * 4, d, s=0.2),
         "head.head.bias": r(CFG["out_dim"] * 4, s=0.01)}
    from test_wan_block_oracle import _params
    for i in range(CFG["num_layers"]):
        for k, v in _params(d, CFG["ffn_dim"], seed + 10 + i).items():
            P[f"blocks.{i}.{k}"] = v
        if zero_branches:
            for k in ("self_attn.o", "cross_attn.o", "ffn.2"):
                P[f"blocks.{i}.{k}.weight"].zero_()
                P[f"blocks.{i}.{k}.bias"].zero_()
    return P


def test_patch_embed_matches_conv3d():
    g = torch.Generator().manual_seed(0)
    u = torch.randn(4, 2, 8, 6, generator=g).to(torch.bfloat16).double()
    w = torch.randn(16, 4, 1, 2, 2, generator=g).to(torch.bfloat16).double()
    b = torch.randn(16, generator=g).to(torch.bfloat16).double()
    emb, grid = WM.patch_embed(u, w, b, (1, 2, 2))
    ref = F.conv3d(u[None], w, b, stride=(1, 2, 2))[0]            # [16, 2, 4, 3]
    assert grid == (2, 4, 3)
    assert torch.equal(emb, bf(ref.flatten(1).T))


def test_unpatchify_index_loop():
    grid, patch, c = (2, 3, 2), (1, 2, 2), 3
    x = torch.randn(12, c * 4)
    out = WM.unpatchify(x, grid, patch, c)
    for f in range(2):
        for h in range(3):
            for w in range(2):
                tok = (f * 3 + h) * 2 + w
                for q in range(2):
                    for r in range(2):
                        for ch in range(c):
                            assert out[ch, f, 2 * h + q, 2 * w + r] == x[tok, ((0 * 2 + q) * 2 + r) * c + ch]


def test_model_with_silent_blocks_is_head_of_patch_embedding():
    P = model_params(0, zero_branches=True)
    g = torch.Generator().manual_seed(1)
    lat = torch.randn(4, 2, 16, 16, generator=g).to(torch.bfloat16)
    src = torch.randn(4, 2, 16, 16, generator=g).to(torch.bfloat16)
    ctx = [torch.randn(10, CFG["text_dim"], generator=g).to(torch.bfloat16)]
    t = torch.tensor([500.0])
    S = 2 * 2 * 8 * 8
    out = WM.wan_model_forward(P, CFG, [lat], t, ctx, S, [src], W.wan_freqs(128))[0]
    emb, grid = WM.patch_embed(lat, P["patch_embedding.weight"], P["patch_embedding.bias"], (1, 2, 2))
    temb = WM.sinusoidal_embedding_1d(CFG["freq_dim"], t)
    e = F.linear(F.silu(F.linear(temb, P["time_embedding.0.weight"], P["time_embedding.0.bias"])),
                 P["time_embedding.2.weight"], P["time_embedding.2.bias"])
    em = (P["head.modulation"] + e.unsqueeze(1)).chunk(2, dim=1)
    hd = F.linear(layer_norm(emb[None], 1e-6) * (1 + em[1]) + em[0], P["head.head.weight"],
                  P["head.head.bias"])[0]
    ref = WM.unpatchify(hd, grid, (1, 2, 2), CFG["out_dim"])
    assert torch.allclose(out, ref, rtol=0, atol=1e-12)
