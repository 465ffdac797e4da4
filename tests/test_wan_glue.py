"""CPU pinning of the Wan glue oracle (RMSNorm, 3D RoPE, alpha gate; oracle/wan_glue.py).

Each check fixes the oracle by something other than its own formula: closed forms at chosen
points, a scalar brute-force loop that evaluates cos / sin of the reference's angle formula
per element, and invariants of rotations and of RMS normalisation.
"""
import math

import pytest
import torch

from oracle import wan_glue as W

pytestmark = pytest.mark.cpu


def test_rope_params_closed_form():
    f = W.rope_params(16, 44)
    assert f.shape == (16, 22)
    assert torch.allclose(f.abs(), torch.ones(16, 22, dtype=torch.float64), atol=1e-15)
    assert torch.all(f[0] == 1)
    ang = 5 * 10000.0 ** (-6.0 / 44)          # pos 5, pair 3
    assert abs(f[5, 3].real.item() - math.cos(ang)) < 1e-15
    assert abs(f[5, 3].imag.item() - math.sin(ang)) < 1e-15


def test_wan_freqs_split_matches_parts():
    assert W.rope_split(128) == (22, 21, 21)
    f = W.wan_freqs(128, 32)
    assert f.shape == (32, 64)
    assert torch.equal(f[:, :22], W.rope_params(32, 44))
    assert torch.equal(f[:, 22:43], W.rope_params(32, 42))
    assert torch.equal(f[:, 43:], W.rope_params(32, 42))


def _brute_rope(x, grid, src, tag, head_dim):
    """Scalar loops: angle of pair j = pos_axis(j) * 10000^(-2 j' / dim_axis)."""
    B, S, H, D = x.shape
    c = D // 2
    nf, nh, nw = c - 2 * (c // 3), c // 3, c // 3
    dims = (D - 4 * (D // 6), 2 * (D // 6), 2 * (D // 6))
    out = torch.empty(B, S, H, D, dtype=torch.float64)
    for b in range(B):
        f, h, w = grid[b]
        sf, sh, sw = src[b]
        for p in range(S):
            if p < f * h * w:
                pos = (p // (h * w), (p // w) % h, p % w)
            elif tag == 1 and p < f * h * w + sf * sh * sw:
                r = p - f * h * w
                pos = (r // (sh * sw), (r // sw) % sh, r % sw)
            else:
                pos = None
            for hh in range(H):
                for j in range(c):
                    a, jj = (0, j) if j < nf else ((1, j - nf) if j < nf + nh else (2, j - nf - nh))
                    x0, x1 = float(x[b, p, hh, 2 * j]), float(x[b, p, hh, 2 * j + 1])
                    if pos is None:
                        cs, sn = 1.0, 0.0
                    else:
                        ang = pos[a] * 10000.0 ** (-2.0 * jj / dims[a])
                        cs, sn = math.cos(ang), math.sin(ang)
                    out[b, p, hh, 2 * j] = x0 * cs - x1 * sn
                    out[b, p, hh, 2 * j + 1] = x0 * sn + x1 * cs
    return out


def test_rope_apply_bruteforce_and_invariants():
    torch.manual_seed(0)
    D = 12
    grid = [(2, 3, 2), (1, 2, 3)]
    src = [(1, 2, 2), (2, 1, 2)]
    S = 19                                   # 12 + 4 tokens, then 3 padding tokens (batch 0)
    x = torch.randn(2, S, 2, D)
    freqs = W.wan_freqs(D, 8)
    y = W.rope_apply(x, grid, src, 1, freqs)
    ref = _brute_rope(x, grid, src, 1, D)
    assert (y.double() - ref).abs().max() < 1e-5
    # every pair keeps its modulus
    m0 = x.view(2, S, 2, D // 2, 2).double().pow(2).sum(-1)
    m1 = y.view(2, S, 2, D // 2, 2).double().pow(2).sum(-1)
    assert torch.allclose(m0, m1, rtol=1e-5, atol=1e-6)
    # token (0, 0, 0), the first source token (TAG == 1) and padding are not rotated
    assert torch.equal(y[0, 0], x[0, 0])
    assert torch.equal(y[0, 12], x[0, 12])
    assert torch.equal(y[0, 16:], x[0, 16:])
    # TAG == 0: source tokens are not rotated either
    y0 = W.rope_apply(x, grid, src, 0, freqs)
    assert torch.equal(y0[0, 12:], x[0, 12:])


def test_rope_relative_position_property():
    torch.manual_seed(1)
    D = 128
    grid = [(4, 5, 6)]
    S = 120
    freqs = W.wan_freqs(D, 16)
    q = torch.randn(1, 1, 1, D).expand(1, S, 1, D).contiguous()
    k = torch.randn(1, 1, 1, D).expand(1, S, 1, D).contiguous()
    rq = W.rope_apply(q, grid, [(0, 0, 0)], 1, freqs).double()
    rk = W.rope_apply(k, grid, [(0, 0, 0)], 1, freqs).double()

    def tok(f, h, w):
        return f * 30 + h * 6 + w

    d1 = (rq[0, tok(1, 2, 3), 0] * rk[0, tok(0, 1, 1), 0]).sum()
    d2 = (rq[0, tok(3, 4, 5), 0] * rk[0, tok(2, 3, 3), 0]).sum()     # same offsets (1, 1, 2)
    d3 = (rq[0, tok(3, 4, 5), 0] * rk[0, tok(2, 3, 2), 0]).sum()     # offset (1, 1, 3)
    assert abs(d1 - d2) < 1e-4
    assert abs(d1 - d3) > 1e-3


def test_rms_norm_invariants():
    torch.manual_seed(2)
    y = torch.randn(3, 7, 512) * 4
    w1 = torch.ones(512)
    n = W.rms_norm(y, w1, 0.0, round_to=None)
    assert torch.allclose(n.pow(2).mean(-1), torch.ones(3, 7, dtype=torch.float64), atol=1e-12)
    assert torch.allclose(W.rms_norm(3.7 * y, w1, 0.0, round_to=None), n, atol=1e-12)
    w = torch.rand(512) + 0.5
    nb = W.rms_norm(y, w, 1e-6)
    base = (nb / w.double())
    assert torch.equal(base.to(torch.bfloat16).double(), base)       # bf16 values times w


def test_alpha_gate_closed_form():
    g = W.alpha_gate(torch.tensor([0.0, 1.0, 40.0, -40.0]))
    # sigmoid(1) = 0.7310586 -> bf16 0.73046875; - 0.5 = 0.23046875 (exact); * 0.5
    assert g.tolist() == [0.0, 0.115234375, 0.25, -0.25]


def test_package_rope_table_matches_oracle():
    from icsa_hip import wan
    assert torch.allclose(wan.wan_freqs(128), W.wan_freqs(128), rtol=0, atol=1e-12)

