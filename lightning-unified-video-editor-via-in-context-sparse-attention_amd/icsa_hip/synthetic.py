"""Seeded synthetic inputs of the benchmark configurations (no datasets, no checkpoints).

Sequence layout is ``[target | source]`` (model.py:425 of the reference), each part
``real`` tokens followed by ``pad`` zero tokens.

* ``random``     : Q ~ N(0,1); source K/V ~ N(0,1); target K/V = source K/V + 0.3 N(0,1)
                   (configs 1 and 2).
* ``structured`` : K/V token (f, p) = 0.6 F_f + 0.4 P_p + 0.2 N(0,1) with per-frame F_f and
                   per-position P_p ~ N(0,1) [D] (21 frames x 1560 positions for 32,760
                   tokens); target = source + 0.3 N(0,1); Q built the same way from an
                   independent generator stream (config 3).

Values are produced in float32, then rounded to ``dtype``; the same rounded values go to
the GPU and to the CPU oracle.
"""
from __future__ import annotations

import torch


def _normal(shape, gen, device):
    return torch.randn(*shape, generator=gen, device=device, dtype=torch.float32)


def _structured_part(frames, positions, H, D, gen, device):
    F = _normal((frames, 1, H, D), gen, device)
    P = _normal((1, positions, H, D), gen, device)
    x = 0.6 * F + 0.4 * P + 0.2 * _normal((frames, positions, H, D), gen, device)
    return x.reshape(frames * positions, H, D)


def make_inputs(H: int, real: int, pad: int = 0, D: int = 128, B: int = 1, kind: str = "random",
                seed: int = 0, device="cpu", dtype=torch.bfloat16, frames: int = 21):
    """Returns ``(q, k, v, t_seq_len)`` with q/k/v ``[B, 2*(real+pad), H, D]``."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    part = real + pad
    S = 2 * part
    qs, ks, vs = [], [], []
    for _ in range(B):
        if kind == "random":
            q_real = [_normal((real, H, D), gen, device), _normal((real, H, D), gen, device)]
            k_src = _normal((real, H, D), gen, device)
            v_src = _normal((real, H, D), gen, device)
        elif kind == "structured":
            assert real % frames == 0, "structured inputs need real % frames == 0"
            pos = real // frames
            k_src = _structured_part(frames, pos, H, D, gen, device)
            v_src = _structured_part(frames, pos, H, D, gen, device)
            q_real = [_structured_part(frames, pos, H, D, gen, device),
                      _structured_part(frames, pos, H, D, gen, device)]
        else:
            raise ValueError(f"unknown kind {kind!r}")
        k_tgt = k_src + 0.3 * _normal((real, H, D), gen, device)
        v_tgt = v_src + 0.3 * _normal((real, H, D), gen, device)
        z = torch.zeros(pad, H, D, device=device)
        qs.append(torch.cat([q_real[0], z, q_real[1], z]))
        ks.append(torch.cat([k_tgt, z, k_src, z]))
        vs.append(torch.cat([v_tgt, z, v_src, z]))
    q = torch.stack(qs).to(dtype)
    k = torch.stack(ks).to(dtype)
    v = torch.stack(vs).to(dtype)
    assert q.shape == (B, S, H, D)
    return q, k, v, part


CONFIGS = {
    # CPU oracle case (t = s = 4096)
    1: dict(H=2, real=4096, pad=0, kind="random"),
    # Wan 2.2 14B self-attention shape, 32,760 + 8 pad per part (65,536 tokens)
    2: dict(H=40, real=32760, pad=8, kind="random"),
    # structured scores, 21 frames x 1560 tokens per part
    3: dict(H=40, real=32760, pad=8, kind="structured"),
    # the DiT block's attention call, 65,520 unpadded tokens (t = 32,760,
    # t % 64 != 0 and a partial last block)
    4: dict(H=40, real=32760, pad=0, kind="random"),
}


def config_inputs(cfg: int, device="cpu", dtype=torch.bfloat16, seed: int = 0, H: int = None):
    c = dict(CONFIGS[cfg])
    if H is not None:
        c["H"] = H
    return make_inputs(c["H"], c["real"], c["pad"], kind=c["kind"], seed=seed, device=device,
                       dtype=dtype)
