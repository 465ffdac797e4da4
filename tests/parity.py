"""Comparison helpers shared by the parity tests (tolerances of the north-star bar)."""
import math

import torch

# Attention output bar: bf16 GPU vs fp32-or-better oracle.
MAX_ABS = 2e-2
MEAN_ABS = 1e-3
# Decision bar: ranked choices must be exact wherever the oracle's score gap exceeds this
# (scores in compressed-logit / probability units).
GAP = 1e-6


def compare_out(gpu_out: torch.Tensor, ref: torch.Tensor, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    d = (gpu_out.double().cpu() - ref.double().cpu()).abs()
    assert torch.isfinite(gpu_out.double().cpu()).all(), "non-finite GPU output"
    mx, mn = d.max().item(), d.mean().item()
    assert mx <= max_abs and mn <= mean_abs, f"max_abs {mx:.3e} (bar {max_abs}), mean_abs {mn:.3e} (bar {mean_abs})"
    return mx, mn


def l3_scale(D: int) -> float:
    """Level-3 scores are products of 64-token block sums; dividing by 64*64*sqrt(D) puts
    them in compressed-logit units, where the GAP bar applies."""
    return 64.0 * 64.0 * math.sqrt(D)


def gpu_decisions(views: dict) -> dict:
    z = views["sizes"]
    order = views["order"].long().cpu()
    return dict(sel=views["sel"].long().cpu(), peaked=order[..., :z["n_peaked"]],
                diffuse=order[..., z["n_peaked"]:], l3=views["l3"].long().cpu())
