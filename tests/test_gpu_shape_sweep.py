"""Seeded sweep over ragged shapes and mixed parameters of the fused pipeline.

The other pipeline tests pin one property each (unaligned t, partial last block, f32 v,
degenerate splits, a batch of two).  This sweep draws cases that combine them: source and
target lengths that are not multiples of 64 (zero padding inside the sequence), one to
three heads, batch one or two, and SAR / SRR / flat ratios across the ranges the reference's
configurations use, each checked against the oracle like every other pipeline case
(decisions valid within GAP, outputs within max-abs 2e-2 / mean-abs 1e-3).
"""
import random

import pytest
import torch

from icsa_hip.synthetic import make_inputs
from test_gpu_pipeline import _run_case

pytestmark = pytest.mark.gpu


def _cases(n=10, seed=20261202):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        out.append(dict(
            real=rng.randint(70, 2600),
            pad=rng.choice([0, 0, 8, 37]),
            H=rng.choice([1, 2, 3]),
            B=rng.choice([1, 1, 2]),
            sparsity=rng.choice([0.03125, 0.0625, 0.125, 0.25]),
            srr=rng.choice([0.0625, 0.125, 0.25]),
            flat=rng.choice([0.25, 0.5, 0.75]),
            alpha=round(rng.uniform(0.2, 1.5), 3),
            seed=100 + i,
        ))
    return out


CASES = _cases()


@pytest.mark.parametrize("c", CASES, ids=lambda c: "real{real}-pad{pad}-H{H}-B{B}-sar{sparsity}-srr{srr}-flat{flat}".format(**c))
def test_pipeline_shape_sweep(gpu, c):
    q, k, v, t = make_inputs(H=c["H"], real=c["real"], pad=c["pad"], B=c["B"], kind="random", seed=c["seed"])
    print(f"[case] sweep {c}", flush=True)
    _run_case(gpu, q, k, v, t, alpha=c["alpha"], sparsity=c["sparsity"], srr=c["srr"], flat_ratio=c["flat"])
