#!/usr/bin/env python3
"""Writes the golden fixtures of the in-context sparse attention path.

The reference holds no golden vectors, known-answer tests or fixtures for this path, so
the fixtures are produced by this repository's float64 CPU oracle (``oracle/``, itself
pinned by tests/test_oracle.py) on seeded synthetic inputs.  Inputs are not stored:
each fixture records the generator call (``icsa_hip.synthetic``) and
the SHA-256 of the generated bf16 bytes, so a changed generator is detected rather than
silently compared.  Run from the repository root:

    python tests/golden/make_golden.py

Fixtures
--------
``tiny_default.npz``    H=1, S=1024 (t=512), the reference's default parameters; full output.
``tiny_unaligned.npz``  H=1, S=1000 (t=500: t unaligned, partial last block), SAR 0.25; full
                        output.
``cfg1.npz``            configuration 1 (B=1, H=2, S=8192, D=128): every decision, the
                        scores they rank, a strided subsample of the output and per-block
                        output sums (a checksum of checksums).

Each fixture also stores the smallest score gap around every ranked decision, so a
consumer knows how far its arithmetic may drift before a decision legitimately flips.
"""
import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "lightning-unified-video-editor-via-in-context-sparse-attention_amd"))

import oracle as O  # noqa: E402
from icsa_hip.synthetic import make_inputs  # noqa: E402

SUBSAMPLE_STRIDE = 997

CASES = {
    "tiny_default": dict(gen=dict(H=1, real=512, pad=0, kind="random", seed=3),
                         params=dict(SPARSITY_RATIO=0.0625, srr=0.125, flat_ratio=0.5, alpha_2=0.7),
                         full=True),
    "tiny_unaligned": dict(gen=dict(H=1, real=500, pad=0, kind="random", seed=4),
                           params=dict(SPARSITY_RATIO=0.25, srr=0.125, flat_ratio=0.5, alpha_2=0.7),
                           full=True),
    "cfg1": dict(gen=dict(H=2, real=4096, pad=0, kind="random", seed=0),
                 params=dict(SPARSITY_RATIO=0.0625, srr=0.125, flat_ratio=0.5, alpha_2=1.0),
                 full=False),
}


def inputs_of(gen):
    q, k, v, t = make_inputs(**gen)
    h = hashlib.sha256()
    for x in (q, k, v):
        h.update(x.contiguous().view(torch.int16).numpy().tobytes())
    return q, k, v, t, h.hexdigest()


def kth_gap(scores, k):
    """Smallest gap between the k-th and (k+1)-th ranked score over all rows."""
    if k <= 0 or k >= scores.shape[-1]:
        return float("inf")
    s = torch.sort(scores, dim=-1, descending=True).values
    return float((s[..., k - 1] - s[..., k]).min())


def order_gap(scores, k):
    """Smallest gap between neighbours among the first k+1 ranked scores (ordered lists)."""
    s = torch.sort(scores, dim=-1, descending=True).values[..., :min(k + 1, scores.shape[-1])]
    if s.shape[-1] < 2:
        return float("inf")
    return float((s[..., :-1] - s[..., 1:]).min())


def run_case(spec):
    q, k, v, t, sha = inputs_of(spec["gen"])
    S = q.shape[1]
    p = spec["params"]
    x, info = O.editing_sparse_attention(q, k, v, t, S - t, **p)
    z = info["sizes"]
    D = q.shape[-1]
    l3_scores = info["l3_scores"] / (64.0 * 64.0 * D ** 0.5)   # compressed-logit units
    out = dict(
        meta=np.array(json.dumps(dict(gen=spec["gen"], params=p, sha256=sha, t=t, S=S,
                                      sizes=z.as_dict(), stride=SUBSAMPLE_STRIDE))),
        sel=info["sel"].numpy().astype(np.int32),
        peaked=torch.sort(info["peaked"], -1).values.numpy().astype(np.int32),
        diffuse_order=info["diffuse"].numpy().astype(np.int32),
        l3=info["l3"].numpy().astype(np.int32),
        src_score=info["src_score"].numpy(),
        sharpness=info["sharpness"].numpy(),
        l3_scores=l3_scores.numpy(),
        gaps=np.array([kth_gap(info["src_score"], z.topK), order_gap(info["src_score"], z.topK),
                       kth_gap(info["sharpness"], z.n_peaked), kth_gap(l3_scores, z.top_k)]),
        block_sums=x.view(1, -1, 64, x.shape[2], D).sum(dim=(2, 4)).numpy()
        if S % 64 == 0 else x.sum(dim=-1).numpy(),
        x_sub=x.reshape(-1)[::SUBSAMPLE_STRIDE].float().numpy(),
    )
    if spec["full"]:
        out["x"] = x.float().numpy()
        out["P"] = info["P"].float().numpy()
        out["out_c"] = info["out_c"].float().numpy()
    return out


def main():
    for name, spec in CASES.items():
        arrays = run_case(spec)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path} ({os.path.getsize(path)} bytes), min gaps {arrays['gaps'].tolist()}")


if __name__ == "__main__":
    main()
