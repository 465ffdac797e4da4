"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored decision and output (a regression pin of
the oracle itself).  GPU: the HIP path reproduces the stored decisions exactly (every
fixture's score gaps exceed the decision bar, which the test asserts first) and the
stored outputs within the output bar.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import oracle as O
from icsa_hip.synthetic import make_inputs
from parity import GAP, MAX_ABS, MEAN_ABS

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ["tiny_default", "tiny_unaligned", "cfg1"]


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as f:
        fx = {k: f[k] for k in f.files}
    fx["meta"] = json.loads(str(fx["meta"]))
    return fx


def regenerate(fx):
    q, k, v, t = make_inputs(**fx["meta"]["gen"])
    h = hashlib.sha256()
    for x in (q, k, v):
        h.update(x.contiguous().view(torch.int16).numpy().tobytes())
    assert h.hexdigest() == fx["meta"]["sha256"], "synthetic input generator changed"
    assert t == fx["meta"]["t"]
    return q, k, v, t


def l3_by_block(diffuse_order, l3):
    """{(b, h, block): sorted exact-block list} from lists stored in diffuse order."""
    out = {}
    B, H, n = diffuse_order.shape
    for b in range(B):
        for h in range(H):
            for i in range(n):
                out[(b, h, int(diffuse_order[b, h, i]))] = sorted(int(x) for x in l3[b, h, i])
    return out


@pytest.mark.cpu
@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_golden(name):
    fx = load(name)
    q, k, v, t = regenerate(fx)
    p = fx["meta"]["params"]
    x, info = O.editing_sparse_attention(q, k, v, t, q.shape[1] - t, **p)
    assert np.array_equal(info["sel"].numpy(), fx["sel"])
    assert np.array_equal(torch.sort(info["peaked"], -1).values.numpy(), fx["peaked"])
    assert np.array_equal(info["diffuse"].numpy(), fx["diffuse_order"])
    assert np.array_equal(info["l3"].numpy(), fx["l3"])
    assert np.allclose(info["src_score"].numpy(), fx["src_score"], rtol=1e-12, atol=1e-15)
    assert np.allclose(info["sharpness"].numpy(), fx["sharpness"], rtol=1e-12, atol=1e-15)
    stride = fx["meta"]["stride"]
    assert np.allclose(x.reshape(-1)[::stride].numpy(), fx["x_sub"], rtol=1e-6, atol=1e-6)
    if "x" in fx:
        assert np.allclose(x.numpy(), fx["x"], rtol=1e-6, atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_reproduces_golden(gpu, name):
    from icsa_hip.editing_sparse_attention import _editing_sparse_attention_hip
    fx = load(name)
    assert (fx["gaps"] > GAP).all(), "fixture has near-ties; decisions would not be pinned"
    q, k, v, t = regenerate(fx)
    p = fx["meta"]["params"]
    print(f"[golden] {name} S={q.shape[1]} H={q.shape[2]} t={t} params={p}", flush=True)
    x, views = _editing_sparse_attention_hip(q.to(gpu), k.to(gpu), v.to(gpu), t, p["alpha_2"],
                                             p["SPARSITY_RATIO"], p["srr"], p["flat_ratio"],
                                             keep_workspace=True)
    torch.cuda.synchronize()
    z = views["sizes"]
    order = views["order"].long().cpu().numpy()
    assert np.array_equal(views["sel"].cpu().numpy(), fx["sel"])
    assert np.array_equal(np.sort(order[..., :z["n_peaked"]], -1), fx["peaked"])
    got = l3_by_block(order[..., z["n_peaked"]:], views["l3"].cpu().numpy())
    assert got == l3_by_block(fx["diffuse_order"], fx["l3"])
    xs = x.reshape(-1)[::fx["meta"]["stride"]].double().cpu().numpy()
    d = np.abs(xs - fx["x_sub"])
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (d.max(), d.mean())
    if "x" in fx:
        d = np.abs(x.double().cpu().numpy() - fx["x"])
        assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (d.max(), d.mean())
        P = views["P"].cpu().numpy()
        assert np.allclose(P, fx["P"], rtol=1e-4, atol=1e-7)
    print(f"[golden] {name} ok", flush=True)
