"""icsa_editing_sparse_attention_noalloc against icsa_editing_sparse_attention.

The no-allocation entry point runs the same kernels on the library's static device scratch
instead of a caller workspace, so its output must equal the workspace entry point's bit for
bit.  Two calls in a row on one device share the scratch; the second is smaller and must not
be disturbed by what the first left behind.
"""
import pytest
import torch

from icsa_hip import _lib
from icsa_hip.editing_sparse_attention import _editing_sparse_attention_hip, derived_sizes
from icsa_hip.synthetic import make_inputs
from parity import compare_out

pytestmark = pytest.mark.gpu

CASES = [
    # configuration 2's shape for one GPU's share of the heads (H = 5 of 40 on 8 GPUs)
    dict(inp=dict(H=5, real=32760, pad=8, kind="random", seed=3), sar=0.0625, flat=0.5),
    # smaller, unaligned t with a partial last block, fp32 q / k as the DiT passes them
    dict(inp=dict(H=2, real=4000, pad=0, kind="structured", seed=4, frames=8), sar=0.125, flat=0.25,
         qk_f32=True),
]


def test_noalloc_matches_workspace_entry_point(gpu):
    for i, c in enumerate(CASES):
        q, k, v, t = make_inputs(**c["inp"], device=gpu)
        if c.get("qk_f32"):
            q, k = q.float(), k.float()
        B, S, H, D = q.shape
        need = _lib.lib().icsa_editing_workspace_size(B, S, H, D, t, c["sar"], 0.125, c["flat"],
                                                      0 if q.dtype == torch.bfloat16 else 1,
                                                      0 if k.dtype == torch.bfloat16 else 1,
                                                      0 if v.dtype == torch.bfloat16 else 1)
        print(f"[noalloc] call {i}: B={B} S={S} H={H} t={t} workspace {need / 2**20:.1f} MiB "
              f"of {_lib.NOALLOC_SCRATCH_BYTES / 2**20:.0f} MiB", flush=True)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES
        g = torch.Generator(device=gpu).manual_seed(20 + i)
        alpha = (torch.rand(B, S, 1, 1, device=gpu, generator=g) - 0.5) * 0.5
        x_ws, _ = _editing_sparse_attention_hip(q, k, v, t, alpha, c["sar"], 0.125, c["flat"])
        x_na, _ = _editing_sparse_attention_hip(q, k, v, t, alpha, c["sar"], 0.125, c["flat"],
                                                noalloc=True)
        torch.cuda.synchronize()
        assert torch.isfinite(x_na.float()).all()
        compare_out(x_na, x_ws)
        assert torch.equal(x_na, x_ws), "the no-allocation entry point differs from the workspace one"


def test_noalloc_rejects_oversized_calls(gpu):
    q, k, v, t = make_inputs(H=40, real=32760, pad=8, kind="random", seed=0, device=gpu)
    z = derived_sizes(1, q.shape[1], 40, 128, t)
    assert z["NB"] == 1024
    with pytest.raises(_lib.IcsaError, match="static scratch"):
        _editing_sparse_attention_hip(q, k, v, t, 1.0, noalloc=True)
