"""When the no-allocation entry point's static scratch takes device memory.

The 256 MiB `scratch` array of icsa_editing_sparse_attention_noalloc lives in api.hip, a
translation unit without kernels, so its code object is loaded onto a device only when the
entry point looks the array up (HIP's deferred code-object loading).  A process that only
uses the workspace entry points never holds it.  Measured in a fresh process, with device
free memory read around the calls.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PARENT = os.path.join(ROOT, "lightning-unified-video-editor-via-in-context-sparse-attention_amd")

PROBE = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
from icsa_hip import _lib
from icsa_hip.editing_sparse_attention import _editing_sparse_attention_hip
from icsa_hip.synthetic import make_inputs
dev = torch.device("cuda:0")
def free():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info(0)[0]
q, k, v, t = make_inputs(H=2, real=4096, pad=0, kind="random", seed=1, device=dev)
x, _ = _editing_sparse_attention_hip(q, k, v, t, 1.0)     # kernels loaded, workspace cached
f0 = free()
x, _ = _editing_sparse_attention_hip(q, k, v, t, 1.0)
f1 = free()
y, _ = _editing_sparse_attention_hip(q, k, v, t, 1.0, noalloc=True)
f2 = free()
print("DELTAS", f0 - f1, f1 - f2, int(torch.equal(x, y)), _lib.NOALLOC_SCRATCH_BYTES, flush=True)
"""


def test_scratch_taken_only_by_the_no_alloc_entry(gpu):
    print("[case] scratch residency in a fresh process", flush=True)
    env = dict(os.environ)
    env.pop("HIP_ENABLE_DEFERRED_LOADING", None)           # HIP's default: deferred
    res = subprocess.run([sys.executable, "-c", PROBE, PKG_PARENT], capture_output=True, text=True,
                         timeout=300, env=env)
    line = [l for l in res.stdout.splitlines() if l.startswith("DELTAS")]
    assert res.returncode == 0 and line, res.stdout[-2000:] + res.stderr[-2000:]
    ws_delta, na_delta, equal, scratch = (int(x) for x in line[0].split()[1:])
    print(f"workspace call: {ws_delta / 2**20:.1f} MiB, first no-alloc call: {na_delta / 2**20:.1f} MiB",
          flush=True)
    assert equal == 1
    assert ws_delta < scratch // 4, "a workspace-entry call took the no-alloc scratch's memory"
    assert na_delta >= scratch, "the first no-alloc call did not load the static scratch"
