"""HIP-graph capture of the fused path and of the sparse piecewise kernel.

The library allocates nothing and issues no memset or host synchronisation, so a call can
be captured by a caller's graph.  Each captured graph is replayed several times, with
eager calls and synchronisations between the replays, and every replay must equal the
eager result bit for bit (the kernels are deterministic).  A replay after new data is
copied into the captured inputs must equal an eager call on that data.
"""
import pytest
import torch

from icsa_hip import editing_sparse_attention, sparse_piecewise_attn_1st_intervals_hip
from icsa_hip.synthetic import make_inputs

pytestmark = pytest.mark.gpu


def _capture(fn):
    # one eager call on a side stream first (library set-up happens outside the capture)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _check_replays(g, out, eager, n=3):
    ref = eager()
    for r in range(n):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {r} differs from the eager result"
        other = eager()                      # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(other, ref)


def test_graph_editing_sparse_attention(gpu):
    print("[case] graph capture editing_sparse_attention H=2 S=4096", flush=True)
    q0, k0, v0, t = make_inputs(H=2, real=4096, pad=0, kind="random", seed=21)
    q, k, v = q0.to(gpu), k0.to(gpu), v0.to(gpu)
    s = q.shape[1] - t

    def call():
        return editing_sparse_attention(q, k, v, t, s, alpha_2=0.7, backend="hip")

    g, out = _capture(call)
    _check_replays(g, out, call)
    # new data in the captured inputs
    q1, k1, v1, _ = make_inputs(H=2, real=4096, pad=0, kind="random", seed=22)
    q.copy_(q1.to(gpu)); k.copy_(k1.to(gpu)); v.copy_(v1.to(gpu))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, call()), "replay on new inputs differs from the eager result"


def test_graph_sparse_piecewise(gpu):
    print("[case] graph capture sparse_piecewise_attn_1st_intervals_hip H=2 S=2048", flush=True)
    gen = torch.Generator().manual_seed(23)
    q, k, v = (torch.randn(1, 2, 2048, 128, generator=gen).to(torch.bfloat16).to(gpu) for _ in range(3))

    def call():
        return sparse_piecewise_attn_1st_intervals_hip(q, k, v, 0.0625, 64)

    g, out = _capture(call)
    _check_replays(g, out, call)
    k.copy_(torch.randn(1, 2, 2048, 128, generator=gen).to(torch.bfloat16).to(gpu))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, call()), "replay on new inputs differs from the eager result"


def test_graph_editing_noalloc(gpu):
    # The no-allocation entry point is meant for callers under graph capture: its first call
    # on a device (the scratch address lookup) happens eagerly in _capture, the captured
    # call then runs on the static scratch.  Replays must equal eager calls of both entry
    # points, also after new data is copied into the captured inputs.
    from icsa_hip.editing_sparse_attention import _editing_sparse_attention_hip
    print("[case] graph capture icsa_editing_sparse_attention_noalloc H=2 S=4096", flush=True)
    q0, k0, v0, t = make_inputs(H=2, real=2048, pad=0, kind="random", seed=24)
    q, k, v = q0.to(gpu), k0.to(gpu), v0.to(gpu)

    def call():
        return _editing_sparse_attention_hip(q, k, v, t, 0.7, noalloc=True)[0]

    def call_ws():
        return _editing_sparse_attention_hip(q, k, v, t, 0.7)[0]

    g, out = _capture(call)
    _check_replays(g, out, call)
    assert torch.equal(out, call_ws()), "no-alloc replay differs from the workspace entry point"
    q1, k1, v1, _ = make_inputs(H=2, real=2048, pad=0, kind="random", seed=25)
    q.copy_(q1.to(gpu)); k.copy_(k1.to(gpu)); v.copy_(v1.to(gpu))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, call_ws()), "replay on new inputs differs from the workspace entry point"
