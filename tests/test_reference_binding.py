"""The reference-side binding of the HIP backend, exercised on the CPU.

The integration guide gives three code blocks that a maintainer pastes into the
reference's ``in_context_sparse_attention/editing_sparse_attention.py`` (imports, the
``Backend`` selector, the ``backend == 'hip'`` dispatch).  This test assembles a stub
reference package from exactly those blocks -- the rest of the module is a freshly written
stand-in whose non-HIP branch returns a marker -- imports it the way the DiT does
(model.py:16), and checks that:

* the module imports without flash-attn, TileLang or Triton kernels (the optional imports);
* ``Backend.validate('hip')`` passes and unknown names still raise ``ValueError``;
* ``backend='hip'`` reaches the HIP path of ``icsa_hip`` with the caller's arguments
  (model.py:173-174 passes ``alpha_2=alpha_1, backend=self.backend``), monkeypatched so no
  GPU is needed;
* the default backend (``'tilelang'``) still takes the reference's own branch.
"""
import os
import re
import sys
import textwrap

import pytest
import torch

pytestmark = pytest.mark.cpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = os.path.join(ROOT, "INTEGRATION.md")


def _patch_block(name: str) -> str:
    text = open(GUIDE).read()
    m = re.search(r"<!-- patch:%s -->\s*```python\n(.*?)```" % re.escape(name), text, re.S)
    assert m, f"patch block {name!r} not found in the integration guide"
    return m.group(1)


def _write_stub_package(root) -> None:
    pkg = root / "in_context_sparse_attention"
    pkg.mkdir()
    (pkg / "__init__.py").write_text(textwrap.dedent("""\
        from .editing_sparse_attention import (
            Backend,
            editing_sparse_attention,
            editing_sparse_attention_tilelang,
        )
        """))
    body = textwrap.dedent('''\
        BLOCK_M = 64


        def editing_sparse_attention(q, k, v, t_seq_len, s_seq_len, alpha_2=1.0, alpha_3=1.0,
                                     SPARSITY_RATIO=0.0625, backend=Backend.TILELANG):
            backend = Backend.validate(backend)
        ''')
    module = (_patch_block("imports") + "\n\n" + _patch_block("backend") + "\n\n" + body
              + _patch_block("dispatch")
              + "    return ('reference branch', backend)\n\n\n"
              + "editing_sparse_attention_tilelang = editing_sparse_attention\n")
    (pkg / "editing_sparse_attention.py").write_text(module)


@pytest.fixture
def stub_reference(tmp_path, monkeypatch):
    _write_stub_package(tmp_path)
    monkeypatch.syspath_prepend(str(tmp_path))
    for name in [m for m in sys.modules if m.split(".")[0] == "in_context_sparse_attention"]:
        monkeypatch.delitem(sys.modules, name)
    import in_context_sparse_attention as ref   # model.py:16
    yield ref
    for name in [m for m in sys.modules if m.split(".")[0] == "in_context_sparse_attention"]:
        del sys.modules[name]


def test_patched_module_imports_and_selector_accepts_hip(stub_reference):
    ref = stub_reference
    esa = sys.modules["in_context_sparse_attention.editing_sparse_attention"]
    import icsa_hip
    assert esa.icsa_hip is icsa_hip
    # nothing CUDA-only is needed to import the patched module
    assert esa._sparse_attn_triton is None and esa.sparse_piecewise_attn_1st_intervals_tilelang is None
    assert ref.Backend.validate("hip") == "hip"
    assert ref.Backend.validate("tilelang") == "tilelang" and ref.Backend.validate("triton") == "triton"
    with pytest.raises(ValueError):
        ref.Backend.validate("cuda")


def test_hip_backend_dispatches_to_icsa_hip(stub_reference, monkeypatch):
    ref = stub_reference
    hip_mod = sys.modules["icsa_hip.editing_sparse_attention"]
    calls = []
    sentinel = torch.full((1, 128, 2, 128), 7.0)

    def fake_hip_path(q, k, v, t_seq_len, alpha_2=1.0, SPARSITY_RATIO=0.0625, srr=0.125,
                      flat_ratio=0.5, **kw):
        calls.append(dict(q=q, k=k, v=v, t=t_seq_len, alpha_2=alpha_2, sar=SPARSITY_RATIO,
                          srr=srr, flat=flat_ratio))
        return sentinel, None

    monkeypatch.setattr(hip_mod, "_editing_sparse_attention_hip", fake_hip_path)
    q = torch.zeros(1, 128, 2, 128)
    k, v = torch.ones_like(q), torch.full_like(q, 2.0)
    alpha_1 = torch.rand(1, 128, 1, 1)
    # the DiT's call (model.py:173-174)
    x = ref.editing_sparse_attention(q, k, v, 64, 64, alpha_2=alpha_1, backend="hip")
    assert x is sentinel
    assert len(calls) == 1
    c = calls[0]
    assert c["q"] is q and c["k"] is k and c["v"] is v and c["t"] == 64
    assert c["alpha_2"] is alpha_1 and c["sar"] == 0.0625
    assert c["srr"] == 0.125 and c["flat"] == 0.5          # the reference's // 8 and // 2
    x = ref.editing_sparse_attention(q, k, v, 64, 64, 1.0, 1.0, 0.125, backend=ref.Backend.HIP)
    assert x is sentinel and calls[-1]["sar"] == 0.125


def test_default_backend_keeps_the_reference_branch(stub_reference):
    ref = stub_reference
    q = torch.zeros(1, 128, 2, 128)
    assert ref.editing_sparse_attention(q, q, q, 64, 64) == ("reference branch", "tilelang")
    assert ref.editing_sparse_attention_tilelang(q, q, q, 64, 64)[1] == "tilelang"


def test_hip_backend_without_the_package_raises(stub_reference, monkeypatch):
    esa = sys.modules["in_context_sparse_attention.editing_sparse_attention"]
    monkeypatch.setattr(esa, "icsa_hip", None)
    q = torch.zeros(1, 128, 2, 128)
    with pytest.raises(ImportError, match="icsa_hip"):
        esa.editing_sparse_attention(q, q, q, 64, 64, backend="hip")
