"""Host-side checks that need no GPU: the C-ABI library loads and exports every symbol the
header declares, its size/layout queries agree with the oracle, argument errors come back
as status codes before any device work, and the Python mirror of the reference interface
keeps the reference's names and error behaviour."""
import ctypes
import os
import re

import pytest
import torch

import oracle as O
from icsa_hip import _lib
from icsa_hip.editing_sparse_attention import (
    SIZE_NAMES, Backend, derived_sizes, editing_sparse_attention)
from icsa_hip.hip_host import (IcsaArgumentError, flash_attn_func,
                               sparse_piecewise_attn_1st_intervals_hip)

pytestmark = pytest.mark.cpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "icsa.h")
PKG = os.path.join(ROOT, "lightning-unified-video-editor-via-in-context-sparse-attention_amd")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(icsa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _declared_functions()
    assert declared, "no declarations parsed from include/icsa.h"
    assert sorted(_lib.EXPORTS) == declared
    for name in declared:
        assert getattr(L, name) is not None
    assert L.icsa_version() == 100


@pytest.mark.parametrize("S,t,sp,srr,flat", [
    (8192, 4096, 0.0625, 0.125, 0.5), (65536, 32768, 0.0625, 0.125, 0.5),
    (65520, 32760, 0.0625, 0.125, 0.5), (151200, 75600, 0.0625, 0.125, 0.5),
    (1000, 500, 0.25, 0.125, 0.5), (64 * 20, 64 * 6, 0.1, 0.25, 0.25), (4096, 0, 0.0625, 0.125, 0.5),
    (4096, 4096, 0.0625, 0.125, 0.5), (65536, 32768, 1 / 32, 0.125, 0.75), (65536, 32768, 1 / 8, 0.125, 0.25),
])
def test_library_sizes_match_oracle(S, t, sp, srr, flat):
    z = derived_sizes(1, S, 40, 128, t, sp, srr, flat)
    o = O.derive_sizes(1, S, 40, 128, t, sp, srr, flat)
    for name in SIZE_NAMES[:-1]:
        assert z[name] == getattr(o, name), name
    assert z["NKVp"] % 64 == 0 and z["NKVp"] >= z["NKV"]


def test_workspace_layout_is_aligned_and_disjoint():
    L = _lib.lib()
    n = len(_lib.WS_SLOTS)
    for (S, t, qd) in ((65536, 32768, _lib.BF16), (65520, 32760, _lib.F32), (8192, 4096, _lib.BF16)):
        offs = (ctypes.c_int64 * n)()
        total = L.icsa_editing_workspace_layout(1, S, 40, 128, t, 0.0625, 0.125, 0.5, qd, qd, qd,
                                                ctypes.cast(offs, ctypes.c_void_p))
        assert total > 0
        assert total == L.icsa_editing_workspace_size(1, S, 40, 128, t, 0.0625, 0.125, 0.5, qd, qd, qd)
        o = list(offs)
        assert all(x % 256 == 0 and 0 <= x <= total for x in o)
        assert o == sorted(o)
    # block sums of the new v: transposed for the V^T tiles of aligned t, row-major for the
    # row tiles the sparse kernel reads in place when t % 64 != 0; a bf16 copy of v only for
    # an f32 v at unaligned t
    vc, vct, vb = (_lib.WS_SLOTS.index(x) for x in ("VC", "VCT", "VB"))
    for t, vd, want_vc, want_vb in ((32768, _lib.BF16, False, False), (32760, _lib.BF16, True, False),
                                    (32768, _lib.F32, False, False), (32760, _lib.F32, True, True)):
        offs = (ctypes.c_int64 * n)()
        L.icsa_editing_workspace_layout(1, 65536, 40, 128, t, 0.0625, 0.125, 0.5, _lib.BF16, _lib.BF16,
                                        vd, ctypes.cast(offs, ctypes.c_void_p))
        assert (offs[vc + 1] > offs[vc]) == want_vc and (offs[vct + 1] > offs[vct]) != want_vc
        assert (offs[vb + 1] > offs[vb]) == want_vb


def test_unaligned_workspace_holds_no_materialised_new_kv():
    # t % 64 != 0 reads the straddling new-KV blocks in place: the workspace of configuration
    # 4's shape is the aligned one's plus the row-major new-KV value sums, nothing of size Tkv
    L = _lib.lib()
    args = (1, 65520, 40, 128)
    aligned = L.icsa_editing_workspace_size(*args, 32768, 0.0625, 0.125, 0.5, _lib.BF16, _lib.BF16, _lib.BF16)
    unaligned = L.icsa_editing_workspace_size(*args, 32760, 0.0625, 0.125, 0.5, _lib.BF16, _lib.BF16, _lib.BF16)
    assert 0 < unaligned < aligned + 8 * 2**20, (aligned, unaligned)


def _status(name, *args):
    rc = getattr(_lib.lib(), name)(*args)
    return rc, _lib.lib().icsa_last_error().decode()


def test_size_queries_reject_bad_arguments():
    out = (ctypes.c_int32 * 12)()
    p = ctypes.cast(out, ctypes.c_void_p)
    rc, msg = _status("icsa_editing_sizes", 1, 1024, 1, 64, 512, 0.0625, 0.125, 0.5, p)
    assert rc == _lib.EUNSUPPORTED and "D=64" in msg
    rc, msg = _status("icsa_editing_sizes", 1, 1024, 1, 128, 2000, 0.0625, 0.125, 0.5, p)
    assert rc == _lib.EINVAL and "t_seq_len" in msg
    rc, _ = _status("icsa_editing_sizes", 0, 1024, 1, 128, 512, 0.0625, 0.125, 0.5, p)
    assert rc == _lib.EINVAL
    rc, _ = _status("icsa_editing_sizes", 1, 1024, 1, 128, 512, 0.0625, 0.125, 0.5, None)
    assert rc == _lib.EINVAL
    assert _lib.lib().icsa_sparse_piecewise_workspace_size(1, 1, 128, 128, 96, 0.1) < 0
    assert _lib.lib().icsa_sparse_piecewise_workspace_size(1, 1, 128, 128, 128, 0.0) < 0
    # ragged lengths (the Triton host) are sized in whole blocks
    assert (_lib.lib().icsa_sparse_piecewise_workspace_size(1, 1, 100, 4645, 128, 0.1)
            == _lib.lib().icsa_sparse_piecewise_workspace_size(1, 1, 128, 4672, 128, 0.1))
    assert (_lib.lib().icsa_sparse_piecewise_attn_bwd_workspace_size(1, 1, 100, 4645, 128)
            == _lib.lib().icsa_sparse_piecewise_attn_bwd_workspace_size(1, 1, 128, 4672, 128) > 0)
    assert _lib.lib().icsa_flash_attn_workspace_size(1, 128, 1, 96) < 0


def _editing_args(q=None, qd=_lib.BF16, D=128, t=512, S=1024, sp=0.0625, ws=None, ws_bytes=0):
    st = (S * 128, 128, 128)
    return [q, qd, *st, q, qd, *st, q, qd, *st, 1, S, 1, D, t, sp, 0.125, 0.5,
            None, _lib.F32, 0, 0, 0, 0, 1.0, q, _lib.BF16, *st, None, None, None,
            ws, ws_bytes, None]


def test_pipeline_entry_rejects_bad_arguments_before_device_work():
    # null pointers, bad dtypes and unsupported shapes are refused before any HIP call
    rc, msg = _status("icsa_editing_sparse_attention", *_editing_args())
    assert rc == _lib.EINVAL and "null" in msg
    rc, msg = _status("icsa_editing_sparse_attention", *_editing_args(qd=7))
    assert rc == _lib.EINVAL and "dtype" in msg
    rc, msg = _status("icsa_editing_sparse_attention", *_editing_args(D=64))
    assert rc == _lib.EUNSUPPORTED
    rc, msg = _status("icsa_sparse_piecewise_attn", None, 0, 0, 0, None, 0, 0, 0, None, 0, 0, 0,
                      1, 1, 100, 128, 128, 0.1, None, None, None, 0, 0, 0, None, 0, None)
    assert rc == _lib.EINVAL and "divisible" in msg


@pytest.mark.skipif(torch.cuda.is_available(), reason="uses non-null host addresses; host-only")
def test_pipeline_entry_rejects_limits_and_small_workspace():
    # Host buffers stand in for device pointers: each call fails validation before any
    # device work, so nothing is dereferenced.
    buf = torch.empty(1 << 12, dtype=torch.uint8)
    p = ctypes.c_void_p((buf.data_ptr() + 255) // 256 * 256)
    rc, msg = _status("icsa_editing_sparse_attention", *_editing_args(q=p, ws=p, ws_bytes=0))
    assert rc == _lib.EWORKSPACE and "workspace" in msg
    rc, msg = _status("icsa_editing_sparse_attention", *_editing_args(q=p, ws=p, S=64 * 5000, t=64 * 2500))
    assert rc == _lib.EUNSUPPORTED
    rc, msg = _status("icsa_editing_sparse_attention", *_editing_args(q=p, ws=p, sp=0.0))
    assert rc == _lib.EINVAL and "sparsity" in msg
    rc, msg = _status("icsa_sparse_piecewise_attn", p, 0, 0, 128, p, 0, 0, 128, p, 0, 0, 128,
                      1, 1, 64, 64 * 4096, 128, 0.1, None, None, p, 0, 0, 128, p, 1 << 30, None)
    assert rc == _lib.EUNSUPPORTED and "NKV" in msg


def test_backend_names_and_dispatch():
    assert Backend.validate("hip") == "hip"
    assert Backend.validate("tilelang") == "tilelang" and Backend.validate("triton") == "triton"
    with pytest.raises(ValueError):
        Backend.validate("cuda")
    q = torch.zeros(1, 128, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        editing_sparse_attention(q, q, q, 64, 64, backend="tilelang")
    # the reference's default backend is 'tilelang' (editing_sparse_attention.py:67-71)
    with pytest.raises(NotImplementedError):
        editing_sparse_attention(q, q, q, 64, 64)
    with pytest.raises(ValueError):
        editing_sparse_attention(q, q, q, 64, 64, backend="nope")
    # CPU tensors are refused, never computed another way
    with pytest.raises(IcsaArgumentError):
        editing_sparse_attention(q, q, q, 64, 64, backend="hip")


def test_host_functions_mirror_reference_asserts():
    x = torch.zeros(1, 1, 128, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):          # reference: assert q.dtype == torch.bfloat16
        sparse_piecewise_attn_1st_intervals_hip(x.float(), x, x)
    with pytest.raises(IcsaArgumentError, match="GPU"):
        sparse_piecewise_attn_1st_intervals_hip(x, x, x)
    with pytest.raises(IcsaArgumentError):
        flash_attn_func(x, x, x, causal=True)


def test_tilelang_hosttopk_mirrors_reference_asserts():
    from icsa_hip import sparse_piecewise_attn_tilelang_hosttopk_hip as hosttopk
    x = torch.zeros(1, 1, 128, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):          # reference: bf16 inputs
        hosttopk(x.float(), x, x)
    with pytest.raises(AssertionError):          # reference: TQ/TKV divisible by BT
        hosttopk(x[:, :, :100], x, x)
    with pytest.raises(AssertionError):          # reference: Vdim divisible by BV
        hosttopk(x, x, x, BV=48)
    with pytest.raises(IcsaArgumentError, match="BN"):
        hosttopk(x, x, x, BN=48)                   # 16, 32 and 64 are the chunk sizes that run
    with pytest.raises(IcsaArgumentError, match="GPU"):
        hosttopk(x, x, x)


def test_product_package_never_imports_the_oracle():
    pat = re.compile(r"^\s*(from|import)\s+oracle\b", re.M)
    for dirpath, _, files in os.walk(PKG):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dirpath, f)).read()
                assert not pat.search(src), f"{f} imports the oracle"


def test_index_list_checks_reject_bad_lists():
    from icsa_hip.hip_host import check_index_lists
    ok = torch.tensor([[[3, 0, 5], [1, 2, 4]]])
    check_index_lists(ok, 6, "idx")
    with pytest.raises(IcsaArgumentError, match="distinct"):
        check_index_lists(torch.tensor([[[3, 0, 3]]]), 6, "idx")
    with pytest.raises(IcsaArgumentError, match="lie in"):
        check_index_lists(torch.tensor([[[3, 0, 6]]]), 6, "idx")
    with pytest.raises(IcsaArgumentError, match="lie in"):
        check_index_lists(torch.tensor([[[-1, 0, 2]]]), 6, "idx")
    check_index_lists(torch.tensor([[[-1, 0, 2]]]), 6, "idx", allow_neg=True)
    # an injected block order must be a permutation of the blocks
    with pytest.raises(IcsaArgumentError):
        check_index_lists(torch.tensor([[[0, 1, 1, 3]]]), 4, "order")


def test_noalloc_entry_rejects_oversized_calls_before_device_work():
    # configuration 2 with all 40 heads needs more than the static scratch; the call fails
    # on its size before any HIP call (the pointers are never read)
    args = _editing_args(S=65536, t=32768)
    args[17] = 40                          # H
    rc, msg = _status("icsa_editing_sparse_attention_noalloc", *args[:-3], None)
    assert rc == _lib.EUNSUPPORTED and "static scratch" in msg
