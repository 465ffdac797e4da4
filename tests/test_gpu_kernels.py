"""GPU parity of the individual entry points (pool, flash attention, sparse host function)."""
import math

import pytest
import torch

import oracle as O
from icsa_hip import (flash_attn_func, gather_kv, pool,
                      sparse_piecewise_attn_1st_intervals_hip,
                      sparse_piecewise_attn_tilelang_hosttopk_hip)
from icsa_hip.hip_host import IcsaArgumentError
from parity import GAP, compare_out, l3_scale

pytestmark = pytest.mark.gpu


def _bf16(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("S", [64, 1000, 4096])
def test_pool_sums_and_transposed_v(gpu, S):
    print(f"[case] pool S={S}", flush=True)
    q, k, v = _bf16(2, S, 3, 128, seed=1), _bf16(2, S, 3, 128, seed=2), _bf16(2, S, 3, 128, seed=3)
    qs, ks, vs, vt = pool(q.to(gpu), k.to(gpu), v.to(gpu), want_vt=True)
    for x, s in ((q, qs), (k, ks), (v, vs)):
        ref, _ = O.pool_blocks(x)
        assert torch.allclose(s.cpu().double(), ref, rtol=1e-6, atol=1e-5)
    # V^T: token tok of block-group g stored at slot kv_slot(tok)
    NB = (S + 63) // 64
    vp = torch.zeros(2, NB * 64, 3, 128, dtype=torch.bfloat16)
    vp[:, :S] = v
    tok = torch.arange(NB * 64)
    slot = (tok & ~12) | ((tok & 4) << 1) | ((tok & 8) >> 1)
    expect = torch.empty(2, 3, 128, NB * 64, dtype=torch.bfloat16)
    expect[..., slot] = vp.permute(0, 2, 3, 1)
    assert torch.equal(vt.cpu(), expect)


@pytest.mark.parametrize("Sq,Sk,H", [(64, 64, 1), (200, 300, 2), (4096, 4096, 2), (130, 4160, 3)])
def test_flash_attn_dense(gpu, Sq, Sk, H):
    print(f"[case] flash Sq={Sq} Sk={Sk} H={H}", flush=True)
    q, k, v = _bf16(1, Sq, H, 128, seed=4), _bf16(1, Sk, H, 128, seed=5), _bf16(1, Sk, H, 128, seed=6)
    out = flash_attn_func(q.to(gpu), k.to(gpu), v.to(gpu), out_dtype=torch.float32)
    ref = O.dense_attention(q.double().permute(0, 2, 1, 3), k.double().permute(0, 2, 1, 3),
                            v.double().permute(0, 2, 1, 3)).permute(0, 2, 1, 3)
    compare_out(out, ref)


@pytest.mark.parametrize("Sk", [65, 128, 129, 191, 192])
def test_flash_attn_few_tiles(gpu, Sk):
    # 2-3 key tiles, full and partial: the schedule's prologue (K(0), K(1), V(0)), its
    # empty-range DMA of the slots past the last tile and the zero fill of the partial tile
    print(f"[case] flash few tiles Sk={Sk}", flush=True)
    q, k, v = _bf16(1, 320, 2, 128, seed=11), _bf16(1, Sk, 2, 128, seed=12), _bf16(1, Sk, 2, 128, seed=13)
    out = flash_attn_func(q.to(gpu), k.to(gpu), v.to(gpu), out_dtype=torch.float32)
    ref = O.dense_attention(q.double().permute(0, 2, 1, 3), k.double().permute(0, 2, 1, 3),
                            v.double().permute(0, 2, 1, 3)).permute(0, 2, 1, 3)
    compare_out(out, ref)


def test_flash_attn_large_logits(gpu):
    # peaked softmax: logits up to ~40 exercise the running-max rescale path
    q, k, v = _bf16(1, 512, 2, 128, seed=7, scale=3.0), _bf16(1, 1024, 2, 128, seed=8, scale=3.0), \
        _bf16(1, 1024, 2, 128, seed=9)
    out = flash_attn_func(q.to(gpu), k.to(gpu), v.to(gpu), out_dtype=torch.float32)
    ref = O.dense_attention(q.double().permute(0, 2, 1, 3), k.double().permute(0, 2, 1, 3),
                            v.double().permute(0, 2, 1, 3)).permute(0, 2, 1, 3)
    compare_out(out, ref)


@pytest.mark.parametrize("TQ,TKV,sparsity", [(512, 1024, 0.25), (1024, 4608, 0.0625), (256, 8192, 0.0625)])
def test_sparse_piecewise_host(gpu, TQ, TKV, sparsity):
    print(f"[case] sparse TQ={TQ} TKV={TKV} sparsity={sparsity}", flush=True)
    q, k, v = _bf16(1, 2, TQ, 128, seed=10), _bf16(1, 2, TKV, 128, seed=11), _bf16(1, 2, TKV, 128, seed=12)
    out, idx = sparse_piecewise_attn_1st_intervals_hip(q.to(gpu), k.to(gpu), v.to(gpu), sparsity,
                                                       return_indices=True)
    ref, ref_idx, scores = O.sparse_piecewise_attn(q, k, v, sparsity, indices=idx.long().cpu())
    top_k = idx.shape[-1]
    assert O.check_topk_valid(scores / l3_scale(128), idx.long().cpu(), top_k, GAP, ordered=False).all()
    compare_out(out, ref)


def test_tilelang_hosttopk_entry(gpu):
    # sparse_piecewise_attn_tilelang_hosttopk's two reference paths (BV == Vdim: fused kernel;
    # BV < Vdim: top-k + interval kernels) compute one function; both map onto the same kernel
    q, k, v = (_bf16(1, 2, n, 128, seed=30 + i).to(gpu) for i, n in enumerate((512, 4608, 4608)))
    want = sparse_piecewise_attn_1st_intervals_hip(q, k, v, 0.0625, 64)
    for bv, srt in ((32, False), (128, True)):
        got = sparse_piecewise_attn_tilelang_hosttopk_hip(q, k, v, 0.0625, BT=64, BV=bv, BN=64,
                                                          sorted_topk=srt)
        assert torch.equal(got, want)
    # BN = 16 / 32 run (their results: test_hosttopk_interval_chunk_size); others are refused
    for bn in (16, 32):
        got = sparse_piecewise_attn_tilelang_hosttopk_hip(q, k, v, 0.0625, BN=bn)
        assert torch.isfinite(got.float()).all()
    with pytest.raises(IcsaArgumentError):
        sparse_piecewise_attn_tilelang_hosttopk_hip(q, k, v, BN=48)


def _interval_skip_margin(q, k, idx):
    """Per query block (q, k: [B, H, T, D] bf16, idx: [B, H, NQ, top_k] exact blocks): the
    minimum over its rows of m_exact - |q| max_j |KC_j| c / 64, in log2 units, with KC_j the
    bf16 block sums of the keys.  Positive: the Cauchy-Schwarz bound proves that no interval
    score reaches the exact max, and the kernel skips its interval max pass for the block;
    negative: it runs both interval passes."""
    c = math.log2(math.e) / math.sqrt(q.shape[-1])
    B, H, TQ, D = q.shape
    NKV = k.shape[2] // 64
    kc = k.float().view(B, H, NKV, 64, D).sum(3).to(torch.bfloat16).float()
    bound = q.float().norm(dim=-1) * kc.norm(dim=-1).amax(-1)[..., None] * c / 64
    out = []
    for b in range(B):
        for h in range(H):
            keys = k[b, h].float().view(NKV, 64, D)
            for blk in range(TQ // 64):
                rows = q[b, h, 64 * blk:64 * blk + 64].float()
                m = (rows @ keys[idx[b, h, blk].long()].reshape(-1, D).T).amax(-1) * c
                out.append((m - bound[b, h, 64 * blk:64 * blk + 64]).min().item())
    return out


def test_sparse_piecewise_interval_bound_skip(gpu):
    # Random queries and keys: the bound holds for every query block, so every workgroup
    # skips the interval max pass; the result must still be the oracle's.
    print("[case] sparse interval-bound skip path", flush=True)
    TQ, TKV = 256, 64 * 64
    q, k, v = _bf16(1, 2, TQ, 128, seed=31), _bf16(1, 2, TKV, 128, seed=32), _bf16(1, 2, TKV, 128, seed=33)
    g = torch.Generator().manual_seed(34)
    idx = torch.stack([torch.randperm(64, generator=g)[:4].sort().values for _ in range(2 * TQ // 64)])
    idx = idx.view(1, 2, TQ // 64, 4).to(torch.int32)
    assert min(_interval_skip_margin(q, k, idx)) > 0.25
    out = sparse_piecewise_attn_1st_intervals_hip(q.to(gpu), k.to(gpu), v.to(gpu), 0.0625,
                                                  indices=idx.to(gpu))
    ref, _, _ = O.sparse_piecewise_attn(q, k, v, 0.0625, indices=idx.long())
    compare_out(out, ref)


def _pipeline_skip_margins(q, k, t, views):
    """_interval_skip_margin for the diffuse blocks of one pipeline call (bf16 q, k on the
    CPU), built from that call's own decisions: the new KV of its source selection and its
    per-block exact lists."""
    z = views["sizes"]
    B, S, H, D = q.shape
    sel, order, l3 = (views[x].long().cpu() for x in ("sel", "order", "l3"))
    tokmap = O.new_kv_token_map(t, S, sel)
    nk = O.gather_new_kv(k, tokmap, torch.float32).to(torch.bfloat16)
    nk = torch.nn.functional.pad(nk, (0, 0, 0, z["TKV_pad"] - nk.shape[2]))
    qp = q.permute(0, 2, 1, 3).reshape(B, H, z["NB"], 64, D)
    diffuse = order[..., z["n_peaked"]:]
    qd = torch.stack([torch.stack([qp[b, h, diffuse[b, h]] for h in range(H)]) for b in range(B)])
    return _interval_skip_margin(qd.reshape(B, H, -1, D), nk, l3)


def test_interval_skip_is_bit_identical(gpu, monkeypatch):
    # The interval-bound skip drops interval pass 1 only where it cannot change the running
    # max, so the output must equal the no-skip schedule bit for bit: the host entry (row-major
    # V tiles) and an aligned pipeline call (V^T tiles), each with the skip on and off (the
    # library's ICSA_DEBUG_NO_INTERVAL_SKIP hook).
    from icsa_hip.editing_sparse_attention import _editing_sparse_attention_hip
    from icsa_hip.synthetic import make_inputs
    print("[case] interval skip on / off: host entry", flush=True)
    TQ, TKV = 256, 64 * 64
    q, k, v = _bf16(1, 2, TQ, 128, seed=31), _bf16(1, 2, TKV, 128, seed=32), _bf16(1, 2, TKV, 128, seed=33)
    g = torch.Generator().manual_seed(34)
    idx = torch.stack([torch.randperm(64, generator=g)[:4].sort().values for _ in range(2 * TQ // 64)])
    idx = idx.view(1, 2, TQ // 64, 4).to(torch.int32).to(gpu)
    args = (q.to(gpu), k.to(gpu), v.to(gpu), 0.0625)
    monkeypatch.delenv("ICSA_DEBUG_NO_INTERVAL_SKIP", raising=False)
    on = sparse_piecewise_attn_1st_intervals_hip(*args, indices=idx)
    monkeypatch.setenv("ICSA_DEBUG_NO_INTERVAL_SKIP", "1")
    off = sparse_piecewise_attn_1st_intervals_hip(*args, indices=idx)
    monkeypatch.delenv("ICSA_DEBUG_NO_INTERVAL_SKIP")
    torch.cuda.synchronize()
    assert torch.equal(on, off)

    print("[case] interval skip on / off: aligned pipeline (V^T tiles)", flush=True)
    q, k, v, t = make_inputs(H=2, real=2048, pad=0, kind="random", seed=41)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    on, views = _editing_sparse_attention_hip(qg, kg, vg, t, 0.5, keep_workspace=True)
    margins = _pipeline_skip_margins(q, k, t, views)
    assert sum(m > 0.25 for m in margins) >= len(margins) // 2, "the skip must fire in this case"
    monkeypatch.setenv("ICSA_DEBUG_NO_INTERVAL_SKIP", "1")
    off, _ = _editing_sparse_attention_hip(qg, kg, vg, t, 0.5)
    monkeypatch.delenv("ICSA_DEBUG_NO_INTERVAL_SKIP")
    torch.cuda.synchronize()
    assert torch.equal(on, off)


@pytest.mark.parametrize("bn", [16, 32, 64])
def test_hosttopk_interval_chunk_size(gpu, bn):
    # BN (sparse_piecewise_attn_tilelang_hosttopk's interval chunk) decides where the
    # non-rescaled interval terms take their running max.  (i) Two interval peaks, blocks 20
    # (logit 2) and 40 (logit 4): one chunk for BN = 64 (plain softmax over the peaks), two
    # for BN = 32 and 16 (the first peak keeps the smaller max) -- the results differ by
    # more than 0.3, and each matches the oracle with that BN.  (ii) Random keys with the
    # exact lists injected as the lowest-scoring blocks, so the running max rises chunk by
    # chunk, against the oracle with that BN.
    print(f"[case] hosttopk BN={bn}", flush=True)
    D, NKV = 128, 128
    q = torch.zeros(1, 1, 64, D)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, NKV * 64, D)
    k[..., 0] = -1000.0 * math.sqrt(D)
    v = torch.zeros(1, 1, NKV * 64, D)
    for blk, logit, d in ((0, 0.0, 0), (20, 2.0, 1), (40, 4.0, 2)):
        k[0, 0, 64 * blk:64 * (blk + 1), 0] = logit * math.sqrt(D)
        v[0, 0, 64 * blk:64 * (blk + 1), d] = 1.0        # output dim d = the block's weight
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    idx = torch.zeros(1, 1, 1, 1, dtype=torch.int32)
    outs = {}
    for b in sorted({bn, 64}):
        outs[b] = sparse_piecewise_attn_1st_intervals_hip(q.to(gpu), k.to(gpu), v.to(gpu), 0.008,
                                                          indices=idx.to(gpu), interval_bn=b)
    ref, _, _ = O.sparse_piecewise_attn(q, k, v, 0.008, indices=idx.long(), bn=bn)
    compare_out(outs[bn], ref)
    if bn != 64:
        assert (outs[bn].float() - outs[64].float()).abs().max().item() > 0.3
    q2, k2, v2 = _bf16(1, 2, 256, D, seed=41), _bf16(1, 2, 130 * 64, D, seed=42), _bf16(1, 2, 130 * 64, D, seed=43)
    qc = q2.double().view(1, 2, 4, 64, D).sum(3)
    kc = k2.double().view(1, 2, 130, 64, D).sum(3)
    low = torch.matmul(qc, kc.transpose(-1, -2)).argsort(-1)[..., :6].sort(-1).values.to(torch.int32)
    out2 = sparse_piecewise_attn_1st_intervals_hip(q2.to(gpu), k2.to(gpu), v2.to(gpu), 0.05,
                                                   indices=low.to(gpu), interval_bn=bn)
    ref2, _, _ = O.sparse_piecewise_attn(q2, k2, v2, 0.05, indices=low.long(), bn=bn)
    compare_out(out2, ref2)


def test_sparse_piecewise_quirk_case(gpu):
    # Keys of a late chunk align with the queries: the interval's running max rises after
    # earlier chunks were accumulated, which the reference does not rescale.  The oracle
    # reproduces that; an implementation that rescaled g_acc / g_l would differ here.
    TQ, TKV = 64, 64 * 192
    q = _bf16(1, 1, TQ, 128, seed=13)
    k = _bf16(1, 1, TKV, 128, seed=14, scale=0.2)
    # block 150 (chunk 2) holds 64 copies of 20 x the mean query: its interval score dwarfs
    # every exact logit, so chunks 0-1 stay weighted by the stale running max
    k[0, 0, 64 * 150:64 * 151] = (20.0 * q[0, 0].float().mean(0)).expand(64, 128).to(torch.bfloat16)
    v = _bf16(1, 1, TKV, 128, seed=15)
    idx = torch.arange(12, dtype=torch.int32).view(1, 1, 1, 12)
    assert max(_interval_skip_margin(q, k, idx)) < -1.0   # both interval passes run
    out = sparse_piecewise_attn_1st_intervals_hip(q.to(gpu), k.to(gpu), v.to(gpu), 0.0625,
                                                  indices=idx.to(gpu))
    ref, _, _ = O.sparse_piecewise_attn(q, k, v, 0.0625, indices=idx.long())
    compare_out(out, ref)


def test_gather_kv_matches_token_map(gpu):
    k, v = _bf16(1, 1000, 2, 128, seed=16), _bf16(1, 1000, 2, 128, seed=17)
    t = 500
    sel = torch.tensor([[[7, 0, 3], [1, 2, 6]]])            # n_t = 7 -> blocks 7+sel (block 15 partial)
    kn, vn = gather_kv(k.to(gpu), v.to(gpu), t, sel)
    tokmap = O.new_kv_token_map(t, 1000, sel)
    ref_k = O.gather_new_kv(k, tokmap, torch.float32).to(torch.bfloat16)
    ref_v = O.gather_new_kv(v, tokmap, torch.float32).to(torch.bfloat16)
    Tkv = ref_k.shape[2]
    assert torch.equal(kn[:, :, :Tkv].cpu(), ref_k) and torch.equal(vn[:, :, :Tkv].cpu(), ref_v)
    assert (kn[:, :, Tkv:] == 0).all()


def test_argument_errors_mirror_reference(gpu):
    q = torch.zeros(1, 1, 64, 128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(AssertionError):
        sparse_piecewise_attn_1st_intervals_hip(q, q, q, block_size=32)
    with pytest.raises(IcsaArgumentError):
        sparse_piecewise_attn_1st_intervals_hip(q.float(), q, q)
    with pytest.raises(IcsaArgumentError):
        sparse_piecewise_attn_1st_intervals_hip(q[:, :, :60], q, q)
