"""Pins the CPU oracle (CPU only, no GPU).

Every oracle function is checked against something other than its own formula: textbook
float64 attention (``scaled_dot_product_attention``), closed forms and invariants, planted
inputs whose answer is known by construction, and the independent scalar-loop restatement
in ``oracle/bruteforce.py``.  Each check is chosen so that a plausible slip (a dropped
term, a wrong index or sign, a transposed operand, a rescaled interval) fails it; the
tests that plant such a slip plant it in a copy of the oracle's arithmetic, on the CPU.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from oracle import bruteforce as BF

pytestmark = pytest.mark.cpu

DT = torch.float64


def _randn(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=DT)


def _sdpa(q, k, v):
    return F.scaled_dot_product_attention(q, k, v)


# ----------------------------------------------------------------------------------------
# derived sizes (editing_sparse_attention.py:89-172, tilelang_host.py:151-171)
# ----------------------------------------------------------------------------------------

# (S, t) -> NB, n_t, n_s, topK, Tkv, k_sparsity, n_peaked, NKV, top_k, hand-derived from the
# reference's integer formulas for the benchmark configurations.
APPENDIX_A = {
    (8192, 4096): (128, 64, 64, 8, 4608, 4, 64, 72, 4),
    (65536, 32768): (1024, 512, 512, 64, 36864, 32, 512, 576, 36),
    (65520, 32760): (1024, 511, 513, 64, 36856, 31, 512, 576, 36),
    (151200, 75600): (2363, 1181, 1182, 147, 85008, 73, 1181, 1329, 83),
}


@pytest.mark.parametrize("S,t", list(APPENDIX_A))
def test_derive_sizes_benchmark_configs(S, t):
    z = O.derive_sizes(1, S, 40, 128, t)
    got = (z.NB, z.n_t, z.n_s, z.topK, z.Tkv, z.k_sparsity, z.n_peaked, z.NKV, z.top_k)
    assert got == APPENDIX_A[(S, t)]
    assert z.n_peaked + z.n_diffuse == z.NB
    assert z.TKV_pad == z.NKV * 64 and z.TKV_pad - z.Tkv in range(64)


def test_derive_sizes_ratio_generalisation_matches_integer_division():
    # srr = 1/8 and flat = 1/2 must reproduce the reference's `// 8` and `// 2` exactly
    for n in range(0, 5000, 7):
        S = 64 * n + 64
        z = O.derive_sizes(1, S, 1, 128, 64 * (n // 3))
        assert z.topK == z.n_s // 8
        assert z.n_peaked == z.NB // 2
        assert z.k_sparsity == max(1, int(z.n_t * 0.0625))


# ----------------------------------------------------------------------------------------
# stage 1: pooling (editing_sparse_attention.py:37-55, 89-111)
# ----------------------------------------------------------------------------------------

def test_pool_constant_blocks_and_partial_last_block():
    S, D = 64 * 3 + 17, 8
    x = torch.zeros(1, S, 1, D, dtype=DT)
    vals = [1.5, -2.0, 0.25, 7.0]
    for n, c in enumerate(vals):
        x[0, 64 * n:min(S, 64 * (n + 1))] = c
    sums, means = O.pool_blocks(x)
    assert torch.equal(means[0, 0, :, 0], torch.tensor(vals, dtype=DT))
    assert sums[0, 0, 3, 0].item() == 17 * 7.0      # divides by the real size (17), not 64
    assert torch.equal(O.block_sizes(S), torch.tensor([64, 64, 64, 17]))


def test_pool_matches_bruteforce_and_exact_power_of_two_scale():
    x = _randn(2, 64 * 5 + 9, 3, 8, seed=1)
    sums, means = O.pool_blocks(x)
    for b in range(2):
        for h in range(3):
            bs, bm = BF.bf_pool(x[b, :, h].numpy())
            assert np.allclose(sums[b, h].numpy(), bs, rtol=0, atol=1e-12)
            assert np.allclose(means[b, h].numpy(), bm, rtol=0, atol=1e-12)
    s32, m32 = O.pool_blocks(x.float(), torch.float32)
    assert torch.equal(s32[:, :, :-1], 64 * m32[:, :, :-1])   # /64 is exact in binary fp


# ----------------------------------------------------------------------------------------
# stage 2: compressed attention, retrieval, split (editing_sparse_attention.py:58-64, 113-172)
# ----------------------------------------------------------------------------------------

def test_compressed_attention_is_textbook_attention():
    qc, kc, vc = (_randn(1, 2, 20, 16, seed=s) for s in (2, 3, 4))
    P, out_c = O.compressed_attention(qc, kc, vc)
    assert torch.allclose(out_c, _sdpa(qc, kc, vc), rtol=0, atol=1e-13)
    assert torch.allclose(P.sum(-1), torch.ones(1, 2, 20, dtype=DT), atol=1e-14)
    bp, bo = BF.bf_compressed(qc[0, 1].numpy(), kc[0, 1].numpy(), vc[0, 1].numpy())
    assert np.allclose(P[0, 1].numpy(), bp, atol=1e-14)
    assert np.allclose(out_c[0, 1].numpy(), bo, atol=1e-13)


def _planted_retrieval(D=16, n_t=8, n_s=16, c=4.0):
    """Target queries align with the keys of source blocks 11 (twice as strongly) and 3;
    every other key is zero.  The ranked top-2 of the per-head column mass is [11, 3]."""
    t, S = 64 * n_t, 64 * (n_t + n_s)
    q = torch.zeros(1, S, 1, D, dtype=DT)
    k = torch.zeros(1, S, 1, D, dtype=DT)
    v = _randn(1, S, 1, D, seed=5)
    q[0, :t, 0, 0] = c
    q[0, :t, 0, 1] = 2 * c
    k[0, t + 64 * 3:t + 64 * 4, 0, 0] = c
    k[0, t + 64 * 11:t + 64 * 12, 0, 1] = c
    return q, k, v, t


def test_source_selection_planted_answer():
    q, k, v, t = _planted_retrieval()
    x, info = O.editing_sparse_attention(q, k, v, t, q.shape[1] - t, SPARSITY_RATIO=0.25)
    z = info["sizes"]
    assert z.topK == 2
    assert info["sel"][0, 0].tolist() == [11, 3]
    # analytic column mass: every target row has logits 8 (block 11), 4 (block 3), 0 (others)
    NB = z.NB
    den = math.exp(8) + math.exp(4) + (NB - 2)
    assert math.isclose(info["src_score"][0, 0, 11].item(), z.n_t * math.exp(8) / den, rel_tol=1e-12)
    assert math.isclose(info["src_score"][0, 0, 3].item(), z.n_t * math.exp(4) / den, rel_tol=1e-12)


def test_source_selection_tie_rule_lower_index_first():
    P = torch.zeros(1, 1, 6, 6, dtype=DT)
    P[0, 0, :2, 2:] = torch.tensor([0.1, 0.3, 0.3, 0.1], dtype=DT)   # n_t = 2, 4 candidates
    sel, score = O.select_source_blocks(P, 2, 3)
    assert sel[0, 0].tolist() == [1, 2, 0]


def test_split_planted_peaked_blocks():
    NB, n_t = 8, 4
    P = torch.full((1, 1, NB, NB), 1.0 / NB, dtype=DT)
    w = [0.2, 0.9, 0.2, 0.5, 0.7, 0.2, 0.95, 0.3]   # mass on target column 2
    for i, wi in enumerate(w):
        P[0, 0, i] = (1 - wi) / (NB - 1)
        P[0, 0, i, 2] = wi
    peaked, diffuse, sharp = O.split_blocks(P, n_t, 1, NB // 2)
    assert peaked[0, 0].tolist() == [6, 1, 4, 3]
    assert diffuse[0, 0].tolist() == [7, 0, 2, 5]      # equal 0.2s: lower index first
    assert torch.allclose(sharp[0, 0], torch.tensor(w, dtype=DT))
    # k_sparsity = 2 adds the second-largest target column (the uniform remainder)
    _, _, sharp2 = O.split_blocks(P, n_t, 2, NB // 2)
    assert torch.allclose(sharp2[0, 0], torch.tensor([wi + (1 - wi) / (NB - 1) for wi in w], dtype=DT))


def test_split_uses_target_columns_only():
    NB, n_t = 6, 3
    P = torch.full((1, 1, NB, NB), 0.01, dtype=DT)
    P[0, 0, 0, 5] = 0.95          # peaked on a *source* column: not counted
    P[0, 0, 1, 1] = 0.5
    peaked, _, sharp = O.split_blocks(P, n_t, 1, 1)
    assert peaked[0, 0].tolist() == [1]
    assert sharp[0, 0, 0].item() == pytest.approx(0.01)


def test_new_kv_token_map_closed_form():
    S, t = 64 * 6 + 20, 64 * 2 + 30          # t unaligned, last block partial
    sel = torch.tensor([[[4, 0, 2]]])        # source block 4 (tokens 384..447) is partial
    tm = O.new_kv_token_map(t, S, sel)
    n_t = t // 64
    assert tm.shape == (1, 1, t + 3 * 64)
    assert tm[0, 0, :t].tolist() == list(range(t))
    for r, j in enumerate(sel[0, 0].tolist()):
        for i in range(64):
            tok = n_t * 64 + 64 * j + i
            assert tm[0, 0, t + 64 * r + i].item() == (tok if tok < S else -1)
    k = _randn(1, S, 1, 4, seed=6)
    nk = O.gather_new_kv(k, tm)
    assert torch.equal(nk[0, 0, t + 64 * 0 + 20:t + 64], torch.zeros(44, 4, dtype=DT))
    assert torch.equal(nk[0, 0, t + 64:t + 128], k[0, n_t * 64:n_t * 64 + 64, 0])


# ----------------------------------------------------------------------------------------
# sparse piecewise kernel (tilelang_host.py:121-274, tilelang_kernels.py:681-997)
# ----------------------------------------------------------------------------------------

def test_sparse_all_blocks_selected_is_dense_attention():
    q = _randn(1, 2, 128, 16, seed=7)
    k = _randn(1, 2, 64 * 5, 16, seed=8)
    v = _randn(1, 2, 64 * 5, 16, seed=9)
    out, idx, _ = O.sparse_piecewise_attn(q, k, v, sparsity=1.0)
    assert idx.shape[-1] == 5
    assert torch.allclose(out, _sdpa(q, k, v), rtol=0, atol=1e-13)


def _blockwise_constant(n_blocks, D, seed):
    base = _randn(1, 1, n_blocks, 1, D, seed=seed)
    return base.expand(1, 1, n_blocks, 64, D).reshape(1, 1, n_blocks * 64, D).contiguous()


@pytest.mark.parametrize("nkv", [7, 70, 130])
def test_sparse_interval_exact_for_blockwise_constant_inputs(nkv):
    # Constant query and key blocks: the top-k blocks hold every row's maximum logit, so the
    # running max never grows inside the interval loop and the interval term is exact.
    q = _blockwise_constant(3, 8, seed=10)
    k = _blockwise_constant(nkv, 8, seed=11)
    v = _randn(1, 1, nkv * 64, 8, seed=12)
    out, _, _ = O.sparse_piecewise_attn(q, k, v, sparsity=0.05)
    assert torch.allclose(out, _sdpa(q, k, v), rtol=0, atol=1e-12)


@pytest.mark.parametrize("nq,nkv,sp,seed", [(2, 4, 0.3, 13), (2, 70, 0.05, 14), (1, 129, 0.02, 15)])
def test_sparse_matches_bruteforce_loops(nq, nkv, sp, seed):
    D = 8
    q = _randn(1, 1, nq * 64, D, seed=seed)
    k = _randn(1, 1, nkv * 64, D, seed=seed + 100)
    v = _randn(1, 1, nkv * 64, D, seed=seed + 200)
    out, idx, _ = O.sparse_piecewise_attn(q, k, v, sparsity=sp)
    ob, ib = BF.bf_sparse_piecewise(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), sp)
    assert idx[0, 0].tolist() == ib
    assert np.allclose(out[0, 0].numpy(), ob, rtol=0, atol=1e-12)


def _quirk_case():
    """One query block, 128 key blocks (two interval chunks).  Exact block 0 has logit 0;
    block 5 (chunk 0) logit 2; block 70 (chunk 1) logit 4; every other block -1000."""
    D = 4
    q = torch.zeros(1, 1, 64, D, dtype=DT)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 128 * 64, D, dtype=DT)
    k[..., 0] = -1000.0 * math.sqrt(D)
    for blk, logit in ((0, 0.0), (5, 2.0), (70, 4.0)):
        k[0, 0, 64 * blk:64 * (blk + 1), 0] = logit * math.sqrt(D)
    v = torch.zeros(1, 1, 128 * 64, D, dtype=DT)
    for blk, d in ((0, 0), (5, 1), (70, 2)):
        v[0, 0, 64 * blk:64 * (blk + 1), d] = 1.0
    return q, k, v, torch.zeros(1, 1, 1, 1, dtype=torch.long)


def test_sparse_interval_accumulators_are_not_rescaled():
    q, k, v, idx = _quirk_case()
    out, _, _ = O.sparse_piecewise_attn(q, k, v, sparsity=0.008, indices=idx)
    e = math.exp(-4.0)
    quirk = torch.tensor([e, 1.0, 1.0, 0.0], dtype=DT) / (e + 2.0)
    assert torch.allclose(out[0, 0], quirk.expand(64, 4), rtol=0, atol=1e-15)
    # a correctly rescaled interval would give dense attention -- clearly different
    z = 1 + math.exp(2) + math.exp(4)
    dense = torch.tensor([1 / z, math.exp(2) / z, math.exp(4) / z, 0.0], dtype=DT)
    assert (out[0, 0, 0] - dense).abs().max() > 0.3
    ob, _ = BF.bf_sparse_piecewise(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), 0.008,
                                   order_exact=[[0]])
    assert np.allclose(ob, quirk.expand(64, 4).numpy(), atol=1e-15)


def _two_peak_case(b1, b2):
    """One query block against 128 key blocks: exact block 0 logit 0, block b1 logit 2,
    block b2 logit 4, every other block -1000; value of block 0 / b1 / b2 = e0 / e1 / e2."""
    D = 4
    q = torch.zeros(1, 1, 64, D, dtype=DT)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 128 * 64, D, dtype=DT)
    k[..., 0] = -1000.0 * math.sqrt(D)
    v = torch.zeros(1, 1, 128 * 64, D, dtype=DT)
    for blk, logit, d in ((0, 0.0, 0), (b1, 2.0, 1), (b2, 4.0, 2)):
        k[0, 0, 64 * blk:64 * (blk + 1), 0] = logit * math.sqrt(D)
        v[0, 0, 64 * blk:64 * (blk + 1), d] = 1.0
    return q, k, v, torch.zeros(1, 1, 1, 1, dtype=torch.long)


@pytest.mark.parametrize("b1,b2,bn,same_chunk", [(5, 40, 64, True), (5, 40, 32, False), (5, 40, 16, False),
                                                 (5, 20, 32, True), (5, 20, 16, False)])
def test_sparse_interval_chunk_size_sets_the_running_max(b1, b2, bn, same_chunk):
    # BN (blocks per interval chunk, tilelang_host.py:127) decides where the non-rescaled
    # interval terms take their running max.  Two interval peaks in one chunk share the
    # chunk's max -- the terms are consistent and the result is plain softmax over the
    # three blocks; in different chunks the first peak's terms keep the older, smaller max
    # (the reference's non-rescaled g_acc / g_l).  Closed forms, oracle and brute force.
    q, k, v, idx = _two_peak_case(b1, b2)
    out, _, _ = O.sparse_piecewise_attn(q, k, v, sparsity=0.008, indices=idx, bn=bn)
    e4, e2 = math.exp(-4.0), math.exp(-2.0)
    if same_chunk:
        want = torch.tensor([e4, e2, 1.0, 0.0], dtype=DT) / (e4 + e2 + 1.0)
    else:
        want = torch.tensor([e4, 1.0, 1.0, 0.0], dtype=DT) / (e4 + 2.0)
    assert torch.allclose(out[0, 0], want.expand(64, 4), rtol=0, atol=1e-15)
    ob, _ = BF.bf_sparse_piecewise(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), 0.008,
                                   order_exact=[[0]], bn=bn)
    assert np.allclose(ob, want.expand(64, 4).numpy(), atol=1e-15)


@pytest.mark.parametrize("bn", [16, 32])
@pytest.mark.parametrize("nq,nkv,sp,seed", [(2, 70, 0.05, 14), (1, 129, 0.02, 15)])
def test_sparse_chunk_size_matches_bruteforce_loops(nq, nkv, sp, seed, bn):
    D = 8
    q = _randn(1, 1, nq * 64, D, seed=seed)
    k = _randn(1, 1, nkv * 64, D, seed=seed + 100)
    v = _randn(1, 1, nkv * 64, D, seed=seed + 200)
    out, idx, _ = O.sparse_piecewise_attn(q, k, v, sparsity=sp, bn=bn)
    ob, ib = BF.bf_sparse_piecewise(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), sp, bn=bn)
    assert idx[0, 0].tolist() == ib
    assert np.allclose(out[0, 0].numpy(), ob, rtol=0, atol=1e-12)


def test_sparse_chunk_size_irrelevant_when_the_exact_max_dominates():
    # blockwise-constant inputs keep every interval score below the exact max: the running
    # max never moves, so every BN gives the same result (and that result is exact)
    q = _blockwise_constant(3, 8, seed=10)
    k = _blockwise_constant(70, 8, seed=11)
    v = _randn(1, 1, 70 * 64, 8, seed=12)
    outs = [O.sparse_piecewise_attn(q, k, v, sparsity=0.05, bn=bn)[0] for bn in (16, 32, 64)]
    assert torch.allclose(outs[0], outs[2], rtol=0, atol=1e-13)
    assert torch.allclose(outs[1], outs[2], rtol=0, atol=1e-13)


def test_planted_rescaling_mistake_is_caught():
    """A copy of the interval update that rescales g_acc/g_l disagrees with the oracle on
    the quirk case, so the quirk check above discriminates."""
    q, k, v, idx = _quirk_case()
    out, _, _ = O.sparse_piecewise_attn(q, k, v, sparsity=0.008, indices=idx)
    s = torch.tensor([0.0, 2.0, 4.0], dtype=DT)     # exact block, chunk 0, chunk 1
    m = s[0]
    l, acc = 64.0, torch.tensor([64.0, 0, 0, 0], dtype=DT)
    g_l, g_acc = 0.0, torch.zeros(4, dtype=DT)
    for c, d in ((1, 1), (2, 2)):
        m_new = torch.maximum(m, s[c])
        a = torch.exp(m - m_new)
        acc, l = acc * a, l * a
        g_acc, g_l = g_acc * a, g_l * a               # the planted slip
        p = torch.exp(s[c] - m_new)
        g_l = g_l + 64 * p
        g_acc[d] += 64 * p
        m = m_new
    wrong = (acc + g_acc) / (l + g_l)
    assert (out[0, 0, 0] - wrong).abs().max() > 0.3


def test_sparse_zero_padded_keys_attended_with_logit_zero():
    # the caller pads TKV with zero tokens; they take part with logit 0 (not masked)
    q = _randn(1, 1, 64, 8, seed=16)
    k = torch.cat([_randn(1, 1, 100, 8, seed=17), torch.zeros(1, 1, 28, 8, dtype=DT)], 2)
    v = torch.cat([_randn(1, 1, 100, 8, seed=18), torch.zeros(1, 1, 28, 8, dtype=DT)], 2)
    out, _, _ = O.sparse_piecewise_attn(q, k, v, sparsity=1.0)
    assert torch.allclose(out, _sdpa(q, k, v), atol=1e-13)
    assert not torch.allclose(out, _sdpa(q, k[:, :, :100], v[:, :, :100]), atol=1e-3)


def test_dense_attention_textbook_and_bruteforce():
    q = _randn(1, 2, 200, 16, seed=19)
    k = _randn(1, 2, 150, 16, seed=20)
    v = _randn(1, 2, 150, 16, seed=21)
    out = O.dense_attention(q, k, v, chunk=64)
    assert torch.allclose(out, _sdpa(q, k, v), atol=1e-13)
    assert np.allclose(out[0, 1].numpy(), BF.bf_dense(q[0, 1].numpy(), k[0, 1].numpy(), v[0, 1].numpy()),
                       atol=1e-13)


# ----------------------------------------------------------------------------------------
# the whole path (editing_sparse_attention.py:67-232)
# ----------------------------------------------------------------------------------------

def _inputs(S, t, D=16, B=1, H=1, seed=30):
    q = _randn(B, S, H, D, seed=seed)
    k = _randn(B, S, H, D, seed=seed + 1)
    v = _randn(B, S, H, D, seed=seed + 2)
    s = S - t
    m = min(t, s)
    k[:, :m] = k[:, t:t + m] + 0.3 * _randn(B, m, H, D, seed=seed + 3)
    v[:, :m] = v[:, t:t + m] + 0.3 * _randn(B, m, H, D, seed=seed + 4)
    return q, k, v


@pytest.mark.parametrize("S,t,sp,srr,flat", [
    (1024, 512, 0.25, 0.125, 0.5),      # aligned
    (1000, 500, 0.25, 0.125, 0.5),      # unaligned t and partial last block
    (64 * 20, 64 * 6, 0.1, 0.25, 0.25), # other ratios
    (64 * 12, 64 * 4, 0.0625, 0.5, 0.75),
])
def test_whole_path_matches_bruteforce(S, t, sp, srr, flat):
    q, k, v = _inputs(S, t)
    x, info = O.editing_sparse_attention(q, k, v, t, S - t, alpha_2=0.7, SPARSITY_RATIO=sp,
                                         srr=srr, flat_ratio=flat)
    xb, ib = BF.bf_editing_sparse_attention(q[0, :, 0].numpy(), k[0, :, 0].numpy(),
                                            v[0, :, 0].numpy(), t, 0.7, sparsity=sp, srr=srr,
                                            flat_ratio=flat)
    assert info["sel"][0, 0].tolist() == ib["sel"]
    assert info["peaked"][0, 0].tolist() == ib["peaked"]
    assert info["diffuse"][0, 0].tolist() == ib["diffuse"]
    if info["l3"] is not None:
        assert info["l3"][0, 0].tolist() == ib["l3"]
    assert np.allclose(x[0, :, 0].numpy(), xb, rtol=0, atol=1e-12)


def test_whole_path_per_head_independent_and_alpha_linear():
    B, H, S, t = 2, 2, 768, 384
    q, k, v = _inputs(S, t, B=B, H=H, seed=40)
    alpha = _randn(B, S, 1, 1, seed=44) * 0.25
    x, info = O.editing_sparse_attention(q, k, v, t, S - t, alpha_2=alpha)
    x0, _ = O.editing_sparse_attention(q, k, v, t, S - t, alpha_2=0.0)
    oc = info["out_c"].repeat_interleave(64, dim=2).permute(0, 2, 1, 3)[:, :S]
    assert torch.allclose(x - x0, alpha * oc, atol=1e-14)
    for b in range(B):
        for h in range(H):
            xs, _ = O.editing_sparse_attention(q[b:b + 1, :, h:h + 1], k[b:b + 1, :, h:h + 1],
                                               v[b:b + 1, :, h:h + 1], t, S - t,
                                               alpha_2=alpha[b:b + 1])
            assert torch.allclose(xs[0, :, 0], x[b, :, h], atol=1e-14)


def test_whole_path_independent_of_block_processing_order():
    S, t = 64 * 16, 64 * 8
    q, k, v = _inputs(S, t, seed=50)
    x, info = O.editing_sparse_attention(q, k, v, t, S - t, SPARSITY_RATIO=0.25)
    g = torch.Generator().manual_seed(0)
    pk = info["peaked"][..., torch.randperm(info["peaked"].shape[-1], generator=g)]
    perm = torch.randperm(info["diffuse"].shape[-1], generator=g)
    df = info["diffuse"][..., perm]
    l3 = info["l3"][..., perm, :].flip(-1)
    x2, _ = O.editing_sparse_attention(q, k, v, t, S - t, SPARSITY_RATIO=0.25,
                                       decisions=dict(peaked=pk, diffuse=df, l3=l3))
    assert torch.allclose(x, x2, atol=1e-13)


def test_whole_path_shape_edge_cases():
    # no diffuse blocks (flat 1.0): every block exact; no source blocks selected (srr tiny)
    S, t = 64 * 6, 64 * 3
    q, k, v = _inputs(S, t, seed=60)
    x, info = O.editing_sparse_attention(q, k, v, t, S - t, flat_ratio=1.0, srr=0.01)
    z = info["sizes"]
    assert z.n_diffuse == 0 and z.topK == 0 and z.Tkv == t
    qh, kh, vh = (a.permute(0, 2, 1, 3) for a in (q, k, v))
    dense = _sdpa(qh, kh[:, :, :t], vh[:, :, :t]).permute(0, 2, 1, 3)
    oc = info["out_c"].repeat_interleave(64, dim=2).permute(0, 2, 1, 3)
    assert torch.allclose(x, dense + oc, atol=1e-13)


def test_topk_checker_rejects_planted_mistakes():
    scores = torch.tensor([[5.0, 1.0, 4.0, 3.0, 0.5]], dtype=DT)
    good = torch.tensor([[0, 2, 3]])
    assert O.check_topk_valid(scores, good, 3, 1e-6, ordered=True).all()
    assert not O.check_topk_valid(scores, torch.tensor([[0, 2, 1]]), 3, 1e-6, ordered=True).all()
    assert not O.check_topk_valid(scores, torch.tensor([[2, 0, 3]]), 3, 1e-6, ordered=True).all()
    assert O.check_topk_valid(scores, torch.tensor([[2, 0, 3]]), 3, 1e-6, ordered=False).all()
    assert not O.check_topk_valid(scores, torch.tensor([[0, 0, 3]]), 3, 1e-6, ordered=False).all()
    assert not O.check_topk_valid(scores, torch.tensor([[0, 2, 7]]), 3, 1e-6, ordered=False).all()
    # within tolerance a near-tie may go either way
    near = torch.tensor([[1.0, 1.0 + 1e-9, 0.0]], dtype=DT)
    assert O.check_topk_valid(near, torch.tensor([[0]]), 1, 1e-6, ordered=True).all()


# ----------------------------------------------------------------------------------------
# the Triton host's contract (triton_host.py:11-30; triton_kernels.py:89-119, 185, 489-539):
# ragged TQ / TKV, floor top_k, keys past TKV masked out of the exact part
# ----------------------------------------------------------------------------------------

def test_sparse_triton_mode_equals_tilelang_for_aligned_lengths():
    q = _randn(1, 2, 128, 16, seed=30)
    k = _randn(1, 2, 64 * 9, 16, seed=31)
    v = _randn(1, 2, 64 * 9, 16, seed=32)
    a = O.sparse_piecewise_attn(q, k, v, 0.25)
    b = O.sparse_piecewise_attn(q, k, v, 0.25, mode="triton")
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_sparse_triton_mode_all_selected_is_attention_over_the_real_keys():
    # TKV = 4 * 64 + 37: five candidate blocks, the last partial; sparsity 1.25 gives
    # top_k = int(1.25 * (TKV // 64)) = 5, so every block is exact and the interval is empty:
    # the result is textbook attention over the 293 real keys (ragged TQ as well)
    q = _randn(1, 2, 133, 16, seed=33)
    k = _randn(1, 2, 293, 16, seed=34)
    v = _randn(1, 2, 293, 16, seed=35)
    out, idx, _ = O.sparse_piecewise_attn(q, k, v, 1.25, mode="triton")
    assert idx.shape[-1] == 5 and out.shape == (1, 2, 133, 16)
    assert torch.allclose(out, _sdpa(q, k, v), rtol=0, atol=1e-13)


@pytest.mark.parametrize("tq,tkv,sp,seed", [(133, 293, 0.5, 36), (64, 64 * 70 + 11, 0.05, 37),
                                            (100, 64 * 129 + 63, 0.02, 38)])
def test_sparse_triton_mode_matches_bruteforce_loops(tq, tkv, sp, seed):
    D = 8
    q = _randn(1, 1, tq, D, seed=seed)
    k = _randn(1, 1, tkv, D, seed=seed + 100)
    v = _randn(1, 1, tkv, D, seed=seed + 200)
    out, idx, _ = O.sparse_piecewise_attn(q, k, v, sparsity=sp, mode="triton")
    ob, ib = BF.bf_sparse_piecewise(q[0, 0].numpy(), k[0, 0].numpy(), v[0, 0].numpy(), sp, triton=True)
    assert idx[0, 0].tolist() == ib
    assert np.allclose(out[0, 0].numpy(), ob, rtol=0, atol=1e-12)


def test_sparse_triton_mode_masks_the_tail_instead_of_attending_zero_keys():
    # a planted mistake -- the tail keys of the partial block attended with logit 0, as
    # TileLang's zero padding does -- differs clearly from the Triton contract
    q = _randn(1, 1, 64, 8, seed=39) * 0.3
    k = _randn(1, 1, 64 * 3 + 5, 8, seed=40) * 0.3
    v = _randn(1, 1, 64 * 3 + 5, 8, seed=41) + 2.0
    idx = torch.tensor([0, 1, 2, 3]).view(1, 1, 1, 4)
    tri, _, _ = O.sparse_piecewise_attn(q, k, v, 1.34, indices=idx, mode="triton")
    kp = torch.cat([k, torch.zeros(1, 1, 59, 8, dtype=DT)], 2)
    vp = torch.cat([v, torch.zeros(1, 1, 59, 8, dtype=DT)], 2)
    pad_logit0, _, _ = O.sparse_piecewise_attn(q, kp, vp, 1.0, indices=idx)
    assert torch.allclose(tri, _sdpa(q, k, v), atol=1e-13)
    assert (tri - pad_logit0).abs().max() > 0.3      # 59 zero keys of 256 pull the mean of v ~ 2 down


def test_sparse_triton_top_k_floor_at_configuration_4():
    # the DiT block's unpadded new KV: Tkv = 36,856 (Appendix A): Triton 35 exact blocks,
    # TileLang (zero-padded to 36,864) 36
    q = _randn(1, 1, 64, 4, seed=42)
    k = _randn(1, 1, 36856, 4, seed=43)
    _, idx_tri, sc = O.sparse_piecewise_attn(q, k, k, 0.0625, mode="triton")
    assert idx_tri.shape[-1] == 35 and sc.shape[-1] == 576
    kp = torch.cat([k, torch.zeros(1, 1, 8, 4, dtype=DT)], 2)
    _, idx_tl, _ = O.sparse_piecewise_attn(q, kp, kp, 0.0625)
    assert idx_tl.shape[-1] == 36
