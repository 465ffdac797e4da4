"""Parity at the benchmark sizes (65,536 / 65,520 / 151,200 tokens, H = 40, D = 128).

The whole CPU oracle is too slow at this size, so the check is split by stage, each
part against float64 arithmetic on the same bf16 inputs (the oracle's own functions,
run in float64 on the GPU as the checker):

* block sums and the compressed softmax P;
* every ranked decision -- source blocks, the peaked/diffuse split, the per-block exact
  lists -- must be a valid ranking of the float64 scores within GAP;
* output rows of eight seeded-random peaked and eight diffuse query blocks in every head
  of every batch entry, plus the peaked blocks of the flash grid's last workgroup and the
  diffuse block whose sparse workgroup starts its sweep furthest along, against float64
  attention for exactly those blocks, built from the GPU's own decisions;
* size-independent properties: two runs are bit-identical, and x is exactly linear in
  alpha_2 (x(alpha) - x(0) = alpha * out_c) on every token.

Configuration 3 (structured K/V) is checked at every point of its sweep, flat ratio in
{0.25, 0.5, 0.75} x SAR in {1/32, 1/16, 1/8}.
"""
import math

import pytest
import torch

import oracle as O
from icsa_hip.editing_sparse_attention import _editing_sparse_attention_hip
from icsa_hip.synthetic import make_inputs
from parity import GAP, MAX_ABS, MEAN_ABS, l3_scale

pytestmark = pytest.mark.gpu

CFG3 = dict(H=40, real=32760, pad=8, kind="structured", seed=0)
CASES = {
    "cfg2": dict(H=40, real=32760, pad=8, kind="random", seed=0),
    "unaligned": dict(H=40, real=32760, pad=0, kind="random", seed=7),
    # configuration 5's attention call: 720p, 75,600 tokens per video, CFG batch B = 2
    # (NB = 2363, NKV = 1329, top_k = 83: the large-row paths of every kernel)
    "cfg5": dict(H=40, real=75600, pad=0, kind="random", seed=9, B=2),
}
for _flat in (0.25, 0.5, 0.75):
    for _sar, _tag in ((1 / 32, "1/32"), (1 / 16, "1/16"), (1 / 8, "1/8")):
        CASES[f"cfg3-flat{_flat}-sar{_tag}"] = dict(CFG3, flat_ratio=_flat, sar=_sar)

SAMPLES_PER_KIND = 8          # seeded-random peaked and diffuse blocks per (batch, head)
SP_SWEEP_CONC = 256           # the sparse kernel's sweep constant (sparse_attn.hip)
FA_QBLK_PER_WG = 4            # query blocks per flash workgroup (flash_attn.hip)


def _block_sums(x, NB):
    """float64 [B, H, NB, D] sums of the 64-token blocks of x [B, S, H, D] (zero padded)."""
    B, S, H, D = x.shape
    xp = torch.zeros(B, NB * 64, H, D, dtype=torch.float64, device=x.device)
    xp[:, :S] = x.double()
    return xp.view(B, NB, 64, H, D).sum(2).permute(0, 2, 1, 3)


def _max_rotation_slots(B, H, n_diffuse, NKV, device):
    """Per (batch, head) the diffuse slot whose sparse workgroup starts its exact-list sweep
    furthest along (the kernel's launch order: work w runs as workgroup 8 (w % per) + w / per,
    per = ceil(n_work / 8), and starts at new-KV block ((wg / 8) NKV / SP_SWEEP_CONC) % NKV)
    -> [B, H] positions in the diffuse list."""
    n_work = B * H * n_diffuse
    per = -(-n_work // 8)
    w = torch.arange(n_work, device=device)
    start = ((w % per) * NKV // SP_SWEEP_CONC) % NKV
    return start.view(B, H, n_diffuse).argmax(-1, keepdim=True)


def _sample(blocks, n, gen):
    """n seeded-random entries of each row of blocks [B, H, m] -> [B, H, min(n, m)]."""
    B, H, m = blocks.shape
    k = min(n, m)
    if k == 0:
        return blocks[..., :0]
    pick = torch.rand(B, H, m, generator=gen, device=blocks.device).argsort(-1)[..., :k]
    return torch.gather(blocks, -1, pick)


@pytest.mark.parametrize("case", list(CASES))
def test_full_size_parity(gpu, case):
    c = dict(CASES[case])
    sar = c.pop("sar", 0.0625)
    flat = c.pop("flat_ratio", 0.5)
    print(f"[fullsize] {case}: generating inputs", flush=True)
    q, k, v, t = make_inputs(**c, device=gpu)
    B, S, H, D = q.shape
    g = torch.Generator(device=gpu).manual_seed(11)
    alpha = (torch.rand(B, S, 1, 1, device=gpu, generator=g) - 0.5) * 0.5
    x, views = _editing_sparse_attention_hip(q, k, v, t, alpha, sar, 0.125, flat, keep_workspace=True)
    x_again, _ = _editing_sparse_attention_hip(q, k, v, t, alpha, sar, 0.125, flat)
    x0, _ = _editing_sparse_attention_hip(q, k, v, t, 0.0, sar, 0.125, flat)
    torch.cuda.synchronize()
    z = O.derive_sizes(B, S, H, D, t, sar, 0.125, flat)
    print(f"[fullsize] {case}: S={S} t={t} sizes={z}", flush=True)
    assert torch.equal(x, x_again), "two runs differ"
    assert torch.isfinite(x.float()).all()

    # ---- stage 1 and the compressed softmax ----
    NB = z.NB
    sizes = O.block_sizes(S).to(device=gpu, dtype=torch.float64).view(1, 1, NB, 1)
    qs, ks, vs = _block_sums(q, NB), _block_sums(k, NB), _block_sums(v, NB)
    assert torch.allclose(views["q_sums"].double(), qs, rtol=1e-5, atol=1e-3)
    assert torch.allclose(views["k_sums"].double(), ks, rtol=1e-5, atol=1e-3)
    assert torch.allclose(views["v_sums"].double(), vs, rtol=1e-5, atol=1e-3)
    P, out_c = O.compressed_attention(qs / sizes, ks / sizes, vs / sizes)
    assert torch.allclose(views["P"].double(), P, rtol=1e-4, atol=1e-7)
    assert torch.allclose(views["out_c"].double(), out_c, rtol=1e-4, atol=1e-5)
    # exact linearity in alpha_2 on every token
    oc = out_c.float().repeat_interleave(64, dim=2).permute(0, 2, 1, 3)[:, :S]
    d = (x.float() - x0.float()) - alpha * oc
    assert d.abs().max().item() <= 2e-2 and d.abs().mean().item() <= 1e-3

    # ---- decisions ----
    sel = views["sel"].long()
    order = views["order"].long()
    peaked, diffuse = order[..., :z.n_peaked], order[..., z.n_peaked:]
    assert torch.equal(order.sort(-1).values, torch.arange(NB, device=gpu).expand_as(order))
    _, src_score = O.select_source_blocks(P, z.n_t, z.topK)
    assert O.check_topk_valid(src_score, sel, z.topK, GAP, ordered=True).all()
    _, _, sharp = O.split_blocks(P, z.n_t, z.k_sparsity, z.n_peaked)
    assert O.check_split_valid(sharp, peaked, GAP).all()
    # new KV (GPU selection, closed-form token map) and its block sums
    tokmap = O.new_kv_token_map(t, S, sel.cpu()).to(gpu)             # [B, H, Tkv]
    pad = z.TKV_pad - z.Tkv
    kh, vh = k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)
    idx = tokmap.clamp(min=0)[..., None].expand(-1, -1, -1, D)
    nk = torch.gather(kh, 2, idx).masked_fill((tokmap < 0)[..., None], 0)
    nv = torch.gather(vh, 2, idx).masked_fill((tokmap < 0)[..., None], 0)
    nk = torch.nn.functional.pad(nk, (0, 0, 0, pad))
    nv = torch.nn.functional.pad(nv, (0, 0, 0, pad))
    bi, hi = torch.arange(B, device=gpu).view(B, 1, 1), torch.arange(H, device=gpu).view(1, H, 1)
    l3 = views["l3"].long()
    if z.n_diffuse > 0:
        kc = nk.double().view(B, H, z.NKV, 64, D).sum(3)
        qc = qs[bi, hi, diffuse]
        l3_scores = torch.matmul(qc, kc.transpose(-1, -2).contiguous())
        assert O.check_topk_valid(l3_scores / l3_scale(D), l3, z.top_k, GAP, ordered=False).all()
    print(f"[fullsize] {case}: decisions valid", flush=True)

    # ---- sampled output blocks of every (batch, head), float64 ----
    gs = torch.Generator(device=gpu).manual_seed(1234)
    pk = _sample(peaked, SAMPLES_PER_KIND, gs)                         # [B, H, np]
    if z.n_peaked > 0:
        # always the peaked blocks of the flash grid's last workgroup (a partial one when
        # n_peaked % 4 != 0: its idle slots must leave the real blocks intact)
        last = list(range(FA_QBLK_PER_WG * ((z.n_peaked - 1) // FA_QBLK_PER_WG), z.n_peaked))
        pk = torch.cat([pk, peaked[..., last]], -1)
    dpos = _sample(torch.arange(z.n_diffuse, device=gpu).expand(B, H, z.n_diffuse).contiguous(),
                   SAMPLES_PER_KIND, gs)                               # positions in `diffuse`
    if z.n_diffuse > 0:                                                # and the largest sweep rotation
        dpos = torch.cat([dpos, _max_rotation_slots(B, H, z.n_diffuse, z.NKV, gpu)], -1)
    dk = torch.gather(diffuse, -1, dpos)                               # [B, H, nd]
    qpad = torch.zeros(B, NB * 64, H, D, dtype=torch.float64, device=gpu)
    qpad[:, :S] = q.double()
    qblk = qpad.view(B, NB, 64, H, D).permute(0, 3, 1, 2, 4)          # [B, H, NB, 64, D]
    errs = []

    def add_err(blocks, ref):                                          # ref [B, H, n, 64, D]
        for b in range(B):
            for h in range(H):
                for j, blk in enumerate(blocks[b, h].tolist()):
                    r0, r1 = 64 * blk, min(S, 64 * blk + 64)
                    want = ref[b, h, j, :r1 - r0] + alpha[b, r0:r1, 0].double() * out_c[b, h, blk].view(1, D)
                    errs.append((x[b, r0:r1, h].double() - want).abs())

    if pk.shape[-1] > 0:
        qp = qblk[bi, hi, pk].reshape(B, H, -1, D)
        s = torch.matmul(qp, nk[:, :, :z.Tkv].double().transpose(-1, -2).contiguous()) / math.sqrt(D)
        op = torch.matmul(torch.softmax(s, -1), nv[:, :, :z.Tkv].double())
        add_err(pk, op.view(B, H, -1, 64, D))
    if dk.shape[-1] > 0:
        qd = qblk[bi, hi, dk].reshape(B, H, -1, D)
        lists = torch.gather(l3, 2, dpos[..., None].expand(-1, -1, -1, z.top_k))
        od, _, _ = O.sparse_piecewise_attn(qd, nk.double(), nv.double(), sar, indices=lists)
        add_err(dk, od.view(B, H, -1, 64, D))
    e = torch.cat(errs)
    print(f"[fullsize] {case}: {len(errs)} sampled blocks, max_abs={e.max().item():.3e} "
          f"mean_abs={e.mean().item():.3e}", flush=True)
    assert e.max().item() <= MAX_ABS and e.mean().item() <= MEAN_ABS
