"""Scalar-loop restatement of the path for tiny shapes (test infrastructure only).

Written independently of ``icsa_oracle`` -- explicit Python loops over rows, keys and
blocks, with the sparse kernel's online softmax carried key by key exactly as the
reference kernel's loop structure describes it (tilelang_kernels.py:863-995;
triton_kernels.py:160-247).  It pins the vectorised oracle on shapes small enough for
loops (a few query/key blocks, D <= 16).  Uses numpy float64 only.
"""
from __future__ import annotations

import math

import numpy as np

BLOCK_M = 64


def _rank(values):
    """Ranked order: larger value first, lower index first on ties."""
    return sorted(range(len(values)), key=lambda i: (-values[i], i))


def bf_pool(x):
    """x [S,D] of one (b,h) -> (sums [NB,D], means [NB,D]); esa.py:89-111."""
    S, D = x.shape
    NB = (S + BLOCK_M - 1) // BLOCK_M
    sums = np.zeros((NB, D))
    for n in range(NB):
        for r in range(n * BLOCK_M, min(S, (n + 1) * BLOCK_M)):
            sums[n] += x[r]
    sizes = [BLOCK_M] * NB
    sizes[-1] = S - (NB - 1) * BLOCK_M
    means = np.stack([sums[n] / sizes[n] for n in range(NB)])
    return sums, means


def bf_softmax_row(logits):
    m = max(logits)
    e = [math.exp(x - m) for x in logits]
    z = sum(e)
    return [x / z for x in e]


def bf_compressed(qc, kc, vc):
    """Row-by-row softmax attention on pooled blocks; esa.py:58-64."""
    NB, D = qc.shape
    P = np.zeros((NB, NB))
    out = np.zeros((NB, D))
    for i in range(NB):
        logits = [float(np.dot(qc[i], kc[j])) / math.sqrt(D) for j in range(NB)]
        P[i] = bf_softmax_row(logits)
        for j in range(NB):
            out[i] += P[i, j] * vc[j]
    return P, out


def bf_sparse_piecewise(q, k, v, sparsity, order_exact=None, triton=False, bn=64):
    """One (b,h) of the sparse kernel, scalar loops.  q [TQ,D], k/v [TKV,D].

    For every query row: online softmax over the selected blocks key by key, then the
    interval chunks (``bn`` compressed blocks each, 64 by default) with the non-rescaled
    g_acc/g_l.
    ``order_exact`` optionally fixes the per-block index lists (any order).
    ``triton``: the Triton host's contract (triton_kernels.py:489-539): TQ and TKV need not
    be multiples of 64; a block's sums run over its real rows, the exact loop visits only
    keys below TKV (triton_kernels.py:185), and top_k = max(1, int(sparsity * (TKV // 64))).
    """
    TQ, D = q.shape
    TKV = k.shape[0]
    if not triton:
        assert TQ % BLOCK_M == 0 and TKV % BLOCK_M == 0
    NQ, NKV = -(-TQ // BLOCK_M), -(-TKV // BLOCK_M)
    QC = np.array([q[n * 64:min(TQ, (n + 1) * 64)].sum(0) for n in range(NQ)])
    KC = np.array([k[n * 64:min(TKV, (n + 1) * 64)].sum(0) for n in range(NKV)])
    VC = np.array([v[n * 64:min(TKV, (n + 1) * 64)].sum(0) for n in range(NKV)])
    top_k = max(1, int(sparsity * (TKV // BLOCK_M if triton else NKV)))
    scale = 1.0 / math.sqrt(D)
    out = np.zeros((TQ, D))
    idx_all = []
    for n in range(NQ):
        if order_exact is not None:
            sel = [int(x) for x in order_exact[n]]
        else:
            scores = [float(np.dot(QC[n], KC[j])) for j in range(NKV)]
            sel = _rank(scores)[:top_k]
        idx_all.append(sorted(sel))
        for r in range(n * 64, min(TQ, (n + 1) * 64)):
            m, l, acc = -math.inf, 0.0, np.zeros(D)
            for blk in sel:
                for key in range(blk * 64, min(TKV, (blk + 1) * 64)):
                    s = float(np.dot(q[r], k[key])) * scale
                    m_new = max(m, s)
                    a = math.exp(m - m_new) if m != -math.inf else 0.0
                    p = math.exp(s - m_new)
                    l = l * a + p
                    acc = acc * a + p * v[key]
                    m = m_new
            g_acc, g_l = np.zeros(D), 0.0
            for c0 in range(0, NKV, bn):
                chunk = range(c0, min(NKV, c0 + bn))
                svals = {}
                for j in chunk:
                    if j in sel:
                        continue
                    svals[j] = float(np.dot(q[r], KC[j])) / 64.0 * scale
                cmax = max(svals.values()) if svals else -math.inf
                m_new = max(m, cmax)
                a = math.exp(m - m_new)
                acc = acc * a
                l = l * a
                m = m_new
                for j, s in svals.items():
                    p = math.exp(s - m)
                    g_l += 64.0 * p
                    g_acc = g_acc + p * VC[j]
            den = l + g_l
            out[r] = 0.0 if den == 0 else (acc + g_acc) / den
    return out, idx_all


def bf_dense(q, k, v):
    D = q.shape[1]
    out = np.zeros((q.shape[0], v.shape[1]))
    for r in range(q.shape[0]):
        p = bf_softmax_row([float(np.dot(q[r], k[j])) / math.sqrt(D) for j in range(k.shape[0])])
        for j in range(k.shape[0]):
            out[r] += p[j] * v[j]
    return out


def bf_editing_sparse_attention(q, k, v, t, alpha, sparsity=0.0625, srr=0.125, flat_ratio=0.5):
    """Whole path for one (b,h): q,k,v [S,D] float64, ``alpha`` scalar.

    esa.py:89-232 restated with loops.  Returns (x [S,D], decisions dict).
    """
    S, D = q.shape
    NB = (S + 63) // 64
    _, qc = bf_pool(q)
    _, kc = bf_pool(k)
    _, vc = bf_pool(v)
    P, out_c = bf_compressed(qc, kc, vc)
    n_t = t // 64
    n_s = NB - n_t
    topK = int(n_s * srr)
    src = [sum(P[i, n_t + j] for i in range(n_t)) for j in range(n_s)]
    sel = _rank(src)[:topK]
    # new KV: target tokens then the selected source blocks of the zero-padded sequence
    kp = np.zeros((NB * 64, D)); kp[:S] = k
    vp = np.zeros((NB * 64, D)); vp[:S] = v
    nk, nv = [k[i] for i in range(t)], [v[i] for i in range(t)]
    for r in sel:
        for i in range(64):
            nk.append(kp[n_t * 64 + r * 64 + i])
            nv.append(vp[n_t * 64 + r * 64 + i])
    nk, nv = np.array(nk).reshape(-1, D), np.array(nv).reshape(-1, D)
    Tkv = nk.shape[0]
    k_sp = max(1, int(n_t * sparsity))
    sharp = [sum(sorted(P[i, :n_t], reverse=True)[:k_sp]) for i in range(NB)]
    order = _rank(sharp)
    n_pk = int(NB * flat_ratio)
    peaked, diffuse = order[:n_pk], order[n_pk:]
    qp = np.zeros((NB * 64, D)); qp[:S] = q
    out = np.zeros((NB * 64, D))
    pad = (64 - Tkv % 64) % 64
    nk_sp = np.concatenate([nk, np.zeros((pad, D))])
    nv_sp = np.concatenate([nv, np.zeros((pad, D))])
    if diffuse:
        qd = np.concatenate([qp[b * 64:(b + 1) * 64] for b in diffuse])
        od, l3 = bf_sparse_piecewise(qd, nk_sp, nv_sp, sparsity)
        for n, b in enumerate(diffuse):
            out[b * 64:(b + 1) * 64] = od[n * 64:(n + 1) * 64]
    else:
        l3 = []
    for b in peaked:
        out[b * 64:(b + 1) * 64] = bf_dense(qp[b * 64:(b + 1) * 64], nk, nv)
    x = np.zeros((S, D))
    for s in range(S):
        x[s] = out[s] + alpha * out_c[s // 64]
    return x, dict(sel=sel, peaked=peaked, diffuse=diffuse, l3=l3, src_score=src,
                   sharpness=sharp, P=P, out_c=out_c)
