"""Trie-verification attention on the CPU (numpy) -- oracle restatements.

attn_hyb      restates the reference kernel _attn_hyb (respect/kernels/attention.py:15-71):
              prompt keys in BN-wide tiles with online softmax and p rounded to
              bf16 before the PV product (:36-50); node slots folded one slot at
              a time in slot order with fp32 p (:52-67); out = bf16(acc / l) (:69-71).
              Tensor-core dot products are modelled as exact sums rounded once
              to fp32 (bf16 x bf16 products are exact in fp32).
attn_blocked  restates the development kernel _fused_attn
              (respect/kernels/reference_blocked.py:14-80): node slots reduced
              tile by tile like the prompt -- the layout-dependent negative control.
attn_exact    float64 masked softmax attention (the mathematical definition).

Inputs are float32 arrays holding bf16 values: q [H, M, D], kp/vp [HK, P, D],
kn/vn [HK, NN, D], msk [M, NN] bool.  Head h uses kv head h // (H // HK).

Pinned by (tests/test_oracle.py): attn_hyb vs attn_exact within bf16 rounding
bounds on random inputs (a dropped term, wrong sign, swapped operand or wrong
scale fails it); single allowed key => out == v exactly; equal scores =>
out == bf16(mean v); masked node slots are exact no-ops (layout invariance of
attn_hyb); attn_blocked *does* change with the layout (the control detects
layout dependence); brute-force per-row fp64 recomputation on tiny inputs.
"""
from __future__ import annotations

import numpy as np

from .bf16 import round_bf16


def _kv_for_heads(x: np.ndarray, H: int) -> np.ndarray:
    HK = x.shape[0]
    return np.repeat(x, H // HK, axis=0)


def _dot32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """fp32 matrix product with exact accumulation rounded once: 'hmd,hnd->hmn'."""
    return np.einsum("hmd,hnd->hmn", a.astype(np.float64), b.astype(np.float64)).astype(np.float32)


def attn_hyb(q, kp, vp, kn, vn, msk, sm_scale=None, BN: int = 128, BNB: int = 16) -> np.ndarray:
    """Logical-order trie attention of attention.py:15-96; returns float32 bf16 values [H, M, D]."""
    q = np.asarray(q, np.float32)
    H, M, D = q.shape
    HK, P, _ = kp.shape
    NN = kn.shape[1]
    assert NN % BNB == 0, "attention.py:79 requires NN % BNB == 0"
    scale = np.float32(D ** -0.5 if sm_scale is None else sm_scale)
    KP, VP = _kv_for_heads(kp, H), _kv_for_heads(vp, H)
    KN, VN = _kv_for_heads(kn, H), _kv_for_heads(vn, H)
    msk = np.asarray(msk, dtype=bool)
    m_i = np.full((H, M), -np.inf, np.float32)
    l_i = np.zeros((H, M), np.float32)
    acc = np.zeros((H, M, D), np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        for start in range(0, P, BN):
            k = KP[:, start:start + BN]
            v = VP[:, start:start + BN]
            qk = _dot32(q, k) * scale
            m_new = np.maximum(m_i, qk.max(axis=2))
            alpha = np.exp(m_i - m_new)
            p = np.exp(qk - m_new[..., None])
            pv = np.einsum("hmn,hnd->hmd", round_bf16(p).astype(np.float64),
                           v.astype(np.float64)).astype(np.float32)
            acc = acc * alpha[..., None] + pv
            l_i = l_i * alpha + p.sum(axis=2, dtype=np.float32)
            m_i = m_new
        for start in range(0, NN, BNB):
            qk = _dot32(q, KN[:, start:start + BNB]) * scale
            qk = np.where(msk[None, :, start:start + BNB], qk, np.float32(-np.inf))
            for j in range(BNB):
                qkj = qk[..., j]
                m_new = np.maximum(m_i, qkj)
                alpha = np.exp(m_i - m_new)
                p = np.exp(qkj - m_new)
                v = VN[:, start + j]
                acc = acc * alpha[..., None] + p[..., None] * v[:, None, :]
                l_i = l_i * alpha + p
                m_i = m_new
        out = acc / l_i[..., None]
    return round_bf16(out)


def attn_blocked(q, kp, vp, kn, vn, msk, sm_scale=None, BN: int = 64) -> np.ndarray:
    """Tile-wise node reduction of reference_blocked.py:14-80 (negative control)."""
    q = np.asarray(q, np.float32)
    H, M, D = q.shape
    HK, P, _ = kp.shape
    NN = kn.shape[1]
    scale = np.float32(D ** -0.5 if sm_scale is None else sm_scale)
    msk = np.asarray(msk, dtype=bool)
    m_i = np.full((H, M), -np.inf, np.float32)
    l_i = np.zeros((H, M), np.float32)
    acc = np.zeros((H, M, D), np.float32)

    def tile(k, v, allow):
        nonlocal m_i, l_i, acc
        qk = _dot32(q, k) * scale
        if allow is not None:
            qk = np.where(allow[None], qk, np.float32(-np.inf))
        m_new = np.maximum(m_i, qk.max(axis=2))
        alpha = np.exp(m_i - m_new)
        p = np.exp(qk - m_new[..., None])
        pv = np.einsum("hmn,hnd->hmd", round_bf16(p).astype(np.float64),
                       v.astype(np.float64)).astype(np.float32)
        acc = acc * alpha[..., None] + pv
        l_i = l_i * alpha + p.sum(axis=2, dtype=np.float32)
        m_i = m_new

    KP, VP = _kv_for_heads(kp, H), _kv_for_heads(vp, H)
    KN, VN = _kv_for_heads(kn, H), _kv_for_heads(vn, H)
    with np.errstate(invalid="ignore", over="ignore"):
        for start in range(0, P, BN):
            tile(KP[:, start:start + BN], VP[:, start:start + BN], None)
        for start in range(0, NN, BN):
            tile(KN[:, start:start + BN], VN[:, start:start + BN], msk[:, start:start + BN])
        out = acc / l_i[..., None]
    return round_bf16(out)


def attn_exact(q, kp, vp, kn, vn, msk, sm_scale=None) -> np.ndarray:
    """float64 softmax(q k^T * scale) v over the prompt keys and the allowed node slots."""
    q = np.asarray(q, np.float64)
    H, M, D = q.shape
    scale = D ** -0.5 if sm_scale is None else float(sm_scale)
    K = np.concatenate([_kv_for_heads(kp, H), _kv_for_heads(kn, H)], axis=1).astype(np.float64)
    V = np.concatenate([_kv_for_heads(vp, H), _kv_for_heads(vn, H)], axis=1).astype(np.float64)
    P = kp.shape[1]
    allow = np.concatenate([np.ones((M, P), bool), np.asarray(msk, bool)], axis=1)
    s = np.einsum("hmd,hnd->hmn", q, K) * scale
    s = np.where(allow[None], s, -np.inf)
    s = s - s.max(axis=2, keepdims=True)
    e = np.exp(s)
    return np.einsum("hmn,hnd->hmd", e, V) / e.sum(axis=2)[..., None]


def attn_rows_bruteforce(q, kp, vp, kn, vn, msk, sm_scale=None) -> np.ndarray:
    """Per-row, per-head loop over explicitly gathered allowed keys (tiny inputs only)."""
    q = np.asarray(q, np.float64)
    H, M, D = q.shape
    HK = kp.shape[0]
    scale = D ** -0.5 if sm_scale is None else float(sm_scale)
    out = np.zeros((H, M, D))
    for h in range(H):
        g = h // (H // HK)
        for m in range(M):
            keys = [kp[g, t] for t in range(kp.shape[1])]
            vals = [vp[g, t] for t in range(vp.shape[1])]
            for t in range(kn.shape[1]):
                if msk[m, t]:
                    keys.append(kn[g, t])
                    vals.append(vn[g, t])
            s = np.array([float(np.dot(q[h, m], np.asarray(k, np.float64))) * scale for k in keys])
            w = np.exp(s - s.max())
            w /= w.sum()
            out[h, m] = sum(wi * np.asarray(v, np.float64) for wi, v in zip(w, vals))
    return out


def attn_error_bound(q, kp, vp, kn, vn, msk, sm_scale=None) -> np.ndarray:
    """Per-element bound on |out - attn_exact| for any kernel that follows the reference's
    rounding points (prompt p rounded to bf16 before PV, fp32 accumulation, one bf16
    rounding of the output):

        2^-9 * sum_prompt p_i |v_i| / sum_all p_i     (bf16 p: relative error <= 2^-9)
      + 2^-20 * sum_all p_i |v_i| / sum_all p_i       (fp32 accumulation and exp)
      + 1 bf16 ulp of the exact value                 (final rounding, with margin)

    p_i are the exact softmax weights.  The bound is deterministic, not statistical.
    """
    q = np.asarray(q, np.float64)
    H, M, D = q.shape
    scale = D ** -0.5 if sm_scale is None else float(sm_scale)
    P = kp.shape[1]
    K = np.concatenate([_kv_for_heads(kp, H), _kv_for_heads(kn, H)], axis=1).astype(np.float64)
    V = np.abs(np.concatenate([_kv_for_heads(vp, H), _kv_for_heads(vn, H)], axis=1).astype(np.float64))
    allow = np.concatenate([np.ones((M, P), bool), np.asarray(msk, bool)], axis=1)
    s = np.einsum("hmd,hnd->hmn", q, K) * scale
    s = np.where(allow[None], s, -np.inf)
    e = np.exp(s - s.max(axis=2, keepdims=True))
    l = e.sum(axis=2)[..., None]
    wv_prompt = np.einsum("hmn,hnd->hmd", e[..., :P], V[:, :P]) / l
    wv_all = np.einsum("hmn,hnd->hmd", e, V) / l
    exact = attn_exact(q, kp, vp, kn, vn, msk, sm_scale)
    from .bf16 import ulp
    return 2.0 ** -9 * wv_prompt + 2.0 ** -20 * wv_all + ulp(exact)
