"""Pins the attention oracle (oracle/ref.py: rope_f64, sdpa_f64) on the CPU.

rope: the reference test's hand-worked rotation (rope.gpu.test.ts:107-114),
pair norms kept, rotations composing by angle. sdpa: closed forms (one
visible key, equal scores, the sink's share of the denominator, rows that
see nothing) and an independent per-row formulation (softmax over the
visible slice with the sink as an extra logit whose value row is 0) over
the reference test's mask and input options (checkSdpa.ts:34-52).
"""
import math

import numpy as np
import pytest

from oracle import ref


def test_rope_hand_worked():
    # Position 1, headDim 2: (1, 0) turns to (cos 1, sin 1)... the reference
    # test's two rows: row 0 angle 0, row 1 angle 1.
    x = np.array([[1.0, 0.0], [0.0, 1.0]])
    cos = np.array([1.0, 1.0, math.cos(1), math.cos(1)])
    sin = np.array([0.0, 0.0, math.sin(1), math.sin(1)])
    got = ref.rope_f64(x, cos, sin, 2).reshape(-1)
    np.testing.assert_allclose(got, [1, 0, -math.sin(1), math.cos(1)], atol=1e-15)


def _tables(rows, hd, scale=1.0):
    ang = np.arange(rows)[:, None] * 10000.0 ** (-2 * np.arange(hd // 2) / hd)[None, :]
    c = np.repeat(np.cos(ang), 2, axis=1) * scale
    s = np.repeat(np.sin(ang), 2, axis=1) * scale
    return c.reshape(-1), s.reshape(-1), ang


def test_rope_keeps_pair_norms_and_composes():
    rng = np.random.default_rng(0)
    rows, hd = 7, 10
    x = rng.standard_normal((rows, 3 * hd))
    c, s, ang = _tables(rows, hd)
    y = ref.rope_f64(x, c, s, hd)
    n0 = x[:, 0::2] ** 2 + x[:, 1::2] ** 2
    n1 = y[:, 0::2] ** 2 + y[:, 1::2] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-12)
    # rotating by a, then by b, is rotating by a + b
    c2, s2 = np.repeat(np.cos(2 * ang), 2, 1).reshape(-1), np.repeat(np.sin(2 * ang), 2, 1).reshape(-1)
    np.testing.assert_allclose(ref.rope_f64(y, c, s, hd), ref.rope_f64(x, c2, s2, hd), atol=1e-12)


def test_rope_window_of_a_wider_slab():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((9, 8 * 16))
    c, s, _ = _tables(9, 16)
    full = ref.rope_f64(x, c, s, 16)
    part = ref.rope_f64(x, c, s, 16, src_start=64, width=32)
    np.testing.assert_array_equal(part, full[:, 64:96])


def _sdpa_slices(q, k, v, qh, kvh, hd, wl, wr, off, sinks, segs, kb):
    """Row by row, head by head: scipy-free softmax over the visible slice
    with the sink appended as one more logit (its value row 0)."""
    q_len, kv_len = q.shape[0], k.shape[0]
    g = qh // kvh
    out = np.zeros((q_len, qh * hd))
    for i in range(q_len):
        qpos = off + i
        lo = 0 if wl == math.inf else max(0, qpos - wl)
        hi = kv_len - 1 if wr == math.inf else min(kv_len - 1, qpos + wr)
        if segs is not None:
            lo, hi = max(lo, int(segs[2 * i])), min(hi, int(segs[2 * i + 1]) - 1)
        for h in range(qh):
            c = h // g
            keys = list(range(lo, hi + 1))
            logits = [float(np.dot(q[i, h * hd:(h + 1) * hd], k[j, c * hd:(c + 1) * hd])) +
                      (kb[2] if kb and kb[0] <= j < kb[1] else 0.0) for j in keys]
            rows = [v[j, c * hd:(c + 1) * hd] for j in keys]
            if sinks is not None:
                logits.append(float(sinks[h]) * math.log(2))
                rows.append(np.zeros(hd))
            if not logits:
                continue
            m = max(logits)
            w = np.exp(np.array(logits) - m)
            out[i, h * hd:(h + 1) * hd] = (w[:, None] * np.array(rows)).sum(0) / w.sum()
    return out


OPTIONS = [
    dict(), dict(wr=0), dict(wl=3, wr=0), dict(wl=2, wr=1), dict(sinks=True, wr=0),
    dict(segs=True), dict(segs=True, wr=0), dict(kb=True, wr=0),
    dict(kb=True, sinks=True, segs=True), dict(kvh=1, wr=0), dict(qh=6, kvh=2, sinks=True, wr=0),
    dict(kvh=4), dict(off=14, kv=20, q=6, wr=0), dict(q=6, kv=4, wl=0, sinks=True),
]


@pytest.mark.parametrize("o", OPTIONS, ids=[str(o) for o in OPTIONS])
def test_sdpa_matches_the_per_row_formulation(o):
    q_len, kv_len = o.get("q", 13), o.get("kv", o.get("q", 13))
    qh, kvh, hd = o.get("qh", 4), o.get("kvh", 2), 5
    rng = np.random.default_rng(7)
    q = rng.standard_normal((q_len, qh * hd)) * 2 / math.sqrt(hd)
    k = rng.standard_normal((kv_len, kvh * hd))
    v = rng.standard_normal((kv_len, kvh * hd))
    wl, wr, off = o.get("wl", math.inf), o.get("wr", math.inf), o.get("off", 0)
    sinks = rng.standard_normal(qh) * 2 if o.get("sinks") else None
    segs = None
    if o.get("segs"):
        segs = np.array([[0, kv_len // 2] if r < q_len // 2 else [kv_len // 2, kv_len]
                         for r in range(q_len)], np.float64).reshape(-1)
    kb = (kv_len // 4, kv_len // 2, 2.0) if o.get("kb") else None
    got = ref.sdpa_f64(q, k, v, qh, kvh, hd, wl, wr, off, sinks, segs, kb)
    want = _sdpa_slices(q, k, v, qh, kvh, hd, wl, wr, off, sinks, segs, kb)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-13)


def test_sdpa_closed_forms():
    rng = np.random.default_rng(3)
    T, hd = 9, 4
    k = rng.standard_normal((T, hd))
    v = rng.standard_normal((T, hd))
    q = rng.standard_normal((T, hd))
    # window (0, 0): each row sees only its own key → its v row
    np.testing.assert_allclose(ref.sdpa_f64(q, k, v, 1, 1, hd, 0, 0), v, atol=1e-15)
    # q = 0: equal scores → the mean of the visible v rows (causal: prefix means)
    z = np.zeros_like(q)
    want = np.cumsum(v, 0) / np.arange(1, T + 1)[:, None]
    np.testing.assert_allclose(ref.sdpa_f64(z, k, v, 1, 1, hd, math.inf, 0), want, atol=1e-14)
    # with a sink σ the n equal weights share the denominator with 2^σ
    sig = 1.5
    n = np.arange(1, T + 1)[:, None]
    got = ref.sdpa_f64(z, k, v, 1, 1, hd, math.inf, 0, sinks=np.array([sig]))
    np.testing.assert_allclose(got, want * n / (n + 2.0 ** sig), atol=1e-14)
    # a key bias of b on one key of two: weights e^b : 1
    q2, k2, v2 = np.zeros((1, hd)), np.zeros((2, hd)), np.array([[1.0] * hd, [0.0] * hd])
    got = ref.sdpa_f64(q2, k2, v2, 1, 1, hd, key_bias=(0, 1, 2.0))
    np.testing.assert_allclose(got, np.full((1, hd), math.e ** 2 / (math.e ** 2 + 1)), atol=1e-15)


def test_sdpa_rows_that_see_nothing_are_zero():
    rng = np.random.default_rng(4)
    q, k, v = rng.standard_normal((6, 8)), rng.standard_normal((4, 4)), rng.standard_normal((4, 4))
    # rows 4 and 5 sit past the 4 keys with windowLeft 0
    for sinks in (None, np.array([0.5, -1.0])):
        got = ref.sdpa_f64(q, k, v, 2, 1, 4, 0, math.inf, sinks=sinks)
        assert np.all(got[4:] == 0) and np.all(np.isfinite(got))
