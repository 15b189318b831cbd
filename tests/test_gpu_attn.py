"""Parity of the attention ops through the C ABI against the f64 oracle
(oracle/ref.py: rope_f64, sdpa_f64).

sdpa: every mask and input option of the reference's attention suite
(test/core/kernels/attention/checkSdpa.ts:34-52) on its shapes (t = 37,
200, 300 at headDim 40, 4 query heads, 2 kv heads, attn.gpu.test.ts:27-48)
and its special shapes (:50-120, headDim ≤ 128), plus the privacy-filter
block's attention (14 query heads on 2 kv heads, headDim 64, window ±128,
sinks); inputs are the reference test's seeded randomF32 (q scaled by
2/√headDim), tolerance its own (f32 atol 2e-5, rtol 1e-4; f16 2e-3, 4e-3).
rope: the reference's cases (rope.gpu.test.ts:80-134) at its tolerance.
"""
import math

import numpy as np
import pytest
import torch

import runntime_amd as rt
from oracle import ref

pytestmark = pytest.mark.gpu

DEV = "cuda"
TD = {"f32": torch.float32, "f16": torch.float16}
TOL = {"f32": dict(atol=2e-5, rtol=1e-4), "f16": dict(atol=2e-3, rtol=4e-3)}


def say(msg):
    print(msg, flush=True)


def rnd(v, dtype):
    return v.astype(np.float16).astype(np.float32) if dtype == "f16" else v


def dev(a, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dt)


def check_sdpa(c, dtype="f32"):
    q_len, kv_len, qh, kvh, hd = c["qLen"], c["kvLen"], c["qHeads"], c["kvHeads"], c["headDim"]
    wl, wr = c.get("windowLeft", math.inf), c.get("windowRight", math.inf)
    off = c.get("qPosOffset", 0)
    say(f"sdpa {dtype} {c}")
    scale = 2 / math.sqrt(hd)
    q = rnd(ref.lcg_f32(q_len * qh * hd, 1) * np.float32(scale), dtype).reshape(q_len, qh * hd)
    k = rnd(ref.lcg_f32(kv_len * kvh * hd, 2), dtype).reshape(kv_len, kvh * hd)
    v = rnd(ref.lcg_f32(kv_len * kvh * hd, 3), dtype).reshape(kv_len, kvh * hd)
    sinks = ref.lcg_f32(qh, 4) * 2 if c.get("sinks") else None
    segs = None
    if c.get("segments"):
        qhalf, kvhalf = q_len // 2, kv_len // 2
        segs = np.array([[0, kvhalf] if r < qhalf else [kvhalf, kv_len] for r in range(q_len)],
                        np.float32).reshape(-1)
    kb = (kv_len // 4, kv_len // 2, 2.0) if c.get("keyBias") else None
    opts = dict(qHeads=qh, kvHeads=kvh, headDim=hd, windowLeft=wl, windowRight=wr,
                qPosOffset=off, sinks=dev(sinks) if sinks is not None else None,
                segments=dev(segs) if segs is not None else None)
    t = TD[dtype]
    if c.get("packed"):
        qkv = np.concatenate([q, k, v], axis=1)
        got = rt.sdpaPacked(dev(qkv, t), opts)
    else:
        if kb:
            opts["keyBias"] = dict(start=kb[0], end=kb[1], value=kb[2])
        got = rt.sdpa(dev(q, t), dev(k, t), dev(v, t), opts)
    torch.cuda.synchronize()
    want = ref.sdpa_f64(q, k, v, qh, kvh, hd, wl, wr, off, sinks, segs, kb)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, **TOL[dtype])


OPTIONS = [
    ("full", {}),
    ("causal", dict(windowRight=0)),
    ("a sliding window", dict(windowLeft=3, windowRight=0)),
    ("a two-sided window", dict(windowLeft=2, windowRight=1)),
    ("sinks", dict(sinks=True, windowRight=0)),
    ("segments", dict(segments=True)),
    ("segments and causal", dict(segments=True, windowRight=0)),
    ("packed qkv", dict(packed=True, windowRight=0)),
    ("packed qkv, sinks and segments", dict(packed=True, sinks=True, segments=True)),
    ("a key bias", dict(keyBias=True, windowRight=0)),
    ("a key bias, sinks and segments", dict(keyBias=True, sinks=True, segments=True)),
    ("every query head on one kv head", dict(kvHeads=1, windowRight=0)),
    ("three query heads per kv head", dict(qHeads=6, kvHeads=2, sinks=True, windowRight=0)),
    ("as many kv heads as query heads", dict(kvHeads=4)),
]


@pytest.mark.parametrize("dtype,t", [("f32", 37), ("f32", 300), ("f32", 200), ("f16", 200),
                                     ("f16", 37)])
@pytest.mark.parametrize("name,o", OPTIONS, ids=[o[0] for o in OPTIONS])
def test_sdpa_options(dtype, t, name, o):
    c = dict(qLen=t, kvLen=t, qHeads=4, kvHeads=2, headDim=40)
    c.update(o)
    check_sdpa(c, dtype)


SHAPES = [
    ("headDim 1", dict(qLen=5, kvLen=5, qHeads=2, kvHeads=1, headDim=1)),
    ("cross-attention over 1700 keys", dict(qLen=5, kvLen=1700, qHeads=2, kvHeads=1, headDim=8)),
    ("qPosOffset into a longer cache",
     dict(qLen=6, kvLen=20, qHeads=2, kvHeads=1, headDim=8, windowRight=0, qPosOffset=14)),
    ("rows that see no key, with sinks",
     dict(qLen=6, kvLen=4, qHeads=2, kvHeads=1, headDim=8, windowLeft=0, sinks=True)),
    ("rows that see no key, with sinks, 120 rows",
     dict(qLen=120, kvLen=100, qHeads=2, kvHeads=1, headDim=8, windowLeft=0, sinks=True)),
    ("at the 96-key chunk", dict(qLen=96, kvLen=96, qHeads=2, kvHeads=1, headDim=8, windowRight=0)),
    ("headDim 128", dict(qLen=33, kvLen=33, qHeads=4, kvHeads=2, headDim=128, sinks=True)),
    ("headDim 72", dict(qLen=50, kvLen=70, qHeads=2, kvHeads=2, headDim=72, windowLeft=9,
                        windowRight=4, qPosOffset=3)),
    ("privacy-filter attention", dict(qLen=300, kvLen=300, qHeads=14, kvHeads=2, headDim=64,
                                      windowLeft=128, windowRight=128, sinks=True)),
    ("privacy-filter attention, packed", dict(qLen=517, kvLen=517, qHeads=14, kvHeads=2,
                                              headDim=64, windowLeft=128, windowRight=128,
                                              sinks=True, packed=True)),
    ("one query row", dict(qLen=1, kvLen=300, qHeads=14, kvHeads=2, headDim=64, sinks=True)),
    ("64 query heads on one kv head", dict(qLen=9, kvLen=9, qHeads=64, kvHeads=1, headDim=16)),
]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("name,c", SHAPES, ids=[s[0] for s in SHAPES])
def test_sdpa_shapes(dtype, name, c):
    check_sdpa(dict(c), dtype)


def test_sdpa_rejects_what_the_kernel_cannot_take():
    q = torch.zeros((4, 2 * 200), device=DEV)
    k = torch.zeros((4, 200), device=DEV)
    with pytest.raises(ValueError, match=r"headDim 200 exceeds the kernel's max \(128\)"):
        rt.sdpa(q, k, k, dict(qHeads=2, kvHeads=1, headDim=200, windowLeft=math.inf,
                              windowRight=math.inf))


# ------------------------------------------------------------------- rope

def rope_tables(rows, hd):
    """The test's tables: angle t · 10000^(−2i/headDim), pair-duplicated."""
    ang = np.arange(rows)[:, None] * 10000.0 ** (-2 * np.arange(hd // 2) / hd)[None, :]
    c = np.repeat(np.cos(ang), 2, axis=1).astype(np.float32)
    s = np.repeat(np.sin(ang), 2, axis=1).astype(np.float32)
    return c, s


def check_rope(rows, cols, hd, src_start=None, width=None, dtype="f32"):
    say(f"rope {dtype} rows={rows} cols={cols} hd={hd} src={src_start} width={width}")
    x = rnd(ref.lcg_f32(rows * cols, 1), dtype).reshape(rows, cols)
    c, s = rope_tables(rows, hd)
    opts = dict(headDim=hd)
    if src_start is not None:
        opts.update(srcStart=src_start, width=width)
    got = rt.rope(dev(x, TD[dtype]), dev(c), dev(s), opts)
    torch.cuda.synchronize()
    want = ref.rope_f64(x, c, s, hd, src_start or 0, width)
    tol = dict(atol=1e-3, rtol=1e-3) if dtype == "f16" else dict(atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, **tol)


ROPE_CASES = [
    ("one pair", (1, 2, 2)),
    ("one head", (5, 64, 64)),
    ("several heads, odd row count", (7, 60, 10)),
    ("pairs not a multiple of the workgroup", (3, 4 * 34, 34)),
    ("a slice of a wider slab", (9, 8 * 16, 16, 4 * 16, 2 * 16)),
    ("the last head of a slab", (3, 48, 16, 32, 16)),
]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("name,a", ROPE_CASES, ids=[c[0] for c in ROPE_CASES])
def test_rope_cases(dtype, name, a):
    check_rope(*a, dtype=dtype)


def test_rope_hand_worked():
    x = dev(np.array([[1, 0], [0, 1]], np.float32))
    c = dev(np.array([[1, 1], [math.cos(1), math.cos(1)]], np.float32))
    s = dev(np.array([[0, 0], [math.sin(1), math.sin(1)]], np.float32))
    got = rt.rope(x, c, s, dict(headDim=2)).cpu().numpy().reshape(-1)
    np.testing.assert_allclose(got, [1, 0, -math.sin(1), math.cos(1)], atol=1e-7, rtol=1e-6)


def test_rope_past_2p24_elements():
    check_rope(4100, 4096, 64)


def test_rope_f16_past_2p24_pairs():
    check_rope(2 ** 14 + 1, 2048, 64, dtype="f16")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_sdpa_long_sequence_sampled_rows(dtype):
    """T = 4096 with the privacy filter's window and sinks; rows checked on
    three ranges, each against the oracle run on those rows as queries at
    their positions (qPosOffset) over all keys."""
    T, qh, kvh, hd = 4096, 14, 2, 64
    say(f"sdpa long {dtype} T={T}")
    rng = np.random.default_rng(8)
    q = rnd((rng.standard_normal((T, qh * hd)) * 2 / math.sqrt(hd)).astype(np.float32), dtype)
    k = rnd(rng.standard_normal((T, kvh * hd)).astype(np.float32), dtype)
    v = rnd(rng.standard_normal((T, kvh * hd)).astype(np.float32), dtype)
    sinks = rng.standard_normal(qh).astype(np.float32)
    t = TD[dtype]
    got = rt.sdpa(dev(q, t), dev(k, t), dev(v, t),
                  dict(qHeads=qh, kvHeads=kvh, headDim=hd, windowLeft=128, windowRight=128,
                       sinks=dev(sinks))).float().cpu().numpy()
    for r0 in (0, 2000, T - 64):
        want = ref.sdpa_f64(q[r0:r0 + 64], k, v, qh, kvh, hd, 128, 128, r0, sinks)
        np.testing.assert_allclose(got[r0:r0 + 64], want, **TOL[dtype])


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("T", [1, 57, 300])
def test_fused_attention_core(dtype, T):
    """moe_attention (rope of the q and k blocks, then banded sdpa over one
    qkv tensor, attnBlock.ts:39-55) against the oracle's rope_f64 and
    sdpa_f64 composed, at the sdpa tolerance."""
    from runntime_amd import _lib
    from runntime_amd.core import _ctx, _xdtype
    from runntime_amd import privacy_filter as pf
    qh, kvh, hd = 14, 2, 64
    say(f"moe_attention {dtype} T={T}")
    rng = np.random.default_rng(T)
    qkv = rnd(rng.standard_normal((T, (qh + 2 * kvh) * hd)).astype(np.float32), dtype)
    sinks = rng.standard_normal(qh).astype(np.float32)
    cos, sin = pf.rope_constants(T)
    t = TD[dtype]
    # every device tensor held until the kernel has run
    dq, ds, dc, dsn = dev(qkv, t), dev(sinks), dev(cos), dev(sin)
    out = torch.empty((T, qh * hd), dtype=t, device=DEV)
    _lib.check(_lib.load().moe_attention(_ctx(dq.device), dq.data_ptr(), _xdtype(dq), T, qh, kvh,
                                         hd, 128, 128, ds.data_ptr(), dc.data_ptr(),
                                         dsn.data_ptr(), out.data_ptr()))
    torch.cuda.synchronize()
    q = ref.rope_f64(qkv, cos, sin, hd, 0, qh * hd)
    k = ref.rope_f64(qkv, cos, sin, hd, qh * hd, kvh * hd)
    v = qkv[:, (qh + kvh) * hd:].astype(np.float64)
    want = ref.sdpa_f64(q, k, v, qh, kvh, hd, 128, 128, 0, sinks)
    np.testing.assert_allclose(out.float().cpu().numpy(), want, **TOL[dtype])
