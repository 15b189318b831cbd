"""numpy front end of the C oracle (moe_oracle.c).

TEST INFRASTRUCTURE ONLY — the checker for the HIP kernels; only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
"""
import ctypes
import os

import numpy as np

from . import build as _build

_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


class _Opt:
    """ndpointer that also accepts None (a NULL pointer)."""

    def __init__(self, base):
        self.base = base

    def from_param(self, v):
        if v is None:
            return None
        return self.base.from_param(v)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_build.OUT):
        _build.build()
    L = ctypes.CDLL(_build.OUT)
    I, I64, U32 = ctypes.c_int, ctypes.c_int64, ctypes.c_uint32
    F = _Opt(_f32p)
    sigs = {
        "orc_lcg_f32": [_f32p, I64, U32],
        "orc_pack_quantw_nk": [_i8p, I, I, I, _u32p],
        "orc_pack_quantw_ekn": [_i8p, I, I, I, I, _u32p],
        "orc_unpack_quantw": [_u32p, I, I, I, I, _i8p],
        "orc_topk": [_f32p, I, I, I, _f32p],
        "orc_router_logits": [_f32p, _f32p, F, I, I, I, _f32p],
        "orc_moe_up_f64": [_f32p, _f32p, _u32p, _f32p, F, _u32p, _f32p, F, I, I, I, I, I, I, I,
                           _f32p],
        "orc_moe_down_f64": [_f32p, _f32p, _u32p, _f32p, F, F, I, I, I, I, I, I, I, _f32p],
        "orc_moe_up_f32ref": [_f32p, _f32p, _u32p, _f32p, F, _u32p, _f32p, F, I, I, I, I, I, I,
                              I, _f32p],
        "orc_moe_down_f32ref": [_f32p, _f32p, _u32p, _f32p, F, F, I, I, I, I, I, I, I, _f32p],
        "orc_dispatch": [_f32p, I, I, I, _i32p, _i32p, _i32p],
        "orc_moe_layer_f64": [_f32p, _f32p, F, _u32p, _f32p, F, _u32p, _f32p, F, _u32p, _f32p, F,
                              F, I, I, I, I, I, I, I, I, _f32p, _f32p, _f32p],
    }
    sigs["orc_rmsnorm"] = [_f32p, I64, I, I, _f32p, I, ctypes.c_float, F, ctypes.c_float, _f32p]
    for name, args in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = None
    L.orc_swiglu_f64.argtypes = [ctypes.c_double, ctypes.c_double]
    L.orc_swiglu_f64.restype = ctypes.c_double
    _lib = L
    return L


def _f(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def lcg_f32(n, seed):
    out = np.empty(n, np.float32)
    lib().orc_lcg_f32(out, n, seed)
    return out


def pack_nk(ints_nk, k, n, bits):
    words = np.zeros(k * n * bits // 32, np.uint32)
    lib().orc_pack_quantw_nk(np.ascontiguousarray(ints_nk, np.int8), k, n, bits, words)
    return words


def pack_ekn(q, bits):
    E, K, N = q.shape
    words = np.zeros(E * K * N * bits // 32, np.uint32)
    lib().orc_pack_quantw_ekn(np.ascontiguousarray(q, np.int8), E, K, N, bits, words)
    return words


def unpack(words, E, K, N, bits):
    q = np.zeros((E, K, N), np.int8)
    lib().orc_unpack_quantw(np.ascontiguousarray(words, np.uint32), E, K, N, bits, q)
    return q


def topk(logits, k):
    T, E = logits.shape
    route = np.zeros((T, 2 * k), np.float32)
    lib().orc_topk(_f(logits), T, E, k, route)
    return route


def router_logits(x, w, b=None):
    T, d = x.shape
    E = w.shape[1]
    out = np.zeros((T, E), np.float32)
    lib().orc_router_logits(_f(x), _f(w), _f(b), T, d, E, out)
    return out


def swiglu(g, l):
    return lib().orc_swiglu_f64(float(g), float(l))


def moe_up(x, route, glu, lin, bits, g, E, f32ref=False):
    """glu/lin: (words uint32, scales f32 [E·K/g, N], bias f32 [E, N] or None)."""
    T, K = x.shape
    k = route.shape[1] // 2
    N = glu[1].shape[-1]
    act = np.zeros((T * k, N), np.float32)
    fn = lib().orc_moe_up_f32ref if f32ref else lib().orc_moe_up_f64
    fn(_f(x), _f(route), np.ascontiguousarray(glu[0], np.uint32), _f(glu[1]), _f(glu[2]),
       np.ascontiguousarray(lin[0], np.uint32), _f(lin[1]), _f(lin[2]), T, K, N, E, k, bits, g,
       act)
    return act


def moe_down(act, route, down, residual, bits, g, E, f32ref=False):
    rows, K = act.shape
    k = route.shape[1] // 2
    T = rows // k
    N = down[1].shape[-1]
    out = np.zeros((T, N), np.float32)
    fn = lib().orc_moe_down_f32ref if f32ref else lib().orc_moe_down_f64
    fn(_f(act), _f(route), np.ascontiguousarray(down[0], np.uint32), _f(down[1]), _f(down[2]),
       _f(residual), T, K, N, E, k, bits, g, out)
    return out


def dispatch(route, E):
    T = route.shape[0]
    k = route.shape[1] // 2
    perm = np.zeros(T * k, np.int32)
    inv = np.zeros(T * k, np.int32)
    offsets = np.zeros(E + 1, np.int32)
    lib().orc_dispatch(_f(route), T, k, E, perm, inv, offsets)
    return perm, inv, offsets


def rmsnorm(x, weight, eps, group=None, residual=None, scale=1.0, dtype=np.float32):
    """rmsNorm in the canonical order. x, weight, residual hold values of
    `dtype` (f32 or f16); the result is rounded to `dtype` as the kernel
    stores it."""
    rows, cols = x.shape
    group = cols if group is None else group
    out = np.zeros((rows, cols), np.float32)
    lib().orc_rmsnorm(_f(x), rows, cols, group, _f(weight), int(np.asarray(weight).size),
                      float(eps), _f(residual), float(scale), out)
    return out.astype(dtype)


def matmul_gather_f64(a, w, bias, idx, K):
    """matmulGatherRef (test/core/kernels/matmul/matmulGather.gpu.test.ts
    :10-28) in f64: out[i] = a[i]·W[e_i] + bias[e_i], W = rows [e·K,
    (e+1)·K) of w [E·K, N]. Rows whose index is not an expert are zero."""
    a = np.asarray(a, np.float64)
    w = np.asarray(w, np.float64)
    bias = None if bias is None else np.asarray(bias, np.float64)
    E = w.shape[0] // K
    N = w.shape[1]
    out = np.zeros((a.shape[0], N))
    for i, f in enumerate(np.asarray(idx, np.float64)):
        if not (f >= 0 and f < E and float(int(f)) == f):
            continue
        e = int(f)
        out[i] = a[i] @ w[e * K:(e + 1) * K]
        if bias is not None:
            out[i] += bias.reshape(E, N)[e]
    return out


def moe_block_float_f64(x, xn, route, glu, lin, down, k):
    """EagerMoeMlp.forward's float branch (src/zoo/privacy-filter/moeMlp.ts
    :85-100) in f64 on the normalised rows xn and a route: for each slot,
    swiglu(gather(xn, glu), gather(xn, lin)) → gather(·, down), weighted by
    the slot's gate and summed in slot order, + x. glu/lin/down: (w, bias)."""
    T, d = xn.shape
    K = d
    I = glu[0].shape[1]
    y = np.zeros((T, d))
    for s in range(k):
        ids = route[:, s]
        g = matmul_gather_f64(xn, glu[0], glu[1], ids, K)
        l_ = matmul_gather_f64(xn, lin[0], lin[1], ids, K)
        gc = np.minimum(g, 7.0)
        lc = np.clip(l_, -7.0, 7.0)
        act = gc / (1.0 + np.exp(-1.702 * gc)) * (lc + 1.0)
        o = matmul_gather_f64(act, down[0], down[1], ids, I)
        valid = np.array([f >= 0 and f < down[0].shape[0] // I and float(int(f)) == f
                          for f in ids])
        y += np.where(valid[:, None], o * route[:, k + s][:, None], 0.0)
    return np.asarray(x, np.float64) + y


def rope_f64(x, cos, sin, head_dim, src_start=0, width=None):
    """ropeRef (test/core/kernels/attention/rope.gpu.test.ts:25-46) in f64:
    each interleaved pair (x[2p], x[2p+1]) of columns [srcStart, srcStart +
    width) rotated by the pair-duplicated table entry of its column."""
    x = np.asarray(x, np.float64)
    rows, cols = x.shape
    width = cols if width is None else width
    c = np.asarray(cos, np.float64).reshape(rows, head_dim)
    s = np.asarray(sin, np.float64).reshape(rows, head_dim)
    col = np.arange(0, width, 2)
    cc, ss = c[:, col % head_dim], s[:, col % head_dim]
    x0, x1 = x[:, src_start + col], x[:, src_start + col + 1]
    out = np.empty((rows, width))
    out[:, 0::2] = x0 * cc - x1 * ss
    out[:, 1::2] = x1 * cc + x0 * ss
    return out


def sdpa_f64(q, k, v, q_heads, kv_heads, head_dim, window_left=np.inf, window_right=np.inf,
             q_pos_offset=0, sinks=None, segs=None, key_bias=None):
    """sdpaRef (test/core/kernels/attention/checkSdpa.ts:55-103) in f64:
    softmax(q·kᵀ) v per query row and head over the keys the window and the
    row's segment leave visible; q and k arrive pre-scaled; a sink adds
    exp(sink · ln 2) to the denominator alone; the key bias (start, end,
    value) adds value to the scores of its keys; a row that sees no key is
    0. Vectorised over heads and keys with a mask per row."""
    q = np.asarray(q, np.float64).reshape(-1, q_heads, head_dim)
    k = np.asarray(k, np.float64).reshape(-1, kv_heads, head_dim)
    v = np.asarray(v, np.float64).reshape(-1, kv_heads, head_dim)
    q_len, kv_len = q.shape[0], k.shape[0]
    group = q_heads // kv_heads
    kh = np.repeat(np.arange(kv_heads), group)                 # kv head of each q head
    scores = np.einsum("ihx,jhx->hij", q, k[:, kh, :])          # [H, qLen, kvLen]
    if key_bias is not None:
        s0, e0, val = key_bias
        scores[:, :, s0:e0] += val
    j = np.arange(kv_len)
    out = np.zeros((q_len, q_heads, head_dim))
    for i in range(q_len):
        qpos = q_pos_offset + i
        lo = max(0, qpos - window_left) if np.isfinite(window_left) else 0
        hi = min(kv_len - 1, qpos + window_right) if np.isfinite(window_right) else kv_len - 1
        if segs is not None:
            lo = max(lo, int(segs[2 * i]))
            hi = min(hi, int(segs[2 * i + 1]) - 1)
        vis = (j >= lo) & (j <= hi)
        sc = np.where(vis[None, :], scores[:, i, :], -np.inf)   # [H, kvLen]
        sink = (np.asarray(sinks, np.float64) * np.log(2.0) if sinks is not None
                else np.full(q_heads, -np.inf))
        m = np.maximum(sink, sc.max(axis=1))
        ok = np.isfinite(m)
        mm = np.where(ok, m, 0.0)
        p = np.where(vis[None, :], np.exp(sc - mm[:, None]), 0.0)
        den = p.sum(axis=1) + np.exp(sink - mm)
        num = np.einsum("hj,jhx->hx", p, v[:, kh, :])
        out[i] = np.where(ok[:, None], num / np.where(ok, den, 1.0)[:, None], 0.0)
    return out.reshape(q_len, q_heads * head_dim)


def viterbi_decode(start, end, trans, log_probs):
    """ViterbiDecoder.decode (src/zoo/privacy-filter/viterbi.ts:85-148) in
    numpy: f64 scores over f32 log-probabilities, ties to the lower previous
    label (the first maximum) and the lower last label; with no finite
    score left, the per-token argmax."""
    lp = np.asarray(log_probs, np.float32)
    T, n = lp.shape
    if T == 0:
        return []
    lp64 = lp.astype(np.float64)
    scores = lp64[0] + start
    back = np.zeros((max(T - 1, 0), n), np.int32)
    for t in range(1, T):
        cand = scores[:, None] + trans
        bi = np.argmax(cand, axis=0)
        back[t - 1] = bi
        scores = cand[bi, np.arange(n)] + lp64[t]
    if not np.isfinite(scores).any():
        return [int(j) for j in np.argmax(lp, axis=1)]
    last = int(np.argmax(scores + end))
    path = [0] * T
    path[T - 1] = last
    for t in range(T - 2, -1, -1):
        last = int(back[t, path[t + 1]])
        path[t] = last
    return path
