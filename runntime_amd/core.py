"""The MoE ops of `runntime/core`, on MI355X.

Same names, argument meaning and error messages as the reference's
graph ops (packages/runntime/src/core/graph/ops/):
  topk(x, k)                                  reduce.ts:93-100
  moeUp(x, route, glu, lin, {bits, groupSize})  matmul.ts:220-244
  moeDown(act, route, out, residual, opts)    matmul.ts:246-272
  rmsNorm(x, weight, eps, {group, residual, scale})  reduce.ts:61-92
plus the fused layer (EagerMoeMlp's quantized branch, zoo/privacy-filter/
moeMlp.ts:82-121), the whole block with its pre-norm (moe_block,
moeMlp.ts:79-121) and the router+topk fusion.

The reference builds lazy nodes and runs them later; here each op enqueues
its HIP kernels at once on torch's current stream and returns the output
tensor (the graph/executor layer is the caller's). Tensors are torch
tensors on a ROCm device; quantW weights are `QuantW` values.

Generalisation: the reference compiles in k = 4 experts per token. Here k
is 1..16; `topk` takes it, moeUp/moeDown read it from the route's
[T, 2k] shape. At k = 4 everything reduces to the reference's behaviour.
"""
import ctypes
import json

import math

import torch

from . import _lib
from .errors import RunntimeError
from .quantw import QuantExpertWeight, QuantW

MAX_K = 16


def _dims(t):
    return list(t.dims) if isinstance(t, QuantW) else list(t.shape)


def _dtype_name(t) -> str:
    if isinstance(t, QuantW):
        return "quantW"
    return {torch.float32: "f32", torch.float16: "f16", torch.int32: "i32"}.get(t.dtype, str(t.dtype))


def _want2d(name, x, allow):
    """wantND(name, x, 2, allow) (src/core/graph/ops/shared.ts:46-70)."""
    dims = _dims(x)
    dt = _dtype_name(x)
    if len(dims) != 2 or dt not in allow:
        raise ValueError(
            f"{name}: expected a 2D {' or '.join(allow)} tensor, got "
            f"dims={json.dumps(dims, separators=(',', ':'))} dtype={dt}")
    return dims[0], dims[1], dt


def _route_k(route) -> int:
    """k of a [T, 2k] route, or the reference's 4 when the shape is not one."""
    dims = _dims(route)
    if len(dims) == 2 and dims[1] % 2 == 0 and 1 <= dims[1] // 2 <= MAX_K:
        return dims[1] // 2
    return 4


def _check_expert_weight(op, wt: QuantExpertWeight, k_in: int, route, t: int, k: int, opts):
    """checkExpertWeight (src/core/graph/ops/matmul.ts:274-315). Returns
    (N, experts)."""
    bits, group_size = opts["bits"], opts["groupSize"]
    if bits not in (8, 4):
        raise ValueError(f"{op}: bits must be 8 or 4, got {bits}")
    w = wt.w
    wd = w.dims if isinstance(w, QuantW) else None
    if not isinstance(w, QuantW) or len(wd) != 2 or wd[0] % k_in != 0:
        raise ValueError(f"{op}: w must be a quantW [E·{k_in}, N] weight")
    r, n = wd
    experts = r // k_in
    if w.elems != (r * n * bits) // 32:
        raise ValueError(f"{op}: quantW weight elems {w.elems} != rows·cols·{bits}/32")
    if k_in % 4 != 0 or n % 4 != 0:
        raise ValueError(f"{op}: K {k_in} and N {n} must be multiples of 4")
    if group_size <= 0 or group_size % 4 != 0 or k_in % group_size != 0:
        raise ValueError(
            f"{op}: groupSize {group_size} must be a multiple of 4 that divides K {k_in}")
    sc = wt.scales
    if _dtype_name(sc) != "f32" or sc.numel() != (experts * k_in * n) // group_size:
        raise ValueError(f"{op}: scales must be f32 [{(experts * k_in) // group_size}, {n}]")
    b = wt.bias
    if b is not None and (_dtype_name(b) != "f32" or b.numel() != experts * n):
        raise ValueError(f"{op}: bias must be f32 [{experts}, {n}]")
    rd = _dims(route)
    if _dtype_name(route) != "f32" or len(rd) != 2 or rd[0] != t or rd[1] != 2 * k:
        raise ValueError(f"{op}: route must be topk's f32 [{t}, {2 * k}] output")
    return n, experts


def _device_of(*tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        tt = t.words if isinstance(t, QuantW) else t
        if tt.device.type != "cuda":
            raise RunntimeError("INVALID_ARGUMENT",
                                f"tensors must be on a ROCm device, got {tt.device}")
        if dev is None:
            dev = tt.device
        elif tt.device != dev:
            raise RunntimeError("INVALID_ARGUMENT", "tensors are on different devices")
        if tt.numel() == 0:
            raise RunntimeError("INVALID_ARGUMENT", "tensor: the shape has no elements")
        if not tt.is_contiguous():
            raise RunntimeError("INVALID_ARGUMENT", "tensors must be contiguous")
    return dev


def _ctx(dev: torch.device) -> int:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(idx).cuda_stream
    return _lib.context(idx, stream)


def _ptr(t):
    if t is None:
        return None
    return (t.words if isinstance(t, QuantW) else t).data_ptr()


def _weight_c(wt: QuantExpertWeight) -> _lib.ExpertWeightC:
    return _lib.ExpertWeightC(_ptr(wt.w), _ptr(wt.scales), _ptr(wt.bias))


def _xdtype(t) -> int:
    return _lib.MOE_F16 if t.dtype == torch.float16 else _lib.MOE_F32


# ----------------------------------------------------------------- the ops


def topk(x: torch.Tensor, k: int) -> torch.Tensor:
    """Router top-k plus softmax over the selected logits, lowest index on
    ties. Returns f32 [M, 2k]: ids first, then weights, descending by logit
    (reduce.ts:93-100; kernel topkSelect.ts:21-92)."""
    m, n, _ = _want2d("topk", x, ("f32", "f16"))
    if not (1 <= k <= MAX_K):
        raise ValueError(f"topk: k must be in 1..{MAX_K}, got {k}")
    if n < k:
        raise ValueError(f"topk: need at least {k} columns, got {n}")
    dev = _device_of(x)
    route = torch.empty((m, 2 * k), dtype=torch.float32, device=dev)
    lib = _lib.load()
    _lib.check(lib.moe_topk(_ctx(dev), x.data_ptr(), _xdtype(x), m, n, k, route.data_ptr()))
    return route


def router_topk(x: torch.Tensor, w: torch.Tensor, b, k: int) -> torch.Tensor:
    """topk(linear(x, w, b), k) fused: x [T, d] f32/f16, w f32 [d, E] (the
    router Linear's weight after the load-time transpose,
    src/core/nn/layers.ts:176-217), b f32 [E] or None. Logits use this
    library's canonical f32 summation order."""
    t, d, _ = _want2d("router", x, ("f32", "f16"))
    wd = _dims(w)
    if _dtype_name(w) != "f32" or len(wd) != 2 or wd[0] != d:
        raise ValueError(f"router: weight must be f32 [{d}, E]")
    e = wd[1]
    if b is not None and (_dtype_name(b) != "f32" or b.numel() != e):
        raise ValueError(f"router: bias must be f32 [{e}]")
    if not (1 <= k <= MAX_K):
        raise ValueError(f"topk: k must be in 1..{MAX_K}, got {k}")
    if e < k:
        raise ValueError(f"topk: need at least {k} columns, got {e}")
    dev = _device_of(x, w, b)
    route = torch.empty((t, 2 * k), dtype=torch.float32, device=dev)
    lib = _lib.load()
    _lib.check(lib.moe_router_topk(_ctx(dev), x.data_ptr(), _xdtype(x), w.data_ptr(), _ptr(b), t,
                                   d, e, k, route.data_ptr()))
    return route


def moeUp(x, route, glu: QuantExpertWeight, lin: QuantExpertWeight, opts) -> torch.Tensor:
    """MoE input projections and clamped SwiGLU. route is topk's [T, 2k]. For
    token t and slot s with expert e, row t·k + s of the [T·k, N] result is
    swiglu(x[t]·glu.w[e] + glu.bias[e], x[t]·lin.w[e] + lin.bias[e])
    (src/core/graph/ops/matmul.ts:220-244). x is f32 as in the reference;
    f16 is accepted too."""
    t, kin, _ = _want2d("moeUp", x, ("f32", "f16"))
    k = _route_k(route)
    n, experts = _check_expert_weight("moeUp", glu, kin, route, t, k, opts)
    _check_expert_weight("moeUp", lin, kin, route, t, k, opts)
    if lin.w.dims[0] != glu.w.dims[0] or lin.w.dims[1] != n:
        raise ValueError("moeUp: glu and lin weights must have the same shape")
    dev = _device_of(x, route, glu.w, glu.scales, glu.bias, lin.w, lin.scales, lin.bias)
    act = torch.empty((t * k, n), dtype=torch.float32, device=dev)
    g, l_ = _weight_c(glu), _weight_c(lin)
    lib = _lib.load()
    _lib.check(lib.moe_up(_ctx(dev), x.data_ptr(), _xdtype(x), route.data_ptr(), ctypes.byref(g),
                          ctypes.byref(l_), t, kin, n, experts, k, opts["bits"],
                          opts["groupSize"], act.data_ptr()))
    return act


def moeDown(act, route, out: QuantExpertWeight, residual, opts) -> torch.Tensor:
    """MoE output projection. Mixes the k slots by gate weight and adds the
    residual: out[t] = residual[t] + Σ_s gate_s·(act[t·k + s]·w[e_s] + bias[e_s])
    (src/core/graph/ops/matmul.ts:246-272). act is moeUp's [T·k, K]; out is
    [T, N]."""
    rows, kin, _ = _want2d("moeDown", act, ("f32",))
    k = _route_k(route)
    if rows % k != 0:
        raise ValueError(f"moeDown: act rows {rows} must be a multiple of {k}")
    t = rows // k
    n, experts = _check_expert_weight("moeDown", out, kin, route, t, k, opts)
    if residual is not None and (_dtype_name(residual) != "f32" or residual.numel() != t * n):
        raise ValueError(f"moeDown: residual must be f32 [{t}, {n}]")
    dev = _device_of(act, route, out.w, out.scales, out.bias, residual)
    y = torch.empty((t, n), dtype=torch.float32, device=dev)
    w = _weight_c(out)
    lib = _lib.load()
    _lib.check(lib.moe_down(_ctx(dev), act.data_ptr(), route.data_ptr(), ctypes.byref(w),
                            _ptr(residual), t, kin, n, experts, k, opts["bits"],
                            opts["groupSize"], y.data_ptr()))
    return y


def moe_layer(x, router_w, router_b, glu: QuantExpertWeight, lin: QuantExpertWeight,
              down: QuantExpertWeight, residual, k: int, bits: int = 8,
              group_size_up=None, group_size_down=None, return_route: bool = False,
              out=None, route=None, noalloc: bool = False):
    """The routed layer in one call (EagerMoeMlp.forward's quantized branch
    after the norm, zoo/privacy-filter/moeMlp.ts:82-121):
    route = topk(x·Wr + br, k); act = moeUp(x, route, glu, lin);
    out = moeDown(act, route, down, residual). Group sizes default to one
    scale per output channel (K of each projection). `out` (f32 [T, d]) and
    `route` (f32 [T, 2k]) may be given to write into existing buffers.
    noalloc: run moe_layer_noalloc, whose workspace is the library's static
    per-GPU scratch (no device allocation by the call; give `out` and
    `route` to allocate nothing here either)."""
    t, d, _ = _want2d("moe_layer", x, ("f32", "f16"))
    rw = _dims(router_w)
    if _dtype_name(router_w) != "f32" or len(rw) != 2 or rw[0] != d:
        raise ValueError(f"moe_layer: router weight must be f32 [{d}, E]")
    e = rw[1]
    if not isinstance(glu.w, QuantW) or glu.w.dims[0] != e * d:
        raise ValueError(f"moe_layer: glu.w must be a quantW [E·{d}, I] weight")
    i = glu.w.dims[1]
    gu = group_size_up or d
    gd = group_size_down or i
    if route is None:
        route = torch.empty((t, 2 * k), dtype=torch.float32, device=x.device)
    elif (_dtype_name(route) != "f32" or route.numel() != t * 2 * k
          or not route.is_contiguous()):
        raise ValueError(f"moe_layer: route must be contiguous f32 [{t}, {2 * k}]")
    _check_expert_weight("moe_layer", glu, d, route, t, k, {"bits": bits, "groupSize": gu})
    _check_expert_weight("moe_layer", lin, d, route, t, k, {"bits": bits, "groupSize": gu})
    _check_expert_weight("moe_layer", down, i, route, t, k, {"bits": bits, "groupSize": gd})
    if residual is not None and (_dtype_name(residual) != "f32" or residual.numel() != t * d):
        raise ValueError(f"moe_layer: residual must be f32 [{t}, {d}]")
    dev = _device_of(x, router_w, router_b, glu.w, lin.w, down.w, residual)
    if out is None:
        out = torch.empty((t, d), dtype=torch.float32, device=dev)
    elif _dtype_name(out) != "f32" or out.numel() != t * d or not out.is_contiguous():
        raise ValueError(f"moe_layer: out must be contiguous f32 [{t}, {d}]")
    g, l_, dn = _weight_c(glu), _weight_c(lin), _weight_c(down)
    lib = _lib.load()
    fn = lib.moe_layer_noalloc if noalloc else lib.moe_layer
    _lib.check(fn(_ctx(dev), x.data_ptr(), _xdtype(x), router_w.data_ptr(), _ptr(router_b),
                  ctypes.byref(g), ctypes.byref(l_), ctypes.byref(dn), _ptr(residual), t, d, i, e,
                  k, bits, gu, gd, route.data_ptr(), out.data_ptr()))
    return (out, route) if return_route else out


def rmsNorm(x, weight, eps: float = 1e-6, opts=None) -> torch.Tensor:
    """RMSNorm over the last dim: x · rsqrt(mean(x²) + eps) · weight, summed
    in f32 even for f16 x (src/core/graph/ops/reduce.ts:61-92). opts.group
    normalizes each run of `group` columns on its own; the weight is then
    `group` long (shared by every run) or N long (a slice per run).
    opts.residual and opts.scale turn the output into
    (residual + norm(x)) · scale. Same dtype as x."""
    opts = opts or {}
    m, n, dtype = _want2d("rmsNorm", x, ("f32", "f16"))
    group = opts.get("group", n)
    residual = opts.get("residual")
    scale = opts.get("scale", 1)
    if not isinstance(group, int) or group < 1 or n % group != 0:
        raise ValueError(f"rmsNorm: group {group} must divide the row width {n}")
    wl = weight.numel()
    if _dtype_name(weight) != dtype or (wl != group and wl != n):
        lens = f"{n}" if group == n else f"{group} or {n}"
        raise ValueError(
            f"rmsNorm: weight must be {dtype} with {lens} elems, got ({wl},{_dtype_name(weight)})")
    if not (eps > 0):
        raise ValueError(f"rmsNorm: eps must be positive, got {eps}")
    if residual is not None and (_dtype_name(residual) != dtype or residual.numel() != m * n):
        raise ValueError(f"rmsNorm: residual must be {dtype} [{m}, {n}]")
    dev = _device_of(x, weight, residual)
    out = torch.empty((m, n), dtype=x.dtype, device=dev)
    lib = _lib.load()
    _lib.check(lib.moe_rmsnorm(_ctx(dev), x.data_ptr(), _xdtype(x), m, n, weight.data_ptr(), wl,
                               float(eps), group, _ptr(residual), float(scale), out.data_ptr()))
    return out


def moe_block(x, norm_w, eps, router_w, router_b, glu: QuantExpertWeight,
              lin: QuantExpertWeight, down: QuantExpertWeight, k: int, bits: int = 8,
              group_size_up=None, group_size_down=None, return_route: bool = False):
    """EagerMoeMlp.forward for the quantized formats
    (src/zoo/privacy-filter/moeMlp.ts:79-121) in one call:
    xn = rmsNorm(x, norm_w, eps); route = topk(xn·Wr + br, k);
    out = moeDown(moeUp(xn, route, glu, lin), route, down, x). The residual
    is x in its own dtype; out is f32 [T, d]. The privacy filter's eps is
    1e-5 (moeMlp.ts:23)."""
    t, d, dtype = _want2d("moe_block", x, ("f32", "f16"))
    if _dtype_name(norm_w) != dtype or norm_w.numel() != d:
        raise ValueError(f"rmsNorm: weight must be {dtype} with {d} elems, got "
                         f"({norm_w.numel()},{_dtype_name(norm_w)})")
    if not (eps > 0):
        raise ValueError(f"rmsNorm: eps must be positive, got {eps}")
    rw = _dims(router_w)
    if _dtype_name(router_w) != "f32" or len(rw) != 2 or rw[0] != d:
        raise ValueError(f"moe_block: router weight must be f32 [{d}, E]")
    e = rw[1]
    if not isinstance(glu.w, QuantW) or glu.w.dims[0] != e * d:
        raise ValueError(f"moe_block: glu.w must be a quantW [E·{d}, I] weight")
    i = glu.w.dims[1]
    gu = group_size_up or d
    gd = group_size_down or i
    route = torch.empty((t, 2 * k), dtype=torch.float32, device=x.device)
    _check_expert_weight("moe_block", glu, d, route, t, k, {"bits": bits, "groupSize": gu})
    _check_expert_weight("moe_block", lin, d, route, t, k, {"bits": bits, "groupSize": gu})
    _check_expert_weight("moe_block", down, i, route, t, k, {"bits": bits, "groupSize": gd})
    dev = _device_of(x, norm_w, router_w, router_b, glu.w, lin.w, down.w)
    out = torch.empty((t, d), dtype=torch.float32, device=dev)
    g, l_, dn = _weight_c(glu), _weight_c(lin), _weight_c(down)
    lib = _lib.load()
    _lib.check(lib.moe_block(_ctx(dev), x.data_ptr(), _xdtype(x), norm_w.data_ptr(), float(eps),
                             router_w.data_ptr(), _ptr(router_b), ctypes.byref(g),
                             ctypes.byref(l_), ctypes.byref(dn), t, d, i, e, k, bits, gu, gd,
                             route.data_ptr(), out.data_ptr()))
    return (out, route) if return_route else out


def matmulGather(a, w, expertIdx, opts) -> torch.Tensor:
    """Indexed matmul plus bias: out[i] = a[i]·W[e_i] + bias[e_i], W = rows
    [e·K, (e+1)·K) of w [E·K, N], e_i looked up per row
    (src/core/graph/ops/matmul.ts:180-210). a, w and bias share one float
    dtype; expertIdx is f32. The bias must be [E, N] (the reference checks
    only its dtype, a known bug its test records)."""
    bias = opts["bias"]
    m, k, dtype = _want2d("matmulGather", a, ("f32", "f16"))
    r, n, wdt = _want2d("matmulGather.w", w, ("f32", "f16"))
    if wdt != dtype:
        raise ValueError(f"matmulGather: w is {wdt} but a is {dtype}")
    if n % 4 != 0:
        raise ValueError(f"matmulGather: n {n} must be divisible by 4")
    if r % k != 0:
        raise ValueError(f"matmulGather: w rows {r} not a multiple of K {k}")
    if _dtype_name(bias) != dtype:
        raise ValueError(f"matmulGather: bias must be {dtype}, got {_dtype_name(bias)}")
    e = r // k
    if bias.numel() != e * n:
        raise ValueError(f"matmulGather: bias must be [{e}, {n}], got {bias.numel()} elems")
    if _dtype_name(expertIdx) != "f32" or expertIdx.numel() != m:
        raise ValueError(f"matmulGather: expertIdx must be f32 with {m} elems, got "
                         f"{expertIdx.numel()}")
    dev = _device_of(a, w, bias, expertIdx)
    out = torch.empty((m, n), dtype=a.dtype, device=dev)
    lib = _lib.load()
    _lib.check(lib.moe_matmul_gather(_ctx(dev), a.data_ptr(), _xdtype(a), w.data_ptr(),
                                     bias.data_ptr(), expertIdx.data_ptr(), m, k, n, e,
                                     out.data_ptr()))
    return out


def moe_block_float(x, norm_w, eps, router_w, router_b, glu_w, glu_b, lin_w, lin_b, out_w, out_b,
                    k: int = 4, return_route: bool = False):
    """EagerMoeMlp.forward for float weights (src/zoo/privacy-filter/
    moeMlp.ts:79-100): rmsNorm, router + topk, per slot the glu/lin gathers,
    clamped SwiGLU and the out gather, weighted by the gates and summed, + x.
    x, norm_w and the expert weights share dtype: glu_w, lin_w [E·d, I],
    out_w [E·I, d], biases [E, I] / [E, d] or None; router W f32 [d, E].
    Returns f32 [T, d]."""
    t, d, dtype = _want2d("moe_block_float", x, ("f32", "f16"))
    if _dtype_name(norm_w) != dtype or norm_w.numel() != d:
        raise ValueError(f"rmsNorm: weight must be {dtype} with {d} elems, got "
                         f"({norm_w.numel()},{_dtype_name(norm_w)})")
    if not (eps > 0):
        raise ValueError(f"rmsNorm: eps must be positive, got {eps}")
    rw = _dims(router_w)
    if _dtype_name(router_w) != "f32" or len(rw) != 2 or rw[0] != d:
        raise ValueError(f"moe_block_float: router weight must be f32 [{d}, E]")
    e = rw[1]
    rows, i, wdt = _want2d("matmulGather.w", glu_w, ("f32", "f16"))
    if wdt != dtype:
        raise ValueError(f"matmulGather: w is {wdt} but a is {dtype}")
    if rows != e * d:
        raise ValueError(f"moe_block_float: glu weight must be [{e}·{d}, I], got {rows} rows")
    for name, wt, shape in (("lin", lin_w, (e * d, i)), ("out", out_w, (e * i, d))):
        if _dtype_name(wt) != dtype or tuple(wt.shape) != shape:
            raise ValueError(f"moe_block_float: {name} weight must be {dtype} {list(shape)}")
    for name, bt, nn_ in (("glu", glu_b, i), ("lin", lin_b, i), ("out", out_b, d)):
        if bt is not None and (_dtype_name(bt) != dtype or bt.numel() != e * nn_):
            raise ValueError(f"moe_block_float: {name} bias must be {dtype} [{e}, {nn_}]")
    dev = _device_of(x, norm_w, router_w, router_b, glu_w, lin_w, out_w, glu_b, lin_b, out_b)
    route = torch.empty((t, 2 * k), dtype=torch.float32, device=dev)
    out = torch.empty((t, d), dtype=torch.float32, device=dev)
    lib = _lib.load()
    _lib.check(lib.moe_block_float(_ctx(dev), x.data_ptr(), _xdtype(x), norm_w.data_ptr(),
                                   float(eps), router_w.data_ptr(), _ptr(router_b),
                                   glu_w.data_ptr(), _ptr(glu_b), lin_w.data_ptr(), _ptr(lin_b),
                                   out_w.data_ptr(), _ptr(out_b), t, d, i, e, k,
                                   route.data_ptr(), out.data_ptr()))
    return (out, route) if return_route else out


def pack_quant_w_device(ints: torch.Tensor, bits: int = 8) -> QuantW:
    """packQuantW (src/core/weights/quantPack.ts:12-28) on the device for a
    whole layer: `ints` is int8 [E, n, k] (each expert output-first, torch's
    Linear layout) or [n, k] for one expert, on the GPU. Returns the quantW
    weight of logical dims [E·k, n] (experts concatenated expert-major)."""
    if ints.dtype != torch.int8 or ints.dim() not in (2, 3) or not ints.is_cuda:
        raise ValueError("packQuantW: ints must be a device int8 [E, n, k] or [n, k] tensor")
    e, n, k = (1, *ints.shape) if ints.dim() == 2 else tuple(ints.shape)
    ints = ints.contiguous()
    words = torch.empty(e * k * n * bits // 32, dtype=torch.int32, device=ints.device)
    lib = _lib.load()
    _lib.check(lib.moe_pack_quantw(_ctx(ints.device), ints.data_ptr(), e, k, n, bits,
                                   words.data_ptr()))
    return QuantW(words, (e * k, n))


def dispatch(route, num_experts: int):
    """The dispatch permutation the layer builds for `route` (diagnostic):
    (perm int32 [T·k], offsets int32 [E + 1])."""
    t, c = _dims(route)
    k = c // 2
    dev = _device_of(route)
    perm = torch.empty(t * k, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    lib = _lib.load()
    _lib.check(lib.moe_dispatch(_ctx(dev), route.data_ptr(), t, num_experts, k, perm.data_ptr(),
                                offsets.data_ptr()))
    return perm, offsets


def _call_stride(t, calls: int, base_dims: int) -> int:
    """Element stride between calls: a tensor with one more leading dim than
    `base_dims` is per call (its leading size must be `calls`), else shared."""
    if t is None:
        return 0
    tt = t.words if isinstance(t, QuantW) else t
    if tt.dim() == base_dims + 1:
        if tt.shape[0] != calls:
            raise ValueError(f"moe_layer_batched: leading dim {tt.shape[0]} != calls {calls}")
        return tt.stride(0)
    if tt.dim() != base_dims:
        raise ValueError(f"moe_layer_batched: expected {base_dims} or {base_dims + 1} dims, "
                         f"got {tt.dim()}")
    return 0


def moe_layer_batched(x, router_w, router_b, glu: QuantExpertWeight, lin: QuantExpertWeight,
                      down: QuantExpertWeight, residual, k: int, bits: int = 8,
                      group_size_up=None, group_size_down=None, out=None, route=None):
    """`calls` independent moe_layer calls in one set of launches
    (moe_layer_batched in include/runntime_moe.h). x is [calls, T, d]; every
    other tensor is either per call (a leading `calls` dim) or shared. The
    quantW words of a per-call weight are [calls, words]. Returns
    (out [calls, T, d], route [calls, T, 2k])."""
    if x.dim() != 3:
        raise ValueError("moe_layer_batched: x must be [calls, T, d]")
    calls, t, d = x.shape
    rw = router_w.shape
    e = rw[-1]
    i = glu.w.dims[1]
    gu = group_size_up or d
    gd = group_size_down or i
    dev = _device_of(x, router_w, router_b, glu.w, glu.scales, lin.w, down.w, residual)
    if out is None:
        out = torch.empty((calls, t, d), dtype=torch.float32, device=dev)
    if route is None:
        route = torch.empty((calls, t, 2 * k), dtype=torch.float32, device=dev)
    st = _lib.CallStridesC(
        x=x.stride(0), router_w=_call_stride(router_w, calls, 2),
        router_b=_call_stride(router_b, calls, 1),
        glu_w=_call_stride(glu.w, calls, 1), glu_scales=_call_stride(glu.scales, calls, 2),
        glu_bias=_call_stride(glu.bias, calls, 2),
        lin_w=_call_stride(lin.w, calls, 1), lin_scales=_call_stride(lin.scales, calls, 2),
        lin_bias=_call_stride(lin.bias, calls, 2),
        down_w=_call_stride(down.w, calls, 1), down_scales=_call_stride(down.scales, calls, 2),
        down_bias=_call_stride(down.bias, calls, 2),
        residual=_call_stride(residual, calls, 2), route=route.stride(0), out=out.stride(0))
    g, l_, dn = _weight_c(glu), _weight_c(lin), _weight_c(down)
    lib = _lib.load()
    _lib.check(lib.moe_layer_batched(
        _ctx(dev), calls, ctypes.byref(st), x.data_ptr(), _xdtype(x), router_w.data_ptr(),
        _ptr(router_b), ctypes.byref(g), ctypes.byref(l_), ctypes.byref(dn), _ptr(residual), t, d,
        i, e, k, bits, gu, gd, route.data_ptr(), out.data_ptr()))
    return out, route


# ------------------------------------------------------------ weight upload


class UploadedExpertWeight:
    """A QuantExpertWeight whose device buffers the library owns
    (moe_weights_upload): the reference's Parameter, which owns its GPU
    buffer and frees it on dispose() (src/core/nn/module.ts:20-65). `view()`
    gives the device pointers the C ABI takes; after `dispose()` it raises
    RESOURCE_DISPOSED."""

    def __init__(self, handle: int, E: int, K: int, N: int, bits: int, group_size: int):
        self.handle, self.E, self.K, self.N = handle, E, K, N
        self.bits, self.group_size = bits, group_size

    def view(self) -> _lib.ExpertWeightC:
        v = _lib.ExpertWeightC()
        _lib.check(_lib.load().moe_weights_view(self.handle, ctypes.byref(v)))
        return v

    def dispose(self) -> None:
        _lib.check(_lib.load().moe_weights_dispose(self.handle))

    def __del__(self):
        if getattr(self, "handle", None):
            _lib.load().moe_weights_release(self.handle)
            self.handle = None


def upload_expert_weight(host_w, scales, bias, E: int, K: int, N: int, bits: int,
                         group_size: int, raw_int8: bool = False,
                         device: int = 0) -> UploadedExpertWeight:
    """Uploads host buffers (numpy): quantW words (uint32, E·K·N·bits/32),
    or int8 [E][N][K] with raw_int8 (packed on the device as packQuantW);
    scales f32 [E·K/groupSize, N]; bias f32 [E, N] or None."""
    import numpy as np
    hw = np.ascontiguousarray(host_w)
    sc = np.ascontiguousarray(scales, dtype=np.float32)
    bs = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    ctx = _lib.context(device, 0)
    out = ctypes.c_void_p()
    _lib.check(_lib.load().moe_weights_upload(
        ctx, hw.ctypes.data if hw.size else None, 1 if raw_int8 else 0,
        sc.ctypes.data if sc.size else None, None if bs is None else bs.ctypes.data,
        E, K, N, bits, group_size, ctypes.byref(out)))
    return UploadedExpertWeight(out.value, E, K, N, bits, group_size)


# ------------------------------------------------------------------ attention
# The attention ops of the privacy-filter block (src/core/graph/ops/
# attention.ts). WINDOW_INF is the reference's lowering of Infinity
# (src/core/graph/ops/shared.ts:37); a window at or past it is unbounded.
WINDOW_INF = 0x3FFFFFFF


def rope(x, cos, sin, opts) -> torch.Tensor:
    """Rotary embedding of the interleaved pairs of x's columns [srcStart,
    srcStart + width) (src/core/graph/ops/attention.ts:220-262): cos and sin
    are f32 [T, headDim] pair-duplicated tables with any scale folded in."""
    head_dim = opts["headDim"]
    t, xw, dtype = _want2d("rope", x, ("f32", "f16"))
    src_start = opts.get("srcStart", 0) or 0
    w = opts.get("width", xw)
    w = xw if w is None else w
    if not isinstance(head_dim, int) or head_dim <= 0 or head_dim % 2 != 0:
        raise ValueError(f"rope: headDim {head_dim} must be a positive even integer")
    if not isinstance(src_start, int) or src_start < 0 or src_start % 2 != 0:
        raise ValueError(f"rope: srcStart {src_start} must be a non-negative even integer")
    if not isinstance(w, int) or w <= 0 or src_start + w > xw:
        raise ValueError(f"rope: window [{src_start}, {src_start + w}) exceeds {xw} input cols")
    if w % head_dim != 0:
        raise ValueError(f"rope: width {w} must be a multiple of headDim {head_dim}")
    for name, v in (("cos", cos), ("sin", sin)):
        if _dtype_name(v) != "f32" or v.numel() != t * head_dim:
            raise ValueError(f"rope: {name} must be f32 [T,headDim] = {t * head_dim} elems, "
                             f"got {v.numel()}")
    dev = _device_of(x, cos, sin)
    out = torch.empty((t, w), dtype=x.dtype, device=dev)
    lib = _lib.load()
    _lib.check(lib.moe_rope(_ctx(dev), x.data_ptr(), _xdtype(x), t, xw, head_dim, src_start, w,
                            cos.data_ptr(), sin.data_ptr(), out.data_ptr()))
    return out


def _lower_window(op, name, w):
    if w == math.inf:
        return -1
    if not isinstance(w, int) or isinstance(w, bool) or w < 0:
        raise ValueError(f"{op}: {name} {w} must be a non-negative integer or Infinity")
    return -1 if w >= WINDOW_INF else w


def _sdpa_common(op, q_len, kv_len, dtype, opts, packed):
    q_heads, kv_heads, head_dim = opts["qHeads"], opts["kvHeads"], opts["headDim"]
    if kv_heads <= 0 or q_heads % kv_heads != 0:
        raise ValueError(f"{op}: qHeads {q_heads} not divisible by kvHeads {kv_heads}")
    if head_dim > 128:
        raise ValueError(f"{op}: headDim {head_dim} exceeds the kernel's max (128)")
    wl = _lower_window(op, "windowLeft", opts["windowLeft"])
    wr = _lower_window(op, "windowRight", opts["windowRight"])
    off = opts.get("qPosOffset", 0) or 0
    if not isinstance(off, int) or off < 0:
        raise ValueError(f"{op}: qPosOffset {off} must be a non-negative integer")
    if wr >= 0 and off + q_len > kv_len:
        raise ValueError(f"{op}: qPosOffset+qLen {off + q_len} exceeds key rows kvLen {kv_len}")
    sinks, segments = opts.get("sinks"), opts.get("segments")
    if sinks is not None and (_dtype_name(sinks) != "f32" or sinks.numel() != q_heads):
        raise ValueError(f"{op}: sinks must be f32 with {q_heads} elems, got {sinks.numel()}")
    if segments is not None:
        if _dtype_name(segments) != "f32" or segments.numel() != 2 * q_len:
            raise ValueError(f"{op}: segments must be f32 [qLen, 2] = {2 * q_len} elems, got "
                             f"({segments.numel()},{_dtype_name(segments)})")
        if q_len == 1 and not packed:
            raise ValueError(f"{op}: segments need qLen > 1 (decode has no segment route)")
    max_segment = opts.get("maxSegment", 0) or 0
    if max_segment != 0:
        if segments is None:
            raise ValueError(f"{op}: maxSegment needs segments")
        if not isinstance(max_segment, int) or max_segment < 1:
            raise ValueError(f"{op}: maxSegment {max_segment} must be a positive integer")
    return q_heads, kv_heads, head_dim, wl, wr, off, sinks, segments


def _sdpa_launch(dev, q, q_rs, k, k_rs, v, v_rs, q_len, kv_len, q_heads, kv_heads, head_dim, wl,
                 wr, off, sinks, segments, kb, dtype_t):
    out = torch.empty((q_len, q_heads * head_dim), dtype=dtype_t, device=dev)
    lib = _lib.load()
    kbs, kbe, kbv = (kb["start"], kb["end"], float(kb["value"])) if kb else (0, 0, 0.0)
    _lib.check(lib.moe_sdpa(_ctx(dev), _xdtype(out), q, q_rs, k, k_rs, v, v_rs, q_len, kv_len,
                            q_heads, kv_heads, head_dim, wl, wr, off,
                            sinks.data_ptr() if sinks is not None else None,
                            segments.data_ptr() if segments is not None else None,
                            1 if kb else 0, kbs, kbe, kbv, out.data_ptr()))
    return out


def sdpa(q, k, v, opts) -> torch.Tensor:
    """Scaled-dot-product attention over the band-mask family with GQA,
    sinks, segments and a key bias (src/core/graph/ops/attention.ts:28-145).
    q [qLen, qHeads·headDim], k and v [kvLen, kvHeads·headDim] share a float
    dtype; q and k arrive pre-scaled."""
    q_len, qw, dtype = _want2d("sdpa", q, ("f32", "f16"))
    q_heads, head_dim = opts["qHeads"], opts["headDim"]
    if qw != q_heads * head_dim:
        raise ValueError(f"sdpa: q cols {qw} != qHeads*headDim {q_heads * head_dim}")
    kv_heads = opts["kvHeads"]
    if kv_heads <= 0 or q_heads % kv_heads != 0:
        raise ValueError(f"sdpa: qHeads {q_heads} not divisible by kvHeads {kv_heads}")
    kv_len, kw, kdt = _want2d("sdpa.k", k, ("f32", "f16"))
    if kw != kv_heads * head_dim:
        raise ValueError(f"sdpa: k cols {kw} != kvHeads*headDim {kv_heads * head_dim}")
    vt, vw, vdt = _want2d("sdpa.v", v, ("f32", "f16"))
    if kdt != dtype or vdt != dtype:
        raise ValueError(f"sdpa: q, k and v must share a dtype, got {dtype}/{kdt}/{vdt}")
    if vt != kv_len:
        raise ValueError(f"sdpa: v rows {vt} != k rows {kv_len}")
    if vw != kv_heads * head_dim:
        raise ValueError(f"sdpa: v cols {vw} != kvHeads*headDim {kv_heads * head_dim}")
    q_heads, kv_heads, head_dim, wl, wr, off, sinks, segments = _sdpa_common(
        "sdpa", q_len, kv_len, dtype, opts, packed=False)
    kb = opts.get("keyBias")
    if kb is not None:
        s0, e0, val = kb["start"], kb["end"], kb["value"]
        if (not isinstance(s0, int) or not isinstance(e0, int) or s0 < 0 or s0 > e0
                or e0 > kv_len):
            raise ValueError(f"sdpa: keyBias keys [{s0}, {e0}) must lie within the {kv_len} keys")
        if not math.isfinite(val):
            raise ValueError(f"sdpa: keyBias value {val} must be finite")
        if q_len == 1:
            raise ValueError("sdpa: keyBias needs qLen > 1 (decode has no key bias route)")
    dev = _device_of(q, k, v, *(t for t in (sinks, segments) if t is not None))
    return _sdpa_launch(dev, q.data_ptr(), qw, k.data_ptr(), kw, v.data_ptr(), vw, q_len, kv_len,
                        q_heads, kv_heads, head_dim, wl, wr, off, sinks, segments, kb, q.dtype)


def sdpaPacked(qkv, opts) -> torch.Tensor:
    """sdpa over one fused qkv tensor read in place: q, k and v are column
    blocks of [T, (qHeads + 2·kvHeads)·headDim] (src/core/graph/ops/
    attention.ts:146-214). Self-attention only."""
    t, w, dtype = _want2d("sdpaPacked", qkv, ("f32", "f16"))
    q_heads, kv_heads, head_dim = opts["qHeads"], opts["kvHeads"], opts["headDim"]
    packed_w = (q_heads + 2 * kv_heads) * head_dim
    if w != packed_w:
        raise ValueError(f"sdpaPacked: qkv cols {w} != (qHeads + 2*kvHeads)*headDim = {packed_w}")
    if kv_heads <= 0 or q_heads % kv_heads != 0:
        raise ValueError(f"sdpaPacked: qHeads {q_heads} not divisible by kvHeads {kv_heads}")
    if head_dim > 128:
        raise ValueError(f"sdpaPacked: headDim {head_dim} exceeds the kernel's max (128)")
    if t == 1:
        raise ValueError("sdpaPacked: qLen must be > 1 (decode has no packed route)")
    q_heads, kv_heads, head_dim, wl, wr, off, sinks, segments = _sdpa_common(
        "sdpaPacked", t, t, dtype, opts, packed=True)
    dev = _device_of(qkv, *(x for x in (sinks, segments) if x is not None))
    es = qkv.element_size()
    base = qkv.data_ptr()
    qw, kw = q_heads * head_dim, kv_heads * head_dim
    return _sdpa_launch(dev, base, w, base + qw * es, w, base + (qw + kw) * es, w, t, t, q_heads,
                        kv_heads, head_dim, wl, wr, off, sinks, segments, None, qkv.dtype)
