"""The C-ABI library and the host-side op checks, without a GPU.

The library must load and export every entry point include/runntime_moe.h
declares. The ops' argument checks mirror the reference's graph-op tests
(test/core/graph/ops/matmul.test.ts:276-409, topkSelect.gpu.test.ts:92-98):
they run before any device work, so CPU tensors exercise them."""
import ctypes
import os
import re

import pytest
import torch

import runntime_amd as rt
from runntime_amd import _lib
from runntime_amd.quantw import QuantExpertWeight, QuantW

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    with open(os.path.join(ROOT, "include", "runntime_moe.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"MOE_API\s+[\w\s\*]*?\b(moe_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    names = declared_symbols()
    assert set(names) == set(_lib.EXPORTED), names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.moe_version() == 1


def test_nm_dynamic_exports():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (moe_\w+)", out))
    assert set(declared_symbols()) <= exported


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device error path")
def test_ctx_without_device_is_not_initialized():
    lib = _lib.load()
    out = ctypes.c_void_p()
    rc = lib.moe_ctx_create(0, None, ctypes.byref(out))
    assert rc == 3  # MOE_NOT_INITIALIZED
    assert b"no HIP device" in lib.moe_last_error()
    with pytest.raises(rt.RunntimeError) as ei:
        _lib.check(rc)
    assert ei.value.code == "NOT_INITIALIZED"


def test_null_context_is_rejected():
    lib = _lib.load()
    rc = lib.moe_sync(None)
    assert rc == 3
    rc = lib.moe_topk(None, None, 0, 1, 4, 4, None)
    assert rc == 3


# ------------------------------------------------- op checks (graph-build)


def _input(dims, dtype=torch.float32):
    return torch.zeros(dims, dtype=dtype)


def _quant(rows, cols, bits=8):
    return QuantW(torch.zeros(rows * cols * bits // 32, dtype=torch.int32), (rows, cols))


MOE = {"bits": 8, "groupSize": 4}


def _experts(k, n, bits=8):
    # One routed layer for 2 experts of [K, N] (matmul.test.ts:283-287).
    return QuantExpertWeight(_quant(2 * k, n, bits), _input([2 * k // 4, n]), _input([2, n]))


ROUTE = _input([3, 8])
X = _input([3, 8])
GLU = _experts(8, 16)
LIN = _experts(8, 16)


MOE_UP_REJECTS = [
    dict(x=_input([3, 8], torch.float64), error=r"expected a 2D f32 or f16 tensor"),
    dict(glu=QuantExpertWeight(_input([16, 16]), GLU.scales, GLU.bias),
         error=r"w must be a quantW \[E·8, N\] weight"),
    dict(glu=QuantExpertWeight(_quant(12, 16), GLU.scales, GLU.bias),
         error=r"w must be a quantW \[E·8, N\] weight"),
    dict(glu=QuantExpertWeight(_quant(16, 16, 4), GLU.scales, GLU.bias),
         error=r"elems 32 != rows·cols·8/32"),
    dict(glu=_experts(8, 6), lin=_experts(8, 6), error=r"K 8 and N 6 must be multiples of 4"),
    dict(opts={"groupSize": 3}, error=r"groupSize 3 must be a multiple of 4 that divides K 8"),
    dict(glu=QuantExpertWeight(GLU.w, _input([2, 16]), GLU.bias), error=r"scales must be f32 \[4, 16\]"),
    dict(glu=QuantExpertWeight(GLU.w, GLU.scales, _input([16])), error=r"bias must be f32 \[2, 16\]"),
    dict(route=_input([3, 3]), error=r"route must be topk's f32 \[3, 8\] output"),
    dict(lin=_experts(8, 8), error=r"glu and lin weights must have the same shape"),
]


@pytest.mark.parametrize("case", MOE_UP_REJECTS)
def test_moe_up_rejects(case):
    # matmul.test.ts:311-371 (f16 activations are accepted here: an extension)
    x = case.get("x", X)
    route = case.get("route", ROUTE)
    glu = case.get("glu", GLU)
    lin = case.get("lin", LIN)
    opts = {**MOE, **case.get("opts", {})}
    with pytest.raises(ValueError, match=case["error"]):
        rt.moeUp(x, route, glu, lin, opts)


def _desc(v):
    """moe_value_desc of a tensor or QuantW (ValueMeta: dtype, dims, elems)."""
    if isinstance(v, QuantW):
        dt, dims, elems = 2, list(v.dims), v.elems
    else:
        dt = {torch.float32: 0, torch.float16: 1}.get(v.dtype, 9)
        dims, elems = list(v.shape), v.numel()
    d = _lib.ValueDescC()
    d.dtype, d.rank, d.elems = dt, len(dims), elems
    for i, n in enumerate(dims[:4]):
        d.dims[i] = n
    return d


@pytest.mark.parametrize("case", [c for c in MOE_UP_REJECTS
                                  if "x" not in c and "same shape" not in c["error"]])
def test_c_abi_check_expert_weight_messages(case):
    """moe_check_expert_weight (the checkExpertWeight a native executor runs)
    fails the same cases with the same messages as the host mirror, and
    passes the valid weight with N and the expert count."""
    lib = _lib.load()
    route = case.get("route", ROUTE)
    glu = case.get("glu", GLU)
    opts = {**MOE, **case.get("opts", {})}
    n, e = ctypes.c_int64(), ctypes.c_int64()
    rc = lib.moe_check_expert_weight(b"moeUp", _desc(glu.w), _desc(glu.scales), _desc(glu.bias),
                                     _desc(route), 8, 3, 4, opts["bits"], opts["groupSize"],
                                     ctypes.byref(n), ctypes.byref(e))
    assert rc == 1, case
    msg = lib.moe_last_error().decode()
    assert re.search(case["error"], msg), msg
    assert msg.startswith("moeUp: ")
    ok = lib.moe_check_expert_weight(b"moeUp", _desc(GLU.w), _desc(GLU.scales), _desc(GLU.bias),
                                     _desc(ROUTE), 8, 3, 4, 8, 4, ctypes.byref(n), ctypes.byref(e))
    assert ok == 0 and (n.value, e.value) == (16, 2)


ACT = _input([12, 16])
OUT = _experts(16, 8)
RES = _input([3, 8])


@pytest.mark.parametrize("case", [
    dict(act=_input([10, 16]), error=r"act rows 10 must be a multiple of 4"),
    dict(residual=_input([3, 4]), error=r"residual must be f32 \[3, 8\]"),
    dict(route=_input([2, 8]), error=r"route must be topk's f32 \[3, 8\] output"),
    dict(out=QuantExpertWeight(OUT.w, OUT.scales, _input([3, 8])), error=r"bias must be f32 \[2, 8\]"),
])
def test_moe_down_rejects(case):
    # matmul.test.ts:384-409
    with pytest.raises(ValueError, match=case["error"]):
        rt.moeDown(case.get("act", ACT), case.get("route", ROUTE), case.get("out", OUT),
                   case.get("residual", RES), MOE)


@pytest.mark.parametrize("k,cols,error", [
    (0, 8, r"k must be in 1..16, got 0"),
    (17, 32, r"k must be in 1..16, got 17"),
    (4, 3, r"need at least 4 columns, got 3"),
])
def test_topk_rejects(k, cols, error):
    # topkSelect.gpu.test.ts:92-98 (k = 2 is accepted here: the reference
    # compiles in k = 4, this build takes k in 1..16)
    with pytest.raises(ValueError, match=error):
        rt.topk(_input([2, cols]), k)


def test_cpu_tensors_are_rejected_after_checks():
    x = _input([2, 8])
    with pytest.raises(rt.RunntimeError) as ei:
        rt.topk(x, 4)
    assert ei.value.code == "INVALID_ARGUMENT"


def test_runntime_error_codes():
    e = rt.RunntimeError("EXECUTION_FAILED", "boom")
    assert rt.is_runntime_error(e) and rt.is_runntime_error(e, "EXECUTION_FAILED")
    assert not rt.is_runntime_error(e, "INVALID_ARGUMENT")
    assert not rt.is_runntime_error(ValueError("x"))
    with pytest.raises(ValueError):
        rt.RunntimeError("NOPE", "x")


def test_pack_quant_w_device_rejects_host_or_wrong_dtype():
    with pytest.raises(ValueError, match="packQuantW: ints must be a device int8"):
        rt.pack_quant_w_device(torch.zeros((2, 8, 8), dtype=torch.int8))
    with pytest.raises(ValueError, match="packQuantW"):
        rt.pack_quant_w_device(torch.zeros((2, 8, 8), dtype=torch.int32))


def test_weights_null_handle_paths():
    """moe_weights_view on no handle is NOT_INITIALIZED; releasing none is a no-op."""
    lib = _lib.load()
    v = _lib.ExpertWeightC()
    assert lib.moe_weights_view(None, ctypes.byref(v)) == 3
    assert b"handle is NULL" in lib.moe_last_error()
    assert lib.moe_weights_release(None) == 0


@pytest.mark.parametrize("case", [
    dict(x=_input([4])[None, None], error=r"rmsNorm: expected a 2D f32 or f16 tensor"),
    dict(opts={"group": 3}, error=r"rmsNorm: group 3 must divide the row width 8"),
    dict(w=_input([4]), error=r"rmsNorm: weight must be f32 with 8 elems, got \(4,f32\)"),
    dict(w=_input([3]), opts={"group": 4}, error=r"weight must be f32 with 4 or 8 elems, got \(3,f32\)"),
    dict(w=_input([8]).half(), error=r"weight must be f32 with 8 elems, got \(8,f16\)"),
    dict(eps=0, error=r"rmsNorm: eps must be positive, got 0"),
    dict(opts={"residual": _input([4, 4])}, error=r"rmsNorm: residual must be f32 \[4, 8\]"),
])
def test_rmsnorm_rejects(case):
    # test/core/graph/ops/reduce.test.ts:116-170 and ops/reduce.ts:67-91
    with pytest.raises(ValueError, match=case["error"]):
        rt.rmsNorm(case.get("x", _input([4, 8])), case.get("w", _input([8])), case.get("eps", 1e-6),
                   case.get("opts"))


def test_moe_block_rejects_a_bad_norm_weight():
    x = _input([2, 8])
    with pytest.raises(ValueError, match=r"rmsNorm: weight must be f32 with 8 elems"):
        rt.moe_block(x, _input([4]), 1e-5, _input([8, 2]), None, GLU, LIN, OUT, 2)
    with pytest.raises(ValueError, match=r"rmsNorm: eps must be positive"):
        rt.moe_block(x, _input([8]), 0.0, _input([8, 2]), None, GLU, LIN, OUT, 2)


@pytest.mark.parametrize("case", [
    dict(w=_input([8, 6]), bias=_input([2, 6]), error=r"matmulGather: n 6 must be divisible by 4"),
    dict(w=_input([10, 8]), error=r"matmulGather: w rows 10 not a multiple of K 4"),
    dict(idx=_input([3]), error=r"matmulGather: expertIdx must be f32 with 2 elems, got 3"),
    dict(w=_input([8, 8]).half(), error=r"matmulGather: w is f16 but a is f32"),
    dict(bias=_input([2, 8]).half(), error=r"matmulGather: bias must be f32, got f16"),
    dict(bias=_input([1, 8]), error=r"matmulGather: bias must be \[2, 8\], got 8 elems"),
])
def test_matmul_gather_rejects(case):
    # matmulGather.gpu.test.ts:142-170 and ops/matmul.ts:188-203; the last
    # case is the [E, N] bias check the reference test marks as a known bug.
    with pytest.raises(ValueError, match=case["error"]):
        rt.matmulGather(case.get("a", _input([2, 4])), case.get("w", _input([8, 8])),
                        case.get("idx", _input([2])), {"bias": case.get("bias", _input([2, 8]))})


# ---- attention ops: refusals with the reference's messages
# (rope.gpu.test.ts:136-177, graph/ops/attention.ts:28-214); they raise
# before any device work.
@pytest.mark.parametrize("opts,err", [
    (dict(headDim=3), r"headDim 3 must be a positive even integer"),
    (dict(headDim=4, srcStart=1, width=4), r"srcStart 1 must be a non-negative even integer"),
    (dict(headDim=4, srcStart=8, width=8), r"window \[8, 16\) exceeds 12 input cols"),
    (dict(headDim=4, width=6), r"width 6 must be a multiple of headDim 4"),
])
def test_rope_refusals(opts, err):
    import runntime_amd as rt
    x = torch.zeros((2, 12))
    table = torch.zeros((2, opts["headDim"]))
    with pytest.raises(ValueError, match=err):
        rt.rope(x, table, table, opts)


def test_rope_refuses_tables_of_the_wrong_size():
    import runntime_amd as rt
    x = torch.zeros((2, 8))
    table = torch.zeros((1, 4))
    with pytest.raises(ValueError, match=r"cos must be f32 \[T,headDim\] = 8 elems, got 4"):
        rt.rope(x, table, table, dict(headDim=4))


def _sdpa_args(**kw):
    import math
    o = dict(qHeads=4, kvHeads=2, headDim=8, windowLeft=math.inf, windowRight=math.inf)
    o.update(kw)
    return o


@pytest.mark.parametrize("q_cols,opts,err", [
    (30, _sdpa_args(), r"sdpa: q cols 30 != qHeads\*headDim 32"),
    (32, _sdpa_args(kvHeads=3), r"sdpa: qHeads 4 not divisible by kvHeads 3"),
    (32, _sdpa_args(windowLeft=-1), r"sdpa: windowLeft -1 must be a non-negative integer or Infinity"),
    (32, _sdpa_args(windowRight=1.5), r"sdpa: windowRight 1.5 must be a non-negative integer or Infinity"),
    (32, _sdpa_args(qPosOffset=-2), r"sdpa: qPosOffset -2 must be a non-negative integer"),
    (32, _sdpa_args(windowRight=0, qPosOffset=3), r"sdpa: qPosOffset\+qLen 8 exceeds key rows kvLen 5"),
    (32, _sdpa_args(maxSegment=4), r"sdpa: maxSegment needs segments"),
])
def test_sdpa_refusals(q_cols, opts, err):
    import runntime_amd as rt
    q = torch.zeros((5, q_cols))
    k = torch.zeros((5, 16))
    with pytest.raises(ValueError, match=err):
        rt.sdpa(q, k, k, opts)


def test_sdpa_refuses_mixed_dtypes_and_sinks():
    import runntime_amd as rt
    q, k = torch.zeros((5, 32)), torch.zeros((5, 16))
    with pytest.raises(ValueError, match=r"q, k and v must share a dtype, got f32/f16/f32"):
        rt.sdpa(q, k.half(), k, _sdpa_args())
    with pytest.raises(ValueError, match=r"sinks must be f32 with 4 elems, got 3"):
        rt.sdpa(q, k, k, _sdpa_args(sinks=torch.zeros(3)))
    with pytest.raises(ValueError, match=r"keyBias keys \[2, 9\) must lie within the 5 keys"):
        rt.sdpa(q, k, k, _sdpa_args(keyBias=dict(start=2, end=9, value=1.0)))
    with pytest.raises(ValueError, match=r"sdpaPacked: qkv cols 40 != \(qHeads \+ 2\*kvHeads\)\*headDim = 64"):
        rt.sdpaPacked(torch.zeros((5, 40)), _sdpa_args())
    with pytest.raises(ValueError, match=r"sdpaPacked: qLen must be > 1"):
        rt.sdpaPacked(torch.zeros((1, 64)), _sdpa_args())
