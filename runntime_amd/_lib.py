"""Loads libmoe.so and declares its C ABI (include/runntime_moe.h) for ctypes.

The library must have been built (``python -m runntime_amd.build``); there is
no fallback: without it every op raises RunntimeError('NOT_INITIALIZED').
"""
import ctypes
import os
import threading

from .errors import STATUS_CODES, RunntimeError

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmoe.so")

MOE_F32 = 0
MOE_F16 = 1
# MOE_NULL_STREAM: the null (legacy default) stream as a stream argument.
MOE_NULL_STREAM = 1
# include/runntime_moe.h MOE_NOALLOC_SCRATCH_BYTES
NOALLOC_SCRATCH_BYTES = 16 << 20

# Every symbol include/runntime_moe.h declares.
EXPORTED = (
    "moe_version", "moe_last_error", "moe_ctx_create", "moe_ctx_set_stream",
    "moe_ctx_reserve", "moe_ctx_destroy", "moe_sync", "moe_topk", "moe_router_topk",
    "moe_up", "moe_down", "moe_layer", "moe_dispatch", "moe_prof_enable", "moe_prof_read",
    "moe_layer_batched", "moe_ctx_reserve_batched", "moe_pack_quantw",
    "moe_weights_upload", "moe_weights_view", "moe_weights_dispose", "moe_weights_release",
    "moe_block", "moe_rmsnorm", "moe_matmul_gather", "moe_block_float", "moe_rope",
    "moe_sdpa", "moe_linear", "moe_viterbi_decode", "moe_attention", "moe_ctx_pin_workspace",
    "moe_check_expert_weight", "moe_buffer_alloc", "moe_buffer_free", "moe_buffer_write",
    "moe_buffer_read", "moe_layer_noalloc",
)
PROF_GROUPS = ("topk", "router", "dispatch", "up", "down", "combine", "norm")


class CallStridesC(ctypes.Structure):
    """moe_call_strides: element strides between the calls of a batch."""
    _fields_ = [(n, ctypes.c_int64) for n in (
        "x", "router_w", "router_b", "glu_w", "glu_scales", "glu_bias", "lin_w", "lin_scales",
        "lin_bias", "down_w", "down_scales", "down_bias", "residual", "route", "out")]


class ValueDescC(ctypes.Structure):
    """moe_value_desc: a Value's ValueMeta (dtype code, dims, elems)."""
    _fields_ = [("dtype", ctypes.c_int), ("rank", ctypes.c_int), ("dims", ctypes.c_int64 * 4),
                ("elems", ctypes.c_int64)]


class ExpertWeightC(ctypes.Structure):
    """moe_expert_weight: quantW words, f32 scales, f32 bias (or NULL)."""
    _fields_ = [("w", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("bias", ctypes.c_void_p)]


_lock = threading.Lock()
_lib = None
_ctxs = {}


def load() -> ctypes.CDLL:
    """The loaded library, with argument types declared."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RunntimeError(
                "NOT_INITIALIZED",
                f"{LIB_PATH} is not built; run `python -m runntime_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        P, I, V = ctypes.c_void_p, ctypes.c_int, None
        W = ctypes.POINTER(ExpertWeightC)
        sigs = {
            "moe_version": ([], I),
            "moe_last_error": ([], ctypes.c_char_p),
            "moe_ctx_create": ([I, P, ctypes.POINTER(P)], I),
            "moe_ctx_set_stream": ([P, P], I),
            "moe_ctx_reserve": ([P, I, I, I, I, I], I),
            "moe_ctx_destroy": ([P], I),
            "moe_sync": ([P], I),
            "moe_topk": ([P, P, I, I, I, I, P], I),
            "moe_router_topk": ([P, P, I, P, P, I, I, I, I, P], I),
            "moe_up": ([P, P, I, P, W, W, I, I, I, I, I, I, I, P], I),
            "moe_down": ([P, P, P, W, P, I, I, I, I, I, I, I, P], I),
            "moe_layer": ([P, P, I, P, P, W, W, W, P, I, I, I, I, I, I, I, I, P, P], I),
            "moe_layer_noalloc": ([P, P, I, P, P, W, W, W, P, I, I, I, I, I, I, I, I, P, P], I),
            "moe_dispatch": ([P, P, I, I, I, P, P], I),
            "moe_pack_quantw": ([P, P, I, I, I, I, P], I),
            "moe_prof_enable": ([P, I], I),
            "moe_layer_batched": ([P, I, ctypes.POINTER(CallStridesC), P, I, P, P, W, W, W, P, I,
                                   I, I, I, I, I, I, I, P, P], I),
            "moe_ctx_reserve_batched": ([P, I, I, I, I, I, I], I),
            "moe_ctx_pin_workspace": ([P, I], I),
            "moe_check_expert_weight": ([ctypes.c_char_p] + [ctypes.POINTER(ValueDescC)] * 4 +
                                        [ctypes.c_int64, ctypes.c_int64, I, I, I,
                                         ctypes.POINTER(ctypes.c_int64),
                                         ctypes.POINTER(ctypes.c_int64)], I),
            "moe_buffer_alloc": ([P, ctypes.c_size_t, ctypes.POINTER(P)], I),
            "moe_buffer_free": ([P, P], I),
            "moe_buffer_write": ([P, P, P, ctypes.c_size_t], I),
            "moe_buffer_read": ([P, P, P, ctypes.c_size_t], I),
            "moe_prof_read": ([P, I, P, P], I),
            "moe_weights_upload": ([P, P, I, P, P, I, I, I, I, I, ctypes.POINTER(P)], I),
            "moe_weights_view": ([P, W], I),
            "moe_weights_dispose": ([P], I),
            "moe_weights_release": ([P], I),
            "moe_block": ([P, P, I, P, ctypes.c_float, P, P, W, W, W, I, I, I, I, I, I, I, I, P,
                           P], I),
            "moe_rmsnorm": ([P, P, I, I, I, P, I, ctypes.c_float, I, P, ctypes.c_float, P], I),
            "moe_matmul_gather": ([P, P, I, P, P, P, I, I, I, I, P], I),
            "moe_block_float": ([P, P, I, P, ctypes.c_float, P, P, P, P, P, P, P, P, I, I, I, I, I,
                                 P, P], I),
            "moe_rope": ([P, P, I, I, I, I, I, I, P, P, P], I),
            "moe_linear": ([P, P, P, P, P, I, I, I, P], I),
            "moe_viterbi_decode": ([P, P, P, P, I, I, P], I),
            "moe_attention": ([P, P, I, I, I, I, I, ctypes.c_int64, ctypes.c_int64, P, P, P, P], I),
            "moe_sdpa": ([P, I, P, ctypes.c_int64, P, ctypes.c_int64, P, ctypes.c_int64, I, I, I,
                          I, I, ctypes.c_int64, ctypes.c_int64, I, P, P, I, I, I, ctypes.c_float,
                          P], I),
        }
        for name, (args, res) in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
        return lib


def check(rc: int) -> None:
    """Raises the RunntimeError a non-zero moe_status stands for."""
    if rc == 0:
        return
    msg = load().moe_last_error().decode("utf-8", "replace")
    raise RunntimeError(STATUS_CODES.get(rc, "EXECUTION_FAILED"), msg)


def context(device: int, stream_handle: int) -> int:
    """The library context of `device`, switched to enqueue on `stream_handle`
    (a hipStream_t as an int). 0 is the null stream, as torch reports its
    default stream: the library then enqueues on that same null stream, so
    its kernels are ordered with torch's work (the context's own stream is
    non-blocking and would not be)."""
    lib = load()
    with _lock:
        ctx = _ctxs.get(device)
        if ctx is None:
            out = ctypes.c_void_p()
            check(lib.moe_ctx_create(device, None, ctypes.byref(out)))
            ctx = out.value
            _ctxs[device] = ctx
    check(lib.moe_ctx_set_stream(ctx, stream_handle or MOE_NULL_STREAM))
    return ctx


def pin_workspace(device: int, pin: bool) -> None:
    """Pins (or unpins) the workspace of `device`'s context: while pinned, a
    call that needs more workspace raises instead of moving it."""
    lib = load()
    ctx = context(device, 0)
    check(lib.moe_ctx_pin_workspace(ctx, 1 if pin else 0))
