"""Per-kernel-group timing of libmoe (the reference's GpuPerfSink,
src/core/gpu/perf.ts:1-23): HIP event pairs around each launch group on the
context's stream."""
import ctypes

import torch

from . import _lib


def _ctx(device=None) -> int:
    idx = torch.cuda.current_device() if device is None else device
    return _lib.context(idx, torch.cuda.current_stream(idx).cuda_stream)


def enable(on: bool = True, device=None) -> None:
    _lib.check(_lib.load().moe_prof_enable(_ctx(device), 1 if on else 0))


def read(reset: bool = True, device=None) -> dict:
    """{group: (total_ms, launches)} for the groups that ran."""
    ms = (ctypes.c_double * 8)()
    cnt = (ctypes.c_int64 * 8)()
    _lib.check(_lib.load().moe_prof_read(_ctx(device), 1 if reset else 0, ms, cnt))
    return {name: (ms[i], cnt[i]) for i, name in enumerate(_lib.PROF_GROUPS) if cnt[i]}


def reserve(T, d, I, E, k, device=None) -> None:
    """Grows the context workspace for layers up to these sizes, so calls
    (and graph captures) of no larger shapes allocate nothing."""
    _lib.check(_lib.load().moe_ctx_reserve(_ctx(device), T, d, I, E, k))


def reserve_batched(calls, T, d, I, E, k, device=None) -> None:
    """reserve() for moe_layer_batched with up to `calls` calls."""
    _lib.check(_lib.load().moe_ctx_reserve_batched(_ctx(device), calls, T, d, I, E, k))
