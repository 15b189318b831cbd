"""moe_layer_noalloc (the allocation-free entry point: its workspace is the
library's static per-GPU scratch) against moe_layer through the C ABI: the
same kernels on the same arguments, so the outputs and routes are equal bit
for bit, on two calls in a row (the second smaller, over the scratch the
first left behind), and a shape whose workspace exceeds the scratch is
refused with the size it needs."""
import numpy as np
import pytest
import torch

import runntime_amd as rt
from runntime_amd import _lib
from runntime_amd.synth import CONFIGS, MoeConfig, make_inputs

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _pair(cfg, seed):
    inp = make_inputs(cfg, seed=seed, bias_rand=True)
    g = torch.Generator().manual_seed(seed)
    inp.residual.copy_(torch.randn(tuple(inp.residual.shape), generator=g))
    args = (inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down, inp.residual, cfg.k)
    t, d = cfg.T, cfg.d
    out = torch.empty((t, d), dtype=torch.float32, device=inp.x.device)
    route = torch.empty((t, 2 * cfg.k), dtype=torch.float32, device=inp.x.device)
    rt.moe_layer(*args, out=out, route=route, noalloc=True)
    want, want_route = rt.moe_layer(*args, return_route=True)
    torch.cuda.synchronize()
    return out.cpu().numpy(), route.cpu().numpy(), want.cpu().numpy(), want_route.cpu().numpy()


def test_noalloc_equals_moe_layer_twice():
    # config 3 (T = 8, d = 2048, E = 64, k = 8, I = 1408, f16 x), then a
    # smaller call (T = 5, config 1's shape) over the scratch the first used
    big = CONFIGS[3]
    small = MoeConfig("c1_T5", 5, 512, 8, 2, 1024, "f32")
    for cfg, seed in ((big, 3), (small, 5)):
        say(f"moe_layer_noalloc {cfg.name}")
        got, got_route, want, want_route = _pair(cfg, seed)
        assert np.array_equal(got_route, want_route), cfg.name
        assert np.array_equal(got, want), cfg.name


def test_noalloc_refuses_a_shape_over_the_scratch():
    cfg = CONFIGS[4]  # T = 4096: act alone is 369 MB
    say("moe_layer_noalloc over the scratch")
    inp = make_inputs(cfg, seed=4)
    with pytest.raises(rt.RunntimeError) as ei:
        rt.moe_layer(inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down, None, cfg.k,
                     noalloc=True)
    assert ei.value.code == "INVALID_ARGUMENT"
    assert f"the static scratch holds {_lib.NOALLOC_SCRATCH_BYTES}" in str(ei.value)


def test_noalloc_refuses_another_stream_with_work_queued():
    """Two streams on one GPU would share the scratch: a call on a second
    stream while the first still has queued work is refused; once the first
    has finished, the second may use it."""
    cfg = MoeConfig("c1_T5", 5, 512, 8, 2, 1024, "f32")
    inp = make_inputs(cfg, seed=9)
    args = (inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down, inp.residual, cfg.k)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    say("moe_layer_noalloc on stream 1 behind a bounded sleep")
    with torch.cuda.stream(s1):
        torch.cuda._sleep(200_000_000)  # ~0.1 s of a busy stream, bounded
        rt.moe_layer(*args, noalloc=True)
    with torch.cuda.stream(s2):
        with pytest.raises(rt.RunntimeError) as ei:
            rt.moe_layer(*args, noalloc=True)
    assert ei.value.code == "INVALID_ARGUMENT"
    assert "has not finished" in str(ei.value)
    s1.synchronize()
    with torch.cuda.stream(s2):
        out = rt.moe_layer(*args, noalloc=True)
    s2.synchronize()
    want = rt.moe_layer(*args)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want.cpu().numpy())


def test_noalloc_under_graph_capture_allocates_nothing():
    """moe_layer_noalloc captured into a graph on a fresh context whose
    workspace is empty: a workspace that has to grow inside a capture raises,
    so any allocation on this path would fail the capture. Every replay
    equals moe_layer."""
    import ctypes
    cfg = CONFIGS[3]
    inp = make_inputs(cfg, seed=12, bias_rand=True)
    args = (inp.x, inp.router_w, inp.router_b, inp.glu, inp.lin, inp.down, inp.residual, cfg.k)
    want = rt.moe_layer(*args)
    torch.cuda.synchronize()
    out = torch.empty((cfg.T, cfg.d), dtype=torch.float32, device="cuda")
    route = torch.empty((cfg.T, 2 * cfg.k), dtype=torch.float32, device="cuda")
    lib = _lib.load()
    fresh = ctypes.c_void_p()
    dev = torch.cuda.current_device()
    _lib.check(lib.moe_ctx_create(dev, None, ctypes.byref(fresh)))
    saved = _lib._ctxs[dev]
    _lib._ctxs[dev] = fresh.value
    try:
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        say("capturing moe_layer_noalloc on a context with no workspace")
        with torch.cuda.graph(g, stream=s):
            rt.moe_layer(*args, out=out, route=route, noalloc=True)
        torch.cuda.synchronize()
        for i in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), want.cpu().numpy()), f"replay {i}"
        del g
        torch.cuda.synchronize()
    finally:
        _lib._ctxs[dev] = saved
        lib.moe_ctx_destroy(fresh)
