"""A checkpoint in the hosted privacy-filter layout drives the kernels:
block 0 of a file with the model's shapes (E = 128, d = I = 640, int8 in
groups of 640, top-4; src/zoo/models.ts:71-73, moeMlp.ts:23-75), loaded onto
the GPU and run as EagerMoeMlp.forward; expert ids bit-exact, outputs at the
layer bar against the oracle on the same file's arrays."""
import numpy as np
import pytest
import torch

from oracle import ref
from runntime_amd import checkpoint as ck
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("act", ["f32", "f16"])
def test_privacy_filter_block_from_checkpoint(tmp_path, act):
    E, d, I, T = 128, 640, 640, 5
    say(f"privacy-filter block from a checkpoint, {act} activations")
    rng = np.random.default_rng(21)
    q = {n: rng.integers(-127, 128, size=s).astype(np.int8)
         for n, s in (("glu", (E, d, I)), ("lin", (E, d, I)), ("out", (E, I, d)))}
    ex = {n: (ref.pack_ekn(q[n], 8), rng.uniform(5e-4, 2e-3, (E, q[n].shape[2])).astype(np.float32),
              (0.1 * rng.standard_normal((E, q[n].shape[2]))).astype(np.float32))
          for n in q}
    gate = (0.02 * rng.standard_normal((E, d))).astype(np.float32)
    gate_b = (0.1 * rng.standard_normal(E)).astype(np.float32)
    npd = np.float16 if act == "f16" else np.float32
    norm = (1 + 0.1 * rng.standard_normal(d)).astype(npd)
    p = str(tmp_path / "pf_int8g640.safetensors")
    ck.save_moe_block(p, 0, norm, gate, gate_b, ex)
    blk = ck.load_moe_block(p, device="cuda", experts=E, hidden=d)
    assert (blk.group_up, blk.group_down, blk.k) == (640, 640, 4)
    x = rng.standard_normal((T, d)).astype(npd)
    out, route = blk.forward(torch.from_numpy(x).cuda(), return_route=True)
    torch.cuda.synchronize()
    xf = x.astype(np.float32)
    xn = ref.rmsnorm(xf, norm.astype(np.float32), 1e-5, dtype=npd).astype(np.float32)
    want_route = ref.topk(ref.router_logits(xn, np.ascontiguousarray(gate.T), gate_b), 4)
    got_route = route.cpu().numpy()
    assert np.array_equal(got_route[:, :4], want_route[:, :4]), "expert ids differ"
    w = {n: ex[n] for n in ex}
    a = ref.moe_up(xn, want_route, w["glu"], w["lin"], 8, d, E)
    want = ref.moe_down(a, want_route, w["out"], xf, 8, I, E)
    assert_close(out.cpu().numpy(), want, what=f"block from checkpoint ({act})")
