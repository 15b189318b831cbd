"""The Node binding on the GPU: the reference's op chain of one routed layer
(router matmul → topk → moeUp → moeDown, src/zoo/privacy-filter/
moeMlp.ts:82-117) dispatched by the TypeScript HipExecutor
(runntime_amd/napi/hipExecutor.ts, types stripped) through the real N-API
addon into libmoe.so, at config 1's shape, checked against the CPU oracle:
  - logits within 1e-5 relative of the oracle's f32 router;
  - expert ids bit-exact with the oracle's topk of the logits the GPU
    produced (so a near-tie in the router's last bits cannot flip the
    check), gates within 1e-6;
  - act and out within the reference's kernel-test bar atol 1e-5·K,
    rtol 1e-4 (moeQuantW.gpu.test.ts:100,127) of the oracle on that route."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from oracle import ref
from runntime_amd.synth import CONFIGS, make_inputs
from tests.helpers import assert_close
from tests.napi.strip_types import strip

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NAPI = os.path.join(ROOT, "runntime_amd", "napi")
NODE = shutil.which("node")


@pytest.mark.skipif(NODE is None, reason="node is not installed on this machine")
def test_executor_layer_on_the_gpu(tmp_path):
    cfg = CONFIGS[1]
    T, d, E, k, I = cfg.T, cfg.d, cfg.E, cfg.k, cfg.I
    inp = make_inputs(cfg, seed=17, device="cpu", keep_q=True, bias_rand=True)
    rng = np.random.default_rng(17)
    res = rng.standard_normal((T, d)).astype(np.float32)
    x = inp.x.float().numpy()
    rw = inp.router_w.numpy()
    words = {n: ref.pack_ekn(inp.q[n].numpy(), 8) for n in ("glu", "lin", "down")}
    sc = {n: getattr(inp, n).scales.numpy() for n in ("glu", "lin", "down")}
    bs = {n: getattr(inp, n).bias.numpy() for n in ("glu", "lin", "down")}
    files = {"x": x, "rw": rw, "gw": words["glu"], "gs": sc["glu"], "lw": words["lin"],
             "ls": sc["lin"], "bcat": np.concatenate([bs["glu"], bs["lin"]]),
             "dw": words["down"], "ds": sc["down"], "db": bs["down"], "res": res}
    for name, a in files.items():
        np.ascontiguousarray(a).tofile(tmp_path / f"{name}.bin")
    (tmp_path / "meta.json").write_text(json.dumps({"T": T, "d": d, "E": E, "k": k, "I": I}))
    js = tmp_path / "hipExecutor.mjs"
    js.write_text(strip(open(os.path.join(NAPI, "hipExecutor.ts")).read()))
    print(f"node HipExecutor on the GPU: config 1 (T={T}, d={d}, E={E}, k={k}, I={I})", flush=True)
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "napi", "gpu_check.mjs"), str(js),
                        os.path.join(NAPI, "runntime_moe.node"), str(tmp_path)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-2000:])
    got = {n: np.fromfile(tmp_path / f"{n}.out", np.float32) for n in ("logits", "route", "act", "out")}
    logits = got["logits"].reshape(T, E)
    np.testing.assert_allclose(logits, ref.router_logits(x, rw, None), rtol=1e-5, atol=1e-6)
    route = got["route"].reshape(T, 2 * k)
    want_route = ref.topk(logits, k)
    assert np.array_equal(route[:, :k], want_route[:, :k]), "expert ids differ"
    np.testing.assert_allclose(route[:, k:], want_route[:, k:], atol=1e-6, rtol=1e-5)
    w = {n: (words[n], sc[n], bs[n]) for n in ("glu", "lin", "down")}
    act = ref.moe_up(x, want_route, w["glu"], w["lin"], 8, d, E)
    assert_close(got["act"].reshape(T * k, I), act, atol=1e-5 * d, rtol=1e-4, what="act")
    out = ref.moe_down(act, want_route, w["down"], res, 8, I, E)
    assert_close(got["out"].reshape(T, d), out, atol=1e-5 * I, rtol=1e-4, what="out")
