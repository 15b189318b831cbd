"""The Node binding (runntime_amd/napi/): the N-API addon over the C ABI,
loaded by `node`, and the TypeScript Executor that dispatches the
reference's pending nodes to it (src/core/graph/evalCore.ts:14-43).

Without a GPU these check what runs on the host: the addon's exports and
error shape (RunntimeError with the reference's codes, src/core/error.ts),
checkExpertWeight's messages against the reference's regexes
(test/core/graph/ops/matmul.test.ts:276-409), and that the executor makes
one addon call per node with the operands in the order each op builder
records them (ops/matmul.ts:236-242, :265-270, ops/reduce.ts:90-100,
ops/matmul.ts:86-96), against a recording mock of the addon."""
import json
import os
import re
import shutil
import subprocess

import pytest
import torch

from tests.napi.strip_types import strip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NAPI = os.path.join(ROOT, "runntime_amd", "napi")
ADDON = os.path.join(NAPI, "runntime_moe.node")
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_node(script, *args):
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "napi", script), *args],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout.strip().splitlines()[-1])


@pytest.fixture(scope="module")
def addon_report():
    assert os.path.exists(ADDON), "the addon is not built (runntime_amd/build.py builds it)"
    return run_node("addon_check.mjs", ADDON)


def test_addon_exports(addon_report):
    assert addon_report["version"] == 1
    assert set(addon_report["exports"]) >= {
        "ctxCreate", "ctxDestroy", "sync", "bufferAlloc", "bufferFree", "bufferWrite",
        "bufferRead", "checkExpertWeight", "topk", "routerTopk", "moeUp", "moeDown", "moeLayer",
        "moeBlock", "rmsNorm", "linear", "packQuantW", "attention", "weightsUpload",
        "weightsView", "weightsDispose"}


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device error path")
def test_addon_context_without_device(addon_report):
    r = addon_report["ctxCreate"]
    assert not r["ok"] and r["name"] == "RunntimeError" and r["code"] == "NOT_INITIALIZED"
    assert "no HIP device" in r["message"]


def test_addon_errors(addon_report):
    r = addon_report["nullCtxUp"]
    assert (r["ok"], r["code"], r["message"]) == (False, "NOT_INITIALIZED", "moeUp: context is NULL")
    r = addon_report["badPointer"]
    assert not r["ok"] and r["code"] == "INVALID_ARGUMENT"


# The reference's regexes for checkExpertWeight (matmul.test.ts:311-371).
CHECKS = {
    "bits": r"bits must be 8 or 4, got 5",
    "w not quantW": r"w must be a quantW \[E·8, N\] weight",
    "w rows": r"w must be a quantW \[E·8, N\] weight",
    "elems": r"elems 32 != rows·cols·8/32",
    "K N multiple of 4": r"K 8 and N 6 must be multiples of 4",
    "groupSize": r"groupSize 3 must be a multiple of 4 that divides K 8",
    "scales": r"scales must be f32 \[4, 16\]",
    "bias": r"bias must be f32 \[2, 16\]",
    "route": r"route must be topk's f32 \[3, 8\] output",
}


def test_addon_check_expert_weight(addon_report):
    got = dict(addon_report["checks"])
    assert got["good"] == {"ok": True, "value": {"n": 16, "experts": 2}}
    for name, rx in CHECKS.items():
        r = got[name]
        assert not r["ok"] and r["code"] == "INVALID_ARGUMENT", (name, r)
        assert re.search(rx, r["message"]) and r["message"].startswith("moeUp: "), (name, r)


def test_addon_refuses_malformed_meta_and_wide_integers(addon_report):
    got = dict(addon_report["malformed"])
    want = {"rank 5": "at most 4 is supported", "fractional dim": "dims[0] must be a non-negative",
            "string elems": "elems must be a non-negative integer",
            "int64 overflow": "out of int64 range"}
    for name, text in want.items():
        r = got[name]
        assert not r["ok"] and r["code"] == "INVALID_ARGUMENT" and text in r["message"], (name, r)


def test_executor_dispatch_operands(tmp_path):
    src = open(os.path.join(NAPI, "hipExecutor.ts")).read()
    js = tmp_path / "hipExecutor.mjs"
    js.write_text(strip(src))
    rec = dict(run_node("executor_check.mjs", str(js)))
    # T 3, K 8, N 16, E 2, int8, groupSize 8; inputs at 100..700, out 900;
    # lin's bias is the second half of the concatenated bias (700 + 2·16·4)
    assert rec["moeUp"] == [["moeUp", "7n", "100n", 0, "200n", "300n", "400n", "700n", "500n",
                             "600n", "828n", 3, 8, 16, 2, 4, 8, 8, "900n"]]
    # act [12, 16] → T 3, K 16; w [32, 8] → N 8
    assert rec["moeDown"] == [["moeDown", "7n", "110n", "210n", "310n", "410n", "510n", "610n",
                               3, 16, 8, 2, 4, 8, 16, "910n"]]
    assert rec["topk"] == [["topk", "7n", "120n", 1, 3, 32, 4, "920n"]]
    assert rec["rmsNorm"] == [["rmsNorm", "7n", "130n", 0, 3, 8, "230n", 8, 1e-5, 8, "330n", 1,
                               "930n"]]
    assert rec["matmul"] == [["linear", "7n", "140n", "240n", "340n", "0n", 3, 8, 2, "940n"]]
    assert rec["add"] == {"error": "HipExecutor: op 'add' is not on the MoE path"}
    assert rec["pool"] == [["bufferAlloc", "7n", 96]]  # one allocation, reused after release
    assert rec["readback f16"] == [1.0, -2.0, 2.0 ** -24]
