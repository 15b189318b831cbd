"""safetensors reading and the MoE block loader, on files written here.

The header, quantization-setting and int-weight cases follow the reference's
reader tests (test/core/weights/safetensors.test.ts: header entries, header
lengths, `runntime.quant` settings, I8/U8 weights with F16 scales); the
loader's checks follow src/core/nn/loadStateDict.ts:180-215 and the Linear's
layout check (src/core/nn/layers.ts:196-217)."""
import json
import struct

import numpy as np
import pytest
import torch

from oracle import ref
from runntime_amd import checkpoint as ck
from runntime_amd import safetensors as st
from runntime_amd.errors import RunntimeError


def raw_file(tmp_path, header, payload=b""):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    p = tmp_path / "f.safetensors"
    p.write_bytes(struct.pack("<Q", len(h)) + h + payload)
    return str(p)


@pytest.mark.parametrize("entry,error", [
    ({"dtype": "Q7", "shape": [4], "data_offsets": [0, 4]}, r"unsupported dtype \"Q7\""),
    ({"dtype": "U8", "shape": [-1], "data_offsets": [0, 4]}, r"malformed shape"),
    ({"dtype": "U8", "shape": [4], "data_offsets": [0]}, r"malformed data_offsets"),
    ({"dtype": "U8", "shape": [4], "data_offsets": [-4, 0]}, r"malformed data_offsets"),
    ({"dtype": "U8", "shape": [4], "data_offsets": [8, 4]}, r"running backwards"),
    ({"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}, r"spans 4 bytes but shape \[2\] of F32 needs 8"),
    ({"dtype": "F16", "shape": [3], "data_offsets": [0, 8]}, r"spans 8 bytes but shape \[3\] of F16 needs 6"),
    ("notanobject", r"is not an object"),
])
def test_header_entry_rejects(tmp_path, entry, error):
    with pytest.raises(ValueError, match=error):
        st.SafetensorsFile(raw_file(tmp_path, {"w": entry}, bytes(8)))


@pytest.mark.parametrize("data,error", [
    (struct.pack("<Q", 0), r"implausible header length 0"),
    (struct.pack("<Q", 200 * 1024 * 1024), r"implausible header length"),
    (struct.pack("<Q", 2 ** 63), r"implausible header length"),
    (b"<!doctype html><html></html>", r"not a safetensors payload"),
    (bytes(4), r"past end 4"),
    (struct.pack("<Q", 100) + b"{}", r"past end 10"),
    (struct.pack("<Q", 5) + b"{nope", r"not valid JSON"),
    (struct.pack("<Q", 4) + b"null", r"header is not a JSON object"),
    (struct.pack("<Q", 2) + b"[]", r"header is not a JSON object"),
])
def test_header_rejects(tmp_path, data, error):
    p = tmp_path / "f.safetensors"
    p.write_bytes(data)
    with pytest.raises(ValueError, match=error):
        st.SafetensorsFile(str(p))


def int8_file(tmp_path, metadata=None, tensors=None):
    tensors = tensors or {
        "w": ("I8", [2, 4], np.array([1, -2, 3, -4, 5, -6, 7, -8], np.int8)),
        "w_scale": ("F16", [2, 2], np.array([0.5, 1, 2, 4], np.float16)),
    }
    p = str(tmp_path / "q.safetensors")
    st.write(p, tensors, metadata)
    return p


VALID = {"version": 1, "bits": 8, "groupSize": 2, "scheme": "symmetric"}


def quant(v):
    return {"runntime.quant": json.dumps(v) if not isinstance(v, str) else v}


@pytest.mark.parametrize("metadata,error", [
    ({"runntime.quant": "{bits"}, r"JSON"),
    (quant([1, 8]), r"not a JSON object"),
    (quant({**VALID, "version": 2}), r"version"),
    (quant({k: v for k, v in VALID.items() if k != "version"}), r"version"),
    (quant({**VALID, "bits": 2}), r"bits 4 or 8"),
    (quant({**VALID, "bits": "8"}), r"bits 4 or 8"),
    (quant({**VALID, "groupSize": 0}), r"groupSize"),
    (quant({**VALID, "groupSize": 1.5}), r"groupSize"),
    (quant({**VALID, "groupSize": "2"}), r"groupSize"),
    (quant({**VALID, "scheme": "asymmetric"}), r"scheme"),
])
def test_quant_setting_rejects(tmp_path, metadata, error):
    with pytest.raises(RunntimeError, match=error) as ei:
        st.SafetensorsFile(int8_file(tmp_path, metadata))
    assert ei.value.code == "CHECKPOINT_MISMATCH"


@pytest.mark.parametrize("dtype", ["I8", "U8"])
def test_int_tensor_without_setting(tmp_path, dtype):
    p = str(tmp_path / "n.safetensors")
    st.write(p, {"w": (dtype, [2], np.zeros(2, np.uint8))})
    with pytest.raises(RunntimeError, match=rf"w is {dtype}.*no 'runntime.quant'") as ei:
        st.SafetensorsFile(p)
    assert ei.value.code == "CHECKPOINT_MISMATCH"


SCALE = ("F16", [2, 2], np.zeros(4, np.float16))


@pytest.mark.parametrize("tensors,error", [
    ({"w": ("I8", [4], np.zeros(4, np.int8)), "w_scale": SCALE}, r"needs a 2D shape"),
    ({"w": ("I8", [2, 3], np.zeros(6, np.int8)), "w_scale": SCALE},
     r"3 columns, not a multiple of groupSize 2"),
    ({"w": ("I8", [2, 4], np.zeros(8, np.int8))}, r"has no w_scale"),
    ({"w": ("I8", [2, 4], np.zeros(8, np.int8)), "w_scale": ("F32", [2, 2], np.zeros(4, np.float32))},
     r"needs an F16 w_scale of shape \[2, 2\], got F32 \[2, 2\]"),
    ({"w": ("I8", [2, 4], np.zeros(8, np.int8)), "w_scale": ("F16", [2, 1], np.zeros(2, np.float16))},
     r"needs an F16 w_scale of shape \[2, 2\], got F16 \[2, 1\]"),
])
def test_quant_weight_rejects(tmp_path, tensors, error):
    with pytest.raises(RunntimeError, match=error) as ei:
        st.SafetensorsFile(int8_file(tmp_path, quant(VALID), tensors))
    assert ei.value.code == "CHECKPOINT_MISMATCH"


def test_i8_in_an_int4_file(tmp_path):
    t = {"w": ("I8", [2, 2], np.zeros(4, np.int8)), "w_scale": ("F16", [2, 2], np.zeros(4, np.float16))}
    with pytest.raises(RunntimeError, match=r"is I8, but int4 is stored as U8"):
        st.SafetensorsFile(int8_file(tmp_path, quant({**VALID, "bits": 4}), t))


def test_int8_and_int4_values(tmp_path):
    f = st.SafetensorsFile(int8_file(tmp_path, quant(VALID)))
    q = f.quant["w"]
    assert q.bits == 8 and q.group_size == 2 and q.shape == [2, 4]
    assert q.ints().tolist() == [[1, -2, 3, -4], [5, -6, 7, -8]]
    assert q.scales().tolist() == [[0.5, 1.0], [2.0, 4.0]]
    assert "w_scale" not in f.names
    # int4: two signed nibbles per byte, low nibble first (0x8F → -1, -8)
    p = str(tmp_path / "q4.safetensors")
    st.write(p, {"w": ("U8", [1, 2], np.array([0x8F, 0x71], np.uint8)),
                 "w_scale": ("F16", [1, 2], np.ones(2, np.float16))},
             quant({"version": 1, "bits": 4, "scheme": "symmetric"}))
    q4 = st.SafetensorsFile(p).quant["w"]
    assert q4.shape == [1, 4] and q4.group_size == 2
    assert q4.ints().tolist() == [[-1, -8, 1, 7]]


def test_bf16_widens_to_f32(tmp_path):
    v = np.array([1.5, -2.25, 3e-3], np.float32)
    bits = (v.view(np.uint32) >> 16).astype(np.uint16)
    p = str(tmp_path / "b.safetensors")
    st.write(p, {"x": ("BF16", [3], bits)})
    got = st.SafetensorsFile(p).array("x")
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, (bits.astype(np.uint32) << 16).view(np.float32))


# ------------------------------------------------------------- the loader

def small_block(E=8, d=64, I=128, seed=3, bits=8):
    rng = np.random.default_rng(seed)
    lim = 127 if bits == 8 else 7
    q = {n: rng.integers(-lim, lim + 1, size=s).astype(np.int8)
         for n, s in (("glu", (E, d, I)), ("lin", (E, d, I)), ("out", (E, I, d)))}
    ex = {}
    for n in ("glu", "lin", "out"):
        K, N = q[n].shape[1:]
        ex[n] = (ref.pack_ekn(q[n], bits), rng.uniform(5e-4, 2e-3, (E, N)).astype(np.float32),
                 (0.1 * rng.standard_normal((E, N))).astype(np.float32))
    gate = (0.02 * rng.standard_normal((E, d))).astype(np.float32)  # torch layout [E, d]
    gate_b = (0.1 * rng.standard_normal(E)).astype(np.float32)
    norm = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    return norm, gate, gate_b, ex, q


def test_load_round_trip(tmp_path):
    norm, gate, gate_b, ex, _ = small_block()
    p = str(tmp_path / "pf.safetensors")
    ck.save_moe_block(p, 3, norm, gate, gate_b, ex)
    b = ck.load_moe_block(p, layer=3, device="cpu", experts=8, hidden=64)
    assert (b.E, b.d, b.I, b.bits, b.group_up, b.group_down) == (8, 64, 128, 8, 64, 128)
    assert b.norm_w.dtype == torch.float32 and np.array_equal(b.norm_w.numpy(), norm)
    assert np.array_equal(b.router_w.numpy(), gate.T)  # transposed to [d, E] at load
    assert np.array_equal(b.router_b.numpy(), gate_b)
    for w, n in ((b.glu, "glu"), (b.lin, "lin"), (b.down, "out")):
        assert np.array_equal(w.w.words.numpy().view(np.uint32), ex[n][0])
        assert np.array_equal(w.scales.numpy(), ex[n][1])
        assert np.array_equal(w.bias.numpy(), ex[n][2])
    assert b.glu.w.dims == (8 * 64, 128) and b.down.w.dims == (8 * 128, 64)


def test_load_norm_weight_name_and_f16(tmp_path):
    norm, gate, gate_b, ex, _ = small_block()
    p = str(tmp_path / "pf.safetensors")
    ck.save_moe_block(p, 0, norm.astype(np.float16), gate, None, ex, norm_name="weight")
    b = ck.load_moe_block(p, device="cpu")
    assert b.norm_w.dtype == torch.float16 and b.router_b is None


def test_load_int4_experts_and_groups(tmp_path):
    E, d, I = 4, 64, 64
    rng = np.random.default_rng(1)
    ex = {}
    for n, (K, N) in (("glu", (d, I)), ("lin", (d, I)), ("out", (I, d))):
        q = rng.integers(-8, 8, size=(E, K, N)).astype(np.int8)
        ex[n] = (ref.pack_ekn(q, 4), rng.uniform(0.5, 1, (E * K // 16, N)).astype(np.float32), None)
    p = str(tmp_path / "q4.safetensors")
    ck.save_moe_block(p, 0, np.ones(d, np.float32), np.zeros((E, d), np.float32), None, ex)
    b = ck.load_moe_block(p, device="cpu")
    assert (b.bits, b.group_up, b.group_down) == (4, 16, 16) and b.glu.bias is None


def test_load_quantized_gate(tmp_path):
    """A gate stored as I8 + F16 scales (the runntime.quant format)
    dequantizes to f32 before the transpose."""
    norm, _, _, ex, _ = small_block()
    E, d = 8, 64
    rng = np.random.default_rng(5)
    qg = rng.integers(-127, 128, size=(E, d)).astype(np.int8)
    sg = rng.uniform(1e-4, 2e-4, (E, d // 32)).astype(np.float16)
    pre = "block.0.mlp."
    t = {pre + "norm.scale": ("F32", [d], norm), pre + "gate.weight": ("I8", [E, d], qg),
         pre + "gate.weight_scale": ("F16", [E, d // 32], sg)}
    for n, (w, s, bb) in ex.items():
        t[pre + f"{n}Weight"] = ("U32", [w.size], w)
        t[pre + f"{n}Scales"] = ("F32", list(s.shape), s)
        t[pre + f"{n}Bias"] = ("F32", list(bb.shape), bb)
    p = str(tmp_path / "qg.safetensors")
    st.write(p, t, {"runntime.quant": json.dumps({"version": 1, "bits": 8, "scheme": "symmetric"})})
    b = ck.load_moe_block(p, device="cpu")
    want = (qg.reshape(E, 2, 32).astype(np.float32) * sg.astype(np.float32)[:, :, None]).reshape(E, d)
    assert np.array_equal(b.router_w.numpy(), want.T)


@pytest.mark.parametrize("break_it,error", [
    (lambda t, pre: t.pop(pre + "gluWeight"), r"missing tensor 'block.0.mlp.gluWeight'"),
    (lambda t, pre: t.pop(pre + "gate.weight"), r"missing tensor 'block.0.mlp.gate.weight'"),
    (lambda t, pre: t.__setitem__(pre + "linWeight", ("U32", [10], np.zeros(10, np.uint32))),
     r"'block.0.mlp.linWeight' checkpoint shape \[10\] \(10 elems\) != model \[512,128\] \(16384 words\)"),
    (lambda t, pre: t.__setitem__(pre + "outBias", ("F32", [3], np.zeros(3, np.float32))),
     r"'block.0.mlp.outBias' checkpoint shape \[3\]"),
    (lambda t, pre: t.__setitem__(pre + "gluScales", ("F32", [3, 128], np.zeros(384, np.float32))),
     r"has 3 rows, which do not divide"),
    (lambda t, pre: t.__setitem__(pre + "gluWeight", ("I32", [16384], np.zeros(16384, np.int32))),
     r"is I32; the quantized MoE weights load as pre-packed U32"),
])
def test_load_rejects(tmp_path, break_it, error):
    norm, gate, gate_b, ex, _ = small_block()
    pre = "block.0.mlp."
    t = {pre + "norm.scale": ("F32", [64], norm), pre + "gate.weight": ("F32", [8, 64], gate),
         pre + "gate.bias": ("F32", [8], gate_b)}
    for n, (w, s, bb) in ex.items():
        t[pre + f"{n}Weight"] = ("U32", [w.size], w)
        t[pre + f"{n}Scales"] = ("F32", list(s.shape), s)
        t[pre + f"{n}Bias"] = ("F32", list(bb.shape), bb)
    break_it(t, pre)
    p = str(tmp_path / "bad.safetensors")
    st.write(p, t)
    with pytest.raises(RunntimeError, match=error) as ei:
        ck.load_moe_block(p, device="cpu")
    assert ei.value.code == "CHECKPOINT_MISMATCH"


def test_load_rejects_a_transposed_gate(tmp_path):
    norm, gate, gate_b, ex, _ = small_block()
    p = str(tmp_path / "pf.safetensors")
    ck.save_moe_block(p, 0, norm, gate.T.copy(), gate_b, ex)  # [d, E] instead of torch's [E, d]
    with pytest.raises(RunntimeError, match=r"Linear: block.0.mlp.gate.weight has shape \[64, 8\], "
                                            r"expected torch layout \[8, 64\]"):
        ck.load_moe_block(p, device="cpu", experts=8, hidden=64)
