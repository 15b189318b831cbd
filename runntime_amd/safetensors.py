"""safetensors files: the header checks, the quantized-file setting and the
int-weight/scale pairing of ruNNtime's reader, with numpy reads (no pickle,
nothing executed from the file).

Reference: src/core/weights/safetensors.ts —
  tensorInfoOf (:67-105): dtype, shape and data_offsets of every entry, the
    byte span checked against the shape;
  parseSafetensorsHeader (:107-150): an 8-byte little-endian header length
    (at most 100 MB), a JSON object, `__metadata__` apart;
  quantConfigOf (:652-696): the `runntime.quant` metadata
    {"version": 1, "bits": 8|4, "groupSize": N, "scheme": "symmetric"};
  fileQuantTensor (:470-520): an I8 (int8) or U8 (two int4 per byte, low
    nibble first) weight [out, cols] with an F16 `<name>_scale` [out, groups];
  fromSafetensors (:698-772): int weights need the setting; scales pair with
    their weights and get no entry of their own.
Header problems raise ValueError (the reference's plain Error); setting and
pairing problems raise RunntimeError('CHECKPOINT_MISMATCH').
"""
import json
import os
import struct
from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

from .errors import RunntimeError

MAX_HEADER_BYTES = 100 * 1024 * 1024
QUANT_METADATA_KEY = "runntime.quant"

DTYPE_BYTES = {"F64": 8, "F32": 4, "F16": 2, "BF16": 2, "U32": 4, "I64": 8, "I32": 4,
               "I16": 2, "I8": 1, "U8": 1, "BOOL": 1}
_NP = {"F64": np.float64, "F32": np.float32, "F16": np.float16, "BF16": np.uint16,
       "U32": np.uint32, "I64": np.int64, "I32": np.int32, "I16": np.int16, "I8": np.int8,
       "U8": np.uint8, "BOOL": np.bool_}


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


@dataclass
class TensorInfo:
    dtype: str
    shape: list
    begin: int  # absolute file offsets
    end: int


def _tensor_info(name: str, value, data_start: int) -> TensorInfo:
    def bad(why):
        raise ValueError(f"safetensors: header entry '{name}' {why}")

    if not isinstance(value, dict):
        bad("is not an object")
    dtype = value.get("dtype")
    if not isinstance(dtype, str) or dtype not in DTYPE_BYTES:
        bad(f"has unsupported dtype {json.dumps(dtype)}")
    shape = value.get("shape")
    if not isinstance(shape, list) or not all(_is_int(n) and n >= 0 for n in shape):
        bad(f"has a malformed shape {json.dumps(shape)}")
    offs = value.get("data_offsets")
    if (not isinstance(offs, list) or len(offs) != 2
            or not all(_is_int(n) and n >= 0 for n in offs)):
        bad(f"has malformed data_offsets {json.dumps(offs)}")
    lo, hi = offs
    if hi < lo:
        bad(f"has data_offsets [{lo}, {hi}] running backwards")
    elems = int(np.prod(shape)) if shape else 1
    want = elems * DTYPE_BYTES[dtype]
    if hi - lo != want:
        bad(f"spans {hi - lo} bytes but shape [{', '.join(map(str, shape))}] of {dtype} needs {want}")
    return TensorInfo(dtype, list(shape), data_start + lo, data_start + hi)


def parse_header(buf: bytes):
    """(metadata, {name: TensorInfo}) of a whole-file byte string, entries in
    file order."""
    if len(buf) < 8:
        raise ValueError(f"safetensors: read [0, 8) past end {len(buf)}")
    head = buf[:8]
    (n,) = struct.unpack("<Q", head)
    if n <= 0 or n > MAX_HEADER_BYTES:
        if all(b in (0x09, 0x0A, 0x0D) or 0x20 <= b <= 0x7E for b in head):
            raise ValueError(
                f"safetensors: got text starting {json.dumps(head.decode('ascii'))} instead of a "
                "binary header — this is not a safetensors payload")
        raise ValueError(f"safetensors: implausible header length {n}")
    if 8 + n > len(buf):
        raise ValueError(f"safetensors: read [8, {8 + n}) past end {len(buf)}")
    try:
        header = json.loads(buf[8:8 + n].decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise ValueError(f"safetensors: header is not valid JSON: {e}") from e
    if not isinstance(header, dict):
        raise ValueError("safetensors: header is not a JSON object")
    data_start = 8 + n
    metadata, entries = {}, []
    for name, value in header.items():
        if name == "__metadata__":
            metadata = value
            continue
        entries.append((name, _tensor_info(name, value, data_start)))
    entries.sort(key=lambda e: e[1].begin)
    return metadata, dict(entries)


def quant_config(metadata) -> Optional[dict]:
    """The file's quantization setting ({bits, groupSize}, either may be
    None), or None for a float file."""
    raw = metadata.get(QUANT_METADATA_KEY) if isinstance(metadata, dict) else None
    if raw is None:
        return None

    def bad(why):
        raise RunntimeError("CHECKPOINT_MISMATCH",
                            f"safetensors: '{QUANT_METADATA_KEY}' metadata {json.dumps(raw)} {why}")

    if not isinstance(raw, str):
        bad("is not a string")
    try:
        cfg = json.loads(raw)
    except json.JSONDecodeError:
        bad("is not valid JSON")
    if not isinstance(cfg, dict):
        bad("is not a JSON object")
    if cfg.get("version") != 1 or isinstance(cfg.get("version"), bool):
        bad("has a version other than 1")
    bits = cfg.get("bits")
    if bits is not None and (not _is_int(bits) or bits not in (4, 8)):
        bad("needs bits 4 or 8")
    g = cfg.get("groupSize")
    if g is not None and (not _is_int(g) or g <= 0):
        bad("needs a positive integer groupSize")
    if cfg.get("scheme") != "symmetric":
        bad("needs scheme 'symmetric'")
    return {"bits": bits, "groupSize": g}


@dataclass
class QuantTensor:
    """An int weight [out, cols] with F16 scales [out, cols / groupSize]."""
    name: str
    shape: list
    bits: int
    group_size: int
    _ints: object = field(repr=False)
    _scales: object = field(repr=False)

    def ints(self) -> np.ndarray:
        """Signed values, one per element, [out, cols] int8."""
        return self._ints()

    def scales(self) -> np.ndarray:
        """f32 [out, cols / groupSize] (from the stored f16)."""
        return self._scales()


def _unpack_int4(b: np.ndarray) -> np.ndarray:
    """Two signed nibbles per byte, low nibble first (safetensors.ts:456-466)."""
    lo = ((b & 0x0F).astype(np.int16) ^ 8) - 8
    hi = ((b >> 4).astype(np.int16) ^ 8) - 8
    out = np.empty(b.size * 2, np.int8)
    out[0::2] = lo.reshape(-1)
    out[1::2] = hi.reshape(-1)
    return out


class SafetensorsFile:
    """An opened file: `metadata`, float/word tensors by name (`array`),
    quantized weights (`quant`)."""

    def __init__(self, path: str):
        self.path = path
        self._mm = np.memmap(path, dtype=np.uint8, mode="r")
        head = bytes(self._mm[:min(len(self._mm), 8)])
        if len(head) == 8:
            (n,) = struct.unpack("<Q", head)
            hdr_end = 8 + n if 0 < n <= MAX_HEADER_BYTES else 8
        else:
            hdr_end = 8
        self.metadata, infos = parse_header(bytes(self._mm[:min(len(self._mm), hdr_end)]))
        size = os.path.getsize(path)
        for name, info in infos.items():
            if info.end > size:
                raise ValueError(f"safetensors: tensor {name} reads [{info.begin}, {info.end}) "
                                 f"past end {size}")
        self.infos = infos
        cfg = quant_config(self.metadata)
        is_int = lambda i: i.dtype in ("I8", "U8")
        scale_names = {f"{n}_scale" for n, i in infos.items() if is_int(i)}
        self.quant: Dict[str, QuantTensor] = {}
        self.names = []
        for name, info in infos.items():
            if name in scale_names:
                continue
            self.names.append(name)
            if not is_int(info):
                continue
            if cfg is None:
                raise RunntimeError("CHECKPOINT_MISMATCH",
                                    f"safetensors: tensor {name} is {info.dtype}, but the file has "
                                    f"no '{QUANT_METADATA_KEY}' metadata")
            self.quant[name] = self._quant_tensor(name, info, infos.get(f"{name}_scale"), cfg)

    def _raw(self, info: TensorInfo) -> np.ndarray:
        return np.asarray(self._mm[info.begin:info.end])

    def _quant_tensor(self, name, info, scale, cfg) -> QuantTensor:
        def bad(why):
            raise RunntimeError("CHECKPOINT_MISMATCH", f"safetensors: quantized tensor {name} {why}")

        bits = cfg["bits"] if cfg["bits"] is not None else (8 if info.dtype == "I8" else 4)
        want = "I8" if bits == 8 else "U8"
        if info.dtype != want:
            bad(f"is {info.dtype}, but int{bits} is stored as {want}")
        if len(info.shape) != 2:
            bad(f"needs a 2D shape, got [{', '.join(map(str, info.shape))}]")
        out = info.shape[0]
        cols = info.shape[1] if bits == 8 else info.shape[1] * 2
        if scale is None:
            bad(f"has no {name}_scale")
        groups = scale.shape[1] if len(scale.shape) == 2 else 0
        g = cfg["groupSize"]
        if g is None:
            g = cols / groups if groups else float("nan")
        if not (isinstance(g, (int, float)) and g == g and float(g).is_integer() and g > 0):
            bad(f"needs an F16 {name}_scale [{out}, groups] with groups dividing {cols}, "
                f"got {scale.dtype} [{', '.join(map(str, scale.shape))}]")
        g = int(g)
        if cols % g:
            bad(f"has {cols} columns, not a multiple of groupSize {g}")
        sshape = [out, cols // g]
        if scale.dtype != "F16" or list(scale.shape) != sshape:
            bad(f"needs an F16 {name}_scale of shape [{', '.join(map(str, sshape))}], "
                f"got {scale.dtype} [{', '.join(map(str, scale.shape))}]")

        def ints():
            b = self._raw(info)
            v = b.view(np.int8) if bits == 8 else _unpack_int4(b)
            return v.reshape(out, cols).copy()

        def scales():
            return self._raw(scale).view(np.float16).astype(np.float32).reshape(sshape)

        return QuantTensor(name, [out, cols], bits, g, ints, scales)

    def array(self, name: str) -> np.ndarray:
        """A float or integer tensor as stored (BF16 widened to f32), shaped."""
        info = self.infos.get(name)
        if info is None or name in self.quant:
            raise KeyError(name)
        a = self._raw(info).view(_NP[info.dtype])
        if info.dtype == "BF16":
            a = (a.astype(np.uint32) << 16).view(np.float32)
        return a.reshape(info.shape).copy()


def write(path: str, tensors: Dict[str, tuple], metadata: Optional[dict] = None) -> None:
    """Writes {name: (dtype, shape, ndarray of the stored element type)} as a
    safetensors file (BF16 given as uint16 bits)."""
    header, blobs, off = {}, [], 0
    if metadata:
        header["__metadata__"] = metadata
    for name, (dtype, shape, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode("utf-8")
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
