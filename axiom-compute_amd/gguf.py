"""GGUF model files: the native reader (libaxh.so, include/axh_gguf.h) wrapped
for Python, and a small writer for producing test and benchmark files.

GGUF is ggml's on-disk format (published specification: ggml docs/gguf.md).
The reference has no loader ("GGUF file parsing - separate",
ROADMAP.md:230-234); these are the pieces that let real Q4_K_M / Q5_K_M
checkpoints (which mix Q4_K, Q5_K and Q6_K tensors) reach the kernels.
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterable, Optional, Union

from . import axh as _axh

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}

# ggml tensor types (GGUF ids)
GGML_F32, GGML_F16, GGML_Q4_0 = 0, 1, 2
GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 12, 13, 14
GGML_BF16 = 30


@dataclass(frozen=True)
class TensorInfo:
    name: str
    type: int
    shape: tuple  # ne[0] first (innermost, one row)
    offset: int   # absolute file offset
    nbytes: int

    @property
    def n_rows(self) -> int:
        r = 1
        for d in self.shape[1:]:
            r *= d
        return r

    @property
    def n_cols(self) -> int:
        return self.shape[0]


def _decode_value(t: int, item_t: int, count: int, addr: int) -> Any:
    if t in _SCALAR:
        fmt = _SCALAR[t]
        return struct.unpack(fmt, ctypes.string_at(addr, struct.calcsize(fmt)))[0]
    if t == STRING:
        return ctypes.string_at(addr, count).decode("utf-8", errors="replace")
    if t == ARRAY:
        out, at = [], addr
        for _ in range(count):
            if item_t in _SCALAR:
                fmt = _SCALAR[item_t]
                out.append(struct.unpack(fmt, ctypes.string_at(at, struct.calcsize(fmt)))[0])
                at += struct.calcsize(fmt)
            elif item_t == STRING:
                n = struct.unpack("<Q", ctypes.string_at(at, 8))[0]
                out.append(ctypes.string_at(at + 8, n).decode("utf-8", errors="replace"))
                at += 8 + n
            else:
                raise ValueError("nested GGUF arrays are not decoded")
        return out
    raise ValueError(f"unknown GGUF value type {t}")


class GgufFile:
    """A GGUF file mapped by the native reader.  `tensors` and `metadata` are
    read at open; tensor bytes stay in the mapping until close()."""

    def __init__(self, path: Union[str, Path]):
        self._lib = _axh.load_library()
        h = ctypes.c_void_p()
        _axh._check(self._lib.axh_gguf_open(str(path).encode(), ctypes.byref(h)))
        self._h = h.value
        self.path = Path(path)
        self.version = self._lib.axh_gguf_version(self._h)
        self.alignment = self._lib.axh_gguf_alignment(self._h)
        self.data_offset = self._lib.axh_gguf_data_offset(self._h)
        self.tensors: dict[str, TensorInfo] = {}
        self._index: dict[str, int] = {}
        info = _axh._GgufTensorInfo()
        for i in range(self._lib.axh_gguf_tensor_count(self._h)):
            _axh._check(self._lib.axh_gguf_tensor_at(self._h, i, ctypes.byref(info)))
            name = info.name.decode("utf-8", errors="replace")
            self.tensors[name] = TensorInfo(name, info.type, tuple(info.ne[: info.n_dims]),
                                            info.offset, info.nbytes)
            self._index[name] = i
        self.metadata: dict[str, Any] = {}
        self.metadata_types: dict[str, int] = {}
        kv = _axh._GgufKvInfo()
        for i in range(self._lib.axh_gguf_kv_count(self._h)):
            _axh._check(self._lib.axh_gguf_kv_at(self._h, i, ctypes.byref(kv)))
            key = kv.key.decode("utf-8", errors="replace")
            self.metadata[key] = _decode_value(kv.type, kv.item_type, kv.count, kv.value)
            self.metadata_types[key] = kv.type

    def tensor_bytes(self, name: str) -> bytes:
        t = self.tensors[name]
        p = self._lib.axh_gguf_tensor_data(self._h, self._index[name])
        return ctypes.string_at(p, t.nbytes)

    def upload(self, ctx, name: str, dst=None):
        """Copies tensor `name` into device memory (a new DeviceBuffer unless
        `dst` is given) and returns the buffer."""
        t = self.tensors[name]
        buf = dst if dst is not None else ctx.alloc(max(16, t.nbytes))
        cap = buf.nbytes if hasattr(buf, "nbytes") else t.nbytes
        _axh._check(self._lib.axh_gguf_upload_tensor(ctx._raw, self._h, self._index[name],
                                                     _axh._ptr(buf), cap))
        return buf

    def close(self) -> None:
        if self._h:
            self._lib.axh_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- writer -------------------------------------------------------------------
def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(t: int, v: Any, item_t: Optional[int] = None) -> bytes:
    if t in _SCALAR:
        return struct.pack(_SCALAR[t], v)
    if t == STRING:
        return _pack_string(v)
    if t == ARRAY:
        assert item_t is not None
        return struct.pack("<IQ", item_t, len(v)) + b"".join(_pack_value(item_t, e) for e in v)
    raise ValueError(f"unknown GGUF value type {t}")


def write_gguf(path: Union[str, Path], metadata: Iterable[tuple], tensors: Iterable[tuple],
               alignment: int = 32, version: int = 3) -> None:
    """Writes a GGUF file.  metadata: (key, type, value[, item_type]) tuples;
    tensors: (name, ggml_type, shape with ne[0] first, raw bytes).  A
    general.alignment entry, if given, must match `alignment`."""
    meta = list(metadata)
    tens = list(tensors)
    out = bytearray(struct.pack("<IIQQ", 0x46554747, version, len(tens), len(meta)))
    for m in meta:
        key, t, v = m[0], m[1], m[2]
        out += _pack_string(key) + struct.pack("<I", t) + _pack_value(t, v, m[3] if len(m) > 3
                                                                     else None)
    offsets, at = [], 0
    for name, gt, shape, data in tens:
        offsets.append(at)
        at += -(-len(data) // alignment) * alignment
    for (name, gt, shape, data), off in zip(tens, offsets):
        out += _pack_string(name) + struct.pack("<I", len(shape))
        out += b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", gt, off)
    out += b"\0" * (-len(out) % alignment)
    for (name, gt, shape, data), off in zip(tens, offsets):
        out += bytes(data)
        out += b"\0" * (-len(out) % alignment)
    Path(path).write_bytes(bytes(out))
