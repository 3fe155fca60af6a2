"""Writes tests/golden/tiny_v3.gguf and tiny_v3.json: a small GGUF v3 file
assembled byte by byte from the published GGUF specification (ggml
docs/gguf.md), and the facts the specification fixes for it (header fields,
aligned data-section start, each tensor's absolute offset and size, every
metadata value).  Independent of the package's writer and reader.

Tensor payloads are deterministic (numpy PCG64, seed 20240611) with valid
f16 block scales, so matvec tests can use them directly.

Run:  python tests/golden/make_gguf_fixture.py
"""
from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ALIGN = 64  # general.alignment (not the default 32, so the key is honoured)

rng = np.random.default_rng(20240611)


def f16le(v: float) -> bytes:
    return np.array([v], dtype="<f2").tobytes()


def q4k_blocks(n: int) -> bytes:  # 144 B: d, dmin, scales[12], qs[128]
    out = b""
    for _ in range(n):
        out += f16le(rng.uniform(0.001, 0.05)) + f16le(rng.uniform(0, 0.02))
        out += rng.integers(0, 256, 140, dtype=np.uint8).tobytes()
    return out


def q5k_blocks(n: int) -> bytes:  # 176 B: d, dmin, scales[12], qh[32], qs[128]
    out = b""
    for _ in range(n):
        out += f16le(rng.uniform(0.001, 0.05)) + f16le(rng.uniform(0, 0.02))
        out += rng.integers(0, 256, 172, dtype=np.uint8).tobytes()
    return out


def q6k_blocks(n: int) -> bytes:  # 210 B: ql[128], qh[64], scales[16], d
    out = b""
    for _ in range(n):
        out += rng.integers(0, 256, 208, dtype=np.uint8).tobytes() + f16le(rng.uniform(1e-4, 2e-3))
    return out


def gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


# (key, type id, packed value, expected JSON value)
META = [
    ("general.architecture", 8, gstr("llama"), "llama"),
    ("general.alignment", 4, struct.pack("<I", ALIGN), ALIGN),
    ("test.u8", 0, struct.pack("<B", 200), 200),
    ("test.i8", 1, struct.pack("<b", -7), -7),
    ("test.u16", 2, struct.pack("<H", 65535), 65535),
    ("test.i16", 3, struct.pack("<h", -32768), -32768),
    ("test.i32", 5, struct.pack("<i", -123456), -123456),
    ("test.f32", 6, struct.pack("<f", 0.5), 0.5),
    ("test.bool", 7, struct.pack("<?", True), True),
    ("test.u64", 10, struct.pack("<Q", 2 ** 63 + 5), 2 ** 63 + 5),
    ("test.i64", 11, struct.pack("<q", -(2 ** 40)), -(2 ** 40)),
    ("test.f64", 12, struct.pack("<d", -2.25), -2.25),
    ("llama.context_length", 4, struct.pack("<I", 8192), 8192),
    ("tokenizer.ggml.tokens", 9, struct.pack("<IQ", 8, 3) + gstr("<s>") + gstr("a") + gstr(""),
     ["<s>", "a", ""]),
    ("test.u32_array", 9, struct.pack("<IQ", 4, 3) + struct.pack("<3I", 1, 2, 3), [1, 2, 3]),
]

# (name, ggml type, ne (ne[0] first), payload)
TENSORS = [
    ("blk.0.ffn_down.weight", 12, (512, 3), q4k_blocks(6)),
    ("blk.0.attn_v.weight", 13, (256, 2), q5k_blocks(2)),
    ("output.weight", 14, (512, 5), q6k_blocks(10)),
    ("token_embd.weight", 0, (4, 2), np.arange(8, dtype="<f4").tobytes()),
]


def main() -> None:
    head = struct.pack("<4sIQQ", b"GGUF", 3, len(TENSORS), len(META))
    for key, t, packed, _ in META:
        head += gstr(key) + struct.pack("<I", t) + packed
    rel, at = [], 0
    for _, _, _, data in TENSORS:
        rel.append(at)
        at += (len(data) + ALIGN - 1) // ALIGN * ALIGN
    for (name, t, ne, _), off in zip(TENSORS, rel):
        head += gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", t, off)
    data_off = (len(head) + ALIGN - 1) // ALIGN * ALIGN
    blob = bytearray(head + b"\0" * (data_off - len(head)))
    for (_, _, _, data), off in zip(TENSORS, rel):
        assert len(blob) == data_off + off
        blob += data + b"\0" * ((-len(data)) % ALIGN)
    (HERE / "tiny_v3.gguf").write_bytes(bytes(blob))
    facts = {
        "version": 3,
        "alignment": ALIGN,
        "data_offset": data_off,
        "file_bytes": len(blob),
        "tensors": [
            {"name": n, "type": t, "shape": list(ne), "offset": data_off + off,
             "nbytes": len(d), "sha256": hashlib.sha256(d).hexdigest()}
            for (n, t, ne, d), off in zip(TENSORS, rel)
        ],
        "metadata": {k: [t, v] for k, t, _, v in META},
    }
    (HERE / "tiny_v3.json").write_text(json.dumps(facts, indent=1) + "\n")


if __name__ == "__main__":
    main()
