"""GGUF reader (native, libaxh.so) and writer: CPU tests.

Pinned against tests/golden/tiny_v3.gguf, a file assembled byte by byte
from the published GGUF specification by tests/golden/make_gguf_fixture.py
(independent of the package's writer), with the facts the specification
fixes for it in tiny_v3.json.  Malformed files must fail to open with a
typed error, never crash or read out of bounds.
"""
from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURE = GOLDEN / "tiny_v3.gguf"
FACTS = json.loads((GOLDEN / "tiny_v3.json").read_text())


@pytest.fixture(scope="module")
def gg(axc):
    import importlib

    return importlib.import_module(axc.__name__ + ".gguf")


def test_fixture_header_tensors_and_metadata(gg):
    with gg.GgufFile(FIXTURE) as f:
        assert f.version == FACTS["version"] == 3
        assert f.alignment == FACTS["alignment"] == 64
        assert f.data_offset == FACTS["data_offset"]
        assert list(f.tensors) == [t["name"] for t in FACTS["tensors"]]
        for t in FACTS["tensors"]:
            info = f.tensors[t["name"]]
            assert (info.type, list(info.shape), info.offset, info.nbytes) == (
                t["type"], t["shape"], t["offset"], t["nbytes"])
            assert hashlib.sha256(f.tensor_bytes(t["name"])).hexdigest() == t["sha256"]
        raw = FIXTURE.read_bytes()
        t0 = FACTS["tensors"][0]
        assert f.tensor_bytes(t0["name"]) == raw[t0["offset"]:t0["offset"] + t0["nbytes"]]
        assert set(f.metadata) == set(FACTS["metadata"])
        for key, (typ, val) in FACTS["metadata"].items():
            assert f.metadata_types[key] == typ, key
            assert f.metadata[key] == val, key
        down = f.tensors["blk.0.ffn_down.weight"]
        assert (down.n_rows, down.n_cols) == (3, 512)


def test_ggml_type_sizes(axc):
    table = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
             8: (32, 34), 9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144),
             13: (256, 176), 14: (256, 210), 15: (256, 292), 30: (1, 2)}
    for t, want in table.items():
        assert axc.axh.ggml_type_size(t) == want, t
    with pytest.raises(axc.DispatchError):
        axc.axh.ggml_type_size(19)  # IQ1_S: not sized by this reader


def test_writer_round_trip(gg, tmp_path):
    q = np.random.default_rng(3).integers(0, 256, 2 * 144, dtype=np.uint8).tobytes()
    meta = [("general.architecture", gg.STRING, "llama"),
            ("a.list", gg.ARRAY, ["x", "yz", ""], gg.STRING),
            ("a.f32s", gg.ARRAY, [0.5, -1.0], gg.F32),
            ("a.u64", gg.U64, 2 ** 50), ("a.bool", gg.BOOL, False)]
    tens = [("w", gg.GGML_Q4_K, (256, 2), q), ("e", gg.GGML_F32, (3,), b"\0" * 12)]
    for align, version in ((32, 3), (256, 2)):
        p = tmp_path / f"w{align}.gguf"
        m = meta + ([("general.alignment", gg.U32, align)] if align != 32 else [])
        gg.write_gguf(p, m, tens, alignment=align, version=version)
        with gg.GgufFile(p) as f:
            assert f.version == version and f.alignment == align
            assert f.metadata["a.list"] == ["x", "yz", ""] and f.metadata["a.u64"] == 2 ** 50
            assert f.metadata["a.f32s"] == [0.5, -1.0] and f.metadata["a.bool"] is False
            assert f.tensor_bytes("w") == q and f.tensors["w"].shape == (256, 2)
            assert all(t.offset % align == 0 for t in f.tensors.values())


def _expect_open_error(gg, axc, path):
    with pytest.raises(axc.DispatchError) as e:
        gg.GgufFile(path)
    return e.value


def test_every_truncation_fails_cleanly(gg, axc, tmp_path):
    raw = FIXTURE.read_bytes()
    end = max(t["offset"] + t["nbytes"] for t in FACTS["tensors"])
    p = tmp_path / "cut.gguf"
    for n in list(range(0, FACTS["data_offset"] + 8)) + list(range(FACTS["data_offset"], end, 37)) \
            + [end - 1]:
        p.write_bytes(raw[:n])
        _expect_open_error(gg, axc, p)
    p.write_bytes(raw[:end])  # trailing padding of the last tensor is optional
    with gg.GgufFile(p) as f:
        assert len(f.tensors) == len(FACTS["tensors"])


def _header(n_tensors, n_kv, version=3):
    return struct.pack("<4sIQQ", b"GGUF", version, n_tensors, n_kv)


def _s(x: str) -> bytes:
    return struct.pack("<Q", len(x)) + x.encode()


def _tensor(name, ne, t, off):
    return _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne) + \
        struct.pack("<IQ", t, off)


def _file(head: bytes, data: bytes = b"", align: int = 32) -> bytes:
    return head + b"\0" * (-len(head) % align) + data


@pytest.mark.parametrize("case", [
    "magic", "v1", "v4", "dims0", "dims5", "misaligned", "partial_block", "dup_tensor",
    "dup_key", "align_not_pow2", "align_wrong_type", "huge_string", "huge_counts",
    "bad_value_type", "past_end", "zero_dim", "f32_size_wraps", "f64_size_wraps",
])
def test_malformed_files_are_typed_errors(gg, axc, tmp_path, case):
    q = b"\1" * 144
    ok_t = _tensor("w", (256,), 12, 0)
    blobs = {
        "magic": b"GGUX" + _header(1, 0)[4:] + ok_t,
        "v1": _header(1, 0, version=1) + ok_t,
        "v4": _header(1, 0, version=4) + ok_t,
        "dims0": _header(1, 0) + _s("w") + struct.pack("<IIQ", 0, 12, 0),
        "dims5": _header(1, 0) + _tensor("w", (256, 1, 1, 1, 1), 12, 0),
        "misaligned": _header(1, 0) + _tensor("w", (256,), 12, 16),
        "partial_block": _header(1, 0) + _tensor("w", (100,), 12, 0),
        "dup_tensor": _header(2, 0) + ok_t + _tensor("w", (256,), 12, 160),
        "dup_key": _header(0, 2) + (_s("k") + struct.pack("<IB", 0, 1)) * 2,
        "align_not_pow2": _header(0, 1) + _s("general.alignment") + struct.pack("<II", 4, 48),
        "align_wrong_type": _header(0, 1) + _s("general.alignment") + struct.pack("<IQ", 10, 64),
        "huge_string": _header(0, 1) + struct.pack("<Q", 2 ** 62) + b"k",
        "huge_counts": _header(2 ** 40, 2 ** 40),
        "bad_value_type": _header(0, 1) + _s("k") + struct.pack("<II", 13, 0),
        "past_end": _header(1, 0) + _tensor("w", (512,), 12, 0),
        "zero_dim": _header(1, 0) + _tensor("w", (256, 0), 12, 0),
        # element count * element bytes wraps in 64 bits (to 0 and to 8 bytes)
        "f32_size_wraps": _header(1, 0) + _tensor("w", (2 ** 62,), 0, 0),
        "f64_size_wraps": _header(1, 0) + _tensor("w", (2 ** 61 + 1,), 28, 0),
    }
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(_file(blobs[case], q))
    err = _expect_open_error(gg, axc, p)
    assert err.variant in ("MetadataParseError", "MetadataSchemaMismatch"), err


def test_missing_file_is_io_error(gg, axc, tmp_path):
    err = _expect_open_error(gg, axc, tmp_path / "absent.gguf")
    assert err.variant == "MetadataIoError"
