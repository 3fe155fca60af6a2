"""Python mirror of the reference runtime surface over the axh C ABI.

Names follow crates/axc-runtime of rudybear/axiom-compute:
  VulkanContext::new / new_with_options  -> HipContext.new / new_with_options
  VulkanContextOptions                   -> HipContextOptions
  prepare_kernel -> KernelHandle         -> HipContext.prepare_kernel
  dispatch_handle                        -> HipContext.dispatch_handle
  dispatch(DispatchRequest)              -> HipContext.dispatch
  DispatchError (25 variants)            -> DispatchError with .variant
The Q4 hot path (resident device buffers, asynchronous launches) is exposed as
HipContext.q4k_matvec / q4_0_matvec / q4k_dequant / q4_0_dequant.

The product path is the HIP library libaxh.so next to this file: importing
this module fails loudly when it has not been built; there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from pathlib import Path
from typing import Iterable, Optional, Sequence

_HERE = Path(__file__).resolve().parent
# AXH_LIBRARY selects another build of the library (e.g. the sanitizer build).
LIB_PATH = Path(os.environ["AXH_LIBRARY"]) if os.environ.get("AXH_LIBRARY") else _HERE / "libaxh.so"
HEADER_PATH = _HERE.parent / "include" / "axh.h"

# status code -> reference DispatchError variant name (error.rs:27-195)
VARIANTS = {
    1: "VulkanEntryFailed",
    2: "NoVulkanInstance",
    3: "NoSupportedDevice",
    4: "NoComputeQueue",
    5: "DeviceCreationFailed",
    6: "ShaderModuleCreationFailed",
    7: "DescriptorSetLayoutFailed",
    8: "DescriptorPoolFailed",
    9: "PipelineLayoutFailed",
    10: "PipelineCreationFailed",
    11: "BufferAllocationFailed",
    12: "MemoryMapFailed",
    13: "NoCompatibleMemoryType",
    14: "CommandBufferRecordFailed",
    15: "QueueSubmitFailed",
    16: "FenceTimeout",
    17: "ReadbackFailed",
    18: "BindingCountMismatch",
    19: "PushConstantSizeMismatch",
    20: "WorkgroupCountExceedsDeviceLimit",
    21: "MetadataIoError",
    22: "MetadataParseError",
    23: "MetadataSchemaMismatch",
    24: "PipelineCacheLoadFailed",
    25: "StagingCopyFailed",
    100: "InvalidArgument",
}

ACCESS_READ_ONLY, ACCESS_WRITE_ONLY, ACCESS_READ_WRITE = 0, 1, 2
# Q4_K matvec kernel families (the `family` hole, include/axh.h AXH_Q4K_FAMILY_*).
(FAMILY_DEFAULT, FAMILY_PERSISTENT, FAMILY_ONE_PASS, FAMILY_ONE_PASS_X, FAMILY_WORKGROUP,
 FAMILY_SPLIT_K, FAMILY_COLUMNS, FAMILY_TILED) = range(8)


class DispatchError(RuntimeError):
    """A non-zero axh_status; `.variant` is the reference variant name."""

    def __init__(self, status: int, message: str):
        self.status = int(status)
        self.variant = VARIANTS.get(self.status, "Unknown")
        super().__init__(f"{self.variant}: {message}")


class _Options(ctypes.Structure):
    _fields_ = [
        ("code_object_cache_dir", ctypes.c_char_p),
        ("device_index", ctypes.c_int32),
        ("fence_timeout_ms", ctypes.c_uint64),
    ]


class _Plan(ctypes.Structure):
    _fields_ = [
        ("n_buffers", ctypes.c_uint32),
        ("access", ctypes.POINTER(ctypes.c_uint8)),
        ("push_constant_total_bytes", ctypes.c_uint32),
        ("workgroup_size", ctypes.c_uint32 * 3),
        ("dynamic_lds_bytes", ctypes.c_uint32),
    ]


class _Variant(ctypes.Structure):
    _fields_ = [
        ("rows_per_wave", ctypes.c_uint32),
        ("waves_per_workgroup", ctypes.c_uint32),
        ("prefetch", ctypes.c_uint32),
        ("nontemporal", ctypes.c_uint32),
        ("family", ctypes.c_uint32),
        ("sb_per_lane", ctypes.c_uint32),
    ]


_lib: Optional[ctypes.CDLL] = None


class _MatmulVariant(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_uint32), ("waves_per_workgroup", ctypes.c_uint32),
                ("col_tiles", ctypes.c_uint32), ("prefetch", ctypes.c_uint32),
                ("row_tiles", ctypes.c_uint32)]


class _BenchOp(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_uint32), ("q", ctypes.c_void_p), ("q_stride", ctypes.c_uint64),
        ("n_copies", ctypes.c_uint32), ("q2_offset", ctypes.c_uint64), ("x", ctypes.c_void_p),
        ("x16", ctypes.c_void_p), ("y", ctypes.c_void_p), ("n_rows", ctypes.c_uint32),
        ("units", ctypes.c_uint32), ("batch", ctypes.c_uint32),
        ("variant", ctypes.c_void_p), ("matmul_variant", ctypes.c_void_p),
    ]


BENCH_OPS = {"q4k": 1, "q4_0": 2, "q5k": 3, "q6k": 4, "gate_up": 5, "matmul_f16": 6,
             "matmul_f32": 7, "read_floor": 8, "launch_empty": 9, "read_shape": 10,
             "gate_up_q4_0": 11, "gate_up_q5k": 12}


class _GgufTensorInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_uint32),
                ("ne", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64),
                ("nbytes", ctypes.c_uint64)]


class _GgufKvInfo(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("type", ctypes.c_uint32),
                ("item_type", ctypes.c_uint32), ("count", ctypes.c_uint64),
                ("value", ctypes.c_void_p)]


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load libaxh.so (raises ImportError if it has not been built)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(f"{p} is missing: run __graft_entry__.build() (HIP path not built)")
    lib = ctypes.CDLL(str(p))
    c = ctypes
    vp, sz, u32, u64, st = c.c_void_p, c.c_size_t, c.c_uint32, c.c_uint64, c.c_int
    sigs = {
        "axh_last_error": (c.c_char_p, []),
        "axh_status_name": (c.c_char_p, [c.c_int]),
        "axh_abi_version": (u32, []),
        "axh_context_create": (st, [c.POINTER(_Options), c.POINTER(vp)]),
        "axh_context_destroy": (None, [vp]),
        "axh_context_device_name": (c.c_char_p, [vp]),
        "axh_context_stream": (vp, [vp]),
        "axh_context_max_workgroup_count": (None, [vp, c.POINTER(u32)]),
        "axh_prepare_kernel": (st, [vp, vp, sz, c.POINTER(_Plan), u32, c.c_char_p, c.POINTER(vp)]),
        "axh_kernel_retain": (None, [vp]),
        "axh_kernel_release": (None, [vp]),
        "axh_kernel_cache_key": (u64, [vp]),
        "axh_kernel_pool_bytes": (u64, [vp, u32]),
        "axh_dispatch_handle": (st, [vp, vp, c.POINTER(u32), c.POINTER(vp), c.POINTER(sz), sz,
                                     c.POINTER(sz), sz, c.POINTER(vp), vp, sz]),
        "axh_dispatch": (st, [vp, vp, sz, c.POINTER(_Plan), c.POINTER(u32), c.POINTER(vp),
                              c.POINTER(sz), sz, c.POINTER(sz), sz, c.POINTER(vp), vp, sz,
                              c.c_char_p]),
        "axh_validate_request": (st, [c.POINTER(_Plan), c.POINTER(u32), sz, sz, sz,
                                      c.POINTER(u32)]),
        "axh_buffer_alloc": (st, [vp, sz, c.POINTER(vp)]),
        "axh_buffer_free": (st, [vp, vp]),
        "axh_upload": (st, [vp, vp, vp, sz]),
        "axh_download": (st, [vp, vp, vp, sz]),
        "axh_copy_device": (st, [vp, vp, vp, sz]),
        "axh_launch": (st, [vp, vp, c.POINTER(u32), c.POINTER(vp), sz, vp, sz, vp]),
        "axh_synchronize": (st, [vp, vp]),
        "axh_device_synchronize": (st, [vp]),
        "axh_event_create": (st, [vp, c.POINTER(vp)]),
        "axh_event_record": (st, [vp, vp, vp]),
        "axh_event_synchronize": (st, [vp, vp]),
        "axh_event_elapsed_ms": (st, [vp, vp, c.POINTER(c.c_float)]),
        "axh_event_destroy": (None, [vp]),
        "axh_q4k_matvec": (st, [vp, vp, vp, vp, u32, u32, c.POINTER(_Variant), vp]),
        "axh_q4k_matvec_noalloc": (st, [vp, vp, vp, vp, u32, u32, vp]),
        "axh_capture_begin": (st, [vp]),
        "axh_capture_end": (st, [vp, c.POINTER(vp)]),
        "axh_graph_launch": (st, [vp, vp, vp]),
        "axh_graph_node_count": (u64, [vp]),
        "axh_graph_destroy": (None, [vp]),
        "axh_q4k_matvec_kernel_name": (st, [u32, u32, c.POINTER(_Variant), c.c_char_p, sz]),
        "axh_q4k_matvec_default_variant": (st, [u32, u32, c.POINTER(_Variant)]),
        "axh_q4_0_matvec_kernel_name": (st, [u32, u32, c.POINTER(_Variant), c.c_char_p, sz]),
        "axh_q4k_gate_up": (st, [vp, vp, vp, vp, vp, u32, u32, c.POINTER(_Variant), vp]),
        "axh_q4_0_gate_up": (st, [vp, vp, vp, vp, vp, u32, u32, c.POINTER(_Variant), vp]),
        "axh_q5k_gate_up": (st, [vp, vp, vp, vp, vp, u32, u32, c.POINTER(_Variant), vp]),
        "axh_q5k_matvec": (st, [vp, vp, vp, vp, u32, u32, c.POINTER(_Variant), vp]),
        "axh_q6k_matvec": (st, [vp, vp, vp, vp, u32, u32, c.POINTER(_Variant), vp]),
        "axh_q5k_matvec_kernel_name": (st, [u32, u32, c.POINTER(_Variant), c.c_char_p, sz]),
        "axh_q6k_matvec_kernel_name": (st, [u32, u32, c.POINTER(_Variant), c.c_char_p, sz]),
        "axh_q5k_matvec_variant_count": (u32, []),
        "axh_q5k_matvec_variant_at": (st, [u32, c.POINTER(_Variant)]),
        "axh_q6k_matvec_variant_count": (u32, []),
        "axh_q6k_matvec_variant_at": (st, [u32, c.POINTER(_Variant)]),
        "axh_matvec_ggml": (st, [vp, u32, vp, vp, vp, u32, u64, vp]),
        "axh_q5k_dequant": (st, [vp, vp, vp, u64, vp]),
        "axh_q6k_dequant": (st, [vp, vp, vp, u64, vp]),
        "axh_ggml_type_size": (st, [u32, c.POINTER(u32), c.POINTER(u32)]),
        "axh_gguf_open": (st, [c.c_char_p, c.POINTER(vp)]),
        "axh_gguf_close": (None, [vp]),
        "axh_gguf_version": (u32, [vp]),
        "axh_gguf_alignment": (u32, [vp]),
        "axh_gguf_data_offset": (u64, [vp]),
        "axh_gguf_tensor_count": (u64, [vp]),
        "axh_gguf_kv_count": (u64, [vp]),
        "axh_gguf_tensor_at": (st, [vp, u64, c.POINTER(_GgufTensorInfo)]),
        "axh_gguf_find_tensor": (st, [vp, c.c_char_p, c.POINTER(u64)]),
        "axh_gguf_tensor_data": (vp, [vp, u64]),
        "axh_gguf_upload_tensor": (st, [vp, vp, u64, vp, u64]),
        "axh_gguf_kv_at": (st, [vp, u64, c.POINTER(_GgufKvInfo)]),
        "axh_gguf_find_kv": (st, [vp, c.c_char_p, c.POINTER(u64)]),
        "axh_q4k_gate_up_kernel_name": (st, [u32, u32, c.POINTER(_Variant), c.c_char_p, sz]),
        "axh_q4_0_gate_up_kernel_name": (st, [u32, u32, c.POINTER(_Variant), c.c_char_p, sz]),
        "axh_q5k_gate_up_kernel_name": (st, [u32, u32, c.POINTER(_Variant), c.c_char_p, sz]),
        "axh_q4k_gate_up_variant_count": (u32, []),
        "axh_q4k_gate_up_variant_at": (st, [u32, c.POINTER(_Variant)]),
        "axh_q4k_matmul_f16": (st, [vp, vp, vp, vp, u32, u32, u32, c.POINTER(_MatmulVariant),
                                    vp]),
        "axh_q4k_matmul_f32": (st, [vp, vp, vp, vp, vp, u32, u32, u32,
                                    c.POINTER(_MatmulVariant), vp]),
        "axh_f32_to_f16": (st, [vp, vp, vp, u64, vp]),
        "axh_q4k_matmul_kernel_name": (st, [u32, u32, u32, c.POINTER(_MatmulVariant),
                                            c.c_char_p, sz]),
        "axh_q4k_matmul_variant_count": (u32, []),
        "axh_q4k_matmul_variant_at": (st, [u32, c.POINTER(_MatmulVariant)]),
        "axh_q4_0_matvec": (st, [vp, vp, vp, vp, u32, u32, c.POINTER(_Variant), vp]),
        "axh_q4k_dequant": (st, [vp, vp, vp, u64, vp]),
        "axh_q4_0_dequant": (st, [vp, vp, vp, u64, vp]),
        "axh_f16_widen": (st, [vp, vp, vp, u64, vp]),
        "axh_read_floor": (st, [vp, vp, u64, vp, u32, vp]),
        "axh_launch_empty": (st, [vp, vp, u32, vp]),
        "axh_read_floor_shape": (st, [vp, vp, u64, u32, u32, u32, vp, u32, vp]),
        "axh_cu_count": (u32, [vp]),
        "axh_q4k_matvec_variant_count": (u32, []),
        "axh_q4k_matvec_variant_at": (st, [u32, c.POINTER(_Variant)]),
        "axh_q4_0_matvec_variant_count": (u32, []),
        "axh_q4_0_matvec_variant_at": (st, [u32, c.POINTER(_Variant)]),
        "axh_builtin_code_object": (vp, [c.POINTER(sz)]),
        "axh_bench_loop": (st, [vp, c.POINTER(_BenchOp), u32, u32, u32, c.POINTER(c.c_float)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def _check(status: int) -> None:
    if status != 0:
        msg = load_library().axh_last_error().decode(errors="replace")
        raise DispatchError(status, msg)


def status_name(status: int) -> str:
    return load_library().axh_status_name(status).decode()


def builtin_code_object() -> bytes:
    """The embedded gfx950 code object holding every kernel of the library."""
    lib = load_library()
    n = ctypes.c_size_t()
    p = lib.axh_builtin_code_object(ctypes.byref(n))
    return ctypes.string_at(p, n.value)


@dataclass(frozen=True)
class Variant:
    """Strategy holes of the matvec kernels (0 = default)."""

    rows_per_wave: int = 0
    waves_per_workgroup: int = 0
    prefetch: int = 0
    nontemporal: int = 0
    family: int = 0       # FAMILY_* (Q4_K and Q4_0 matvec); 0 = the shape's choice
    sb_per_lane: int = 0  # one-pass families: superblocks (Q4_0: octets) a lane walks per row

    def _c(self) -> _Variant:
        return _Variant(self.rows_per_wave, self.waves_per_workgroup, self.prefetch,
                        self.nontemporal, self.family, self.sb_per_lane)


def _variant_from_c(v: "_Variant") -> "Variant":
    return Variant(v.rows_per_wave, v.waves_per_workgroup, v.prefetch, v.nontemporal, v.family,
                   v.sb_per_lane)


def q4k_matvec_default_variant(n_rows: int, sb_per_row: int) -> "Variant":
    """The hole assignment axh_q4k_matvec uses for this shape with no variant."""
    v = _Variant()
    _check(load_library().axh_q4k_matvec_default_variant(n_rows, sb_per_row, ctypes.byref(v)))
    return _variant_from_c(v)


def q4k_matvec_kernel_name(n_rows: int, sb_per_row: int,
                           variant: Optional[Variant] = None) -> str:
    """Entry point axh_q4k_matvec launches for this shape and variant."""
    lib = load_library()
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(lib.axh_q4k_matvec_kernel_name(n_rows, sb_per_row, ctypes.byref(v) if v else None,
                                          buf, 64))
    return buf.value.decode()


@dataclass(frozen=True)
class MatmulVariant:
    """Strategy holes of the batched matmul kernels (0 = default).  kind: 3
    K-split, 5 K-split tile, 7 streaming rows (K <= 4096), 8 32x32 tiles, 9
    long rows (kinds 1, 2, 4 and 6 were removed); row_tiles is kinds 3, 5, 8
    and 9's only (kind 9: 16-row tiles per workgroup; its col_tiles counts
    4-column groups).  The default kind follows the grid each kind
    would launch on 256 CUs (q4k_matmul_kernel_name names the choice)."""

    kind: int = 0
    waves_per_workgroup: int = 0
    col_tiles: int = 0
    prefetch: int = 0
    row_tiles: int = 0

    def _c(self) -> _MatmulVariant:
        return _MatmulVariant(self.kind, self.waves_per_workgroup, self.col_tiles, self.prefetch,
                              self.row_tiles)


def compiled_matmul_variants() -> list[MatmulVariant]:
    lib = load_library()
    out = []
    for i in range(lib.axh_q4k_matmul_variant_count()):
        v = _MatmulVariant()
        _check(lib.axh_q4k_matmul_variant_at(i, ctypes.byref(v)))
        out.append(MatmulVariant(v.kind, v.waves_per_workgroup, v.col_tiles, v.prefetch,
                                 v.row_tiles))
    return out


def q4k_matmul_kernel_name(n_rows: int, sb_per_row: int, batch: int,
                           variant: Optional[MatmulVariant] = None) -> str:
    """Entry point axh_q4k_matmul_f16 launches for this shape and variant."""
    lib = load_library()
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(lib.axh_q4k_matmul_kernel_name(n_rows, sb_per_row, batch,
                                          ctypes.byref(v) if v else None, buf, 64))
    return buf.value.decode()


def q4_0_matvec_kernel_name(n_rows: int, blocks_per_row: int,
                            variant: Optional[Variant] = None) -> str:
    """Entry point axh_q4_0_matvec launches for this shape and variant."""
    lib = load_library()
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(lib.axh_q4_0_matvec_kernel_name(n_rows, blocks_per_row,
                                           ctypes.byref(v) if v else None, buf, 64))
    return buf.value.decode()


def q4k_gate_up_kernel_name(n_rows: int, sb_per_row: int,
                            variant: Optional[Variant] = None) -> str:
    """Entry point axh_q4k_gate_up launches for this shape and variant."""
    lib = load_library()
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(lib.axh_q4k_gate_up_kernel_name(n_rows, sb_per_row, ctypes.byref(v) if v else None,
                                           buf, 64))
    return buf.value.decode()


def q4_0_gate_up_kernel_name(n_rows: int, blocks_per_row: int,
                             variant: Optional[Variant] = None) -> str:
    """Entry point axh_q4_0_gate_up launches for this shape and variant."""
    lib = load_library()
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(lib.axh_q4_0_gate_up_kernel_name(n_rows, blocks_per_row,
                                            ctypes.byref(v) if v else None, buf, 64))
    return buf.value.decode()


def q5k_gate_up_kernel_name(n_rows: int, sb_per_row: int,
                            variant: Optional[Variant] = None) -> str:
    """Entry point axh_q5k_gate_up launches for this shape and variant."""
    lib = load_library()
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(lib.axh_q5k_gate_up_kernel_name(n_rows, sb_per_row, ctypes.byref(v) if v else None,
                                           buf, 64))
    return buf.value.decode()


def _kernel_name(fn: str, n_rows: int, units: int, variant: Optional[Variant]) -> str:
    lib = load_library()
    v = variant._c() if variant else None
    buf = ctypes.create_string_buffer(64)
    _check(getattr(lib, fn)(n_rows, units, ctypes.byref(v) if v else None, buf, 64))
    return buf.value.decode()


def q5k_matvec_kernel_name(n_rows: int, sb_per_row: int,
                           variant: Optional[Variant] = None) -> str:
    """Entry point axh_q5k_matvec launches for this shape and variant."""
    return _kernel_name("axh_q5k_matvec_kernel_name", n_rows, sb_per_row, variant)


def q6k_matvec_kernel_name(n_rows: int, sb_per_row: int,
                           variant: Optional[Variant] = None) -> str:
    """Entry point axh_q6k_matvec launches for this shape and variant."""
    return _kernel_name("axh_q6k_matvec_kernel_name", n_rows, sb_per_row, variant)


def ggml_type_size(ggml_type: int) -> tuple[int, int]:
    """(elements, bytes) per block of a ggml type."""
    lib = load_library()
    e, b = ctypes.c_uint32(), ctypes.c_uint32()
    _check(lib.axh_ggml_type_size(ggml_type, ctypes.byref(e), ctypes.byref(b)))
    return e.value, b.value


def compiled_variants(kind: str = "q4k") -> list[Variant]:
    """Compiled hole assignments of the "q4k", "q4_0", "q5k" or "q6k" matvec,
    or of the fused "gate_up" kernel."""
    lib = load_library()
    if kind not in ("q4k", "q4_0", "q5k", "q6k", "gate_up"):
        raise ValueError(f"unknown kernel family {kind!r}")
    count = getattr(lib, f"axh_{kind}_matvec_variant_count" if kind != "gate_up"
                    else "axh_q4k_gate_up_variant_count")
    at = getattr(lib, f"axh_{kind}_matvec_variant_at" if kind != "gate_up"
                 else "axh_q4k_gate_up_variant_at")
    out = []
    for i in range(count()):
        v = _Variant()
        _check(at(i, ctypes.byref(v)))
        out.append(Variant(v.rows_per_wave, v.waves_per_workgroup, v.prefetch, v.nontemporal))
    return out


@dataclass
class BindingPlan:
    """ParamBindingPlan (crates/axc-hir/src/param.rs:119-126) + launch facts."""

    buffers: Sequence[int]  # ACCESS_* per binding, in binding order
    push_constant_total_bytes: int
    workgroup_size: tuple = (64, 1, 1)
    dynamic_lds_bytes: int = 0
    _keep: list = field(default_factory=list, repr=False)

    def _c(self) -> _Plan:
        arr = (ctypes.c_uint8 * max(1, len(self.buffers)))(*self.buffers)
        self._keep = [arr]
        return _Plan(len(self.buffers), ctypes.cast(arr, ctypes.POINTER(ctypes.c_uint8)),
                     self.push_constant_total_bytes,
                     (ctypes.c_uint32 * 3)(*self.workgroup_size), self.dynamic_lds_bytes)


def validate_request(plan: BindingPlan, workgroups, n_inputs: int, n_outputs: int,
                     push_constant_bytes: int, max_workgroup_count=(0xFFFFFFFF,) * 3) -> None:
    """Pure request validation (dispatch.rs:56-95); raises DispatchError."""
    lib = load_library()
    cp = plan._c()
    wg = (ctypes.c_uint32 * 3)(*workgroups)
    mx = (ctypes.c_uint32 * 3)(*max_workgroup_count)
    _check(lib.axh_validate_request(ctypes.byref(cp), wg, n_inputs, n_outputs,
                                    push_constant_bytes, mx))


@dataclass
class HipContextOptions:
    """VulkanContextOptions (context.rs:76-109)."""

    code_object_cache_dir: Optional[str] = None
    physical_device_index: int = -1
    fence_timeout_ms: int = 0


@dataclass
class DispatchRequest:
    """DispatchRequest (dispatch.rs:33-50) with a code object in place of SPIR-V."""

    code_object: bytes
    binding_plan: BindingPlan
    workgroups: tuple
    inputs: Sequence[bytes]
    output_sizes: Sequence[int]
    push_constants: bytes
    entry_point: str


def _ptr(obj) -> int:
    """Device address of a DeviceBuffer, an object with data_ptr() or a raw int."""
    if obj is None:
        return 0
    if isinstance(obj, int):
        return obj
    if hasattr(obj, "ptr"):
        return int(obj.ptr)
    if hasattr(obj, "data_ptr"):
        return int(obj.data_ptr())
    raise TypeError(f"not a device pointer: {type(obj)!r}")


def _stream(s) -> Optional[int]:
    """A hipStream_t of this library's HIP runtime, as an int (None = context stream)."""
    if s is None:
        return None
    if isinstance(s, int):
        return s
    raise TypeError(f"not a stream handle: {type(s)!r}")


class Event:
    """HIP event of the context's runtime (GPU timestamps on a stream)."""

    def __init__(self, ctx: "HipContext"):
        self._ctx = ctx
        raw = ctypes.c_void_p()
        _check(ctx._lib.axh_event_create(ctx._raw, ctypes.byref(raw)))
        self._raw = int(raw.value)

    def record(self, stream=None) -> None:
        _check(self._ctx._lib.axh_event_record(self._ctx._raw, self._raw, _stream(stream)))

    def synchronize(self) -> None:
        _check(self._ctx._lib.axh_event_synchronize(self._ctx._raw, self._raw))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _check(self._ctx._lib.axh_event_elapsed_ms(self._raw, end._raw, ctypes.byref(ms)))
        return float(ms.value)

    def __del__(self):
        try:
            if self._raw:
                self._ctx._lib.axh_event_destroy(self._raw)
                self._raw = 0
        except Exception:
            pass


class Graph:
    """Launches captured on a context stream, replayed with launch()."""

    def __init__(self, ctx: "HipContext", raw: int):
        self._ctx = ctx
        self._raw = raw

    @property
    def node_count(self) -> int:
        return int(self._ctx._lib.axh_graph_node_count(self._raw))

    def launch(self, stream=None) -> None:
        _check(self._ctx._lib.axh_graph_launch(self._ctx._raw, self._raw, _stream(stream)))

    def close(self) -> None:
        if self._raw:
            self._ctx._lib.axh_graph_destroy(self._raw)
            self._raw = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KernelHandle:
    """Reference-counted prepared kernel (KernelHandle, kernel_handle.rs:44-51)."""

    def __init__(self, lib, raw: int):
        self._lib = lib
        self._raw = raw

    @property
    def raw(self) -> int:
        return self._raw

    def clone(self) -> "KernelHandle":
        self._lib.axh_kernel_retain(self._raw)
        return KernelHandle(self._lib, self._raw)

    @property
    def cache_key(self) -> int:
        return int(self._lib.axh_kernel_cache_key(self._raw))

    def pool_bytes(self, binding: int) -> int:
        return int(self._lib.axh_kernel_pool_bytes(self._raw, binding))

    def release(self) -> None:
        if self._raw:
            self._lib.axh_kernel_release(self._raw)
            self._raw = 0

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class DeviceBuffer:
    """Device allocation owned by a context (freed on close/__del__)."""

    def __init__(self, ctx: "HipContext", nbytes: int):
        self._ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _check(ctx._lib.axh_buffer_alloc(ctx._raw, self.nbytes, ctypes.byref(p)))
        self.ptr = int(p.value)

    def close(self) -> None:
        if self.ptr and self._ctx._raw:
            self._ctx._lib.axh_buffer_free(self._ctx._raw, self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipContext:
    """VulkanContext counterpart: one gfx950 device, one stream."""

    def __init__(self, options: Optional[HipContextOptions] = None):
        self._lib = load_library()
        o = options or HipContextOptions()
        co = _Options(o.code_object_cache_dir.encode() if o.code_object_cache_dir else None,
                      o.physical_device_index, o.fence_timeout_ms)
        raw = ctypes.c_void_p()
        _check(self._lib.axh_context_create(ctypes.byref(co), ctypes.byref(raw)))
        self._raw = int(raw.value)

    @classmethod
    def new(cls) -> "HipContext":
        return cls(None)

    @classmethod
    def new_with_options(cls, options: HipContextOptions) -> "HipContext":
        return cls(options)

    @property
    def raw(self) -> int:
        return self._raw

    @property
    def device_name(self) -> str:
        return self._lib.axh_context_device_name(self._raw).decode()

    @property
    def stream(self) -> int:
        return int(self._lib.axh_context_stream(self._raw) or 0)

    @property
    def max_workgroup_count(self) -> tuple:
        out = (ctypes.c_uint32 * 3)()
        self._lib.axh_context_max_workgroup_count(self._raw, out)
        return tuple(out)

    def close(self) -> None:
        if self._raw:
            self._lib.axh_context_destroy(self._raw)
            self._raw = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- kernels -----------------------------------------------------------
    def prepare_kernel(self, code_object: bytes, plan: BindingPlan, push_constant_bytes: int,
                       entry: str) -> KernelHandle:
        cp = plan._c()
        buf = ctypes.create_string_buffer(bytes(code_object), len(code_object))
        raw = ctypes.c_void_p()
        _check(self._lib.axh_prepare_kernel(self._raw, buf, len(code_object), ctypes.byref(cp),
                                            push_constant_bytes, entry.encode(),
                                            ctypes.byref(raw)))
        return KernelHandle(self._lib, int(raw.value))

    def dispatch_handle(self, handle: KernelHandle, workgroups, inputs: Sequence[bytes],
                        output_sizes: Sequence[int], push_constants: bytes) -> list:
        n_in, n_out = len(inputs), len(output_sizes)
        in_bufs = [bytes(b) for b in inputs]
        in_ptrs = (ctypes.c_void_p * max(1, n_in))(
            *[ctypes.cast(ctypes.c_char_p(b), ctypes.c_void_p) if b else None for b in in_bufs])
        in_sz = (ctypes.c_size_t * max(1, n_in))(*[len(b) for b in in_bufs])
        outs = [ctypes.create_string_buffer(max(1, int(s))) for s in output_sizes]
        out_ptrs = (ctypes.c_void_p * max(1, n_out))(*[ctypes.addressof(o) for o in outs])
        out_sz = (ctypes.c_size_t * max(1, n_out))(*[int(s) for s in output_sizes])
        pc = bytes(push_constants)
        pcb = ctypes.create_string_buffer(pc, max(1, len(pc)))
        wg = (ctypes.c_uint32 * 3)(*workgroups)
        _check(self._lib.axh_dispatch_handle(self._raw, handle.raw, wg, in_ptrs, in_sz, n_in,
                                             out_sz, n_out, out_ptrs, pcb, len(pc)))
        return [o.raw[: int(s)] for o, s in zip(outs, output_sizes)]

    def dispatch(self, req: DispatchRequest) -> list:
        validate_request(req.binding_plan, req.workgroups, len(req.inputs),
                         len(req.output_sizes), len(req.push_constants),
                         self.max_workgroup_count)
        h = self.prepare_kernel(req.code_object, req.binding_plan,
                                req.binding_plan.push_constant_total_bytes, req.entry_point)
        try:
            return self.dispatch_handle(h, req.workgroups, req.inputs, req.output_sizes,
                                        req.push_constants)
        finally:
            h.release()

    def launch(self, handle: KernelHandle, workgroups, buffers: Iterable, push_constants: bytes,
               stream=None) -> None:
        ptrs = [_ptr(b) for b in buffers]
        arr = (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)
        pc = bytes(push_constants)
        pcb = ctypes.create_string_buffer(pc, max(1, len(pc)))
        wg = (ctypes.c_uint32 * 3)(*workgroups)
        _check(self._lib.axh_launch(self._raw, handle.raw, wg, arr, len(ptrs), pcb, len(pc),
                                    _stream(stream)))

    # ---- resident buffers --------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def upload(self, dst, data) -> None:
        mv = memoryview(data).cast("B")
        buf = (ctypes.c_char * len(mv)).from_buffer_copy(mv) if mv.readonly else (
            ctypes.c_char * len(mv)).from_buffer(mv)
        _check(self._lib.axh_upload(self._raw, _ptr(dst), buf, len(mv)))

    def download(self, src, nbytes: int) -> bytes:
        out = ctypes.create_string_buffer(max(1, nbytes))
        _check(self._lib.axh_download(self._raw, out, _ptr(src), nbytes))
        return out.raw[:nbytes]

    def copy_device(self, dst, src, nbytes: int) -> None:
        _check(self._lib.axh_copy_device(self._raw, _ptr(dst), _ptr(src), nbytes))

    def synchronize(self, stream=None) -> None:
        _check(self._lib.axh_synchronize(self._raw, _stream(stream)))

    def device_synchronize(self) -> None:
        _check(self._lib.axh_device_synchronize(self._raw))

    def event(self) -> "Event":
        return Event(self)

    def capture(self, fn) -> "Graph":
        """Runs fn() with the context stream in capture mode and returns the
        graph of the launches it issued."""
        _check(self._lib.axh_capture_begin(self._raw))
        g = ctypes.c_void_p()
        try:
            fn()
        except BaseException:
            if self._lib.axh_capture_end(self._raw, ctypes.byref(g)) == 0 and g.value:
                self._lib.axh_graph_destroy(g)
            raise
        _check(self._lib.axh_capture_end(self._raw, ctypes.byref(g)))
        return Graph(self, int(g.value))

    # ---- Q4 operations -----------------------------------------------------
    def q4k_matvec(self, q, x, y, n_rows: int, sb_per_row: int,
                   variant: Optional[Variant] = None, stream=None) -> None:
        v = variant._c() if variant else None
        _check(self._lib.axh_q4k_matvec(self._raw, _ptr(q), _ptr(x), _ptr(y), n_rows, sb_per_row,
                                        ctypes.byref(v) if v else None, _stream(stream)))

    def q4k_matvec_noalloc(self, q, x, y, n_rows: int, sb_per_row: int, stream=None) -> None:
        """Allocation-free matvec (1-32 rows of 1-256 superblocks, per-device scratch)."""
        _check(self._lib.axh_q4k_matvec_noalloc(self._raw, _ptr(q), _ptr(x), _ptr(y), n_rows,
                                                sb_per_row, _stream(stream)))

    def q4k_gate_up(self, q_gate, q_up, x, h, n_rows: int, sb_per_row: int,
                    variant: Optional[Variant] = None, stream=None) -> None:
        """h[r] = silu(q_gate[r] . x) * (q_up[r] . x), silu(g) = g / (1 + exp(-g))."""
        v = variant._c() if variant else None
        _check(self._lib.axh_q4k_gate_up(self._raw, _ptr(q_gate), _ptr(q_up), _ptr(x), _ptr(h),
                                         n_rows, sb_per_row, ctypes.byref(v) if v else None,
                                         _stream(stream)))

    def q4_0_gate_up(self, q_gate, q_up, x, h, n_rows: int, blocks_per_row: int,
                     variant: Optional[Variant] = None, stream=None) -> None:
        """The same fusion over two Q4_0 matrices of blocks_per_row blocks a row."""
        v = variant._c() if variant else None
        _check(self._lib.axh_q4_0_gate_up(self._raw, _ptr(q_gate), _ptr(q_up), _ptr(x), _ptr(h),
                                          n_rows, blocks_per_row, ctypes.byref(v) if v else None,
                                          _stream(stream)))

    def q5k_gate_up(self, q_gate, q_up, x, h, n_rows: int, sb_per_row: int,
                    variant: Optional[Variant] = None, stream=None) -> None:
        """The same fusion over two Q5_K matrices (the one-pass kernels)."""
        v = variant._c() if variant else None
        _check(self._lib.axh_q5k_gate_up(self._raw, _ptr(q_gate), _ptr(q_up), _ptr(x), _ptr(h),
                                         n_rows, sb_per_row, ctypes.byref(v) if v else None,
                                         _stream(stream)))

    def q5k_matvec(self, q, x, y, n_rows: int, sb_per_row: int,
                   variant: Optional[Variant] = None, stream=None) -> None:
        v = variant._c() if variant else None
        _check(self._lib.axh_q5k_matvec(self._raw, _ptr(q), _ptr(x), _ptr(y), n_rows, sb_per_row,
                                        ctypes.byref(v) if v else None, _stream(stream)))

    def q6k_matvec(self, q, x, y, n_rows: int, sb_per_row: int,
                   variant: Optional[Variant] = None, stream=None) -> None:
        v = variant._c() if variant else None
        _check(self._lib.axh_q6k_matvec(self._raw, _ptr(q), _ptr(x), _ptr(y), n_rows, sb_per_row,
                                        ctypes.byref(v) if v else None, _stream(stream)))

    def matvec_ggml(self, ggml_type: int, q, x, y, n_rows: int, n_cols: int,
                    stream=None) -> None:
        """y = W x for a row-major ggml tensor (Q4_0, Q4_K, Q5_K, Q6_K)."""
        _check(self._lib.axh_matvec_ggml(self._raw, ggml_type, _ptr(q), _ptr(x), _ptr(y), n_rows,
                                         n_cols, _stream(stream)))

    def q5k_dequant(self, q, w, n_superblocks: int, stream=None) -> None:
        _check(self._lib.axh_q5k_dequant(self._raw, _ptr(q), _ptr(w), n_superblocks,
                                         _stream(stream)))

    def q6k_dequant(self, q, w, n_superblocks: int, stream=None) -> None:
        _check(self._lib.axh_q6k_dequant(self._raw, _ptr(q), _ptr(w), n_superblocks,
                                         _stream(stream)))

    def q4_0_matvec(self, q, x, y, n_rows: int, blocks_per_row: int,
                    variant: Optional[Variant] = None, stream=None) -> None:
        v = variant._c() if variant else None
        _check(self._lib.axh_q4_0_matvec(self._raw, _ptr(q), _ptr(x), _ptr(y), n_rows,
                                         blocks_per_row, ctypes.byref(v) if v else None,
                                         _stream(stream)))

    def q4k_matmul(self, q, x, y, n_rows: int, sb_per_row: int, batch: int,
                   variant: Optional[MatmulVariant] = None, stream=None) -> None:
        """y (batch x n_rows f32) = RN_f16(W) x (batch x K f16 vectors)."""
        v = variant._c() if variant else None
        _check(self._lib.axh_q4k_matmul_f16(self._raw, _ptr(q), _ptr(x), _ptr(y), n_rows,
                                            sb_per_row, batch, ctypes.byref(v) if v else None,
                                            _stream(stream)))

    def q4k_matmul_f32(self, q, x, x16, y, n_rows: int, sb_per_row: int, batch: int,
                       variant: Optional[MatmulVariant] = None, stream=None) -> None:
        """As q4k_matmul for f32 activations: x is rounded to f16 (RN) into
        x16 (batch * K * 2 bytes), then the f16 matmul runs on x16."""
        v = variant._c() if variant else None
        _check(self._lib.axh_q4k_matmul_f32(self._raw, _ptr(q), _ptr(x), _ptr(x16), _ptr(y),
                                            n_rows, sb_per_row, batch,
                                            ctypes.byref(v) if v else None, _stream(stream)))

    def f32_to_f16(self, x, h, n: int, stream=None) -> None:
        """h = RN_f16(x) for n values."""
        _check(self._lib.axh_f32_to_f16(self._raw, _ptr(x), _ptr(h), n, _stream(stream)))

    def q4k_dequant(self, q, w, n_superblocks: int, stream=None) -> None:
        _check(self._lib.axh_q4k_dequant(self._raw, _ptr(q), _ptr(w), n_superblocks,
                                         _stream(stream)))

    def q4_0_dequant(self, q, w, n_blocks: int, stream=None) -> None:
        _check(self._lib.axh_q4_0_dequant(self._raw, _ptr(q), _ptr(w), n_blocks, _stream(stream)))

    def f16_widen(self, h, f, n: int, stream=None) -> None:
        _check(self._lib.axh_f16_widen(self._raw, _ptr(h), _ptr(f), n, _stream(stream)))

    def cu_count(self) -> int:
        return int(self._lib.axh_cu_count(self._raw))

    def read_floor(self, q, nbytes: int, out, out_words: int, stream=None) -> None:
        """Stream nbytes of q with the matvec's launch shape (measurement helper)."""
        _check(self._lib.axh_read_floor(self._raw, _ptr(q), nbytes, _ptr(out), out_words,
                                        _stream(stream)))

    def bench_loop(self, op: str, q, q_stride: int, n_copies: int, x, y, n_rows: int = 0,
                   units: int = 0, batch: int = 0, variant=None, q2_offset: int = 0, x16=None,
                   warmup: int = 20, groups: int = 10, calls_per_group: int = 20) -> list:
        """Times `groups` x `calls_per_group` back-to-back calls of one operation
        launched from the library's own loop (axh_bench_loop); returns the
        per-group times in ms."""
        v = variant._c() if variant is not None else None
        o = _BenchOp(BENCH_OPS[op], _ptr(q), q_stride, n_copies, q2_offset, _ptr(x),
                     _ptr(x16) if x16 is not None else None, _ptr(y), n_rows, units, batch,
                     None, None)
        if v is not None:
            if isinstance(variant, MatmulVariant):
                o.matmul_variant = ctypes.cast(ctypes.byref(v), ctypes.c_void_p)
            else:
                o.variant = ctypes.cast(ctypes.byref(v), ctypes.c_void_p)
        out = (ctypes.c_float * groups)()
        _check(self._lib.axh_bench_loop(self._raw, ctypes.byref(o), warmup, groups,
                                        calls_per_group, out))
        return [float(t) for t in out]

    def read_floor_shape(self, q, nbytes: int, threads: int, loads: int, grid: int, out,
                         out_words: int, stream=None) -> None:
        """The read floor at another launch shape (measurement helper)."""
        _check(self._lib.axh_read_floor_shape(self._raw, _ptr(q), nbytes, threads, loads, grid,
                                              _ptr(out), out_words, _stream(stream)))

    def launch_empty(self, out, out_words: int, stream=None) -> None:
        """An empty kernel with the matvec's launch shape (measurement helper)."""
        _check(self._lib.axh_launch_empty(self._raw, _ptr(out), out_words, _stream(stream)))


def header_functions(header: Path = HEADER_PATH) -> list[str]:
    """Names of every function declared in include/axh.h."""
    import re

    text = header.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(axh_[a-z0-9_]+)\s*\(", text)))
