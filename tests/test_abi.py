"""C-ABI checks that need no GPU: the library loads, exports every function
the headers declare, and validates requests before touching a device
(reference: crates/axc-runtime/src/dispatch.rs:56-95 and its unit tests at
dispatch.rs:193,217; crates/axc-runtime/tests/dispatch_error_paths.rs)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _header_functions(path: Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(axh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function(axc):
    lib = axc.load_library()
    names = []
    for h in sorted((ROOT / "include").glob("*.h")):
        names += _header_functions(h)
    assert len(names) > 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_status_names_mirror_reference_dispatch_error_variants(axc):
    expected = [
        "VulkanEntryFailed", "NoVulkanInstance", "NoSupportedDevice", "NoComputeQueue",
        "DeviceCreationFailed", "ShaderModuleCreationFailed", "DescriptorSetLayoutFailed",
        "DescriptorPoolFailed", "PipelineLayoutFailed", "PipelineCreationFailed",
        "BufferAllocationFailed", "MemoryMapFailed", "NoCompatibleMemoryType",
        "CommandBufferRecordFailed", "QueueSubmitFailed", "FenceTimeout", "ReadbackFailed",
        "BindingCountMismatch", "PushConstantSizeMismatch", "WorkgroupCountExceedsDeviceLimit",
        "MetadataIoError", "MetadataParseError", "MetadataSchemaMismatch",
        "PipelineCacheLoadFailed", "StagingCopyFailed",
    ]  # error.rs:27-195, in order
    assert [axc.axh.status_name(i) for i in range(1, 26)] == expected
    assert axc.axh.status_name(0) == "Ok"
    assert [axc.axh.VARIANTS[i] for i in range(1, 26)] == expected


def _plan(axc, n=3, pc=4):
    return axc.BindingPlan([axc.axh.ACCESS_READ_ONLY] * (n - 1) + [axc.axh.ACCESS_READ_WRITE],
                           pc, (64, 1, 1))


def test_validate_accepts_matching_request(axc):
    axc.validate_request(_plan(axc), (1, 1, 1), 3, 3, 4, (65535, 65535, 65535))


def test_validate_binding_count_mismatch_inputs(axc):
    with pytest.raises(axc.DispatchError) as e:
        axc.validate_request(_plan(axc), (1, 1, 1), 2, 3, 4)
    assert e.value.variant == "BindingCountMismatch"
    assert "expected 3, got 2" in str(e.value)


def test_validate_binding_count_mismatch_outputs(axc):
    with pytest.raises(axc.DispatchError) as e:
        axc.validate_request(_plan(axc), (1, 1, 1), 3, 4, 4)
    assert e.value.variant == "BindingCountMismatch"
    assert "expected 3, got 4" in str(e.value)


def test_validate_push_constant_size_mismatch(axc):
    with pytest.raises(axc.DispatchError) as e:
        axc.validate_request(_plan(axc, pc=4), (1, 1, 1), 3, 3, 8)
    assert e.value.variant == "PushConstantSizeMismatch"
    assert "expected 4 bytes, got 8" in str(e.value)


def test_validate_workgroup_count_exceeds_limit(axc):
    with pytest.raises(axc.DispatchError) as e:
        axc.validate_request(_plan(axc), (70000, 1, 1), 3, 3, 4, (65535, 65535, 65535))
    assert e.value.variant == "WorkgroupCountExceedsDeviceLimit"


def test_validation_order_binding_before_push_constants(axc):
    """Both wrong: the binding count is reported first (dispatch.rs:60-83)."""
    with pytest.raises(axc.DispatchError) as e:
        axc.validate_request(_plan(axc), (1, 1, 1), 1, 3, 99)
    assert e.value.variant == "BindingCountMismatch"


def test_builtin_code_object_holds_every_variant_kernel(axc):
    co = axc.builtin_code_object()
    assert co[:4] == b"\x7fELF"
    variants = axc.compiled_variants("q4k")
    assert len(set(variants)) == len(variants)  # one entry per hole assignment
    for v in variants:
        name = (f"axh_q4k_matvec_flat_r{v.rows_per_wave}_w{v.waves_per_workgroup}"
                f"_p{v.prefetch}_n{1 if v.nontemporal == 1 else 0}")
        assert name.encode() in co or (name + "_x2").encode() in co, name
    for v in axc.compiled_variants("q4_0"):
        name = f"axh_q4_0_matvec_r{v.rows_per_wave}_w{v.waves_per_workgroup}"
        assert name.encode() in co, name
    for nit in range(1, 17):  # one-pass kernels for rows of 1..128 superblocks
        assert f"axh_q4k_matvec_one_i{nit}".encode() in co
        assert f"axh_q4k_matvec_onex_i{nit}".encode() in co
        if nit >= 3:  # x two chunks ahead
            assert f"axh_q4k_matvec_onep_i{nit}".encode() in co
    for name in ("q4km_dequant_matvec", "q4_0_dequant_matvec", "axh_q4k_dequant",
                 "axh_q4_0_dequant", "axh_f16_widen", "axh_q4k_matvec_tiled_r2_w8_p2",
                 "axh_q4k_matvec_tiled_r1_w4_p2"):
        assert name.encode() in co, name


def test_kernel_selection_by_shape_and_variant(axc):
    """The entry point axh_q4k_matvec launches (no device work): persistent
    kernel while a row's x fits one workgroup's LDS, tiled kernel beyond."""
    name = axc.q4k_matvec_kernel_name
    # 32..32768 rows: one pass, one pair of rows per wave, a workgroup per 16 rows;
    # x two chunks ahead from four steps up to one workgroup per CU (4096 rows)
    assert name(4096, 56) == "axh_q4k_matvec_onep_i7"
    assert name(2048, 33) == "axh_q4k_matvec_onep_i5"
    assert name(4096, 128) == "axh_q4k_matvec_onep_i16"
    # up to 1024 rows of 24+ superblocks (17+ from 513 rows, 13+ up to 512
    # rows): the tiled kernel, one row per wave
    assert name(32, 33) == "axh_q4k_matvec_tiled_r1_w4_p2"
    assert name(1024, 24) == name(1024, 17) == "axh_q4k_matvec_tiled_r1_w4_p2"
    assert name(512, 13) == name(32, 13) == "axh_q4k_matvec_tiled_r1_w4_p2"
    assert name(1024, 16) == name(513, 16) == "axh_q4k_matvec_one_i2"
    assert name(512, 12) == "axh_q4k_matvec_one_i2"
    assert name(1025, 23) == "axh_q4k_matvec_one_i3"
    # 24576-32768 rows of 25-32 superblocks: the persistent kernel, 4 waves
    assert name(24576, 25) == name(32768, 32) == "axh_q4k_matvec_flat_r1_w4_p1_n0"
    assert name(24575, 32) == "axh_q4k_matvec_onex_i4"
    assert name(28672, 24) == "axh_q4k_matvec_onex_i3"
    assert name(32769, 32) == "axh_q4k_matvec_flat_r2_w4_p1_n0"
    assert name(1025, 24) == "axh_q4k_matvec_one_i3"
    assert name(4097, 56) == "axh_q4k_matvec_one_i7"
    assert name(4096, 32) == "axh_q4k_matvec_onep_i4"
    assert name(4096, 24) == "axh_q4k_matvec_one_i3"
    assert name(4096, 16) == "axh_q4k_matvec_one_i2"
    # 4097-6143 rows: x staged whole up to 24 superblocks, the persistent kernel
    # with one row per lane group for 25-32, one pass again beyond
    assert name(4097, 24) == "axh_q4k_matvec_onex_i3"
    assert name(6143, 16) == "axh_q4k_matvec_onex_i2"
    assert name(5120, 8) == "axh_q4k_matvec_onex_i1"
    assert name(4097, 25) == "axh_q4k_matvec_flat_r1_w4_p1_n0"
    assert name(6143, 32) == "axh_q4k_matvec_flat_r1_w4_p1_n0"
    assert name(5120, 33) == "axh_q4k_matvec_one_i5"
    # 4097-8191 rows of 74+ superblocks (one one-pass workgroup per CU): persistent
    assert name(4097, 74) == "axh_q4k_matvec_flat_r1_w16_p2_n0"
    assert name(8191, 128) == "axh_q4k_matvec_flat_r1_w16_p2_n0"
    assert name(5000, 73) == "axh_q4k_matvec_one_i10"
    assert name(8192, 112) == "axh_q4k_matvec_one_i14"
    # from 6144 rows of at most 32 superblocks: x staged whole behind one barrier
    assert name(32768, 1) == "axh_q4k_matvec_onex_i1"
    assert name(6144, 16) == "axh_q4k_matvec_onex_i2"
    assert name(14336, 16) == "axh_q4k_matvec_onex_i2"
    assert name(14336, 32) == "axh_q4k_matvec_onex_i4"
    assert name(14336, 33) == "axh_q4k_matvec_one_i5"
    assert name(8192, 56) == "axh_q4k_matvec_one_i7"
    # taller matrices: the persistent kernels
    assert name(32769, 16) == "axh_q4k_matvec_onex_i2"  # whole-x one pass up to 65536 rows
    assert name(65536, 16) == "axh_q4k_matvec_onex_i2"
    assert name(40000, 17).startswith("axh_q4k_matvec_flat_")
    assert name(40000, 33).startswith("axh_q4k_matvec_flat_")
    assert name(65537, 16).startswith("axh_q4k_matvec_flat_")
    assert name(128256, 16) == "axh_q4k_matvec_flat_r2_w4_p2_n0"  # the head keeps prefetch 2
    assert name(65536, 56) == "axh_q4k_matvec_flat_r1_w8_p2_n0"
    assert name(65536, 128) == "axh_q4k_matvec_flat_r1_w16_p2_n0"
    # the early-refill (prefetch 1) kernels stage x in chunks: any row fits
    assert name(4096, 56, axc.Variant(2, 4, 1, 2)) == "axh_q4k_matvec_flat_r2_w4_p1_n0"
    assert name(1, 256) == "axh_q4k_matvec_sk_s16"  # few long rows: split-K
    assert name(1, 1024) == "axh_q4k_matvec_tiled_r1_w4_p2"
    assert name(4096, 1024) == "axh_q4k_matvec_tiled_r2_w8_p2"
    assert name(4096, 56, axc.Variant(2, 4, 4, 1)) == "axh_q4k_matvec_tiled_r2_w8_p2"  # 56*8 > 4*64
    assert name(4096, 16, axc.Variant(2, 4, 4, 1)) == "axh_q4k_matvec_flat_r2_w4_p4_n1"
    # two staged x sub-blocks per thread when one is not enough
    assert name(4096, 56, axc.Variant(2, 4, 2, 2)) == "axh_q4k_matvec_flat_r2_w4_p2_n0_x2"
    assert name(4096, 16, axc.Variant(2, 4, 2, 2)) == "axh_q4k_matvec_flat_r2_w4_p2_n0"
    # few rows: one workgroup for 1-4 long rows, split-K past 128 superblocks,
    # the tiled kernel otherwise
    assert name(1, 128) == "axh_q4k_matvec_wg_w8_x2_r1"
    assert name(2, 33) == "axh_q4k_matvec_wg_w8_x2_r2"
    assert name(3, 64) == "axh_q4k_matvec_wg_w8_x2_r4"
    assert name(4, 128) == "axh_q4k_matvec_wg_w8_x2_r4"
    assert name(5, 129) == name(31, 256) == "axh_q4k_matvec_sk_s16"
    for rows, sb in ((4, 63), (5, 128), (31, 64), (1, 32), (8, 63), (8, 56), (31, 1)):
        assert name(rows, sb) == "axh_q4k_matvec_tiled_r1_w4_p2", (rows, sb)
    assert name(8, 56, axc.Variant(family=axc.FAMILY_COLUMNS)) == "axh_q4k_matvec_cols_r4_w4_n0_x1"
    assert name(31, 1, axc.Variant(family=axc.FAMILY_COLUMNS)) == "axh_q4k_matvec_cols_r4_w1_n0_x1"
    assert name(32, 1) == "axh_q4k_matvec_one_i1"
    co = axc.builtin_code_object()
    for rows in (1, 31, 64):
        for sb in (1, 16, 56, 128, 129, 4096):
            assert name(rows, sb).encode() in co
    with pytest.raises(axc.DispatchError):
        name(64, 16, axc.Variant(3, 4, 2, 2))


def test_variant_index_out_of_range_is_typed_error(axc):
    lib = axc.load_library()
    v = axc.axh._Variant()
    assert lib.axh_q4k_matvec_variant_at(10_000, ctypes.byref(v)) == 100
    assert b"out of range" in lib.axh_last_error()


def test_null_context_calls_fail_cleanly(axc):
    lib = axc.load_library()
    assert lib.axh_q4k_matvec(None, None, None, None, 1, 1, None, None) == 100
    assert lib.axh_synchronize(None, None) == 100
    assert lib.axh_upload(None, None, None, 0) == 100
    lib.axh_context_destroy(None)  # no-op
    lib.axh_kernel_release(None)   # no-op


def test_context_without_gpu_reports_typed_error(axc):
    """In a container without a GPU, context creation fails with a typed
    status (no crash); on a GPU box it succeeds."""
    try:
        ctx = axc.HipContext.new()
    except axc.DispatchError as e:
        assert e.variant in ("NoVulkanInstance", "NoSupportedDevice")
    else:
        assert "gfx950" in ctx.device_name or ctx.device_name
        ctx.close()


def test_matmul_kernel_selection(axc):
    """Defaults by the grid each kind would launch on 256 CUs: streaming rows
    (kind 7) in the narrowest column groups that keep its grid one resident
    wave, the K-split kind where its grid is one wave, 32 x 32 MFMA tiles where
    their rows fill 160 workgroups, else K-split tiles with their columns
    halved until the grid fills."""
    name = axc.q4k_matmul_kernel_name
    # K <= 4096, up to 8 columns of 14336 rows: 8-column groups (X staged through 64 KiB)
    assert name(14336, 16, 8) == "axh_q4k_matmul_sr_w8_s2_h"
    assert name(14336, 1, 1) == "axh_q4k_matmul_sr_w8_s2_h"
    assert name(14336, 16, 8, axc.MatmulVariant(7, 8, 1, 1)) == "axh_q4k_matmul_sr_w8_s2"
    assert name(14336, 16, 9) == "axh_q4k_matmul_sr_w8_s2"
    assert name(14336, 16, 16) == "axh_q4k_matmul_sr_w8_s2"
    assert name(14336, 16, 16, axc.MatmulVariant(7, 8, 1, 2)) == "axh_q4k_matmul_sr_w8_s2_h"
    assert name(14336, 16, 32) == "axh_q4k_matmul_sr_w8_s2_n2"  # two column groups
    assert name(14336, 16, 17) == "axh_q4k_matmul_sr_w8_s2_n2"
    # fewer rows: narrower groups still fit one wave, and kind 7 goes past 32 columns
    assert name(1024, 16, 32) == "axh_q4k_matmul_sr_w8_s2_h"  # 64 blocks x 4 groups
    assert name(2048, 16, 32) == "axh_q4k_matmul_sr_w8_s2"
    assert name(1024, 16, 64) == "axh_q4k_matmul_sr_w8_s2"
    assert name(4096, 16, 64) == "axh_q4k_matmul_sr_w8_s2_n2"  # two blocks of 32 columns per CU
    assert name(8192, 16, 64) == "axh_q4k_matmul_kx_r4_n2_k4_p2"  # four: K-split tiles
    # 128 columns: 32 x 32 tiles once 128 x 128 of them fill 160 workgroups
    assert name(14336, 16, 128) == "axh_q4k_matmul_kx_r4_n8_k4_p2"  # 112: K-split tiles
    assert name(20480, 16, 128) == "axh_q4k_matmul_rm_w4_r1_p4"  # 160
    assert name(28672, 32, 128) == "axh_q4k_matmul_rm_w4_r1_p4"
    # K > 4096 over few rows: kind 9 up to 32 columns, its largest tile (32 or
    # 16 rows x 16 or 8 columns) whose grid fills 160 workgroups, at most two
    # waves of them; then the K-split kind while its grid is one wave
    assert name(4096, 56, 8) == "axh_q4k_matmul_lk_c8_x2_w2"
    assert name(4096, 17, 16) == "axh_q4k_matmul_lk_c16_x1_w3"
    with pytest.raises(axc.DispatchError):  # kind 7 keeps K <= 4096 of X in registers
        name(4096, 17, 16, axc.MatmulVariant(7, 8, 1, 1))
    assert name(4096, 56, 32) == "axh_q4k_matmul_lk_c16_x1_w3_r2"  # 128 x 2 workgroups
    assert name(1024, 56, 32) == "axh_q4k_matmul_lk_c8_x2_w2"  # 64 x 4
    assert name(4096, 56, 4) == "axh_q4k_matmul_lk_c4_x2_w2"  # up to 4 columns
    assert name(2048, 56, 8) == "axh_q4k_matmul_lk_c4_x2_w2"  # 8 columns on 128 tiles of 8
    assert name(2049, 56, 8) == "axh_q4k_matmul_lk_c8_x2_w2"
    assert name(8192, 56, 3) == "axh_q4k_matmul_lk_c4_x2_w2"  # 512: two per CU
    assert name(8192, 56, 8) == "axh_q4k_matmul_lk_c8_x2_w2_r2"  # 256 x 1
    assert name(14336, 56, 8) == "axh_q4k_matmul_kx_r4_n1_k4_p3"  # 448 x 1: K-split tiles
    assert name(8192, 56, 32) == "axh_q4k_matmul_kx_r4_n1_k4_p3"  # 256 x 2
    # past 32 columns, where one wave of 16 x 16 or 32 x 16 tiles fills the
    # chip: kind 9 with 16-column tiles (the K-split kind with the same tiles
    # for rows too long for kind 9)
    assert name(1024, 56, 64) == "axh_q4k_matmul_lk_c16_x1_w3"  # 16-row tiles: 64 x 4
    assert name(1024, 56, 128) == "axh_q4k_matmul_lk_c16_x1_w3_r2"  # 32-row tiles: 32 x 8
    assert name(64, 1100, 64) == "axh_q4k_matmul_ks_k8_n1_p1_r1"
    assert name(14336, 56, 32) == "axh_q4k_matmul_kx_r4_n2_k4_p3"  # prefetch 3 at K > 4096
    assert name(4096, 56, 8, axc.MatmulVariant(3, 8, 1, 2, 1)) == "axh_q4k_matmul_ks_k8_n1_p2_r1"
    with pytest.raises(axc.DispatchError):  # kind 9 keeps the chunk offsets below 1 MiB
        name(16, 1024, 8, axc.MatmulVariant(9))
    # ... so a call without a variant never picks it there: rows of 1024 or
    # more superblocks fall through to the K-split kinds
    assert name(64, 1024, 1) == "axh_q4k_matmul_ks_k8_n1_p1_r1"
    assert name(4096, 1200, 8).startswith("axh_q4k_matmul_k")
    assert name(4096, 2048, 2).startswith("axh_q4k_matmul_k")
    assert name(16, 1023, 8).startswith("axh_q4k_matmul_lk_")
    # K-split tiles, columns halved until 160 workgroups
    assert name(14336, 16, 64) == "axh_q4k_matmul_kx_r4_n4_k4_p2"
    assert name(14336, 16, 128) == "axh_q4k_matmul_kx_r4_n8_k4_p2"
    assert name(4096, 16, 128) == "axh_q4k_matmul_kx_r4_n2_k4_p2"
    assert name(4096, 56, 128) == "axh_q4k_matmul_kx_r4_n2_k4_p3"
    assert name(4096, 56, 64) == "axh_q4k_matmul_kx_r4_n1_k4_p3"
    # 32 x 32 MFMA tiles where their rows fill the grid
    assert name(14336, 16, 256) == "axh_q4k_matmul_rm_w4_r1_p4"
    assert name(14336, 16, 512) == "axh_q4k_matmul_rm_w8_r1_p4"
    assert name(8192, 16, 512) == "axh_q4k_matmul_rm_w4_r1_p4"  # 8 waves: 128 workgroups
    assert name(4096, 16, 512) == "axh_q4k_matmul_kx_r4_n8_k4_p2"
    assert name(4096, 16, 256) == "axh_q4k_matmul_kx_r4_n4_k4_p2"
    assert name(14336, 16, 512, axc.MatmulVariant(8, 4, 8, 4, 2)) == "axh_q4k_matmul_rm_w4_r2_p4"
    assert name(14336, 16, 8, axc.MatmulVariant(3, 4, 1, 2)) == "axh_q4k_matmul_ks_k4_n1_p2"
    # kinds 1, 2, 4 and 6 (LDS-tiled, register A, streaming, row-split) were removed
    for kind, w, nt, pf, rt in ((1, 2, 2, 1, 0), (2, 4, 4, 2, 0), (4, 4, 1, 4, 0), (6, 8, 8, 3, 2)):
        with pytest.raises(axc.DispatchError):
            name(14336, 16, 512, axc.MatmulVariant(kind, w, nt, pf, rt))
    vs = axc.compiled_matmul_variants()
    assert len(set(vs)) == len(vs) >= 6
    assert {v.kind for v in vs} == {3, 5, 7, 8, 9}
    assert name(14336, 16, 128, axc.MatmulVariant(5, 4, 8, 2, 4)) == \
        "axh_q4k_matmul_kx_r4_n8_k4_p2"
    assert all((v.row_tiles > 0) == (v.kind in (3, 5, 8, 9)) for v in vs)
    assert name(4096, 56, 32, axc.MatmulVariant(9, 8, 4, 1, 2)) == "axh_q4k_matmul_lk_c16_x1_w3_r2"
    with pytest.raises(axc.DispatchError):  # row tiles are kinds 3, 5, 8 and 9 only
        name(14336, 16, 8, axc.MatmulVariant(7, 8, 1, 1, 1))
    co = axc.builtin_code_object()
    for v in vs:
        assert name(64, 16, 64, v).startswith("axh_q4k_matmul_")


def test_gate_up_kernel_selection(axc):
    """Fused gate/up: persistent kernel only; x staging widened for long rows;
    rows past 128 superblocks and non-temporal requests are typed errors."""
    name = axc.q4k_gate_up_kernel_name
    assert name(14336, 16) == "axh_q4k_gate_up_r1_w4_p1_x1"
    assert name(14336, 56, axc.Variant(1, 4, 1, 0)) == "axh_q4k_gate_up_r1_w4_p1_x1"  # chunked x
    assert name(14336, 56) == "axh_q4k_gate_up_r1_w8_p2_x1"
    assert name(14336, 128) == "axh_q4k_gate_up_r1_w8_p2_x2"
    assert name(14336, 16, axc.Variant(2, 8, 2, 0)) == "axh_q4k_gate_up_r2_w8_p2_x1"
    assert name(14336, 56, axc.Variant(1, 4, 2, 0)) == "axh_q4k_gate_up_r1_w4_p2_x2"
    # up to 12288 rows of up to 64 superblocks: the wave-paired one-pass kernel
    assert name(1024, 16) == name(2048, 16) == "axh_q4k_gate_up_one_i2"
    assert name(2049, 16) == "axh_q4k_gate_up_onex_i2"
    assert name(12288, 64) == "axh_q4k_gate_up_onex_i8"
    assert name(12289, 16) == "axh_q4k_gate_up_r1_w4_p1_x1"
    assert name(4096, 65) == "axh_q4k_gate_up_r1_w8_p2_x2"
    V, one, onex = axc.Variant, axc.FAMILY_ONE_PASS, axc.FAMILY_ONE_PASS_X
    assert name(14336, 16, V(family=onex)) == "axh_q4k_gate_up_onex_i2"
    assert name(14336, 16, V(family=one, sb_per_lane=5)) == "axh_q4k_gate_up_one_i5"
    for bad in ((4, 16, V(family=one, sb_per_lane=1)), (4, 16, V(family=one, sb_per_lane=9)),
                (4, 65, V(family=one)), (4, 16, V(1, 0, 0, 0, one)), (4, 16, V(family=1)),
                (4, 16, V(sb_per_lane=2))):
        with pytest.raises(axc.DispatchError):
            name(*bad)
    co = axc.builtin_code_object()
    for nit in range(1, 9):
        for fmt in ("q4k", "q4_0"):
            assert f"axh_{fmt}_gate_up_one_i{nit}".encode() in co
            assert f"axh_{fmt}_gate_up_onex_i{nit}".encode() in co
    vs = axc.compiled_variants("gate_up")
    assert len(set(vs)) == len(vs) >= 4
    for v in vs:
        assert name(1000, 16, v).encode() in co
    for sb in (1, 16, 64, 128):
        assert name(7, sb).encode() in co
    for bad in ((4, 0, None), (4, 129, None), (4, 16, axc.Variant(0, 0, 0, 1)),
                (4, 16, axc.Variant(3, 4, 2, 0)), (4, 100, axc.Variant(2, 4, 2, 0))):
        with pytest.raises(axc.DispatchError):
            name(*bad)


def test_kquant_kernel_selection(axc):
    """Q5_K / Q6_K: persistent kernel only, x staging widened for long rows,
    typed errors beyond 128 superblocks or for missing variants."""
    co = axc.builtin_code_object()
    for fam, name in (("q5k", axc.q5k_matvec_kernel_name), ("q6k", axc.q6k_matvec_kernel_name)):
        assert name(128256, 16) == f"axh_{fam}_matvec_flat_r1_w4_p1_x1"
        assert name(4096, 56) == ("axh_q5k_matvec_one_i7" if fam == "q5k"
                                  else "axh_q6k_matvec_flat_r1_w8_p1_x1")
        assert name(8192, 56) == f"axh_{fam}_matvec_flat_r1_w8_p1_x1"
        # Q5_K's prefetch-1 kernel stages x in chunks; Q6_K's stages it whole
        assert name(65536, 128) == ("axh_q5k_matvec_flat_r1_w8_p1_x1" if fam == "q5k"
                                    else "axh_q6k_matvec_flat_r1_w8_p2_x2")
        assert name(4096, 56, axc.Variant(1, 4, 2, 0)) == f"axh_{fam}_matvec_flat_r1_w4_p2_x2"
        vs = axc.compiled_variants(fam)
        assert len(set(vs)) == len(vs) >= 3
        for v in vs:
            assert name(100, 16, v).encode() in co
        for bad in ((4, 0, None), (4, 129, None), (4, 16, axc.Variant(0, 0, 0, 1)),
                    (4, 16, axc.Variant(3, 4, 2, 0)), (4, 100, axc.Variant(2, 4, 2, 0))):
            with pytest.raises(axc.DispatchError):
                name(*bad)
    for k in ("axh_q5k_dequant", "axh_q6k_dequant", "axh_f32_to_f16"):
        assert k.encode() in co


def test_q5k_one_pass_family(axc):
    """Q5_K rows of up to 16 superblocks over 768-32768 rows take the
    one-pass kernel by default; the family is reachable by request (hole:
    sb_per_lane 1 or 2) and is Q5_K's only family."""
    co = axc.builtin_code_object()
    name, V, one = axc.q5k_matvec_kernel_name, axc.Variant, axc.FAMILY_ONE_PASS
    assert name(14336, 16) == "axh_q5k_matvec_one_i2"
    assert name(4096, 16) == "axh_q5k_matvec_one_i2"
    assert name(2048, 8) == name(768, 8) == "axh_q5k_matvec_one_i1"
    assert name(1024, 16) == "axh_q5k_matvec_one_i2"
    for rows, sb in ((767, 16), (32769, 16), (2048, 17), (4097, 17), (4096, 65), (8192, 56)):
        assert name(rows, sb).startswith("axh_q5k_matvec_flat_"), (rows, sb)
    # 2049-4096 rows of 17-64 superblocks: one pass too
    assert name(2049, 17) == "axh_q5k_matvec_one_i3"
    assert name(4096, 56) == "axh_q5k_matvec_one_i7"
    assert name(4096, 64) == "axh_q5k_matvec_one_i8"
    assert name(4096, 16, V(1, 4, 1, 0)) == "axh_q5k_matvec_flat_r1_w4_p1_x1"  # flat holes
    assert name(7, 3, V(0, 0, 0, 0, one, 0)) == "axh_q5k_matvec_one_i1"
    assert name(7, 3, V(0, 0, 0, 0, one, 2)) == "axh_q5k_matvec_one_i2"
    assert name(7, 3, V(0, 0, 2, 0, one, 3)) == "axh_q5k_matvec_onep_i3"
    assert name(100, 64, V(0, 0, 1, 0, one, 8)) == "axh_q5k_matvec_one_i8"
    for i in range(1, 9):
        assert f"axh_q5k_matvec_one_i{i}".encode() in co
        assert i < 3 or f"axh_q5k_matvec_onep_i{i}".encode() in co
    for bad in ((100, 65, V(0, 0, 0, 0, one, 0)), (100, 16, V(0, 0, 0, 0, one, 1)),
                (100, 16, V(0, 0, 0, 0, one, 9)), (100, 16, V(1, 0, 0, 0, one, 0)),
                (100, 16, V(0, 0, 2, 0, one, 0)), (100, 16, V(0, 0, 3, 0, one, 3)),
                (100, 16, V(0, 0, 0, 1, one, 0)), (100, 16, V(0, 0, 0, 0, 0, 2))):
        with pytest.raises(axc.DispatchError):
            name(*bad)


def test_q6k_one_pass_family(axc):
    """Q6_K rows of up to 16 superblocks over 256-4096 rows take the one-pass
    kernel by default; the family is reachable by request with the same hole
    (sb_per_lane 1 or 2) and otherwise the persistent kernels run."""
    co = axc.builtin_code_object()
    name, V, one = axc.q6k_matvec_kernel_name, axc.Variant, axc.FAMILY_ONE_PASS
    assert name(1024, 16) == "axh_q6k_matvec_one_i2"  # Llama-3-8B attn_v (GQA)
    assert name(4096, 16) == "axh_q6k_matvec_one_i2"
    assert name(256, 8) == "axh_q6k_matvec_one_i1"
    for rows, sb in ((255, 16), (4097, 16), (14336, 16), (128256, 16), (2048, 17), (4096, 41),
                     (4096, 56), (8193, 24)):
        assert name(rows, sb).startswith("axh_q6k_matvec_flat_"), (rows, sb)
    # 2049-8192 rows of 17-40 superblocks: one pass too
    assert name(2049, 17) == "axh_q6k_matvec_one_i3"
    assert name(4096, 40) == "axh_q6k_matvec_one_i5"
    assert name(8192, 24) == "axh_q6k_matvec_one_i3"
    # at most 2048 rows of 17-64 superblocks, and 14336 rows and more of 33-64:
    # 4 waves, x whole, prefetch 2
    assert name(2048, 24) == "axh_q6k_matvec_flat_r1_w4_p2_x1"
    assert name(1024, 56) == name(14336, 56) == "axh_q6k_matvec_flat_r1_w4_p2_x2"
    assert name(14336, 24) == "axh_q6k_matvec_flat_r1_w4_p1_x1"
    assert axc.q5k_matvec_kernel_name(14336, 40) == "axh_q5k_matvec_flat_r1_w4_p2_x2"
    assert name(4096, 16, V(1, 4, 1, 0)) == "axh_q6k_matvec_flat_r1_w4_p1_x1"  # flat holes
    # up to 1024 rows of 17-32 superblocks: prefetch 2 (Llama-2-70B attn_v is 1024 x 8192)
    assert name(1024, 32) == "axh_q6k_matvec_flat_r1_w4_p2_x1"
    assert name(1, 17) == "axh_q6k_matvec_flat_r1_w4_p2_x1"
    assert name(1025, 32) == "axh_q6k_matvec_flat_r1_w4_p2_x1"
    assert name(1024, 33) == "axh_q6k_matvec_flat_r1_w4_p2_x2"
    assert name(1024, 65) == "axh_q6k_matvec_flat_r1_w8_p2_x2"
    # Q5_K: the same up to 1024 rows of up to 32 superblocks (below 768 rows
    # of up to 16: the one pass takes 768 rows on)
    q5 = axc.q5k_matvec_kernel_name
    assert q5(767, 16) == "axh_q5k_matvec_flat_r1_w4_p2_x1"
    assert q5(1024, 32) == "axh_q5k_matvec_flat_r1_w4_p2_x1"
    assert q5(1025, 32) == "axh_q5k_matvec_flat_r1_w4_p2_x1"
    assert q5(4096, 16) == "axh_q5k_matvec_one_i2"
    assert name(7, 3, V(0, 0, 0, 0, one, 0)) == "axh_q6k_matvec_one_i1"
    assert name(7, 3, V(0, 0, 0, 0, one, 2)) == "axh_q6k_matvec_one_i2"
    assert name(100, 56, V(0, 0, 2, 0, one, 0)) == "axh_q6k_matvec_onep_i7"
    for i in range(1, 9):
        assert f"axh_q6k_matvec_one_i{i}".encode() in co
        assert i < 3 or f"axh_q6k_matvec_onep_i{i}".encode() in co
    for bad in ((100, 65, V(0, 0, 0, 0, one, 0)), (100, 16, V(0, 0, 0, 0, one, 1)),
                (100, 16, V(0, 0, 0, 0, one, 9)), (100, 16, V(0, 0, 2, 0, one, 0)),
                (100, 16, V(0, 0, 0, 0, 0, 2)), (100, 16, V(0, 0, 0, 0, 3, 0))):
        with pytest.raises(axc.DispatchError):
            name(*bad)


def test_q4_0_kernel_selection(axc):
    """Q4_0 defaults: fewer than 32 rows, 32-1024 rows of at most 128 blocks,
    32-256 rows of 193-256 blocks, odd block counts and rows of more than 1024
    blocks take the LDS-tiled kernel (the column kernel only on request);
    otherwise the one-pass kernel over octets of 8 blocks (x whole for 65-128 blocks from 6144 rows, x two chunks ahead for 14-16 steps
    from 4096 rows), persistent for more than 16384 rows of more than 256
    blocks."""
    name = axc.q4_0_matvec_kernel_name
    assert name(1, 2) == name(31, 128) == name(8, 16) == "axh_q4_0_matvec_r1_w4"
    # 32-256 rows of 193-256 blocks
    assert name(32, 193) == name(256, 256) == name(100, 200) == "axh_q4_0_matvec_r1_w4"
    assert name(257, 256) == "axh_q4_0_matvec_one_i4"
    assert name(256, 192) == "axh_q4_0_matvec_one_i3"
    assert name(256, 258) == "axh_q4_0_matvec_one_i5"
    cols = axc.Variant(family=axc.FAMILY_COLUMNS)
    assert name(1, 2, cols) == name(31, 128, cols) == "axh_q4_0_matvec_cols_r1"
    assert name(256, 128) == name(512, 128) == name(300, 2) == name(32, 128) == \
        "axh_q4_0_matvec_r1_w4"
    assert name(31, 130) == "axh_q4_0_matvec_r1_w4"
    assert name(512, 130) == "axh_q4_0_matvec_one_i3"
    assert name(1024, 128) == name(513, 128) == "axh_q4_0_matvec_r1_w4"
    assert name(1025, 128) == "axh_q4_0_matvec_one_i2"
    assert name(4096, 2) == "axh_q4_0_matvec_one_i1"
    assert name(256, 130) == "axh_q4_0_matvec_one_i3"
    assert name(32, 448) == "axh_q4_0_matvec_one_i7"
    assert name(31, 448) == name(16, 1024) == "axh_q4_0_matvec_r1_w4"
    assert name(6143, 128) == "axh_q4_0_matvec_one_i2"
    assert name(6144, 128) == name(128256, 128) == "axh_q4_0_matvec_onex_i2"
    assert name(6144, 64) == "axh_q4_0_matvec_one_i1"
    assert name(6144, 130) == "axh_q4_0_matvec_one_i3"
    assert name(4096, 896) == "axh_q4_0_matvec_onep_i14"
    assert name(4096, 1024) == "axh_q4_0_matvec_onep_i16"
    assert name(4095, 1024) == "axh_q4_0_matvec_one_i16"
    assert name(4096, 832) == "axh_q4_0_matvec_one_i13"
    assert name(16384, 448) == "axh_q4_0_matvec_one_i7"
    assert name(16385, 256) == "axh_q4_0_matvec_one_i4"
    assert name(16385, 258) == name(28672, 448) == "axh_q4_0_matvec_flat_r1_w8_p1_x1"
    # odd block counts and rows past 1024 blocks: the LDS-tiled kernel
    assert name(256, 127) == name(4095, 1026) == "axh_q4_0_matvec_r1_w4"
    assert name(4096, 127) == name(8191, 1100) == name(8192, 255) == "axh_q4_0_matvec_r2_w4"
    assert name(8192, 257) == name(14336, 127) == "axh_q4_0_matvec_r4_w4"
    assert name(256, 128, axc.Variant(1, 1, 0, 0)) == "axh_q4_0_matvec_r1_w1"
    assert name(256, 128, axc.Variant(family=axc.FAMILY_TILED)) == "axh_q4_0_matvec_r1_w4"
    co = axc.builtin_code_object()
    assert b"axh_q4_0_matvec_cols_r1" in co
    for nit in range(1, 17):
        assert f"axh_q4_0_matvec_one_i{nit}".encode() in co
        assert f"axh_q4_0_matvec_onex_i{nit}".encode() in co
        if nit >= 3:
            assert f"axh_q4_0_matvec_onep_i{nit}".encode() in co


def test_q4_0_gate_up_selection(axc):
    """Fused Q4_0 gate/up: the persistent kernel over octets (4 waves, early
    refill by default), its holes, and typed errors for odd or long rows."""
    name, V = axc.q4_0_gate_up_kernel_name, axc.Variant
    co = axc.builtin_code_object()
    assert name(14336, 128) == name(100, 1024) == "axh_q4_0_gate_up_r1_w4_p1_x1"
    assert name(1, 2) == "axh_q4_0_gate_up_one_i1"
    assert name(4096, 128) == name(12288, 128) == "axh_q4_0_gate_up_onex_i2"
    assert name(2048, 512) == "axh_q4_0_gate_up_one_i8"
    assert name(2048, 514) == "axh_q4_0_gate_up_r1_w4_p1_x1"
    assert name(14336, 128, V(family=axc.FAMILY_ONE_PASS)) == "axh_q4_0_gate_up_one_i2"
    for (r, w, pf), want in (((1, 8, 1), "r1_w8_p1_x1"), ((2, 4, 1), "r2_w4_p1_x1"),
                             ((1, 4, 2), "r1_w4_p2_x1"), ((1, 8, 2), "r1_w8_p2_x1")):
        got = name(14336, 128, V(r, w, pf, 0))
        assert got == f"axh_q4_0_gate_up_{want}" and got.encode() in co
    assert name(14336, 448, V(1, 4, 2, 0)) == "axh_q4_0_gate_up_r1_w4_p2_x2"
    for bad in ((4, 127, None), (4, 1026, None), (4, 0, None), (4, 2, V(0, 0, 0, 1)),
                (4, 2, V(4, 4, 1, 0)), (4, 2, V(family=1)), (4, 600, V(1, 8, 2, 0)),
                (4, 600, V(1, 4, 2, 0))):
        with pytest.raises(axc.DispatchError):
            name(*bad)


def test_q5k_gate_up_selection(axc):
    """Fused Q5_K gate/up: the wave-paired one-pass kernel (x chunk by chunk)
    up to 12288 rows of up to 64 superblocks, else the persistent kernel (4
    waves, x whole, prefetch 2; early refill past 64 superblocks); both
    reachable through their holes."""
    name, V = axc.q5k_gate_up_kernel_name, axc.Variant
    co = axc.builtin_code_object()
    assert name(1, 1) == "axh_q5k_gate_up_one_i1"
    assert name(2048, 16) == name(14336 - 2048, 16) == "axh_q5k_gate_up_one_i2"
    assert name(100, 64) == "axh_q5k_gate_up_one_i8"
    assert name(12289, 16) == name(28672, 32) == "axh_q5k_gate_up_r1_w4_p2_x1"
    assert name(28672, 64) == "axh_q5k_gate_up_r1_w4_p2_x2"
    assert name(100, 65) == name(28672, 128) == "axh_q5k_gate_up_r1_w4_p1_x1"
    assert name(14336, 16, V(1, 8, 1, 0)) == "axh_q5k_gate_up_r1_w8_p1_x1"
    assert name(14336, 16, V(family=axc.FAMILY_ONE_PASS)) == "axh_q5k_gate_up_one_i2"
    assert name(14336, 16, V(family=axc.FAMILY_ONE_PASS_X, sb_per_lane=5)) == \
        "axh_q5k_gate_up_onex_i5"
    for nit in range(1, 9):
        assert f"axh_q5k_gate_up_one_i{nit}".encode() in co
        assert f"axh_q5k_gate_up_onex_i{nit}".encode() in co
    for k in ("r1_w4_p1_x1", "r1_w8_p1_x1", "r1_w4_p2_x1", "r1_w4_p2_x2"):
        assert f"axh_q5k_gate_up_{k}".encode() in co
    for bad in ((4, 0, None), (4, 129, None), (4, 16, V(1, 4, 3, 0)), (4, 16, V(family=1)),
                (4, 16, V(family=2, sb_per_lane=9)), (4, 16, V(family=2, sb_per_lane=1)),
                (4, 16, V(sb_per_lane=2)), (4, 70, V(1, 4, 2, 0)), (4, 65, V(family=2)),
                (4, 16, V(0, 0, 0, 1))):
        with pytest.raises(axc.DispatchError):
            name(*bad)


def test_q4_0_family_holes(axc):
    """The Q4_0 families and their holes: persistent (rows_per_wave,
    waves_per_workgroup, prefetch), one pass (sb_per_lane = steps of 64 blocks,
    prefetch = x chunks ahead), one pass with x whole, column, tiled."""
    name, V = axc.q4_0_matvec_kernel_name, axc.Variant
    P, O1, OX = axc.FAMILY_PERSISTENT, axc.FAMILY_ONE_PASS, axc.FAMILY_ONE_PASS_X
    co = axc.builtin_code_object()
    assert name(4096, 128, V(family=P)) == "axh_q4_0_matvec_flat_r1_w8_p1_x1"
    for (r, w, pf), want in (((1, 4, 1), "r1_w4_p1_x1"), ((2, 4, 1), "r2_w4_p1_x1"),
                             ((2, 8, 1), "r2_w8_p1_x1"), ((1, 8, 2), "r1_w8_p2_x1"),
                             ((2, 4, 2), "r2_w4_p2_x2"), ((1, 16, 2), "r1_w16_p2_x1")):
        got = name(4096, 448, V(r, w, pf, 0, P))
        assert got == f"axh_q4_0_matvec_flat_{want}" and got.encode() in co
    assert name(4096, 1024, V(1, 16, 2, 0, P)) == "axh_q4_0_matvec_flat_r1_w16_p2_x1"
    assert name(4096, 128, V(family=O1)) == "axh_q4_0_matvec_one_i2"
    assert name(4096, 128, V(family=O1, sb_per_lane=5)) == "axh_q4_0_matvec_one_i5"
    assert name(4096, 128, V(prefetch=2, family=O1, sb_per_lane=3)) == "axh_q4_0_matvec_onep_i3"
    assert name(4096, 1024, V(prefetch=1, family=O1)) == "axh_q4_0_matvec_one_i16"
    assert name(4096, 128, V(family=OX)) == "axh_q4_0_matvec_onex_i2"
    assert name(4096, 128, V(family=axc.FAMILY_COLUMNS)) == "axh_q4_0_matvec_cols_r1"
    assert name(4096, 448, V(2, 4, 0, 0, axc.FAMILY_TILED)) == "axh_q4_0_matvec_r2_w4"
    for bad in ((4096, 127, V(family=P)), (4096, 1026, V(family=P)), (4096, 127, V(family=O1)),
                (4096, 1026, V(family=OX)), (4096, 130, V(family=O1, sb_per_lane=2)),
                (4096, 128, V(family=O1, sb_per_lane=17)), (4096, 128, V(prefetch=2, family=O1)),
                (4096, 448, V(prefetch=2, family=OX)), (4096, 448, V(prefetch=3, family=O1)),
                (4096, 448, V(1, 0, 0, 0, O1)), (4096, 448, V(0, 0, 0, 1, P)),
                (4096, 448, V(3, 4, 1, 0, P)), (4096, 1024, V(1, 8, 2, 0, P)),
                (4096, 130, V(family=axc.FAMILY_COLUMNS)), (4096, 128, V(1, 4, 0, 0, 6)),
                (4096, 128, V(family=axc.FAMILY_WORKGROUP)), (4096, 128, V(family=5)),
                (4096, 128, V(1, 4, 0, 0, 0, 2)), (119304648, 2, V(family=P))):
        with pytest.raises(axc.DispatchError):
            name(*bad)
