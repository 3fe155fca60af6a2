"""axiom-compute_amd: MI355X (gfx950) Q4_0 / Q4_K_M dequant-matvec path.

The package directory name contains a hyphen, so it is loaded by path; see
`load()` in __graft_entry__.py and tests/conftest.py.  Everything here calls
into libaxh.so (hand-written HIP kernels + C ABI runtime).
"""
from . import axh, gguf  # noqa: F401
from .axh import (  # noqa: F401
    FAMILY_COLUMNS, FAMILY_DEFAULT, FAMILY_ONE_PASS, FAMILY_ONE_PASS_X, FAMILY_PERSISTENT,
    FAMILY_SPLIT_K, FAMILY_TILED, FAMILY_WORKGROUP, BindingPlan, DeviceBuffer, DispatchError,
    DispatchRequest, Graph, HipContext, HipContextOptions, KernelHandle, MatmulVariant, Variant,
    builtin_code_object, compiled_matmul_variants, compiled_variants, ggml_type_size,
    load_library, q4_0_gate_up_kernel_name, q4_0_matvec_kernel_name, q4k_gate_up_kernel_name,
    q4k_matmul_kernel_name, q4k_matvec_default_variant, q4k_matvec_kernel_name,
    q5k_gate_up_kernel_name, q5k_matvec_kernel_name, q6k_matvec_kernel_name, validate_request)
