"""axiom-compute_amd: MI355X (gfx950) Q4_0 / Q4_K_M dequant-matvec path.

The package directory name contains a hyphen, so it is loaded by path; see
`load()` in __graft_entry__.py and tests/conftest.py.  Everything here calls
into libaxh.so (hand-written HIP kernels + C ABI runtime).
"""
from . import axh  # noqa: F401
from . import gguf  # noqa: F401
from .axh import (  # noqa: F401
    BindingPlan,
    DeviceBuffer,
    DispatchError,
    DispatchRequest,
    Graph,
    HipContext,
    HipContextOptions,
    KernelHandle,
    Variant,
    builtin_code_object,
    compiled_variants,
    compiled_matmul_variants,
    MatmulVariant,
    q4k_matmul_kernel_name,
    q4k_gate_up_kernel_name,
    q4k_matvec_kernel_name,
    q5k_matvec_kernel_name,
    q6k_matvec_kernel_name,
    ggml_type_size,
    q4_0_matvec_kernel_name,
    load_library,
    validate_request,
)

__all__ = [
    "axh",
    "BindingPlan",
    "DeviceBuffer",
    "DispatchError",
    "DispatchRequest",
    "Graph",
    "HipContext",
    "HipContextOptions",
    "KernelHandle",
    "Variant",
    "builtin_code_object",
    "compiled_variants",
    "compiled_matmul_variants",
    "MatmulVariant",
    "q4k_matmul_kernel_name",
    "q4k_gate_up_kernel_name",
    "q4k_matvec_kernel_name",
    "q5k_matvec_kernel_name",
    "q6k_matvec_kernel_name",
    "ggml_type_size",
    "gguf",
    "q4_0_matvec_kernel_name",
    "load_library",
    "validate_request",
]
