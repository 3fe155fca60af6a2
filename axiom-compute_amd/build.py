"""Build recipe for the gfx950 path (no cmake/ninja needed).

1. csrc/kernels/*.hip -> gfx950 code objects (hipcc, device only, raw ELF)
2. csrc/runtime/*.cpp + axh_embed.S -> libaxh.so (g++ against libamdhip64),
   with the code objects embedded so the library is self-contained
3. oracle/ -> oracle/liboracle.so (test infrastructure, gcc)

Every step runs on a machine without a GPU.  Outputs stay in the source
tree (libaxh.so next to this file, intermediates in _build/).

`python axiom-compute_amd/build.py --sanitize` also builds the host code
(runtime, GGUF reader, checker, autotuner, winner table) and the oracle with
AddressSanitizer and UndefinedBehaviorSanitizer into separate outputs,
_build/san/libaxh.so and oracle/_san/liboracle.so, for the CPU test suite
(AXH_LIBRARY / AXH_ORACLE_LIBRARY select them; the sanitizer runtimes are
preloaded into the interpreter).  Device code is never built with a
sanitizer.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
BUILD = PKG / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
LIB = PKG / "libaxh.so"

# Packed-FP32 instructions stay off (hipcc flag for device code).
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Kernel code objects: every kernel argument (pointers and 32-bit shape
# words) is preloaded into SGPRs at wave launch, so no wave waits for a
# kernarg load before its first memory request.
KERNEL_FLAGS = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]

KERNELS = ["q4_matvec", "q4_matmul"]

# Host-only sanitizer build (g++ lines only).
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer",
             "-fno-sanitize-recover=undefined", "-g"]
SAN_LIB = BUILD / "san" / "libaxh.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build_kernels() -> dict[str, Path]:
    BUILD.mkdir(exist_ok=True)
    cos = {}
    for name in KERNELS:
        src = PKG / "csrc" / "kernels" / f"{name}.hip"
        out = BUILD / f"{name}.co"
        _run([HIPCC, *HIP_FLAGS, *KERNEL_FLAGS, "--offload-device-only", "--no-gpu-bundle-output",
              "-I", str(PKG / "csrc" / "kernels"), "-o", str(out), str(src)])
        cos[name] = out
    return cos


def build_runtime(cos: dict[str, Path], sanitize: bool = False) -> Path:
    rt = PKG / "csrc" / "runtime"
    embed_o = BUILD / "axh_embed.o"
    # The allocation-free entry point keeps its scratch in a __device__ array,
    # so its file is HIP (host code plus that array's device image).
    noalloc_o = BUILD / "axh_noalloc.o"
    _run([HIPCC, *HIP_FLAGS, "-fPIC", "-c", "-I", str(ROOT / "include"), "-I", str(rt),
          "-o", str(noalloc_o), str(rt / "axh_noalloc.hip")])
    _run(["gcc", "-c", f'-DAXH_Q4_MATVEC_CO="{cos["q4_matvec"]}"',
          f'-DAXH_Q4_MATMUL_CO="{cos["q4_matmul"]}"', "-o", str(embed_o),
          str(rt / "axh_embed.S")])
    out = SAN_LIB if sanitize else LIB
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix(".so.tmp")
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
        *(SAN_FLAGS if sanitize else []),
        "-D__HIP_PLATFORM_AMD__", "-I", str(ROCM / "include"), "-I", str(ROOT / "include"),
        "-I", str(rt),
        str(rt / "axh_runtime.cpp"), str(rt / "axh_ops.cpp"), str(rt / "axh_gguf.cpp"),
        str(PKG / "csrc" / "tune" / "axh_tune.cpp"), str(PKG / "csrc" / "tune" / "axh_winners.cpp"),
        str(PKG / "csrc" / "check" / "axh_check.cpp"),
        str(embed_o), str(noalloc_o),
        "-L", str(ROCM / "lib"), "-Wl,-rpath," + str(ROCM / "lib"), "-lamdhip64", "-pthread",
        "-o", str(tmp),
    ])
    os.replace(tmp, out)
    return out


def build_oracle(sanitize: bool = False) -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle"), *(["san"] if sanitize else [])])
    return ROOT / "oracle" / ("_san/liboracle.so" if sanitize else "liboracle.so")


def build_all() -> None:
    cos = build_kernels()
    build_runtime(cos)
    build_oracle()


def build_sanitized() -> tuple[Path, Path]:
    """The host code and the oracle with ASan + UBSan (separate outputs)."""
    cos = build_kernels()
    return build_runtime(cos, sanitize=True), build_oracle(sanitize=True)


if __name__ == "__main__":
    if "--sanitize" in sys.argv[1:]:
        lib, orc = build_sanitized()
        print(f"built {lib} and {orc}")
    else:
        build_all()
        print(f"built {LIB}")
    sys.exit(0)
