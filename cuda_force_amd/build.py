"""Build the native parts in-tree.

* ``libcudaforge_hip.so`` - every HIP kernel plus the C ABI declared in
  ``include/cudaforge_hip.h``, compiled with hipcc for gfx950 only.
* ``_C*.so`` - the PyTorch dispatcher shim registering the ``cudaforge::``
  operators; plain C++ against the torch headers, linked to the library above
  with an ``$ORIGIN`` rpath.

Run ``python -m cuda_force_amd.build`` (or ``__graft_entry__.build()``). The
reference builds its extension through setup.py + CMake with nvcc
(setup.py:25-93, cuda/CMakeLists.txt:46-102); this tree needs neither: two
compiler invocations per artefact, run in parallel.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"

HIP_SOURCES = (
    "cf_runtime.hip",
    "cf_quant.hip",
    "cf_norm.hip",
    "cf_softmax.hip",
    "cf_reduce.hip",
    "cf_activations.hip",
    "cf_lora.hip",
    "cf_lora_fused.hip",
    "cf_lora_bwd.hip",
    "cf_lora_f32.hip",
    "cf_matmul_f32.hip",
    "cf_scheduler.hip",
    "cf_paged_attention.hip",
    "cf_tensor_core.hip",
    "cf_matmul_fp8.hip",
    "cf_attention.hip",
)

# Per-source additions. The fused LoRA kernel accumulates in VGPRs: the
# compiler's AGPR accumulator allocation rotates registers every K-step.
# (cf_matmul_fp8.hip must not take this flag: its one-wave-per-SIMD kernel
# keeps 256 accumulators per lane in the accumulation registers.)
HIPCC_EXTRA_FLAGS = {
    "cf_lora_fused.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
}

HIP_LIBRARY = PACKAGE_DIR / "libcudaforge_hip.so"
OFFLOAD_ARCH = "gfx950"

# -packed-fp32-ops keeps the compiler from emitting packed fp32 VALU ops
# (v_pk_add/mul/fma_f32), which this hardware pool has miscomputed
# intermittently. No -ffast-math: the quantiser relies on IEEE division and
# the default correctly-rounded sqrt. -fvisibility=hidden: only the C ABI
# (declared default-visible in include/cudaforge_hip.h) is exported.
HIPCC_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-fvisibility-inlines-hidden",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    return str(candidate) if candidate.exists() else "hipcc"


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            "build step failed:\n  " + " ".join(cmd) + "\n" + result.stdout + result.stderr
        )


def extension_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def torch_extension_path() -> Path:
    return PACKAGE_DIR / f"_C{extension_suffix()}"


def build_hip_library(jobs: int = 8) -> Path:
    """Compile every .hip source and link libcudaforge_hip.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()

    def compile_one(name: str) -> Path:
        obj = BUILD_DIR / (Path(name).stem + ".o")
        extra = HIPCC_EXTRA_FLAGS.get(name, ())
        _run([hipcc, *HIPCC_FLAGS, *extra, "-c", str(CSRC / name), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objects = list(pool.map(compile_one, HIP_SOURCES))
    tmp = HIP_LIBRARY.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objects)])
    os.replace(tmp, HIP_LIBRARY)
    return HIP_LIBRARY


def build_torch_extension() -> Path:
    """Compile the dispatcher shim against the installed torch."""
    import torch.utils.cpp_extension as cpp_ext

    BUILD_DIR.mkdir(exist_ok=True)
    includes = cpp_ext.include_paths(device_type="cuda")
    lib_dirs = cpp_ext.library_paths(device_type="cuda")
    python_include = sysconfig.get_paths()["include"]
    out = torch_extension_path()
    tmp = out.with_name(out.name + ".tmp")
    abi = int(getattr(__import__("torch")._C, "_GLIBCXX_USE_CXX11_ABI", True))
    cmd = [
        "g++",
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-parameter",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-I{python_include}",
        f"-I{REPO_ROOT / 'include'}",
        *[f"-I{p}" for p in includes],
        str(CSRC / "torch_ops.cpp"),
        "-o",
        str(tmp),
        f"-L{PACKAGE_DIR}",
        "-lcudaforge_hip",
        *[f"-L{p}" for p in lib_dirs],
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_hip",
        "-ltorch_python",
        "-Wl,-rpath,$ORIGIN",
        *[f"-Wl,-rpath,{p}" for p in lib_dirs],
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_hip_library()
    build_torch_extension()


if __name__ == "__main__":
    build_all()
    print(f"built {HIP_LIBRARY.name} and {torch_extension_path().name}", file=sys.stderr)
