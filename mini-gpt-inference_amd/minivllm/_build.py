"""In-tree build of libminivllm_hip.so (HIP C++ for gfx950) and its PyTorch
binding.

Every ``csrc/*.hip`` source is compiled with hipcc into an object under
``mini-gpt-inference_amd/_build/`` (in parallel), then linked into
``minivllm/_native/libminivllm_hip.so``. The library exports the C ABI
declared in ``include/minivllm_hip.h``.

``csrc/torch_ops.cpp`` (host C++, no device code) is then compiled with the
host compiler against PyTorch's headers into the extension module
``minivllm/_native/_hip_ops<ext>``, which links the library by ``$ORIGIN``.

Packed-FP32 instructions are disabled on the device pass
(``-target-feature -packed-fp32-ops``); hipcc's host pass warns that it does
not know the feature, which is harmless.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
SRC_ROOT = PKG_DIR.parent
CSRC = SRC_ROOT / "csrc"
INCLUDE = SRC_ROOT.parent / "include"
OBJ_DIR = SRC_ROOT / "_build"
LIB_DIR = PKG_DIR / "_native"
LIB_NAME = "libminivllm_hip.so"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# Matrix-core accumulators in ordinary VGPRs: without this the compiler keeps
# the prefill kernel's MFMA results in AGPRs and copies them back and forth
# for the softmax (64 v_accvgpr moves per key tile).
MFMA_FLAGS = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
MFMA_SOURCES = {"paged_prefill.hip"}


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def ops_path() -> Path:
    import sysconfig

    return LIB_DIR / ("_hip_ops" + sysconfig.get_config_var("EXT_SUFFIX"))


def _hipcc() -> str:
    exe = shutil.which("hipcc")
    if exe:
        return exe
    fallback = Path("/opt/rocm/bin/hipcc")
    if fallback.exists():
        return str(fallback)
    raise RuntimeError("hipcc not found: a ROCm toolchain is required to build libminivllm_hip.so")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links the shared library.

    Always recompiles (this is the "does it build" check). Returns the path of
    the library.
    """
    hipcc = _hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    includes = [f"-I{INCLUDE}", f"-I{CSRC}"]

    def compile_one(src: Path) -> Path:
        obj = OBJ_DIR / (src.stem + ".o")
        extra = MFMA_FLAGS if src.name in MFMA_SOURCES else []
        _run([hipcc, *HIP_FLAGS, *extra, *includes, "-c", str(src), "-o", str(obj)], verbose)
        return obj

    workers = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(compile_one, sources))

    out = library_path()
    tmp = out.with_name(out.name + f".tmp{os.getpid()}")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)],
         verbose)
    os.replace(tmp, out)
    build_torch_ops(verbose)
    return out


def build_torch_ops(verbose: bool = False) -> Path:
    """Compiles csrc/torch_ops.cpp into the _hip_ops extension module (needs
    libminivllm_hip.so in place: it links against it)."""
    import sysconfig

    import torch

    cxx = shutil.which("g++") or shutil.which("c++")
    if not cxx:
        raise RuntimeError("no host C++ compiler (g++) for the PyTorch binding")
    tdir = Path(torch.__file__).resolve().parent
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    out = ops_path()
    tmp = out.with_name(out.name + f".tmp{os.getpid()}")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared",
          "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_hip_ops",
          "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
          f"-I{sysconfig.get_paths()['include']}", f"-I{rocm / 'include'}", f"-I{INCLUDE}",
          str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
          f"-L{tdir / 'lib'}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
          f"-L{LIB_DIR}", "-lminivllm_hip", "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
