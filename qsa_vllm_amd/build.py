"""Build ``libqsa_hip.so`` (the C-ABI HIP library) in-tree for gfx950.

Usage: ``python -m qsa_vllm_amd.build`` or ``qsa_vllm_amd.build.build()``.
Every HIP source is compiled to an object with hipcc in parallel, then linked
into one shared library next to this file. No torch types cross that library's
boundary. The torch-op layer over it (``csrc/torch_ops.cpp``, host C++ against
PyTorch's headers) is a second library, ``libqsa_torch_ops.so``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libqsa_hip.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
OBJ_DIR = PACKAGE_DIR / "_build"

SOURCES = ["qsa_errors.hip", "prepare.hip", "topk.hip", "indexer.hip", "sparse_attn.hip",
           "sparse_attn_wide.hip", "hybrid.hip"]

# Packed fp32 VALU ops are disabled: the kernels get no benefit from them and
# some of their forms are not trusted on this hardware.
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libqsa_hip.so")
    return path


def _compile(src: Path, obj: Path, extra: list[str]) -> None:
    cmd = [hipcc(), *HIP_FLAGS, *extra, "-I", str(INCLUDE), "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")


TORCH_OPS_SOURCE = "torch_ops.cpp"
TORCH_OPS_LIB = PACKAGE_DIR / "libqsa_torch_ops.so"


def _torch_paths() -> tuple[Path, bool]:
    import torch

    return Path(torch.__file__).resolve().parent, bool(torch._C._GLIBCXX_USE_CXX11_ABI)


def build_torch_ops(verbose: bool = False) -> Path:
    """Compile the torch-op layer (host C++ against PyTorch's headers, linked
    against ``libqsa_hip.so``) into ``libqsa_torch_ops.so``."""
    torch_dir, cxx11_abi = _torch_paths()
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    cxx = shutil.which("g++") or "g++"
    tmp = TORCH_OPS_LIB.with_name(TORCH_OPS_LIB.name + f".tmp{os.getpid()}")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(cxx11_abi)}",
           "-I", str(INCLUDE), "-I", str(torch_dir / "include"),
           "-I", str(torch_dir / "include" / "torch" / "csrc" / "api" / "include"),
           "-I", str(rocm / "include"),
           str(CSRC / TORCH_OPS_SOURCE), "-o", str(tmp),
           "-L", str(PACKAGE_DIR), "-lqsa_hip", "-L", str(torch_dir / "lib"),
           "-lc10", "-lc10_hip", "-ltorch_cpu", "-L", str(rocm / "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build of {TORCH_OPS_LIB.name} failed:\n{proc.stderr}")
    os.replace(tmp, TORCH_OPS_LIB)
    if verbose:
        print(f"built {TORCH_OPS_LIB}", file=sys.stderr)
    return TORCH_OPS_LIB


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every HIP source and link ``libqsa_hip.so``, then the torch-op
    layer ``libqsa_torch_ops.so``; returns the HIP library's path."""
    extra = list(extra_flags or [])
    OBJ_DIR.mkdir(exist_ok=True)
    objs = [OBJ_DIR / (Path(s).stem + ".o") for s in SOURCES]
    jobs = max(1, min(len(SOURCES), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_compile, CSRC / s, o, extra) for s, o in zip(SOURCES, objs)]
        for f in futures:
            f.result()
    tmp = LIB_PATH.with_name(LIB_NAME + f".tmp{os.getpid()}")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {LIB_NAME} failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    build_torch_ops(verbose)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
