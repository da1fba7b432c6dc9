"""``torch.ops.yulan_qsa_kernels``: loads the torch-op layer ``libqsa_torch_ops.so``.

The ops are defined and implemented in C++ (``csrc/torch_ops.cpp``), as the
reference registers its own (ops/csrc/topk.cu:548-557): ``topk`` and
``topk_expand`` with the reference schemas verbatim, plus this library's
indexer preparation, scoring, whole-selection, sparse attention and helper ops
in the same namespace. Each validates dtypes, devices and layouts (a
RuntimeError, like the reference's ``TORCH_CHECK`` / ``data_ptr<T>()``
failures) and calls the C ABI of ``libqsa_hip.so`` on the current stream of
the tensors' device. Nothing synchronises.

Loading fails loudly when the library is missing: there is no other
implementation of these ops. The helpers below serve the ctypes calls of the
hybrid model's layer kernels (``hybrid_layers.py``).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

from .. import _lib

_NS = "yulan_qsa_kernels"
_TORCH_OPS_LIB = Path(__file__).resolve().parents[1] / "libqsa_torch_ops.so"
_lock = threading.Lock()
_loaded = False


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _stride(t, d):
    """Stride of dim d, 0 for a size-1 dim (never used to address memory; views
    may carry any value there)."""
    return 0 if t.size(d) == 1 else t.stride(d)


def _require(cond, msg):
    if not cond:
        raise RuntimeError(f"{_NS}: {msg}")


def _on_gpu(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        _require(t.is_cuda, f"expected a GPU tensor, got device {t.device}")
        if dev is None:
            dev = t.device
        _require(t.device == dev, "all tensors must be on the same device")
    return dev


def _dtype(t, dtype, name):
    _require(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")


def _vector(t, dtype, name, min_len=None):
    _dtype(t, dtype, name)
    _require(t.dim() == 1, f"{name} must be 1-D")
    _require(t.numel() <= 1 or t.stride(0) == 1, f"{name} must be contiguous")
    if min_len is not None:
        _require(t.numel() >= min_len, f"{name} has {t.numel()} entries, need {min_len}")


def _workspace(nbytes, device):
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def register() -> None:
    """Load ``libqsa_torch_ops.so`` once per process (it defines the ops and
    registers their GPU and Meta kernels)."""
    global _loaded
    if _loaded:
        return
    with _lock:
        if _loaded:
            return
        _lib.load()  # the HIP library first: the op layer links against it
        if not _TORCH_OPS_LIB.exists():
            raise _lib.QSAError(
                f"{_TORCH_OPS_LIB} is missing: build it with `python -m qsa_vllm_amd.build` "
                "(the QSA ops have no other implementation)")
        torch.ops.load_library(str(_TORCH_OPS_LIB))
        _loaded = True


register()
