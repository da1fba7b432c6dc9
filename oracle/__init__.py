"""CPU oracle for the QSA sparse-attention path.

TEST INFRASTRUCTURE ONLY. This package restates the reference algorithm in
eager PyTorch on the CPU so the HIP kernels can be checked against it. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and there only as the reference the results are
compared with or as the timed CPU baseline. The product path (``qsa_vllm_amd``) never imports it and fails
loudly when its HIP library is missing.
"""

from .qsa_oracle import *  # noqa: F401,F403
from .qsa_oracle import __all__ as _path_all
from .qsa_prepare_oracle import norm_rope, prepare, rotary_cache_table  # noqa: F401
from . import hybrid_oracle as hybrid  # noqa: F401

__all__ = list(_path_all) + ["norm_rope", "prepare", "rotary_cache_table", "hybrid"]
