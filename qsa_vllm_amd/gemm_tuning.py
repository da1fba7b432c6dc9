"""Library GEMM choices for the hybrid decoder's projection shapes on gfx950.

The hybrid decoder's projections, MLPs and LM head are plain library GEMMs
(hipBLASLt / rocBLAS through ``torch``). PyTorch's TunableOp can time every
solution both libraries offer for a shape and record the fastest;
``gemm_tuning_gfx950.csv`` holds those records for the serving shapes (the
8304-token mixed batch, the 112-token decode batch and the LM-head rows),
written on one MI355X by::

    python -m qsa_vllm_amd.gemm_tuning

The file starts with validator lines (PyTorch, HIP, hipBLASLt and rocBLAS
versions, GPU architecture). PyTorch rejects the whole file on any other
software stack, and every GEMM then runs the libraries' own choice, as without
it. Shapes the file does not name run the libraries' own choice too: nothing is
timed at run time.
"""

from __future__ import annotations

import argparse
from pathlib import Path

TUNING_FILE = Path(__file__).with_name("gemm_tuning_gfx950.csv")


def enable_tuned_gemms(path: Path | str = TUNING_FILE) -> bool:
    """Route torch's GEMMs through TunableOp with the recorded choices and no
    tuning. Returns whether the file was read and accepted; when it was not,
    TunableOp is switched off again."""
    import torch.cuda.tunable as tunable

    path = Path(path)
    if not path.is_file():
        return False
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    tunable.set_filename(str(path))
    tunable.enable(True)
    if not tunable.read_file(str(path)):
        tunable.enable(False)
        return False
    return True


def disable_tuned_gemms() -> None:
    """Back to the libraries' own GEMM choices."""
    import torch.cuda.tunable as tunable

    tunable.enable(False)


def tune(out: Path) -> None:
    """Times every library solution for the serving shapes of the hybrid
    decoder (one mixed step, one decode step) and records the fastest in
    `out`, which PyTorch writes when the process exits."""
    import torch

    import torch.cuda.tunable as tunable

    from .hybrid import make_serving_hybrid_workload

    out.parent.mkdir(parents=True, exist_ok=True)
    if out.exists():
        out.unlink()
    tunable.set_filename(str(out))
    tunable.tuning_enable(True)
    tunable.enable(True)
    wl = make_serving_hybrid_workload(torch.device("cuda:0"))
    wl.model.forward(wl.build())
    wl.model.forward(wl.build_decode())
    torch.cuda.synchronize()
    print(f"tuned {len(tunable.get_results())} GEMM shapes; results go to {out} at exit",
          flush=True)


def main() -> None:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--out", type=Path, default=TUNING_FILE)
    tune(p.parse_args().out)


if __name__ == "__main__":
    main()
