"""GEMM kernel selection for the layer's hipBLASLt / rocBLAS calls.

The layer's projections, MLP and lm_head stay library GEMMs. PyTorch's
TunableOp (`torch.cuda.tunable`) can time every hipBLASLt and rocBLAS solution
for a GEMM shape and keep the fastest. `tuning/gemm_mi355x.csv` holds such
selections, measured on MI355X for the CyFA-400M prefill (B=8 x T=2048 and the
B=64 x T=2048 decode prompt) and decode (B=64) shapes. Its validator lines pin
the PyTorch, HIP, hipBLASLt and rocBLAS versions and the gfx950 target; with
other versions TunableOp ignores the file and every GEMM takes the library's
default solution, as it does for shapes the file does not list.

`python bench.py --tune-gemms <file>` re-measures the selections.
"""

import os
import tempfile
from pathlib import Path

import torch

DEFAULT_FILE = Path(__file__).with_name("tuning") / "gemm_mi355x.csv"


def use_tuned_gemms(path=None):
    """Route GEMMs through the selections in `path` (no tuning at run time).

    Returns True when the file was read. TunableOp writes its results file when
    the process exits, so its output name is pointed at a scratch path and the
    committed file is never rewritten.
    """
    path = Path(path or DEFAULT_FILE)
    if not torch.cuda.is_available() or not path.exists():
        return False
    tunable = torch.cuda.tunable
    tunable.enable(True)
    tunable.tuning_enable(False)
    ok = tunable.read_file(str(path))
    tunable.set_filename(os.path.join(tempfile.gettempdir(), "cyfa_tunableop_%d.csv"))
    return bool(ok)


def tune_gemms(path):
    """Time the solutions of every GEMM shape run from now on and write the
    selections to `path` at exit (`%d` in the name becomes the device index)."""
    tunable = torch.cuda.tunable
    tunable.enable(True)
    tunable.tuning_enable(True)
    tunable.set_max_tuning_duration(30)
    tunable.set_filename(str(path))
