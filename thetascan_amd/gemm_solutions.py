"""Measured library-GEMM solutions for the mixer's projections on MI355X.

The projection GEMMs around the memory (the stacked q/k/v/gate projection,
the output projection and its input gradient) are plain library GEMMs
(hipBLASLt / rocBLAS).  The libraries pick a solution by heuristic; for the
shapes of a B8 x T4096, d_model 512 step, PyTorch's TunableOp measured
faster solutions than the heuristic's choice on gfx950 (the q/k/v/gate
projection forward, the output projection forward and its input gradient;
the split-K weight gradients are batched fp32-output GEMMs that TunableOp does
not cover).  ``data/gemm_solutions_gfx950.csv`` is that measurement, in
TunableOp's file format, headed by the library versions it was taken with.

:func:`use_measured_gemms` makes PyTorch take those solutions: TunableOp is
switched on with tuning off, so shapes in the table replay their recorded
solution and every other shape keeps the library heuristic; nothing is timed
or explored at run time.  A table whose versions differ from the running
libraries is not loaded (the heuristics stay in force).  The selection changes
which library kernel computes a GEMM, not what it computes: results agree to
the rounding of the bf16 outputs.
"""
from __future__ import annotations

import csv
from pathlib import Path

TABLE = Path(__file__).resolve().parent / "data" / "gemm_solutions_gfx950.csv"


def read_table(path: Path | str = TABLE) -> tuple[dict[str, str], list[tuple[str, str, str, float]]]:
    """(validators, entries) of a TunableOp results file: validators map a
    library to its version; entries are (op, problem, solution, ms)."""
    validators: dict[str, str] = {}
    entries: list[tuple[str, str, str, float]] = []
    with open(path, newline="") as f:
        for row in csv.reader(f):
            if not row:
                continue
            if row[0] == "Validator":
                validators[row[1]] = row[2]
            elif len(row) >= 4:
                entries.append((row[0], row[1], row[2], float(row[3])))
    return validators, entries


def use_measured_gemms(enable: bool = True, path: Path | str = TABLE) -> bool:
    """Replay the measured GEMM solutions (``enable``) or return to the
    library heuristics.  Returns whether the table is in force: False when
    its library versions differ from the running ones or no GPU is present."""
    import torch

    tunable = torch.cuda.tunable
    if not enable:
        tunable.enable(False)
        return False
    if not torch.cuda.is_available():
        return False
    want, _ = read_table(path)
    have = dict(tunable.get_validators())
    if any(have.get(k) != v for k, v in want.items()):
        tunable.enable(False)
        return False
    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    tunable.set_filename(str(path))
    if not tunable.read_file(str(path)):
        tunable.enable(False)
        return False
    return True


def in_force() -> bool:
    """Whether PyTorch currently replays measured GEMM solutions."""
    import torch

    return bool(torch.cuda.tunable.is_enabled()) and not torch.cuda.tunable.tuning_is_enabled()
