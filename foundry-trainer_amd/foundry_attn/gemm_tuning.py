"""Tuned hipBLASLt / rocBLAS solutions for the blocks' frozen-linear GEMMs on
MI355X (gfx950).

The frozen base linears of the double and single blocks are library GEMMs
(``torch.mm``).  PyTorch's TunableOp can pick, per GEMM shape, the fastest
hipBLASLt or rocBLAS solution as measured on the GPU itself.
``gemm_tuning_gfx950.csv`` holds that choice for every GEMM shape of the c4
double block and the klein single block (forward, dX, both streams, with the
adapter-carrying K / N extensions of both blocks), measured on an MI355X.
Its Validator rows name the PyTorch, HIP, hipBLASLt and rocBLAS versions it
was measured with.

``enable()`` loads it read-only, unless the process already runs TunableOp
its own way (then it changes nothing):
- no tuning happens at run time;
- shapes not in the file keep the default heuristic;
- TunableOp refuses a file whose validators do not match the running
  libraries, which leaves the default path in place.

Measured on one box: the single block step 3.73 -> 3.41 ms, the double block
3.92 -> 3.87 ms; after the double block's adapters moved into its GEMMs, the
rows for those extended shapes took its graph-replayed step from about
3.35 to 3.2 ms.  This switches TunableOp on for the whole process (read-only),
which affects only GEMM shapes listed in the file.
"""
from __future__ import annotations

import os
import tempfile

TUNING_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_tuning_gfx950.csv")
_state = None


def enable(path: str = TUNING_FILE) -> bool:
    """Load the tuned GEMM solutions (once per process) on a gfx950 device.
    Returns whether TunableOp now serves them."""
    global _state
    if _state is not None:
        return _state
    _state = False
    import torch
    if not torch.cuda.is_available() or not os.path.exists(path):
        return False
    if not torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName.startswith("gfx950"):
        return False
    t = torch.cuda.tunable
    if t.is_enabled():  # the caller runs TunableOp its own way: leave it alone
        return False
    t.enable(True)
    t.tuning_enable(False)
    t.record_untuned_enable(False)
    # results TunableOp writes at exit go to a scratch path, never over the packaged file
    t.set_filename(os.path.join(tempfile.gettempdir(), f"foundry_tunableop_{os.getpid()}.csv"), False)
    _state = bool(t.read_file(path))
    if not _state:
        t.enable(False)
    return _state
