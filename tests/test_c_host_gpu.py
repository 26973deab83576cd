"""The ABI from a plain-C host: tests/c_host/attn_c_host (built by
__graft_entry__.build()) allocates device buffers with the HIP runtime, runs
fa_attn_fwd / fa_attn_bwd through include/foundry_attn.h alone, and checks
the results against the C oracle at the parity gates (bf16 ragged + masked,
D = 64, the f32 c1 shape, an 8-wave shape, a masked range-split shape with
its forward workspace) plus the ABI's error reporting.
It runs as a child process of this test."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_host", "attn_c_host")


def test_c_host_attention_parity():
    assert os.path.exists(EXE), "tests/c_host/attn_c_host is not built: run __graft_entry__.build()"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=110)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASSED (0 failures)" in r.stdout
