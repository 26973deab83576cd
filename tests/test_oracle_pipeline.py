"""The oracle composed into the reference fixture's whole pipeline (double
block, single block, MSE loss, backward to the inputs; gen_block.py:170-360)
against the fixture itself.

This pins, with reference data, the oracle pieces no single-op fixture
covers: the SwiGLU forward and backward, the LN-mod backward, the gated
residual's backward, and the frozen linears' input gradients, all of which
grad/inputs/{img,txt} depends on.
"""
import numpy as np
import pytest

import fixture_ref
from helpers import load_pipeline_golden, rel_l2

ACTS = ["double.txt_norm1", "double.img_norm1", "double.q", "double.k", "double.attn_img",
        "double.img_post_attn", "double.img_out", "double.txt_out", "single.norm1", "single.q",
        "single.k", "single.attn", "single.mlp", "single.out", "output/img", "output/txt", "loss"]
GRADS = ["grad/inputs/img", "grad/inputs/txt"] + [
    f"grad/{lin}.lora_{p}" for lin in fixture_ref.LORA_LINEARS for p in ("a", "b")]


@pytest.fixture(scope="module")
def fp32():
    f = load_pipeline_golden("fp32")
    return f, fixture_ref.pipeline(f)


def test_pipeline_fp32_forward_matches_fixture(fp32):
    f, (acts, _) = fp32
    for k in ACTS:
        assert rel_l2(np.reshape(acts[k], f[k].shape), f[k]) <= 5e-6, k


def test_pipeline_fp32_gradients_match_fixture(fp32):
    f, (_, grads) = fp32
    for k in GRADS:
        assert rel_l2(grads[k], f[k]) <= 5e-6, k


def test_pipeline_bf16_matches_fixture():
    """bf16: the oracle rounds each op result once; PyTorch's bf16 sequence
    differs in a few places (the gated residual's product), so the gate is
    the bf16 rel-L2 one.  The double block up to its attention output is
    bit-exact."""
    f = load_pipeline_golden("bf16")
    acts, grads = fixture_ref.pipeline(f, bf16=True)
    for k in ("double.txt_norm1", "double.img_norm1", "double.q", "double.k", "double.attn_img"):
        assert rel_l2(np.reshape(acts[k], f[k].shape), f[k]) == 0.0, k
    for k in ACTS:
        assert rel_l2(np.reshape(acts[k], f[k].shape), f[k]) <= 1e-2, k
    for k in GRADS:
        assert rel_l2(grads[k], f[k]) <= 1e-2, k


@pytest.mark.parametrize("mutant", ["swiglu_swap", "ln_drop_proj"])
def test_planted_mistakes_miss_the_fixture(mutant):
    """A swapped SwiGLU gradient or an LN-mod gradient without its projection
    term misses grad/inputs by far more than the gate (>= 1e-3 vs 5e-6)."""
    f = load_pipeline_golden("fp32")
    _, grads = fixture_ref.pipeline(f, mutate=mutant)
    assert rel_l2(grads["grad/inputs/img"], f["grad/inputs/img"]) > 1e-3
    assert rel_l2(grads["grad/inputs/txt"], f["grad/inputs/txt"]) > 1e-3
