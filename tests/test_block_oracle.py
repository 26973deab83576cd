"""CPU check of the composed block-step oracle (oracle/block_ref.py): its
LoRA gradients are directional derivatives of L = sum(y * dY), checked by
central finite differences through the same oracle forward (f32, tiny
block).  This pins the backward wiring (gated residuals, layer_norm_mod,
GELU, out projection, attention, prologue, adapters) as a whole; each piece
is pinned on its own in test_oracle*.py."""
import numpy as np
import pytest

import block_ref
from block_case import make_case, oracle_mods


def _loss(case):
    y, _, _ = block_ref.block_step(case["x"], case["dy"], case["W"], case["H"], case["D"], case["cos"],
                                   case["sin"], case["axes"], case["scale"], bf16=False)
    return sum(float((y[k].astype(np.float64) * case["dy"][k]).sum()) for k in y)


@pytest.mark.parametrize("stream,target,part", [("img", "q", "a"), ("txt", "k", "b"), ("img", "v", "b"),
                                                 ("txt", "out", "a"), ("img", "out", "b")])
def test_block_lora_grads_directional_fd(stream, target, part):
    case = oracle_mods(make_case(C=256, H=2, T=8, rows=2, cols=4, F=512, r=4, bf16=False, seed=3))
    _, grads, _ = block_ref.block_step(case["x"], case["dy"], case["W"], case["H"], case["D"], case["cos"],
                                       case["sin"], case["axes"], case["scale"], bf16=False)
    g = grads[(stream, target)][0 if part == "a" else 1]
    P = case["W"][stream]["lora_" + part][target]
    rng = np.random.default_rng(7)
    d = rng.standard_normal(P.shape).astype(np.float32)
    P0 = P.copy()

    def central(h):
        case["W"][stream]["lora_" + part][target] = P0 + h * d
        lp = _loss(case)
        case["W"][stream]["lora_" + part][target] = P0 - h * d
        lm = _loss(case)
        case["W"][stream]["lora_" + part][target] = P0
        return (lp - lm) / (2 * h)

    # Richardson extrapolation cancels the h^2 term (large along q / k,
    # where the direction bends through the softmax)
    h = 0.05 * float(np.abs(P).mean()) / float(np.abs(d).mean())
    fd = (4 * central(h / 2) - central(h)) / 3
    an = float((g.astype(np.float64) * d).sum())
    print(stream, target, part, fd, an)
    assert abs(fd - an) <= 2e-3 * max(abs(an), 1e-3), (fd, an)


def _richardson(loss_at, h):
    central = lambda hh: (loss_at(hh) - loss_at(-hh)) / (2 * hh)
    return (4 * central(h / 2) - central(h)) / 3


@pytest.mark.parametrize("stream", ["txt", "img"])
def test_block_input_grad_directional_fd(stream):
    """want_dx: dL/dx of the double block (through the frozen qkv projection,
    the adapters, the first layer_norm_mod and the residuals) along a random
    direction."""
    case = oracle_mods(make_case(C=256, H=2, T=8, rows=2, cols=4, F=512, r=4, bf16=False, seed=3))
    _, grads, _ = block_ref.block_step(case["x"], case["dy"], case["W"], case["H"], case["D"], case["cos"],
                                       case["sin"], case["axes"], case["scale"], bf16=False, want_dx=True)
    d = np.random.default_rng(8).standard_normal(case["x"][stream].shape).astype(np.float32)
    x0 = case["x"][stream].copy()

    def loss_at(h):
        case["x"][stream] = x0 + h * d
        v = _loss(case)
        case["x"][stream] = x0
        return v

    fd = _richardson(loss_at, 0.02)
    an = float((grads[(stream, "x")].astype(np.float64) * d).sum())
    print(stream, fd, an)
    assert abs(fd - an) <= 2e-3 * max(abs(an), 1e-3), (fd, an)


def _single_loss(case):
    y = block_ref.single_block_step(case["x"], case["dy"], case["W"], case["H"], case["D"], case["cos"],
                                    case["sin"], case["axes"], case["scale"], bf16=False, want_dx=False)[0]
    return float((y.astype(np.float64) * case["dy"]).sum())


@pytest.mark.parametrize("what", [("to_in", "a"), ("to_in", "b"), ("to_out", "a"), ("to_out", "b"), ("x", None)])
def test_single_block_grads_directional_fd(what):
    """The single-stream block restatement: LoRA gradients of the fused to_in
    (through SwiGLU, attention and the prologue) and to_out, and the input
    gradient, as directional derivatives of L = sum(y * dY)."""
    from block_case import make_single_case, single_oracle_mods
    case = single_oracle_mods(make_single_case(C=256, H=2, T=8, rows=2, cols=4, r=4, bf16=False, seed=4))
    _, grads, _, dx = block_ref.single_block_step(case["x"], case["dy"], case["W"], case["H"], case["D"],
                                                  case["cos"], case["sin"], case["axes"], case["scale"],
                                                  bf16=False, want_dx=True)
    t, part = what
    if t == "x":
        P, g = case["x"], dx
    else:
        P, g = case["W"]["lora_" + part][t], grads[t][0 if part == "a" else 1]
    d = np.random.default_rng(9).standard_normal(P.shape).astype(np.float32)
    P0 = P.copy()

    def loss_at(h):
        P[...] = P0 + h * d
        v = _single_loss(case)
        P[...] = P0
        return v

    h = 0.05 * float(np.abs(P0).mean()) / float(np.abs(d).mean())
    fd = _richardson(loss_at, h)
    an = float((g.astype(np.float64) * d).sum())
    print(what, fd, an)
    assert abs(fd - an) <= 2e-3 * max(abs(an), 1e-3), (fd, an)
