"""GPU checks of the checkpointed stack step (foundry_attn/checkpoint.py,
the reference's checkpointed_backward, lib.rs:541-638) over a small klein
stack: double block -> cat(txt, img) -> single block -> split, seeded by the
reference's MSE loss.

1. Reusing each block's saved attention output and LSE in the recompute
   gives the same loss and gradients, bit for bit, as recomputing the
   attention forward.
2. The stack's LoRA gradients and input gradients match the oracle composed
   from block_ref.block_step and block_ref.single_block_step (the same
   chain rule run on the CPU), at the north-star gate (bf16 rel-L2 1e-2 and
   max-abs 2e-2 x max(1, peak); f32 rel-L2 1e-4).
"""
import numpy as np
import pytest
import torch

import block_ref
import oracle
from block_case import make_case, make_single_case, oracle_mods, single_oracle_mods
from foundry_attn import checkpoint as ck
from helpers import check_gate
from test_block_gpu import dev, device_block, device_single_block, host

pytestmark = pytest.mark.gpu

T, ROWS, COLS, C, H, R = 8, 4, 8, 256, 2, 4


def build(dtype):
    bf = dtype == torch.bfloat16
    dcase = oracle_mods(make_case(C=C, H=H, T=T, rows=ROWS, cols=COLS, r=R, bf16=bf, seed=21))
    scase = single_oracle_mods(make_single_case(C=C, H=H, T=T, rows=ROWS, cols=COLS, r=R, bf16=bf, seed=22))
    rng = np.random.default_rng(23)
    rnd = oracle.bf16_round if bf else (lambda a: a.astype(np.float32))
    targets = [rnd(rng.standard_normal((T, C)).astype(np.float32)),
               rnd(rng.standard_normal((ROWS * COLS, C)).astype(np.float32))]
    return dcase, scase, targets


def stack(dcase, scase, dtype):
    return [ck.DoubleStage(device_block(dcase, dtype)), ck.JoinStage(T),
            ck.SingleStage(device_single_block(scase, dtype)), ck.SplitStage(T)]


def oracle_stack(dcase, scase, targets, bf):
    rnd = oracle.bf16_round if bf else (lambda a: np.asarray(a, np.float32))
    dargs = (dcase["W"], dcase["H"], dcase["D"], dcase["cos"], dcase["sin"], dcase["axes"], dcase["scale"])
    sargs = (scase["W"], scase["H"], scase["D"], scase["cos"], scase["sin"], scase["axes"], scase["scale"])
    zeros = {k: np.zeros_like(v) for k, v in dcase["x"].items()}
    yd = block_ref.block_step(dcase["x"], zeros, *dargs, bf16=bf)[0]
    joint = np.concatenate([yd["txt"], yd["img"]])
    ys = block_ref.single_block_step(joint, np.zeros_like(joint), *sargs, bf16=bf, want_dx=False)[0]
    outs = [ys[:T], ys[T:]]
    loss = sum(float(np.mean((o.astype(np.float64) - t) ** 2)) for o, t in zip(outs, targets))
    ups = [rnd((2.0 * (o.astype(np.float64) - t) / o.size).astype(np.float32)) for o, t in zip(outs, targets)]
    _, sgrads, _, dxj = block_ref.single_block_step(joint, np.concatenate(ups), *sargs, bf16=bf, want_dx=True)
    _, dgrads, _ = block_ref.block_step(dcase["x"], {"txt": dxj[:T], "img": dxj[T:]}, *dargs, bf16=bf,
                                        want_dx=True)
    return loss, dgrads, sgrads


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_saved_attention_equals_recompute(dtype):
    dcase, scase, targets = build(dtype)
    inputs = [dev(dcase["x"]["txt"], dtype), dev(dcase["x"]["img"], dtype)]
    seed = ck.mse_seed([dev(t, dtype) for t in targets])
    results = []
    for save in (False, True):
        st = stack(dcase, scase, dtype)
        loss, in_grads, grads = ck.checkpointed_step(st, inputs, seed, save_attention=save)
        torch.cuda.synchronize()
        results.append((float(loss), [g.clone() for g in in_grads],
                        {k: {kk: tuple(t.clone() for t in vv) for kk, vv in g.items()} for k, g in grads.items()}))
    (l0, x0, g0), (l1, x1, g1) = results
    assert l0 == l1
    for a, b in zip(x0, x1):
        assert torch.equal(a, b)
    assert g0.keys() == g1.keys()
    for k in g0:
        for kk in g0[k]:
            for a, b in zip(g0[k][kk], g1[k][kk]):
                assert torch.equal(a, b), (k, kk)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_checkpointed_stack_matches_oracle(dtype):
    bf = dtype == torch.bfloat16
    dcase, scase, targets = build(dtype)
    st = stack(dcase, scase, dtype)
    inputs = [dev(dcase["x"]["txt"], dtype), dev(dcase["x"]["img"], dtype)]
    loss, in_grads, grads = ck.checkpointed_step(st, inputs, ck.mse_seed([dev(t, dtype) for t in targets]))
    torch.cuda.synchronize()
    wloss, wd, ws = oracle_stack(dcase, scase, targets, bf)
    rl = abs(float(loss) - wloss) / wloss
    print(f"  loss: rel={rl:.2e}", flush=True)
    assert rl <= (1e-2 if bf else 1e-4)
    for name, got in zip(("txt", "img"), in_grads):
        check_gate(f"dx.{name}", host(got), wd[(name, "x")], bf)
    for key, (da, db) in grads[0].items():
        check_gate(f"double {key} dA", host(da), wd[key][0], bf)
        check_gate(f"double {key} dB", host(db), wd[key][1], bf)
    for t, (da, db) in grads[2].items():
        check_gate(f"single {t} dA", host(da), ws[t][0], bf)
        check_gate(f"single {t} dB", host(db), ws[t][1], bf)
    ck.apply_adamw(st, grads)
    torch.cuda.synchronize()
    assert st[0].block.step_count == 1 and st[2].block.step_count == 1


def test_stack_training_lowers_the_loss():
    """Training as the reference's harness does (MSE seed, checkpointed
    backward, AdamW on the LoRA factors; Session::step, throughput.rs:784-803)
    for 20 steps on a fixed target lowers the loss steadily."""
    dcase, scase, targets = build(torch.bfloat16)
    st = stack(dcase, scase, torch.bfloat16)
    inputs = [dev(dcase["x"]["txt"], torch.bfloat16), dev(dcase["x"]["img"], torch.bfloat16)]
    seed = ck.mse_seed([dev(t, torch.bfloat16) for t in targets])
    losses = []
    for _ in range(20):
        loss, _, grads = ck.checkpointed_step(st, inputs, seed)
        ck.apply_adamw(st, grads, lr=3e-3)
        losses.append(float(loss))
    print("  losses", [round(v, 4) for v in losses[::4]], flush=True)
    assert all(np.isfinite(losses))
    assert losses[-1] < 0.8 * losses[0]
    assert sum(b < a for a, b in zip(losses, losses[1:])) >= 18
