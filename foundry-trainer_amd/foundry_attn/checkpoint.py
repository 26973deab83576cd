"""Checkpointed backward over a stack of blocks, on the MI355X path.

Mirrors ``checkpointed_backward`` (crates/foundry-spike/src/lib.rs:541-638):
the stages run forward once, keeping only each stage's inputs; the final
outputs are seeded by a loss; then, from the last stage back, each stage is
recomputed and run backward against the upstream gradient, giving the
gradient for the stage before it and the stage's LoRA gradients.

The reference recomputes every stage's attention forward in that second pass.
Here a stage may keep its attention output and LSE from the forward
(``save_attention``, ≈ 2·S·H·D + 4·H·S bytes per block: 28 MB at S=4608,
24x128 heads) and hand them to the recompute, which then skips the attention
forward: the backward recomputes P from the saved LSE, as it does anyway.
The result is identical to recomputing (the attention kernels are
deterministic), which the tests check bit for bit.

Stages take and return lists of tensors, as the reference's ``Stage.run``:
  DoubleStage   [txt, img] -> [txt, img]   (DoubleBlockLoRA)
  JoinStage     [txt, img] -> [joint]      (cat along tokens, txt first)
  SingleStage   [joint]    -> [joint]      (SingleBlockLoRA)
  SplitStage    [joint]    -> [txt, img]
"""
from __future__ import annotations

from typing import Callable, Dict, List, Optional, Sequence, Tuple

import torch

from .block import DoubleBlockLoRA, SingleBlockLoRA


class DoubleStage:
    def __init__(self, block: DoubleBlockLoRA):
        self.block = block

    def forward(self, inputs, keep_attention: bool):
        y, att = self.block.forward({"txt": inputs[0], "img": inputs[1]}, keep_attention=True) \
            if keep_attention else (self.block.forward({"txt": inputs[0], "img": inputs[1]}), None)
        return [y["txt"], y["img"]], att

    def backward(self, inputs, upstream, attention):
        y, g = self.block.forward_backward({"txt": inputs[0], "img": inputs[1]},
                                           {"txt": upstream[0], "img": upstream[1]}, want_dx=True,
                                           attention=attention)
        lora = {k: v for k, v in g.items() if k[1] != "x"}
        return [y["txt"], y["img"]], [g[("txt", "x")], g[("img", "x")]], lora

    def apply_adamw(self, grads, lr: float) -> None:
        self.block.apply_adamw(grads, lr)


class SingleStage:
    def __init__(self, block: SingleBlockLoRA):
        self.block = block

    def forward(self, inputs, keep_attention: bool):
        if keep_attention:
            y, att = self.block.forward(inputs[0], keep_attention=True)
            return [y], att
        return [self.block.forward(inputs[0])], None

    def backward(self, inputs, upstream, attention):
        y, g = self.block.forward_backward(inputs[0], upstream[0], want_dx=True, attention=attention)
        return [y], [g["x"]], {k: v for k, v in g.items() if k != "x"}

    def apply_adamw(self, grads, lr: float) -> None:
        self.block.apply_adamw(grads, lr)


class JoinStage:
    """cat([txt, img]) along tokens (throughput.rs:545-550 order)."""

    def __init__(self, txt_tokens: int):
        self.T = txt_tokens

    def forward(self, inputs, keep_attention: bool):
        return [torch.cat([inputs[0], inputs[1]], dim=0)], None

    def backward(self, inputs, upstream, attention):
        g = upstream[0]
        return None, [g[:self.T].contiguous(), g[self.T:].contiguous()], {}

    def apply_adamw(self, grads, lr: float) -> None:
        pass


class SplitStage(JoinStage):
    """joint -> [txt, img] (the final narrow of the klein forward)."""

    def forward(self, inputs, keep_attention: bool):
        j = inputs[0]
        return [j[:self.T].contiguous(), j[self.T:].contiguous()], None

    def backward(self, inputs, upstream, attention):
        return None, [torch.cat([upstream[0], upstream[1]], dim=0)], {}


def mse_seed(targets: Sequence[torch.Tensor]) -> Callable:
    """Seed of the reference's loss, sum over outputs of mean((y - t)^2)
    (mse, lib.rs:457-462): returns (loss, upstream gradients in each
    output's dtype), the loss accumulated in f32."""
    def seed(outputs: List[torch.Tensor]):
        loss = torch.zeros((), dtype=torch.float32, device=outputs[0].device)
        ups = []
        for y, t in zip(outputs, targets):
            d = y.float() - t.float()
            loss = loss + (d * d).mean()
            ups.append((d * (2.0 / d.numel())).to(y.dtype))
        return loss, ups
    return seed


def checkpointed_step(stages: Sequence, inputs: Sequence[torch.Tensor], seed: Callable,
                      save_attention: bool = True):
    """Forward through the stages keeping only their inputs (and, with
    save_attention, each block's attention output and LSE), seed the final
    outputs, then recompute and backpropagate stage by stage from the end.

    Returns (loss, input gradients, {stage index: that stage's LoRA grads})."""
    stage_inputs: List[List[torch.Tensor]] = []
    saved: List[Optional[Tuple[torch.Tensor, torch.Tensor]]] = []
    cur = list(inputs)
    for st in stages:
        stage_inputs.append(cur)
        out, att = st.forward(cur, save_attention)
        cur = [t.clone() for t in out]  # block outputs live in per-block buffers
        saved.append(att)
    loss, upstream = seed(cur)
    grads: Dict[int, dict] = {}
    for k in range(len(stages) - 1, -1, -1):
        _, in_grads, g = stages[k].backward(stage_inputs[k], upstream, saved[k])
        grads[k] = g
        upstream = [t.clone() for t in in_grads]
    return loss, upstream, grads


def apply_adamw(stages: Sequence, grads: Dict[int, dict], lr: float = 1e-3) -> None:
    """One AdamW step on every stage's LoRA factors (Session::step,
    throughput.rs:784-803)."""
    for k, st in enumerate(stages):
        if grads.get(k):
            st.apply_adamw(grads[k], lr)
