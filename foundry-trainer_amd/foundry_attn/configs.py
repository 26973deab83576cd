"""The workload shapes of the attention hot path (one per benchmark config).

c1  f32 parity case: B1 H4 D64 S256 (64 txt + 192 img), no RoPE.
c2  FLUX joint attention at 1024 px: B1 H24 D128 S4608 = 512 txt + 64x64 img,
    QK-RMSNorm + axial RoPE (axes 16/56/56 over (txt index, row, col), theta 1e4).
c3  512 px with batch: B4 H24 D128 S1536 = 512 txt + 32x32 img.
c5  aspect-bucketed padded batch: B2 H24 D128 S6656 = 512 txt slots + 64x96 img,
    valid text lengths 77 and 512, key-padding mask.
c4  double-stream DiT block at S4608 (hidden 3072) — block shapes only.

Positions follow the reference harness's joint order (txt first, then img,
crates/foundry-spike/src/bin/throughput.rs:724-748): a text token l sits at
(l, 0, 0) and an image token (r, c) at (0, r, c).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

SEED = 20261028  # the reference fixture seed (tools/fixtures/gen_block.py:51)


@dataclass(frozen=True)
class AttnConfig:
    name: str
    batch: int
    heads: int
    head_dim: int
    txt_len: int
    img_rows: int
    img_cols: int
    dtype: str = "bf16"
    rope: bool = True
    axes: Sequence[int] = (16, 56, 56)
    theta: float = 10000.0
    txt_valid: Optional[Sequence[int]] = None  # per batch item; None = no mask

    @property
    def seq(self) -> int:
        return self.txt_len + self.img_rows * self.img_cols

    @property
    def scale(self) -> float:
        return 1.0 / float(np.sqrt(self.head_dim))

    def positions(self) -> np.ndarray:
        """[S, 3] float32 rope positions, txt then img."""
        t = np.zeros((self.txt_len, 3), np.float32)
        t[:, 0] = np.arange(self.txt_len)
        n_img = self.img_rows * self.img_cols
        i = np.zeros((n_img, 3), np.float32)
        i[:, 1] = np.arange(n_img) // self.img_cols
        i[:, 2] = np.arange(n_img) % self.img_cols
        return np.concatenate([t, i], 0)

    def key_keep(self) -> Optional[np.ndarray]:
        """[B, S] uint8 keep mask (padded text slots excluded) or None."""
        if self.txt_valid is None:
            return None
        m = np.ones((self.batch, self.seq), np.uint8)
        for b, n in enumerate(self.txt_valid):
            m[b, n:self.txt_len] = 0
        return m

    def kept_keys(self) -> List[int]:
        kk = self.key_keep()
        return [self.seq] * self.batch if kk is None else [int(r.sum()) for r in kk]

    def fwd_flops(self) -> float:
        """4 * B * H * S_q * S_kv * D, S_kv = kept keys per batch item."""
        return float(sum(4.0 * self.heads * self.seq * kv * self.head_dim for kv in self.kept_keys()))

    def bwd_flops(self) -> float:
        """Backward counted as 2.5x forward (5 GEMMs incl. the QK^T recompute)."""
        return 2.5 * self.fwd_flops()


C1 = AttnConfig("c1", batch=1, heads=4, head_dim=64, txt_len=64, img_rows=12, img_cols=16,
                dtype="f32", rope=False)
C2 = AttnConfig("c2", batch=1, heads=24, head_dim=128, txt_len=512, img_rows=64, img_cols=64)
C3 = AttnConfig("c3", batch=4, heads=24, head_dim=128, txt_len=512, img_rows=32, img_cols=32)
C5 = AttnConfig("c5", batch=2, heads=24, head_dim=128, txt_len=512, img_rows=64, img_cols=96,
                txt_valid=(77, 512))

CONFIGS = {c.name: c for c in (C1, C2, C3, C5)}


@dataclass(frozen=True)
class BlockConfig:
    """c4: double-stream block, S = 4096 img + 512 txt, hidden 3072, 24 x 128 heads."""
    img_tokens: int = 4096
    txt_tokens: int = 512
    hidden: int = 3072
    heads: int = 24
    head_dim: int = 128
    mlp_ratio: int = 4
    lora_rank: int = 16
    lora_alpha: float = 16.0
    axes: Sequence[int] = (16, 56, 56)
    theta: float = 10000.0


C4 = BlockConfig()
