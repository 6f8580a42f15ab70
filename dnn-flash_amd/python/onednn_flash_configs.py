"""The five attention workloads the library is measured and checked on.

Layout [B,H,T,D] row-major, M = N, Dv = D, scale 1/sqrt(D), inputs iid normal.
Conventions fixed here for every report:
  * ALiBi slope of 0-based head h is 2^(-8(h+1)/H); bias slope_h * (key - query).
  * "N(0, 0.5)" means standard deviation 0.5.
  * The block-sparse workload runs causal=True plus a 64x64 block bitmap
    allowed[qb][kb] = kb <= qb and (qb - kb < 16 or kb < 4): a causal sliding
    window of 16 blocks (1024 tokens) plus 4 global sink blocks.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    dtype: str          # "f32", "bf16", "f16"
    batch: int
    heads: int
    tokens: int
    head_dim: int
    causal: bool
    alibi: bool = False
    softcap: float = 0.0
    block_sparse: bool = False
    std: float = 1.0

    @property
    def scale(self) -> float:
        return 1.0 / float(np.sqrt(self.head_dim))

    def alibi_slopes(self) -> np.ndarray:
        h = np.arange(self.heads, dtype=np.float64)
        return (2.0 ** (-8.0 * (h + 1.0) / self.heads)).astype(np.float32)

    def mask(self) -> np.ndarray | None:
        if not self.block_sparse:
            return None
        nb = self.tokens // 64
        qb = np.arange(nb)[:, None]
        kb = np.arange(nb)[None, :]
        return ((kb <= qb) & ((qb - kb < 16) | (kb < 4))).astype(np.uint8)

    mask_block = (64, 64)

    def useful_pairs_per_head(self) -> int:
        """Unmasked (query, key) pairs of one head, counted exactly."""
        n = self.tokens
        m = self.mask()
        if m is None:
            return n * (n + 1) // 2 if self.causal else n * n
        total = 0
        bs = 64
        for qb in range(m.shape[0]):
            for kb in np.nonzero(m[qb])[0]:
                if kb < qb or not self.causal:
                    total += bs * bs
                else:  # diagonal block with token-level causality
                    total += bs * (bs + 1) // 2
        return total

    def useful_flops(self) -> float:
        return 4.0 * self.head_dim * self.useful_pairs_per_head() * self.batch * self.heads

    def algorithmic_bytes(self) -> int:
        """Read Q, K, V once and write O once."""
        es = 4 if self.dtype == "f32" else 2
        return 4 * self.batch * self.heads * self.tokens * self.head_dim * es


WORKLOADS = {
    "fp32_noncausal_b1h4n512d64": Workload("fp32_noncausal_b1h4n512d64", "f32", 1, 4, 512, 64, False),
    "fp32_causal_b2h8n2048d64": Workload("fp32_causal_b2h8n2048d64", "f32", 2, 8, 2048, 64, True),
    "bf16_causal_b4h32n4096d128": Workload("bf16_causal_b4h32n4096d128", "bf16", 4, 32, 4096, 128, True),
    "bf16_alibi_softcap_b2h16n8192d128": Workload("bf16_alibi_softcap_b2h16n8192d128", "bf16", 2, 16,
                                                   8192, 128, False, alibi=True, softcap=50.0),
    "fp16_blocksparse_b1h16n16384d64": Workload("fp16_blocksparse_b1h16n16384d64", "f16", 1, 16,
                                                 16384, 64, True, block_sparse=True, std=0.5),
}

# Short aliases in the order the workloads are listed in the benchmark brief.
ALIASES = {
    "c1": "fp32_noncausal_b1h4n512d64",
    "c2": "fp32_causal_b2h8n2048d64",
    "c3": "bf16_causal_b4h32n4096d128",
    "c4": "bf16_alibi_softcap_b2h16n8192d128",
    "c5": "fp16_blocksparse_b1h16n16384d64",
}

HEADLINE = "bf16_causal_b4h32n4096d128"

# MI355X published dense peaks (TFLOP/s) and HBM bandwidth (GB/s).
PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6, "f32": 157.3}
PEAK_HBM_GBS = 8000.0


def get(name: str) -> Workload:
    return WORKLOADS[ALIASES.get(name.lower(), name)]
