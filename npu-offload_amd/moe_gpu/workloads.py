"""The MoE-layer workloads the tier is measured and checked on, with their algorithmic HBM bytes.

Shapes follow the reference's Solar-Open-100B decode layer (track2_opt/solar_engine/src/host.rs:5-16: H=4096,
F=1280, E=128, TOPK=8, one shared expert) and a tiny single-layer case runnable on any host.
Weights are ~N(0, 0.02) bf16, activations ~N(0, 1) bf16, the router score bias of the Solar case is
b_e = -1.1 * ln(rank_e) with rank a seeded permutation of 1..E (skewed, hot/cold expert popularity).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import numpy as np


@dataclass(frozen=True)
class Workload:
    name: str
    H: int
    F: int
    E: int
    k: int
    n_shared: int
    T: int = 1
    keep: int = 0          # 0: keep all k ranks; 4 for the approximate int8 mode (ranks >= 4 dropped, renormalised)
    int8: bool = False     # routed experts int8 weight-only, shared stays bf16
    zipf_s: float = 0.0    # router bias exponent (0: no bias)
    sigma_w: float = 0.02
    seed: int = 0

    @property
    def keep_eff(self) -> int:
        return self.keep if 0 < self.keep <= self.k else self.k

    def expert_bytes(self, int8: bool | None = None) -> int:
        q8 = self.int8 if int8 is None else int8
        if q8:
            return 3 * self.F * self.H + (2 * self.F + self.H) * 4
        return 3 * self.F * self.H * 2

    def router_bytes(self) -> int:
        return self.E * self.H * 2

    def algorithmic_bytes(self, distinct_routed: int | None = None) -> int:
        """Weight bytes one layer call must read: router + each distinct selected routed expert once + shared."""
        u = self.keep_eff if distinct_routed is None else distinct_routed
        shared = self.n_shared * self.expert_bytes(int8=False)
        return self.router_bytes() + u * self.expert_bytes() + shared

    def flops(self, n_expert_tokens: int) -> int:
        """2 flops per weight element per (expert, token) pair, + router."""
        return 2 * n_expert_tokens * 3 * self.F * self.H + 2 * self.T * self.E * self.H


TINY = Workload("tiny: H=1024 E=16 top-2 F=512, no shared, batch 1", 1024, 512, 16, 2, 0)
SOLAR = Workload("solar: H=4096 E=128+1 shared top-8 F=1280, bf16, batch 1", 4096, 1280, 128, 8, 1, zipf_s=1.1)
SOLAR_INT8 = replace(SOLAR, name="solar int8 weight-only, ranks>=4 dropped + renormalised, batch 1", int8=True, keep=4)


def solar_batch(T: int) -> Workload:
    return replace(SOLAR, name=f"solar bf16 batch {T}", T=T)


def zipf_bias(E: int, s: float, seed: int) -> np.ndarray:
    """b_e = -s * ln(rank_e), rank = seeded permutation of 1..E (float32)."""
    if s == 0.0:
        return np.zeros(E, np.float32)
    rank = np.random.default_rng(seed + 2).permutation(E) + 1
    return (-s * np.log(rank.astype(np.float64))).astype(np.float32)
