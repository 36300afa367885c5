"""Seeded synthetic inputs for the benchmark workloads.

Skewed routing: router logits drawn as ln p_{pi(e)} + Gumbel(0, 1) with
p_r proportional to r^-s (Zipf) and pi a seeded permutation of the experts,
so that top-k of the logits samples k experts without replacement with
probabilities p (the Gumbel-top-k construction).  Values are computed in
float64 and rounded to float32.
"""
from __future__ import annotations

import numpy as np


def zipf_logits(tokens: int, experts: int, s: float = 1.1, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    p = np.arange(1, experts + 1, dtype=np.float64) ** -s
    p /= p.sum()
    base = np.log(p)[rng.permutation(experts)]
    return (base[None, :] + rng.gumbel(size=(tokens, experts))).astype(np.float32)


def normal(shape, seed: int = 0, std: float = 1.0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * std).astype(np.float32)
