"""Deterministic synthetic inputs for the oracle, the golden fixtures and the tests.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Values come from splitmix64 (Steele, Lea, Flood, "Fast splittable pseudorandom
number generators", OOPSLA 2014) turned into standard normals with the
Box-Muller transform.  Everything is numpy uint64/float64 arithmetic, so the
same (seed, shape) gives the same float32 array on any host with numpy >= 1.17,
independent of torch's RNG.  Fixtures store only outputs; tests regenerate the
inputs from the seeds recorded next to them.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n consecutive outputs of splitmix64 started from state ``seed``."""
    with np.errstate(over="ignore"):
        state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + (np.arange(1, n + 1, dtype=np.uint64) * _GOLDEN)
        z = state
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniform01(seed: int, n: int) -> np.ndarray:
    """Uniform doubles in (0, 1]: the top 53 bits of splitmix64, plus one ulp."""
    z = splitmix64(seed, n)
    return ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """float32 N(mean, std^2) array of ``shape`` (Box-Muller on pairs of uniforms)."""
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = uniform01(seed, 2 * m)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:n] * std + mean).astype(np.float32).reshape(shape)


def moe_inputs(seed: int, num_tokens: int, hidden: int, num_experts: int, inter: int,
               weight_std: float = 0.02, logit_bias_std: float = 0.0):
    """Inputs of one MoE FFN layer as float32 numpy arrays.

    Returns x [T,H] ~ N(0,1), gate weight [E,H], gate_up weight [E,2I,H] and
    down weight [E,H,I], all ~ N(0, weight_std^2).  With ``logit_bias_std`` > 0
    the router logits are skewed without touching the module: a per-expert
    bias b ~ N(0, logit_bias_std^2) is folded into the activations as
    x += Wg^T (Wg Wg^T)^-1 b, so that Wg x_t = Wg z_t + b for every token.
    """
    x = normal(seed * 16 + 1, (num_tokens, hidden))
    wg = normal(seed * 16 + 2, (num_experts, hidden), std=weight_std)
    wgu = normal(seed * 16 + 3, (num_experts, 2 * inter, hidden), std=weight_std)
    wdn = normal(seed * 16 + 4, (num_experts, hidden, inter), std=weight_std)
    if logit_bias_std > 0.0:
        b = normal(seed * 16 + 5, (num_experts,), std=logit_bias_std).astype(np.float64)
        wg64 = wg.astype(np.float64)
        v = wg64.T @ np.linalg.solve(wg64 @ wg64.T, b)
        x = (x.astype(np.float64) + v[None, :]).astype(np.float32)
    return x, wg, wgu, wdn
