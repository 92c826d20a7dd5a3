"""Seeded logit vectors and option sets for the sampler's checks (CPU and
GPU): every branch of model/sampler.c's ml_sample and the inputs that steer
them (ties, -inf, NaN, +inf, underflow)."""
import numpy as np

NAN = np.float32("nan")
INF = np.float32("inf")


def gen_logits(kind, n, rng):
    """seeded logit vectors covering the cases the sampler branches on"""
    if kind == "normal":
        return (rng.standard_normal(n) * rng.uniform(0.5, 6.0)).astype(np.float32)
    if kind == "peaked":
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.integers(0, n)] = 25.0
        return x
    if kind == "ties":   # few distinct values: equal probabilities, ids break the ties
        return (rng.integers(-3, 4, n) * 0.5).astype(np.float32)
    if kind == "flat":
        return np.zeros(n, dtype=np.float32)
    if kind == "neginf":
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.random(n) < 0.3] = -INF
        return x
    if kind == "allneginf":
        return np.full(n, -INF, dtype=np.float32)
    if kind == "nan":
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.integers(0, n)] = NAN
        return x
    if kind == "posinf":
        x = rng.standard_normal(n).astype(np.float32)
        x[rng.integers(0, n)] = INF
        return x
    if kind == "tiny":   # a wide range: many probabilities underflow or are subnormal
        return (rng.standard_normal(n) * 40.0).astype(np.float32)
    raise ValueError(kind)


KINDS = ["normal", "peaked", "ties", "flat", "neginf", "allneginf", "nan", "posinf", "tiny"]
OPTS = {
    "greedy_penalty": dict(temperature=0.0, repeat_penalty=1.3, repeat_last_n=8),
    "mult": dict(temperature=0.8, topp=1.0),
    "mult_topp0": dict(temperature=1.3, topp=0.0, seed=0),
    "topp": dict(temperature=0.8, topp=0.9),
    "topp_half_penalty": dict(temperature=1.0, topp=0.5, repeat_penalty=1.5, repeat_last_n=16),
    "topp_tiny": dict(temperature=1.0, topp=1e-6),
    "topk": dict(temperature=0.7, topk=40, topp=0.9),
    "topk_no_nucleus": dict(temperature=1.1, topk=40, topp=1.0),
    "topk1": dict(temperature=1.5, topk=1),
    "topk_big": dict(temperature=0.9, topk=500, topp=0.95, seed=77),
}
