"""Seeded synthetic inputs shared by the fixture generator, the tests and bench.py.

All draws use ``numpy.random.default_rng(seed)`` with a fixed draw order so the
same arrays are produced here and on the GPU box (same image, same numpy).
Shapes follow the BASELINE configs: hidden H=1536, FFN I=6144 split into E=16
experts of G=384 neurons; weights ~N(0, 0.02), x ~N(0, 1).
"""
from __future__ import annotations

import hashlib

import numpy as np

H, I, E, G = 1536, 6144, 16, 384


def sha256(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def layer_weights(seed: int, H: int = H, I: int = I, E: int = E, balanced_random: bool = True,
                  std: float = 0.02):
    """One MoE-MLP layer in the reference's dense (nn.Linear) layout.

    Returns dict with w_gate/w_up [I,H], w_down [H,I], w_router [E,H] (fp32) and
    expert_ids [I] (neuron -> expert). ``balanced_random`` draws a random balanced
    partition (every expert owns I/E neurons); otherwise contiguous blocks
    (the reference default, src/MoEBlock_origin.py:139-143).
    """
    rng = np.random.default_rng(seed)
    w_gate = rng.normal(0.0, std, (I, H)).astype(np.float32)
    w_up = rng.normal(0.0, std, (I, H)).astype(np.float32)
    w_down = rng.normal(0.0, std, (H, I)).astype(np.float32)
    w_router = rng.normal(0.0, std, (E, H)).astype(np.float32)
    Gs = I // E
    if balanced_random:
        expert_ids = rng.permutation(np.repeat(np.arange(E, dtype=np.int32), Gs)).astype(np.int32)
    else:
        expert_ids = np.repeat(np.arange(E, dtype=np.int32), Gs)
    return dict(w_gate=w_gate, w_up=w_up, w_down=w_down, w_router=w_router, expert_ids=expert_ids)


def tokens(seed: int, n: int, H: int = H) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((n, H)).astype(np.float32)


def zipf_bias(E: int = E, s: float = 1.2) -> np.ndarray:
    """Router bias b_e = log of the Zipf(s) pmf over E experts (skews expert load)."""
    ranks = np.arange(1, E + 1, dtype=np.float64)
    pmf = ranks ** (-s)
    pmf /= pmf.sum()
    return np.log(pmf).astype(np.float32)


def routing_logits(seed: int, n: int, E: int):
    """Logit families used by the routing fixtures: name -> [n, E] fp32."""
    rng = np.random.default_rng(seed)
    fam = {}
    for scale in (0.05, 0.78, 2.0, 6.0):
        fam[f"normal_{scale}"] = (rng.standard_normal((n, E)) * scale).astype(np.float32)
    # many exact ties: values on a coarse grid
    fam["ties"] = (rng.integers(-3, 4, (n, E)) * 0.5).astype(np.float32)
    # all-equal rows and one dominant expert
    eq = np.zeros((n, E), np.float32)
    eq[n // 2:, :] = rng.standard_normal((n - n // 2, 1)).astype(np.float32)
    fam["all_equal"] = eq
    dom = (rng.standard_normal((n, E)) * 0.5).astype(np.float32)
    dom[np.arange(n), rng.integers(0, E, n)] += 12.0
    fam["dominant"] = dom
    # extremes: large magnitudes exercise exp underflow / sigmoid saturation
    fam["extreme"] = (rng.standard_normal((n, E)) * 60.0).astype(np.float32)
    fam["zipf_bias"] = ((rng.standard_normal((n, E)) * 0.78) + zipf_bias(E)[None, :]).astype(np.float32)
    return fam
