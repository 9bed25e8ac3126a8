"""Seeded synthetic inputs for the benchmark configurations.

There is no network and no checkpoint, so every weight and prompt is drawn
from ``numpy.random.default_rng(seed)`` (PCG64 + ziggurat: the same bits on
every platform).  Weights are float32, like the HuggingFace fp32 tensors the
reference reads (rtl/vc707/host/gen_smollm_blockfp_full.py:319,327-328), and
are widened to float64 exactly before quantisation.

Draw order (part of the contract; changing it changes every fixture):
per layer Wq, Wk, Wv, Wo, Wg, Wu, Wd, g1, g2; then embed, norm_w.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .dims import Dims

W_STD = np.float32(0.02)
G_STD = np.float32(0.05)

# (name, rows, cols) of each per-layer matrix, in draw order
def layer_shapes(d: Dims):
    return [("Wq", d.D, d.D), ("Wk", d.KV, d.D), ("Wv", d.KV, d.D), ("Wo", d.D, d.D),
            ("Wg", d.FFN, d.D), ("Wu", d.FFN, d.D), ("Wd", d.D, d.FFN)]


def _w(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32) * W_STD


def _gamma(rng, n):
    return np.float32(1.0) + G_STD * rng.standard_normal(n, dtype=np.float32)


@dataclass
class Fp32Model:
    """Raw float32 weights of a SmolLM2-shaped decoder."""
    dims: Dims
    layers: list          # list of dict name -> float32 array (+ 'g1','g2')
    embed: np.ndarray     # (VOCAB, D) float32
    norm_w: np.ndarray    # (D,) float32


def make_layer(rng, d: Dims):
    lw = {name: _w(rng, (r, c)) for name, r, c in layer_shapes(d)}
    lw["g1"] = _gamma(rng, d.D)
    lw["g2"] = _gamma(rng, d.D)
    return lw


def make_model(d: Dims, seed: int = 0) -> Fp32Model:
    rng = np.random.default_rng(seed)
    layers = [make_layer(rng, d) for _ in range(d.NL)]
    embed = _w(rng, (d.VOCAB, d.D))
    norm_w = _gamma(rng, d.D)
    return Fp32Model(d, layers, embed, norm_w)


def make_prompt(d: Dims, n: int, seed: int = 0) -> np.ndarray:
    """n token ids uniform in [0, VOCAB) (config 3/4 prompts)."""
    return np.random.default_rng(seed + 1_000_003).integers(0, d.VOCAB, size=n).astype(np.int32)


def make_layer_inputs(d: Dims, n_pos: int, seed: int = 0) -> np.ndarray:
    """Config 1: n_pos activation vectors x_p ~ N(0, 1) (float64), to be
    BFP-quantised by the caller (fp_quantize_vec)."""
    return np.random.default_rng(seed + 2_000_003).standard_normal((n_pos, d.D))


def make_matvec_case(n_out: int, n_in: int, seed: int = 0, reps: int = 1):
    """Config 2: W ~ N(0, 0.02) float32 (reps copies), x ~ N(0, 1) float64."""
    rng = np.random.default_rng(seed + 3_000_003)
    W = rng.standard_normal((reps, n_out, n_in), dtype=np.float32) * W_STD
    x = rng.standard_normal((reps, n_in))
    return W, x
