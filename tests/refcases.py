"""Inputs of the reference's golden fixtures, rebuilt for the tests.

The single-layer baker (rtl/vc707/host/gen_smollm_blockfp_bfp.py:186-225)
draws its inputs with the legacy ``np.random.seed(SEED)`` generator in a fixed
order: Wq, Wk, Wv, Wo (x0.3), Wg, Wu, Wd (x0.3), g1, g2 (1 + 0.05 N), the
preloaded K and V cache (x0.5, MAX_CTX rows) and h_in (x1.0).  This module
redraws them in that order and quantises them the way the baker does, so a
test can run the oracle (or the GPU) on exactly the baker's inputs and
compare with its stage dumps (tests/golden/ref_stages_*.npz).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle import bfp_sim as sim

GOLDEN = Path(__file__).resolve().parent / "golden"


def baker_case(name):
    f = np.load(GOLDEN / f"ref_stages_{name}.npz")
    cfg = {k: int(f[k]) for k in ("D", "H_Q", "H_KV", "HD", "FFN", "MAX_CTX", "POS", "KV_POS",
                                  "SEED")}
    D, KV, FFN, MC = cfg["D"], cfg["H_KV"] * cfg["HD"], cfg["FFN"], cfg["MAX_CTX"]
    np.random.seed(cfg["SEED"])

    def randn(*shape, scale):
        return (np.random.randn(*shape) * scale).astype(np.float64)

    W = {}
    W["Wq"] = randn(D, D, scale=0.3)
    W["Wk"] = randn(KV, D, scale=0.3)
    W["Wv"] = randn(KV, D, scale=0.3)
    W["Wo"] = randn(D, D, scale=0.3)
    W["Wg"] = randn(FFN, D, scale=0.3)
    W["Wu"] = randn(FFN, D, scale=0.3)
    W["Wd"] = randn(D, FFN, scale=0.3)
    g1 = np.ones(D, dtype=np.float64) + 0.05 * np.random.randn(D)
    g2 = np.ones(D, dtype=np.float64) + 0.05 * np.random.randn(D)
    K_init = randn(MC, KV, scale=0.5)
    V_init = randn(MC, KV, scale=0.5)
    h_in = randn(D, scale=1.0)
    lw = {n: sim.quantize_W(w) for n, w in W.items()}
    lw["g1"] = sim.fp_quantize_vec(g1)
    lw["g2"] = sim.fp_quantize_vec(g2)
    dims = sim.Dims(D=D, H_Q=cfg["H_Q"], H_KV=cfg["H_KV"], HD=cfg["HD"], FFN=FFN, NL=1,
                    MAX_CTX=MC, VOCAB=256)
    # preloaded cache: per timestep tile_quantize over the whole KV row
    kv = sim.new_kv(dims, MC)
    kq = [sim.tile_quantize(K_init[t]) for t in range(MC)]
    vq = [sim.tile_quantize(V_init[t]) for t in range(MC)]
    for t in range(MC):
        kv["k"][t] = sim.tile_decode(*kq[t]).reshape(cfg["H_KV"], cfg["HD"])
        kv["v"][t] = sim.tile_decode(*vq[t]).reshape(cfg["H_KV"], cfg["HD"])
    hq = sim.tile_quantize(h_in)
    return dict(cfg=cfg, dims=dims, lw=lw, g1=g1, g2=g2, W=W, kv=kv, kq=kq, vq=vq,
                h=sim.tile_decode(*hq), hq=hq, fixture=f)
