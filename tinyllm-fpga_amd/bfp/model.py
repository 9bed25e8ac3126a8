"""HBM-resident BFP model: layer step, decode head and the autoregressive
driver of rtl/vc707/host/gen_smollm_blockfp_full.py (full.py:261-293,
411-443), computed by libbfp.so on one GPU.

Host arrays go in and out as numpy; the model, KV cache and every
intermediate stay in device memory owned by the C context.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import synth
from ._lib import BfpError, DimsC, N_STAGES, StageDumpC, call, lib
from .dims import Dims

STAGES = ("N1", "Q", "K", "V", "ATTN", "O", "H1", "N2", "G", "U", "MLP", "D", "HOUT")
TRACE_LAYER = 20   # stage-trace stamps per (step, layer), bfp_decode_trace
PIPE_TRACE_JOBS, PIPE_TRACE_W = 1024, 8   # the pipelined step's trace: job slots per workgroup, words each
WHICH = {"Wq": 0, "Wk": 1, "Wv": 2, "Wo": 3, "Wg": 4, "Wu": 5, "Wd": 6, "g1": 7, "g2": 8,
         "embed": 9, "norm_w": 10}


def _p(a: np.ndarray) -> int:
    """The address of a's data.  A writable, C-contiguous, non-empty array's
    buffer is taken through ctypes (about 0.9 us a call, against 2 us for
    a.ctypes.data, four of which a single-layer call makes); any other
    array goes through a.ctypes.data."""
    try:
        return C.addressof(C.c_char.from_buffer(a))
    except (TypeError, ValueError, BufferError):
        return a.ctypes.data


def _c16(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int16))


def _c8(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int8))


class BfpModel:
    """One context: weights for ``dims.NL`` layers, KV cache for
    ``max_batch`` sequences of ``dims.MAX_CTX`` positions."""

    def __init__(self, dims: Dims, device: int = 0, max_batch: int = 1):
        self.dims = dims.check()
        self.max_batch = max_batch
        cd = DimsC(dims.D, dims.H_Q, dims.H_KV, dims.HD, dims.FFN, dims.NL, dims.MAX_CTX,
                   dims.VOCAB)
        h = lib().bfp_create(C.byref(cd), device, max_batch)
        if not h:
            raise BfpError("bfp_create", -22, lib().bfp_last_error().decode())
        self._h = C.c_void_p(h)

    # ------------------------------------------------------------ lifetime
    def close(self):
        if getattr(self, "_h", None):
            lib().bfp_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -------------------------------------------------------------- weights
    def load_tensor(self, name, layer=0, fp32=None, m=None, e=None):
        w = WHICH[name]
        if fp32 is not None:
            f = np.ascontiguousarray(np.asarray(fp32, dtype=np.float32))
            call("bfp_load_weights", self._h, w, layer, _p(f), None, None)
        else:
            mm, ee = _c16(m), _c8(e)
            call("bfp_load_weights", self._h, w, layer, None, _p(mm), _p(ee))

    def load_fp32(self, fm: synth.Fp32Model):
        """Load a float32 model (quantize_W / fp_quantize_vec on the device)."""
        if fm.dims != self.dims:
            raise ValueError(f"model dims {fm.dims} != context dims {self.dims}")
        for li, lw in enumerate(fm.layers):
            for name in ("Wq", "Wk", "Wv", "Wo", "Wg", "Wu", "Wd", "g1", "g2"):
                self.load_tensor(name, li, fp32=lw[name])
        self.load_tensor("embed", fp32=fm.embed)
        self.load_tensor("norm_w", fp32=fm.norm_w)

    def load_ddr_image(self, path):
        """Load the reference's DDR3 weight image (<PREFIX>DDR3.bin,
        gen_smollm_blockfp_ddr.py) -- see bfp.image."""
        from .image import WeightImage, load_image
        load_image(self, WeightImage.from_ddr(path, self.dims))

    def load_hex_dir(self, directory, prefix="lbfp_full_"):
        """Load the reference's per-tensor hex set (<PREFIX><TAG>_{m,e}.hex,
        gen_smollm_blockfp_full.py) -- see bfp.image."""
        from .image import WeightImage, load_image
        load_image(self, WeightImage.from_hex_dir(directory, self.dims, prefix))

    def reset_kv(self):
        call("bfp_reset_kv", self._h)

    def kv_io(self, layer, seq, t0, n, k=None, v=None):
        """Read (k, v None) or write KV positions [t0, t0+n): each a pair
        (m (n, H_KV*HD) int16, e (n, H_KV*HD/16) int8)."""
        d = self.dims
        if k is None:
            km = np.zeros((n, d.KV), np.int16)
            ke = np.zeros((n, d.KV // 16), np.int8)
            vm, ve = np.zeros_like(km), np.zeros_like(ke)
            call("bfp_kv_io", self._h, layer, seq, t0, n, _p(km), _p(ke), _p(vm), _p(ve), 0)
            return (km, ke), (vm, ve)
        km, ke = _c16(k[0]).reshape(n, d.KV), _c8(k[1]).reshape(n, d.KV // 16)
        vm, ve = _c16(v[0]).reshape(n, d.KV), _c8(v[1]).reshape(n, d.KV // 16)
        call("bfp_kv_io", self._h, layer, seq, t0, n, _p(km), _p(ke), _p(vm), _p(ve), 1)

    # ----------------------------------------------------------- layer step
    def _stage_len(self, name):
        d = self.dims
        return {"K": d.KV, "V": d.KV, "G": d.FFN, "U": d.FFN, "MLP": d.FFN}.get(name, d.D)

    def kv_io_f64(self, layer, seq, t0, n, k=None, v=None):
        """The cache rows [t0, t0+n) as the reference holds them: float64
        (n, H_KV, HD) arrays.  Read (k, v None) or write (exact encoding;
        ValueError-like BfpError for values that are not BFP tiles)."""
        d = self.dims
        if k is None:
            kk = np.zeros((n, d.H_KV, d.HD), np.float64)
            vv = np.zeros_like(kk)
            call("bfp_kv_io_f64", self._h, layer, seq, t0, n, _p(kk), _p(vv), 0)
            return kk, vv
        kk = np.ascontiguousarray(np.asarray(k, dtype=np.float64)).reshape(n, d.KV)
        vv = np.ascontiguousarray(np.asarray(v, dtype=np.float64)).reshape(n, d.KV)
        call("bfp_kv_io_f64", self._h, layer, seq, t0, n, _p(kk), _p(vv), 1)

    def matvec(self, name, layer, x_m, x_e):
        """matvec_hw_golden with this context's matrix `name` ('Wq'..'Wd')
        of `layer` on BFP input (batch, n_in) / (batch, n_in/16): returns
        the raw BFP output (y_m (batch, n_out), y_e (batch, n_out/16))."""
        d = self.dims
        n_out, n_in = {"Wq": (d.D, d.D), "Wk": (d.KV, d.D), "Wv": (d.KV, d.D), "Wo": (d.D, d.D),
                       "Wg": (d.FFN, d.D), "Wu": (d.FFN, d.D), "Wd": (d.D, d.FFN)}[name]
        x_m = _c16(x_m).reshape(-1, n_in)
        batch = x_m.shape[0]
        x_e = _c8(x_e).reshape(batch, n_in // 16)
        ym = np.empty((batch, n_out), np.int16)
        ye = np.empty((batch, n_out // 16), np.int8)
        call("bfp_matvec", self._h, _p(x_m), _p(x_e), WHICH[name], layer, batch, _p(ym), _p(ye))
        return ym, ye

    def layer_step_bfp(self, layer, pos, h_m, h_e, dump=False, kv_pos=None):
        """fwd_layer on BFP input (batch, D) / (batch, D/16) with RoPE at pos
        and the K/V slot kv_pos (default pos); returns (out_m, out_e,
        stages) where stages maps stage name -> (m, e)."""
        h_m = _c16(h_m).reshape(-1, self.dims.D)
        batch = h_m.shape[0]
        h_e = _c8(h_e).reshape(batch, self.dims.D // 16)
        out_m = np.empty_like(h_m)
        out_e = np.empty_like(h_e)
        stages = {}
        sd = None
        if dump:
            sd = StageDumpC()
            for i, name in enumerate(STAGES):
                n = self._stage_len(name)
                sm = np.empty((batch, n), np.int16)
                se = np.empty((batch, n // 16), np.int8)
                stages[name] = (sm, se)
                sd.m[i] = _p(sm)
                sd.e[i] = _p(se)
        call("bfp_layer_step_kv", self._h, layer, pos, pos if kv_pos is None else kv_pos, batch,
             _p(h_m), _p(h_e), _p(out_m), _p(out_e), C.byref(sd) if sd is not None else None)
        return out_m, out_e, stages

    def rtl_layer_step(self, layer, pos, h_m, h_e, kv_pos=None, dump=False):
        """The FPGA's decoder layer (smollm_layer_bfp.sv, the RTL engines in
        its FSM order) on one BFP input (D,) / (D/16,) at RoPE position pos
        and KV slot kv_pos (default pos); returns (out_m, out_e, stages)."""
        d = self.dims
        h_m = _c16(h_m).reshape(d.D)
        h_e = _c8(h_e).reshape(d.D // 16)
        out_m, out_e = np.empty_like(h_m), np.empty_like(h_e)
        stages, sd = {}, None
        if dump:
            sd = StageDumpC()
            for i, name in enumerate(STAGES):
                n = self._stage_len(name)
                stages[name] = (np.empty(n, np.int16), np.empty(n // 16, np.int8))
                sd.m[i], sd.e[i] = _p(stages[name][0]), _p(stages[name][1])
        call("bfp_rtl_layer_step", self._h, layer, pos, pos if kv_pos is None else kv_pos,
             _p(h_m), _p(h_e), _p(out_m), _p(out_e), C.byref(sd) if sd is not None else None)
        return out_m, out_e, stages

    def rtl_head(self, h_m, h_e, logits=False):
        """The FPGA decode head (smollm_decode_head_bfp.sv: RMSNorm engine
        with the final norm gamma, lm_head on the matvec engine over the
        tile-quantised tied embedding, bfp_gt running argmax) on one BFP
        hidden state; returns token or (token, (logit_m, logit_e)) with one
        exponent per logit."""
        d = self.dims
        h_m = _c16(h_m).reshape(d.D)
        h_e = _c8(h_e).reshape(d.D // 16)
        tok = np.zeros(1, np.int32)
        lm = np.empty(d.VOCAB, np.int16) if logits else None
        le = np.empty(d.VOCAB, np.int8) if logits else None
        call("bfp_rtl_head", self._h, _p(h_m), _p(h_e), _p(lm) if logits else None,
             _p(le) if logits else None, _p(tok))
        return (int(tok[0]), (lm, le)) if logits else int(tok[0])

    def rtl_decode(self, prompt, n_gen, hist=False):
        """The FPGA's token loop (autoregress_bfp_top.sv:357-386) over the
        composed RTL layer and head, on sequence 0 of this context: returns
        the len(prompt) + n_gen per-step predictions, and with hist=True also
        the last layer's output per step ((steps, D), (steps, D/16))."""
        d = self.dims
        ids = np.ascontiguousarray(np.asarray(prompt, np.int32).reshape(-1))
        steps = ids.size + int(n_gen)
        preds = np.zeros(steps, np.int32)
        hm = np.zeros((steps, d.D), np.int16) if hist else None
        he = np.zeros((steps, d.D // 16), np.int8) if hist else None
        call("bfp_rtl_decode", self._h, _p(ids), ids.size, int(n_gen), _p(preds),
             _p(hm) if hist else None, _p(he) if hist else None)
        return (preds, (hm, he)) if hist else preds

    def fwd_layer(self, h, layer, pos, kv_pos=None):
        """The reference's fwd_layer(h, lw, pos, kv, kv_pos) (full.py:261-293)
        with the layer's weights and KV cache resident in the context:
        float64 BFP-exact h (D,) in, float64 out; RoPE at pos, K/V at slot
        kv_pos (default pos).  bfp.api.fwd_layer takes the reference's own
        caller-owned lw and kv instead."""
        from . import api
        m, e = api.tile_encode(h)
        om, oe, _ = self.layer_step_bfp(layer, pos, m.reshape(1, -1), e.reshape(1, -1),
                                        kv_pos=kv_pos)
        return api.tile_decode(om[0], oe[0])

    # ----------------------------------------------------------------- head
    def head(self, h_m, h_e, logits=False):
        """Final norm + float64 logits + argmax (full.py:438-440) for a batch
        of BFP hidden states; returns (argmax ids, logits or None)."""
        h_m = _c16(h_m).reshape(-1, self.dims.D)
        batch = h_m.shape[0]
        h_e = _c8(h_e).reshape(batch, self.dims.D // 16)
        am = np.empty(batch, np.int32)
        lg = np.empty((batch, self.dims.VOCAB), np.float64) if logits else None
        call("bfp_head", self._h, batch, _p(h_m), _p(h_e), _p(lg) if logits else None, _p(am))
        return am, lg

    # --------------------------------------------------------------- decode
    def decode(self, prompts, n_gen, hist=False, graph=True, step_times=False, rtl_loop=False,
               persist=True, trace=False, abort_test=False, pipe=None):
        """Greedy decode (full.py:426-443) of a batch of prompts
        (batch, n_prompt).  Returns (tokens (batch, n_gen), hist) where hist
        is None or (m (batch, steps, NL, D), e (batch, steps, NL, D/16)).

        rtl_loop=True runs the FPGA driver's loop policy instead
        (autoregress_bfp_top.sv:357-386): the step after the prompt feeds
        the last prediction, and the tokens returned are every step's
        prediction, (batch, n_prompt + n_gen).

        persist=False keeps batch 1 off the persistent single-launch kernel
        (decode_path() tells which path the last decode took); pipe=True
        runs batches on the pipelined one-launch step where it covers the
        dimensions, pipe=False on the per-stage launches, None leaves the
        choice to the library (decode_form() tells which ran); trace=True
        records the stage stamps (decode_trace()).

        abort_test=True is a test hook: the decode's abort word is set before
        its first launch, so its bounded waits give up, the kernels run to
        their end and the call raises BfpError (BFP_EIO)."""
        P = np.ascontiguousarray(np.atleast_2d(np.asarray(prompts, dtype=np.int32)))
        batch, n_prompt = P.shape
        steps = n_prompt + n_gen
        n_out = steps if rtl_loop else n_gen
        toks = np.zeros((batch, max(n_out, 1)), np.int32)
        hm = he = None
        d = self.dims
        if hist:
            hm = np.zeros((batch, steps, d.NL, d.D), np.int16)
            he = np.zeros((batch, steps, d.NL, d.D // 16), np.int8)
        flags = ((0 if graph else 1) | (2 if step_times else 0) | (4 if rtl_loop else 0)
                 | (0 if persist else 8) | (16 if trace else 0) | (32 if abort_test else 0)
                 | (0 if pipe is None else (128 if pipe else 64)))
        call("bfp_decode", self._h, _p(P), n_prompt, n_gen, batch, _p(toks),
             _p(hm) if hist else None, _p(he) if hist else None, flags)
        return toks[:, :n_out], ((hm, he) if hist else None)

    def step_times_ms(self):
        """Per-step device times of the last decode(step_times=True)."""
        n = lib().bfp_decode_step_times(self._h, None, 0)
        out = np.zeros(max(n, 0), np.float32)
        if n > 0:
            lib().bfp_decode_step_times(self._h, _p(out), n)
        return out

    def decode_path(self):
        """'persist', 'graph' or 'eager': how the last decode ran."""
        return {0: "graph", 1: "persist", 2: "eager"}.get(lib().bfp_decode_path(self._h), None)

    def decode_form(self):
        """How the last decode's layers were launched: 'persist', 'pipe' (the
        pipelined batched step), 'single', 'multi', or 'mx' followed by
        '+qkv_attn' (Q|K|V and attention in one launch), '+attn_group' (its
        attention a KV group per workgroup) and '+norm_fused' (RMSNorms
        inside the O and D launches)."""
        f = lib().bfp_decode_form(self._h)
        if f < 0:
            return None
        if f == 16:
            return "persist"
        if f == 32:
            return "pipe"
        if f < 2:
            return ("single", "multi")[f]
        return ("mx" + ("+qkv_attn" if f & 4 else "") + ("+attn_group" if f & 64 else "")
                + ("+norm_fused" if f & 8 else ""))

    def decode_trace(self):
        """Stamps (device clock, 100 MHz) of the last decode(trace=True): on
        the persistent path (layer stamps (steps, NL, 20), head stamps
        (steps, 3)) -- layer stamps 0-15 are the stages', 16-19 the first
        attention job's phases; on the pipelined batched step every job of
        the last step's launch (workgroups, PIPE_TRACE_JOBS, 8: job code + 1,
        start, inputs in, end, -, and a matvec's row maxima, tile sums and
        epilogue stored); on the per-stage
        matrix-core launches the blocks' phase stamps (4 kernels, 1024
        blocks, 6) (include/bfp.h, bfp_decode_trace); None when nothing was
        recorded."""
        n = lib().bfp_decode_trace(self._h, None, 0)
        if n <= 0:
            return None
        out = np.zeros(n, np.uint64)
        lib().bfp_decode_trace(self._h, _p(out), n)
        if self.decode_form() == "pipe":
            return out.reshape(-1, PIPE_TRACE_JOBS, PIPE_TRACE_W)
        if self.decode_path() != "persist":
            return out.reshape(4, 1024, 6)
        nl, k = self.dims.NL, TRACE_LAYER
        steps = n // (nl * k + 3)
        return out[:steps * nl * k].reshape(steps, nl, k), out[steps * nl * k:].reshape(steps, 3)

    def decode_time_ms(self):
        t, g = C.c_float(), C.c_float()
        call("bfp_decode_time", self._h, C.byref(t), C.byref(g))
        return t.value, g.value
