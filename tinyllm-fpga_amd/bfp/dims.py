"""Model dimensions of the SmolLM2-135M-shaped decoder.

The reference reads these from environment variables at import
(rtl/vc707/host/gen_smollm_blockfp_full.py:54-60); here they are a value
object passed to the context.
"""
from __future__ import annotations

from dataclasses import dataclass

TILE = 16        # mantissas per shared exponent (bfp_format.svh)
LANES = 16       # rows per output chunk (full.py:66)


@dataclass(frozen=True)
class Dims:
    D: int = 576
    H_Q: int = 9
    H_KV: int = 3
    HD: int = 64
    FFN: int = 1536
    NL: int = 30
    MAX_CTX: int = 64
    VOCAB: int = 49152

    @property
    def KV(self) -> int:
        return self.H_KV * self.HD

    def check(self):
        """Shape rules of the reference (full.py:78-83) plus the ones the
        kernels rely on."""
        for name, v in (("D", self.D), ("KV", self.KV), ("FFN", self.FFN)):
            if v % TILE:
                raise ValueError(f"{name}={v} is not a multiple of {TILE}")
        if self.HD % 32:
            raise ValueError(f"HD={self.HD} must be a multiple of 32")
        if self.H_Q % self.H_KV:
            raise ValueError("H_Q must be a multiple of H_KV")
        if self.H_Q * self.HD != self.D:
            raise ValueError("H_Q*HD must equal D")
        if self.VOCAB % LANES:
            raise ValueError("VOCAB must be a multiple of 16")
        return self
