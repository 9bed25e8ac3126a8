"""MI355X-native block-floating-point decode datapath (host side).

Import the package with ``tinyllm-fpga_amd`` on ``sys.path``::

    import sys; sys.path.insert(0, "<repo>/tinyllm-fpga_amd")
    import bfp
    m, e = bfp.tile_quantize(v)

Modules: ``api`` (the reference simulator's functions on the GPU),
``model`` (HBM-resident model, layer step and decode driver), ``synth``
(seeded synthetic inputs), ``dims`` (model dimensions), ``_lib`` (ctypes
binding of libbfp.so).
"""
from .dims import Dims, TILE, LANES  # noqa: F401


_API = ("tile_quantize", "tile_decode", "fp_quantize_vec", "tile_encode", "quantize_W",
        "matvec_hw_golden", "matvec_bfp", "PackedMatrix", "rmsnorm_fp", "silu_fp", "softmax_fp",
        "rope_fp", "fwd_layer")


def __getattr__(name):
    # the GPU API is imported lazily so that CPU-only tooling (synth, dims)
    # does not load libbfp.so or torch
    if name in _API:
        import importlib
        return getattr(importlib.import_module(".api", __name__), name)
    raise AttributeError(name)
