"""voodoo_quant on MI355X: the gated-mixture Linear of Voodoo dynamic quant
selection, running on hand-written gfx950 kernels (``libvoodoo_hip.so``).

- :mod:`voodoo_quant.layers`  gated layers (drop-in ``MixedQuantLinear``), module walkers
- :mod:`voodoo_quant.cache`   candidate cache (same on-disk format as the reference)
- :mod:`voodoo_quant.ggml`    quant-type registry and the libggml quantizer bridge
- :mod:`voodoo_quant.rtn`     labelled non-ggml encoder used when libggml is absent
- :mod:`voodoo_quant.training.trainer`  the trainer's per-step calls (anneal, size loss, gate optimizer)
- :mod:`voodoo_quant._hip`    ctypes binding of the C ABI (include/voodoo_hip.h)
"""

__version__ = "0.1.0"
