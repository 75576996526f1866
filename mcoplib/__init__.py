"""``mcoplib`` -- the reference's import path for the fused RMSNorm + per-token quantization
operators, so that callers written against MetaX-MACA/mcoplib run unchanged:

    from mcoplib import op as ops                                   (README.md:149)
    import mcoplib._C                                               (README.md:155)
    from mcoplib.custom_ops import rms_norm_dynamic_per_token_quant  (unit_test/test_rms_norm_custom.py:2)

``mcoplib.op``, ``mcoplib._C`` and ``mcoplib.custom_ops`` are the very module objects
``mcoplib_amd.op``, ``mcoplib_amd._C`` and ``mcoplib_amd.custom_ops`` (one implementation, two
names): the hand-written gfx950 kernels of libmcop_norm.so behind the C++ operator layer.
Only this operator family exists under the name; mcoplib's other operators (attention, MoE,
GEMMs, ...) are not part of this package.  Unlike the reference, importing prints nothing.
"""

from mcoplib_amd import __version__, LIBRARY_PATH  # noqa: F401  (loads libmcop_norm.so)
