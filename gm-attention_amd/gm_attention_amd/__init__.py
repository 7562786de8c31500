"""gm-attention's fused hot path on MI355X (gfx950).

The layers and ops keep the reference's names and signatures
(``gm_attention.nn.fused_attention``, ``fused_factored``, the ``SO2*``
modules); the arithmetic of the fused ops runs in ``_lib/libgmhip.so``
(hand-written HIP) through :mod:`gm_attention_amd._native`.
"""

__version__ = "0.1.0"
