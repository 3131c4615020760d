"""MI355X-native FP8 linear path for Bongard's T5Gemma-2 judgment model.

Drop-in modules: ``float8_training`` (torchao Float8Linear path), ``te_linear``
(TransformerEngine te.Linear path) and ``fused_mlp`` (te.LayerNormMLP path), all running
on the hand-written gfx950 HIP kernels in libbongard_fp8.so through ``ops``.
"""

__version__ = "0.1.0"
