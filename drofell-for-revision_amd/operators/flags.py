"""Module-level switches read by the quantized Linear.

Same names and meaning as the reference's ``operators/flags.py:8-10``
(paths relative to ``/root/reference/After-Revision-DROFELL``).
"""

# Keep a dequantised fp16 copy of every weight after post_init; the forward
# then takes the dense route over that copy, as in the reference.
RECONSTRUCTE_WEIGTH_FLOAT16 = False
# bf16 reconstruction is not offered by the HIP backend (fp16 only).
RECONSTRUCTE_WEIGTH_BFLOAT16 = False
# In training, keep the forward's dequantised weight for the backward.
REUSE_RECONSTRUCT_CACHE_WHEN_GRAD = True
# Token slots per KV-cache block (the reference's operators/flags.py:28-29).
BLOCK_SIZE = 32
