"""Optimizers: the 8-bit AdamW step (mirror of rollfast ``optim/adam8.py``)
and full-precision AdamW (mirror of ``optim/adam.py``)."""

from .adam import ScaleByAdamState, adamw, adamw_step, scale_by_adam

from .adam8 import (
    DYNAMIC_SIGNED_CODEBOOK_ID,
    DYNAMIC_UNSIGNED_CODEBOOK_ID,
    SYMMETRIC_INT8_CODEBOOK_ID,
    QuantizedBlocks,
    ScaleByAdam8State,
    adamw8,
    adamw8_step,
    dequantize_blocks,
    estimate_quantized_moment_bytes,
    quantize_blocks,
    quantized_nbytes,
    scale_by_adam8,
    tree_state_nbytes,
)

__all__ = (
    "ScaleByAdamState",
    "adamw",
    "adamw_step",
    "scale_by_adam",
    "DYNAMIC_SIGNED_CODEBOOK_ID",
    "DYNAMIC_UNSIGNED_CODEBOOK_ID",
    "SYMMETRIC_INT8_CODEBOOK_ID",
    "QuantizedBlocks",
    "ScaleByAdam8State",
    "adamw8",
    "adamw8_step",
    "dequantize_blocks",
    "estimate_quantized_moment_bytes",
    "quantize_blocks",
    "quantized_nbytes",
    "scale_by_adam8",
    "tree_state_nbytes",
)
