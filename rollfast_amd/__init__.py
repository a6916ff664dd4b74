"""rollfast_amd: rollfast's 8-bit AdamW step on MI355X (gfx950) HIP kernels.

Drop-in for the reference's adam8 hot path (rollfast ``adamw8``,
``scale_by_adam8``, ``quantize_blocks``, ``dequantize_blocks``,
``apply_updates``) and its full-precision sibling (``adamw``,
``scale_by_adam``): same names, arguments, state pytree and errors, with
torch tensors on a ROCm device in place of jax arrays.  ``adamw8_step`` /
``adamw_step`` fuse ``tx.update`` and ``apply_updates`` into one HBM pass.
"""

from . import prng
from ._base import (
    ApplyIfFiniteState,
    EmptyState,
    GradientTransformation,
    GradientTransformationExtraArgs,
    MaskedNode,
    MaskedState,
    ScaleByScheduleState,
)
from .optim.adam8 import (
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
from .optim.adam import ScaleByAdamState, adamw, adamw_step, scale_by_adam
from .optim.convert import adam8_state_from_adam, adam_state_from_adam8, dequantize_state_tree, quantize_state_tree
from .combine import MultiTransformState, chain, masked, multi_transform
from .transforms import GlobalNormClipState, apply_if_finite, clip_by_global_norm
from .multisteps import MultiSteps, MultiStepsState
from .utils import apply_updates, apply_updates_prefix

__version__ = "0.1.0"

__all__ = (
    "DYNAMIC_SIGNED_CODEBOOK_ID",
    "DYNAMIC_UNSIGNED_CODEBOOK_ID",
    "SYMMETRIC_INT8_CODEBOOK_ID",
    "ApplyIfFiniteState",
    "EmptyState",
    "GlobalNormClipState",
    "GradientTransformation",
    "GradientTransformationExtraArgs",
    "MaskedNode",
    "MaskedState",
    "MultiSteps",
    "MultiStepsState",
    "MultiTransformState",
    "QuantizedBlocks",
    "ScaleByAdam8State",
    "ScaleByAdamState",
    "ScaleByScheduleState",
    "adam8_state_from_adam",
    "adam_state_from_adam8",
    "adamw",
    "adamw8",
    "adamw8_step",
    "adamw_step",
    "apply_if_finite",
    "apply_updates",
    "apply_updates_prefix",
    "chain",
    "clip_by_global_norm",
    "dequantize_blocks",
    "dequantize_state_tree",
    "estimate_quantized_moment_bytes",
    "masked",
    "multi_transform",
    "prng",
    "quantize_blocks",
    "quantize_state_tree",
    "quantized_nbytes",
    "scale_by_adam",
    "scale_by_adam8",
    "tree_state_nbytes",
)
