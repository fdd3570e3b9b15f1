"""The layer ops of ``collab_infer.models.llama`` (collab_infer/models/llama.py:44-88, 305):
RMSNorm, rotary embedding, the half-split rotation and the gated activations, computed by the
gfx950 kernels with the reference's rounding points."""

from ..layers import (  # noqa: F401
    ACTIVATION_CODES,
    RMSNorm,
    RotaryEmbedding,
    apply_rotary,
    gated_activation,
    gated_mul,
)

__all__ = ["RMSNorm", "RotaryEmbedding", "apply_rotary", "gated_activation", "gated_mul"]
