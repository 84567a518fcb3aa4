"""MI355X (gfx950) native Morphottention: fused morpho-attention on HIP kernels.

Drop-in for the reference package ``morphottention``
(``packages/morphottention/torch-ext/morphottention/__init__.py:1-3``).
"""

from .autograd import MorphoAttention, MorphoAttentionFunction, morpho_attention
from .soft_morph import SoftMorphAttention, SoftMorphAttentionFunction, soft_morph_attention

__all__ = ["MorphoAttention", "MorphoAttentionFunction", "morpho_attention", "SoftMorphAttention",
           "SoftMorphAttentionFunction", "soft_morph_attention"]
