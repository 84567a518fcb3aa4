"""``morphottention.autograd`` (reference: ``torch-ext/morphottention/autograd.py``):
the autograd Function, the functional wrapper and the nn.Module, implemented
in ``morphottention_amd.autograd``."""

from morphottention_amd.autograd import MorphoAttention, MorphoAttentionFunction, morpho_attention, variant_bits

__all__ = ["MorphoAttention", "MorphoAttentionFunction", "morpho_attention", "variant_bits"]
