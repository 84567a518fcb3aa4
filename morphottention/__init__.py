"""The reference package's import path, served by this build.

Callers of vhrabar/Morphottention write
``from morphottention import MorphoAttention, MorphoAttentionFunction, morpho_attention``
(``packages/morphottention/torch-ext/morphottention/__init__.py:1-3``; the attn-bench
caller ``attn-bench/src/layers/attention/morpho_attention.py:7``). Those names
resolve here to the MI355X implementation in ``morphottention_amd`` (HIP
kernels behind the same ``torch.ops.morphottention`` schemas), so such code runs
unchanged. The submodules mirror the reference's: ``morphottention.autograd``
and the op loader ``morphottention._ops`` (``ops``, ``add_op_namespace_prefix``).
"""

from .autograd import MorphoAttention, MorphoAttentionFunction, morpho_attention

__all__ = ["MorphoAttention", "MorphoAttentionFunction", "morpho_attention"]
