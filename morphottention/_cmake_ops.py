"""``morphottention._cmake_ops``: the reference's second loader module name.

The reference's autograd module imports ``ops`` and ``add_op_namespace_prefix``
from ``._ops`` (a Hub build) or, failing that, from ``._cmake_ops`` (a local
CMake / PyPI build) (``torch-ext/morphottention/autograd.py:10-13``,
``_cmake_ops.py:15-30``). Both names resolve to the same in-tree loader here:
importing it registers ``torch.ops.morphottention`` from the built ``_C.so``
and raises ImportError when the build is missing.
"""

from morphottention_amd._ops import add_op_namespace_prefix, ops

__all__ = ["ops", "add_op_namespace_prefix"]
