"""``morphottention._ops``: the op namespace and its prefix helper under the
names the reference's autograd module imports (``autograd.py:10-13``, from its
``_ops`` or ``_cmake_ops`` loader). Loading ``morphottention_amd`` registers the
``torch.ops.morphottention`` ops from the in-tree ``_C.so`` and raises
ImportError when the build is missing."""

from morphottention_amd._ops import add_op_namespace_prefix, ops

__all__ = ["ops", "add_op_namespace_prefix"]
