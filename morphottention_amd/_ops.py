"""Op-namespace loader for the in-tree HIP build.

Mirrors the reference loader
(``packages/morphottention/torch-ext/morphottention/_cmake_ops.py:15-30``): it
finds ``_C*.so`` next to this file and loads it with
``torch.ops.load_library``, which registers ``torch.ops.morphottention``. A
missing build raises ``ImportError`` -- there is no CPU fallback.
"""

from __future__ import annotations

import glob
import os

import torch

_NAMESPACE = "morphottention"


def _load_c_extension() -> str:
    pkg_dir = os.path.dirname(os.path.abspath(__file__))
    for pattern in ("_C*.so",):
        matches = sorted(glob.glob(os.path.join(pkg_dir, pattern)))
        if matches:
            torch.ops.load_library(matches[0])
            return matches[0]
    raise ImportError(
        f"morphottention_amd: no built '_C' extension in {pkg_dir}; "
        "build it with `python morphottention_amd/build.py` (hipcc, gfx950)"
    )


LIBRARY_PATH = _load_c_extension()

ops = getattr(torch.ops, _NAMESPACE)


def add_op_namespace_prefix(op_name: str) -> str:
    return f"{_NAMESPACE}::{op_name}"
