"""Checks of the gfx950 code the compiler makes for the kernels (no GPU).

The masked-score loops of the backward once compiled (masked-diagonal
instances) to divergent if-blocks whose bodies were empty: the stores of -inf
had been dropped for the lanes that reached them, so the causal and diagonal
masks were lost while the kernels still ran to completion. A divergent block
with an empty body is ``s_and_saveexec_b64 X, C`` followed at once by
``s_or_b64 exec, exec, X``; none may remain in any kernel.
"""

from __future__ import annotations

import concurrent.futures
import importlib.util
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "morphottention_amd", "csrc")


def _build_module():
    spec = importlib.util.spec_from_file_location("_morpho_build", os.path.join(ROOT, "morphottention_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def empty_divergent_blocks(asm: str) -> dict[str, int]:
    """Kernel name -> number of divergent if-blocks without a body."""
    hits: dict[str, int] = {}
    kernel = None
    lines = asm.splitlines()
    for k, line in enumerate(lines):
        m = re.match(r"^(_Z\w+):", line)
        if m:
            kernel = m.group(1)
        m = re.match(r"^\s+s_and_saveexec_b64 (s\[\d+:\d+\]), ", line)
        if m and k + 1 < len(lines) and re.match(r"^\s+s_or_b64 exec, exec, " + re.escape(m.group(1)) + r"\s*$",
                                                 lines[k + 1]):
            hits[kernel] = hits.get(kernel, 0) + 1
    return hits


def test_scanner_finds_an_empty_block():
    asm = ("_ZN6morpho1kEv:\n\ts_and_saveexec_b64 s[60:61], s[58:59]\n\ts_or_b64 exec, exec, s[60:61]\n"
           "_ZN6morpho1jEv:\n\ts_and_saveexec_b64 s[60:61], s[58:59]\n\tv_mov_b32_e32 v1, s2\n"
           "\ts_or_b64 exec, exec, s[60:61]\n")
    assert empty_divergent_blocks(asm) == {"_ZN6morpho1kEv": 1}


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_no_kernel_has_an_empty_divergent_block(tmp_path):
    b = _build_module()
    sources = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip") and f != "capi.hip")

    def asm_of(src):
        out = tmp_path / (src + ".s")
        subprocess.run([b.HIPCC, *b.flags_for(src), "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", str(out)],
                       check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
        return src, out.read_text()

    with concurrent.futures.ThreadPoolExecutor(max_workers=len(sources)) as ex:
        results = list(ex.map(asm_of, sources))
    for src, asm in results:
        assert re.search(r"^_ZN6morpho\w*_kernel", asm, re.M), src  # the file's kernels were compiled
        assert empty_divergent_blocks(asm) == {}, src
