"""Checks the generated gfx950 assembly (CPU only; this file is not sent to GPU boxes).

Every kernel must write memory through vector instructions only (no scalar
data-cache stores, atomics, write-back or discard), and no packed fp32
arithmetic may be formed.
"""
from __future__ import annotations

import re
import subprocess

from .conftest import ROOT


def test_device_code_has_no_scalar_memory_writes(tmp_path):
    """The gfx950 assembly of every kernel source writes memory through vector instructions only."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("_b", ROOT / "megaqwen-a10_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    bad = re.compile(r"^\s*(s_store|s_buffer_store|s_scratch_store|s_atomic|s_buffer_atomic|s_dcache_wb|s_dcache_discard)",
                     re.M)
    for src in b.sources():
        out = tmp_path / (src.stem + ".s")
        subprocess.run([b.hipcc(), *b.HIPCC_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)],
                       check=True, capture_output=True)
        text = out.read_text()
        assert not bad.search(text), f"{src.name} uses scalar memory writes"
        assert "v_pk_fma_f32" not in text and "v_pk_mul_f32" not in text and "v_pk_add_f32" not in text, src.name
