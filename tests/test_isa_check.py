"""Checks the generated gfx950 assembly (CPU only; this file is not sent to GPU boxes).

Every kernel must write memory through vector instructions only (no scalar
data-cache stores, atomics, write-back or discard), and no packed fp32
arithmetic may be formed. The decode kernels copy their per-layer pointer
tables into LDS before anything else, so none may read LDS before its first
workgroup barrier (a wave would otherwise read table words another wave has
not written yet, and dereference what the previous kernel left in LDS).
"""
from __future__ import annotations

import re
import subprocess

from .conftest import ROOT


def _builder():
    import importlib.util
    spec = importlib.util.spec_from_file_location("_b", ROOT / "megaqwen-a10_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    return b


def _kernel_bodies(text):
    """(name, body) of every function in a gfx950 assembly listing: from the
    function's own label to the next .Lfunc_end label."""
    for name in re.findall(r"^\s*\.type\s+([^,\s]+),@function", text, flags=re.M):
        m = re.search(r"^" + re.escape(name) + r":.*?\n(.*?)^\.Lfunc_end\d+:", text, flags=re.M | re.S)
        if m:
            yield name, m.group(1)


def lds_reads_before_first_barrier(text):
    """Names of the decode kernels in which an LDS read precedes the first s_barrier."""
    bad = []
    for name, body in _kernel_bodies(text):
        if "decode" not in name or "kernel" not in name:
            continue
        first_barrier = body.find("s_barrier")
        head = body if first_barrier < 0 else body[:first_barrier]
        if re.search(r"^\s*ds_(read|load)", head, flags=re.M):
            bad.append(name)
    return bad


def test_decode_kernels_read_lds_only_after_a_barrier(tmp_path):
    b = _builder()
    seen = 0
    for src in b.sources():
        if "decode" not in src.stem:
            continue
        out = tmp_path / (src.stem + ".s")
        subprocess.run([b.hipcc(), *b.HIPCC_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)],
                       check=True, capture_output=True)
        text = out.read_text()
        seen += sum(1 for n, _ in _kernel_bodies(text) if "decode" in n and "kernel" in n)
        assert not lds_reads_before_first_barrier(text), (src.name, lds_reads_before_first_barrier(text))
    assert seen >= 3


def test_lds_order_check_flags_a_read_before_the_barrier():
    listing = ("\t.type\t_Z13decode_kernelv,@function\n_Z13decode_kernelv:\n\tglobal_load_dwordx2 v[0:1], v[2:3], off\n\tds_write_b64 v1, v[0:1]\n"
               "\tds_read_b64 v[4:5], v4\n\ts_barrier\n\ts_endpgm\n.Lfunc_end0:\n")
    assert lds_reads_before_first_barrier(listing) == ["_Z13decode_kernelv"]
    fixed = listing.replace("\tds_read_b64 v[4:5], v4\n\ts_barrier\n", "\ts_barrier\n\tds_read_b64 v[4:5], v4\n")
    assert lds_reads_before_first_barrier(fixed) == []


def test_device_code_has_no_scalar_memory_writes(tmp_path):
    """The gfx950 assembly of every kernel source writes memory through vector instructions only."""
    b = _builder()
    bad = re.compile(r"^\s*(s_store|s_buffer_store|s_scratch_store|s_atomic|s_buffer_atomic|s_dcache_wb|s_dcache_discard)",
                     re.M)
    for src in b.sources():
        out = tmp_path / (src.stem + ".s")
        subprocess.run([b.hipcc(), *b.HIPCC_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)],
                       check=True, capture_output=True)
        text = out.read_text()
        assert not bad.search(text), f"{src.name} uses scalar memory writes"
        assert "v_pk_fma_f32" not in text and "v_pk_mul_f32" not in text and "v_pk_add_f32" not in text, src.name
