"""Compile-time checks of the gfx950 code (CPU only: hipcc cross-compiles without a GPU).

Every kernel of libpthdec.so must run without scratch memory: a spill to scratch in the decode
or prefill kernels costs a memory round trip per spilled value inside the tile loop. The check
compiles each kernel source to gfx950 assembly with the flags of the product build and reads
each kernel's `.private_segment_fixed_size` from the code-object metadata.
"""
import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "mi50-vllm-lab_amd")


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    return None


@pytest.fixture(scope="module")
def gfx950_asm(tmp_path_factory):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    sys.path.insert(0, PKG_DIR)
    try:
        import build as pd_build
    finally:
        sys.path.remove(PKG_DIR)
    flags = [f for f in pd_build.HIP_FLAGS if f not in ("-shared", "-fPIC")]
    tmp = tmp_path_factory.mktemp("asm")
    text = []
    for src in pd_build.KERNEL_SOURCES:
        out = str(tmp / (os.path.basename(src) + ".s"))
        cmd = [hipcc, *flags, "--cuda-device-only", "-S", "-I", os.path.join(ROOT, "include"), src, "-o", out]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, (src, res.stderr[-4000:])
        with open(out) as f:
            text.append(f.read())
    return text


def _kernel_metadata(asms):
    """{kernel name: metadata text} from the amdhsa.kernels lists of the code objects."""
    out = {}
    for asm in asms:
        meta = asm[asm.index("amdhsa.kernels:"):]
        entries = re.split(r"\n  - ", meta)
        for e in entries[1:]:
            m = re.search(r"\.name:\s+(\S+)", e)
            if m:
                out[m.group(1)] = e
    return out


def test_every_kernel_is_built(gfx950_asm):
    names = _kernel_metadata(gfx950_asm)
    for k in ("pd_partial_kernel", "pd_combine_kernel", "pd_prefill_kernel", "pd_cache_write_kernel"):
        assert any(k in n for n in names), (k, sorted(names))
    # decode: one to three 16-row blocks, fast and general block-size paths
    assert sum("pd_partial_kernel" in n for n in names) == 6


def test_no_kernel_uses_scratch(gfx950_asm):
    meta = _kernel_metadata(gfx950_asm)
    scratch = {}
    for name, text in meta.items():
        m = re.search(r"\.private_segment_fixed_size:\s+(\d+)", text)
        assert m, name
        scratch[name] = int(m.group(1))
    assert all(v == 0 for v in scratch.values()), {k: v for k, v in scratch.items() if v}


def test_no_packed_fp32_instructions(gfx950_asm):
    # the build disables the packed-FP32 VALU forms; none may appear in the code
    for asm in gfx950_asm:
        assert not re.search(r"\bv_pk_(add|mul|fma)_f32\b", asm)
