"""The built library's gfx950 kernels keep their working set in registers: no kernel of the automatic
configurations may use scratch (private segment) memory, which would put spills on the streaming path.  Reads
the code object of the in-tree build (the kernel descriptors' .private_segment_fixed_size) with the ROCm LLVM
tools; skipped when the library or the tools are absent.  The one family allowed scratch is the MFMA kernel with
two tiles a wavefront at depth 8 (an explicit-configuration shape no automatic choice uses, 20 bytes)."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "qwen-a100-fastpath_amd", "qwen_fastpath", "libqf_w8a16.so")
ATTN = os.path.join(ROOT, "qwen-a100-fastpath_amd", "qwen_fastpath", "libqf_spec_attn.so")
LLVM = "/opt/rocm/llvm/bin"
# w8a16_mfma_kernel<LAYOUT, NT = 2, WN, WK, DEPTH = 8, ...>
ALLOWED = re.compile(r"^_ZN2qf17w8a16_mfma_kernelILi[01]ELi2ELi\d+ELi\d+ELi8E")


def _kernel_scratch(lib):
    objdump, readelf = os.path.join(LLVM, "llvm-objdump"), os.path.join(LLVM, "llvm-readelf")
    if not (os.path.exists(lib) and os.path.exists(objdump) and os.path.exists(readelf)):
        pytest.skip("built library or ROCm LLVM tools absent")
    with tempfile.TemporaryDirectory() as d:
        copy = os.path.join(d, "lib.so")
        shutil.copy(lib, copy)
        subprocess.run([objdump, "--offloading", copy], cwd=d, check=True, capture_output=True)
        cos = [f for f in os.listdir(d) if "gfx950" in f]
        assert cos, "no gfx950 code object in the library"
        notes = subprocess.run([readelf, "--notes", os.path.join(d, cos[0])], check=True, capture_output=True,
                               text=True).stdout
    names = re.findall(r"\.name:\s+(\S+)", notes)
    sizes = [int(v) for v in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)]
    assert len(names) == len(sizes) and names
    return dict(zip(names, sizes))


def test_w8a16_kernels_use_no_scratch():
    k = _kernel_scratch(LIB)
    bad = {n: s for n, s in k.items() if s and not ALLOWED.match(n)}
    assert not bad, bad
    assert any("w8a16_stream_kernel" in n for n in k) and any("argmax_slots_kernel" in n for n in k)


def test_attention_kernels_use_no_scratch():
    k = _kernel_scratch(ATTN)
    bad = {n: s for n, s in k.items() if s}
    assert not bad, bad
