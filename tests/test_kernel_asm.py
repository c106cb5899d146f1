"""Checks on the gfx950 assembly of the bf16 wide kernel (CPU only: hipcc
cross-compiles without a GPU).

The kernel's K/V tile loads are inline-assembly LDS-DMA loads
(`buffer_load_dwordx4 ... lds`) whose LDS address comes from M0. The asm
writes M0 itself without naming it as clobbered, because the compiler
reserves M0 and ignores such a clobber. That is only sound while the compiled
kernel has no other reader or writer of M0: this test compiles the kernel
with the library's flags and checks that every M0 access is one of those
write-then-load triples.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tenferro-decision-rs_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.fixture(scope="module")
def wide_asm(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "jeff_bf16_wide.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "--cuda-device-only", "-S",
           os.path.join(CSRC, "jeff_bf16_wide.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                   timeout=600)
    return out.read_text().splitlines()


def _code(lines):
    """Instruction lines (comments and directives dropped), in order."""
    out = []
    for l in lines:
        l = l.split(";")[0].strip()
        if l and not l.startswith(".") and not l.endswith(":"):
            out.append(l)
    return out


def test_m0_only_feeds_the_lds_dma_loads(wide_asm):
    code = _code(wide_asm)
    m0 = re.compile(r"\bm0\b")
    writes = [i for i, l in enumerate(code) if m0.search(l)]
    assert writes, "the wide kernel no longer sets M0: update this check"
    for i in writes:
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", code[i]), f"unexpected M0 use: {code[i]}"
        assert code[i + 1] == "s_nop 0", f"M0 write not followed by the asm's nop: {code[i + 1]}"
        assert re.match(r"buffer_load_dwordx4 .* lds$", code[i + 2]), \
            f"M0 write not consumed by an LDS-DMA load: {code[i + 2]}"
    dma = [i for i, l in enumerate(code) if re.match(r"buffer_load_\w+ .* lds$", l)]
    assert sorted(i + 2 for i in writes) == dma, "an LDS-DMA load without its own M0 write"
