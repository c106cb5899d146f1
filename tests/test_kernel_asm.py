"""Checks on the gfx950 assembly of the kernels that use LDS-DMA loads (CPU
only: hipcc cross-compiles without a GPU).

The bf16 wide kernel's K/V tiles and the f32 split-head kernel's prefetched
K/V slices and gate arrive through inline-assembly LDS-DMA loads
(`buffer_load_dwordx4 ... lds`) whose LDS address comes from M0. The asm
writes M0 itself without naming it as clobbered, because the compiler
reserves M0 and ignores such a clobber. That is only sound while the
compiled kernel has no other reader or writer of M0 (the compiler also uses
M0 for indirect register indexing, s_set_gpr_idx_on): this test compiles each
kernel with the library's flags and checks that every M0 access in its body
is one of those write-then-load triples.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tenferro-decision-rs_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# (source file, mangled-name prefix of the kernel that uses load_lds16)
KERNELS = [
    ("jeff_bf16_wide.hip", "_ZN3tfd21jeff_bf16_wide_kernel"),
    ("jeff_attention.hip", "_ZN3tfd21jeff_split_f32_kernelILi256E"),
]


@pytest.fixture(scope="module")
def asm_of(tmp_path_factory):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out_dir = tmp_path_factory.mktemp("asm")
    cache = {}

    def get(src):
        if src not in cache:
            out = out_dir / (src + ".s")
            cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                   "-I" + os.path.join(ROOT, "include"), "-I" + CSRC, "--cuda-device-only", "-S",
                   os.path.join(CSRC, src), "-o", str(out)]
            subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL,
                           timeout=900)
            cache[src] = out.read_text().splitlines()
        return cache[src]

    return get


def _body(lines, prefix):
    """Instruction lines of the kernel whose symbol starts with prefix, from
    its label to its end marker (comments and directives dropped)."""
    start = next(i for i, l in enumerate(lines) if l.startswith(prefix) and l.split(":")[0]
                 and re.match(r"^\S+:", l))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
    out = []
    for l in lines[start + 1:end]:
        l = l.split(";")[0].strip()
        if l and not l.startswith(".") and not l.endswith(":"):
            out.append(l)
    return out


@pytest.mark.parametrize("src,prefix", KERNELS, ids=[k[0] for k in KERNELS])
def test_m0_only_feeds_the_lds_dma_loads(asm_of, src, prefix):
    code = _body(asm_of(src), prefix)
    m0 = re.compile(r"\bm0\b")
    writes = [i for i, l in enumerate(code) if m0.search(l)]
    assert writes, f"{prefix} no longer sets M0: update this check"
    assert not any("s_set_gpr_idx" in l for l in code), "indirect register indexing uses M0"
    for i in writes:
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", code[i]), f"unexpected M0 use: {code[i]}"
        assert code[i + 1] == "s_nop 0", f"M0 write not followed by the asm's nop: {code[i + 1]}"
        assert re.match(r"buffer_load_dwordx4 .* lds$", code[i + 2]), \
            f"M0 write not consumed by an LDS-DMA load: {code[i + 2]}"
    dma = [i for i, l in enumerate(code) if re.match(r"buffer_load_\w+ .* lds$", l)]
    assert sorted(i + 2 for i in writes) == dma, "an LDS-DMA load without its own M0 write"
