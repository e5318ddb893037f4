"""Register spills of the kernels in the built library (CPU test).

A spill costs scratch-memory traffic inside a kernel's inner loop, and a
rewrite that changes no result can introduce one: the rotary-embedding
rotation written with explicit fused multiply-adds made the n_embd-4096
Hadamard kernel spill 178 registers and run 2.2x slower while every parity
test still passed.  This test reads the AMDGPU code-object metadata of
walsh-research_amd/lib/libwalsh_hip.so (the .hip_fatbin section: one clang
offload bundle per source file, each holding a gfx950 ELF whose notes list
every kernel's .vgpr_count and .vgpr_spill_count) and bounds the spill count
of every kernel: zero unless the kernel is listed below with the count it
has today.
"""
import os
import re
import shutil
import struct
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "walsh-research_amd", "lib", "libwalsh_hip.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

# kernels allowed to spill (mangled-name fragment -> most spilled VGPRs):
# backward and fp32 variants off the measured inference path, the n = 8
# Sinkhorn backward (n <= 4 takes sinkhorn_bwd_lds_kernel), and a few
# registers in epilogues outside the inner loops
ALLOWED = {
    "sinkhorn_bwd_kernelILi8E": 244,
    "hadamard_bwd_kernelIfLb0ELb0ELb1E": 141,
    "hadamard_bwd_kernelIfLb0ELb0ELb0E": 139,
    "hadamard_bwd_kernelIfLb0ELb1ELb1E": 134,
    "hadamard_bwd_kernelIfLb0ELb1ELb0E": 128,
    "hadamard_bwd_kernelItLb1ELb0ELb1E": 70,
    "hadamard_bwd_kernelItLb1ELb0ELb0E": 68,
    "hadamard_bwd_kernelItLb1ELb1ELb1E": 14,
    "hadamard_bwd_kernelItLb1ELb1ELb0E": 14,
    "hadamard_wide_kernelIfLb0ELb0E": 55,
    "hadamard_wide_kernelIfLb0ELb1E": 51,
    "hadamard_wide_kernelItLb1ELb0E": 3,
    "hadamard_wide_kernelItLb1ELb1E": 2,
    "hadamard_swiglu_kernelItLb1ELb0ELb1E": 31,
    "hadamard_swiglu_kernelItLb1ELb0ELb0E": 2,
    "hadamard_swiglu_kernelIfLb0ELb1ELb1E": 2,
    "hadamard_swiglu_kernelIfLb0ELb0ELb0E": 2,
    "hadamard_fwd_kernelItLb1ELb0ELb0ELb0ELb0E": 2,
    "hadamard_fwd_kernelIfLb0ELb0ELb0ELb0ELb0E": 2,
    "hadamard_wide3_kernelILi0ELb1E": 3,       # head mixer at head_dim 128
    "gemm256_silu_kernel": 4,                   # epilogue (SiLU), outside the K loop
    "gemm256_beta_kernel": 3,                   # epilogue (beta), outside the K loop
    "gemm256_beta_f32_kernel": 5,               # epilogue (bf16 rounding, beta, float32 stores)
}


def _tool(name):
    path = os.path.join(LLVM, name)
    return path if os.path.exists(path) else shutil.which(name)


def kernel_resources(lib=LIB):
    """{mangled kernel name: (vgpr_count, vgpr_spill_count)} of every gfx950
    kernel in the library."""
    objcopy, readelf = _tool("llvm-objcopy"), _tool("llvm-readelf")
    if not objcopy or not readelf:
        pytest.skip("llvm-objcopy / llvm-readelf not found")
    out = {}
    with tempfile.TemporaryDirectory() as d:
        fat = os.path.join(d, "fat.bin")
        subprocess.run([objcopy, "--dump-section", f".hip_fatbin={fat}", lib], check=True, capture_output=True)
        data = open(fat, "rb").read()
        for bi, st in enumerate(m.start() for m in re.finditer(re.escape(MAGIC), data)):
            # bundle: magic, entry count, then per entry offset, size, triple
            # length and triple; offsets from the bundle's start
            (n,) = struct.unpack_from("<Q", data, st + len(MAGIC))
            p = st + len(MAGIC) + 8
            for _ in range(n):
                off, size, tl = struct.unpack_from("<QQQ", data, p)
                p += 24
                triple = data[p:p + tl].decode()
                p += tl
                if "gfx950" not in triple or size == 0:
                    continue
                co = os.path.join(d, f"co{bi}.o")
                with open(co, "wb") as f:
                    f.write(data[st + off:st + off + size])
                notes = subprocess.run([readelf, "--notes", co], check=True, capture_output=True, text=True).stdout
                for m in re.finditer(r"\.name:\s+(\S+)(.*?)(?=\n\s+- \.|\Z)", notes, re.S):
                    spill = re.search(r"\.vgpr_spill_count:\s+(\d+)", m.group(2))
                    vgpr = re.search(r"\.vgpr_count:\s+(\d+)", m.group(2))
                    if spill and vgpr:
                        out[m.group(1)] = (int(vgpr.group(1)), int(spill.group(1)))
    return out


@pytest.fixture(scope="module")
def resources():
    if not os.path.exists(LIB):
        pytest.skip("library not built (python -c 'import __graft_entry__ as g; g.build()')")
    return kernel_resources()


def test_library_holds_the_hot_kernels(resources):
    names = " ".join(resources)
    for k in ("hadamard_fwd_kernel", "hadamard_wide3_kernel", "hadamard_split3_kernel", "gemm256_beta_kernel",
              "gemm256_silu_kernel", "gemm256_f32_kernel", "mhc_pre2_kernel", "moe_ffn_kernel",
              "router_w2_topk_kernel", "decode_attn_partial_kernel", "prefill_attn_head_kernel"):
        assert k in names, k
    assert len(resources) > 100


def test_spills_within_bounds(resources):
    over = []
    for name, (vgpr, spill) in resources.items():
        allowed = max([v for k, v in ALLOWED.items() if k in name] or [0])
        if spill > allowed:
            over.append((name, vgpr, spill, allowed))
    assert not over, "kernels spilling beyond their bound (name, vgprs, spills, allowed): %s" % over
