"""CPU: resource use of the built gfx950 kernels, read from the code object
metadata of the library's own objects (tiny-llm_amd/_build/obj, built by
__graft_entry__.build()).

The decode attention kernels take a ~3.7 KB argument struct (the inline plan
metadata).  Code that takes its address -- passing it by reference to a
helper -- makes the compiler copy it into per-lane scratch memory (3800
bytes per lane), which halved the kernel's speed once; a group-8 kernel
spilling many VGPRs costs a few percent.  These checks pin both."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OBJ = os.path.join(ROOT, "tiny-llm_amd", "_build", "obj", "kernels")
LLVM = "/opt/rocm/llvm/bin"


def kernels(obj, tmp_path):
    path = os.path.join(OBJ, obj)
    if not os.path.exists(path) or not os.path.exists(os.path.join(LLVM, "llvm-readelf")):
        pytest.skip("built objects or LLVM tools not present")
    # the host object carries the device code object in its .hip_fatbin
    # section, a clang offload bundle
    fatbin = tmp_path / (obj + ".fatbin")
    elf = tmp_path / (obj + ".elf")
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}",
                    path, str(tmp_path / (obj + ".host"))], check=True, capture_output=True)
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    f"--input={fatbin}", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--output={elf}"], check=True, capture_output=True)
    notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", str(elf)], check=True,
                           capture_output=True, text=True).stdout
    out = {}
    for blk in notes.split("- .agpr_count")[1:]:
        name = re.search(r"\.name:\s+(\S+)", blk).group(1)
        if name.endswith(".kd"):
            continue
        out[name] = {k: int(re.search(rf"\.{k}:\s+(\d+)", blk).group(1))
                     for k in ("private_segment_fixed_size", "vgpr_spill_count", "vgpr_count")}
    assert out, "no kernels found"
    return out


def test_decode_kernels_use_no_argument_copy_in_scratch(tmp_path):
    ks = kernels("attention_decode.o", tmp_path)
    decode = {n: r for n, r in ks.items() if "attn_decode" in n or "attn_merge" in n}
    assert len(decode) > 100
    # (head_dim 256 at group 8 spills ~130 VGPRs: ~530 bytes, far below a copy
    # of the arguments)
    big = {n: r["private_segment_fixed_size"] for n, r in decode.items()
           if r["private_segment_fixed_size"] > 1024}
    assert not big, big


def test_default_decode_kernels_spill_little(tmp_path):
    """The VALU score path (the default for every group) at head_dim <= 128,
    per-head and head-fused, spills no VGPRs.  (At head_dim 128 and group 8
    the v_dot2 P.V's 8 heads x 8 dims of accumulators spilled up to 5; the
    MFMA P.V keeps 32 VGPRs of them.)"""
    ks = kernels("attention_decode.o", tmp_path)
    for name, r in ks.items():
        m = re.search(r"attn_decode_kernelILi(\d+)ELi(\d)ELb(\d)ELb0ELi(\d)E", name)
        if not m or int(m.group(1)) > 128:
            continue
        assert r["vgpr_spill_count"] == 0, (name, r)


def test_w8a16_kernels_use_no_scratch(tmp_path):
    """The W8A16 kernels keep their register rings, accumulators and the
    epilogue operands in registers: no per-lane scratch (a segment field
    picked by a run-time index, or a struct indexed the same way, would put
    the kernel argument block there), no VGPR spills."""
    ks = kernels("w8a16_gemm.o", tmp_path)
    dec = {n: r for n, r in ks.items() if "w8a16_dec_kernel" in n}
    assert len(dec) == 16, sorted(dec)
    for name, r in ks.items():
        assert r["private_segment_fixed_size"] == 0, (name, r)
        assert r["vgpr_spill_count"] == 0, (name, r)


def test_prefill_kernels_spill_nothing(tmp_path):
    """Both prefill workgroup forms (8 and 4 waves up to head_dim 128, 4 at
    256) keep their registers: no spills, no private memory."""
    ks = kernels("attention_prefill.o", tmp_path)
    pf = {n: r for n, r in ks.items() if "attn_prefill_kernel" in n}
    # 4 head_dims x 4 groups x 2 layouts, two wave forms below head_dim 256
    assert len(pf) == 3 * 4 * 2 * 2 + 4 * 2, sorted(pf)
    bad = {n: r for n, r in pf.items() if r["vgpr_spill_count"] or r["private_segment_fixed_size"]}
    assert not bad, bad
