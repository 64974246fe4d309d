"""Register budgets the kernels' co-residency depends on, read from the gfx950
code objects of the built library (zealot_amd/_build/*.o).

A mixed runner step runs the chunk prefill (side stream) and the decode (cache
stream) together, each on part of every CU: one four-wave prefill workgroup and
two decode waves a CU.  The plan kernels are one 1024-thread workgroup (four
waves on every SIMD) that must start while those waves are resident; with more
than 64 VGPRs a lane the prefill plan cannot be placed beside a decode wave and
the chunks' attention runs after the decode instead of beside it (a regression
this file guards: 0.73 -> 0.87 ms a mixed step)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "zealot_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
SIMD_VGPRS = 512  # unified VGPR + AGPR file of a gfx950 SIMD, per lane
GRANULE = 8


def _tools():
    bundler = os.path.join(LLVM, "clang-offload-bundler")
    readelf = os.path.join(LLVM, "llvm-readelf")
    objcopy = shutil.which("objcopy") or os.path.join(LLVM, "llvm-objcopy")
    if not all(os.path.exists(t) for t in (bundler, readelf, objcopy)):
        pytest.skip("ROCm LLVM tools not found")
    return bundler, readelf, objcopy


def kernel_registers(obj_name: str, tmp_path) -> dict:
    """{kernel symbol: (vgpr_count, agpr_count, private_segment_fixed_size)} of one object."""
    obj = os.path.join(BUILD, obj_name)
    if not os.path.exists(obj):
        pytest.skip(f"{obj_name} not built (run python -m zealot_amd.build)")
    bundler, readelf, objcopy = _tools()
    fb = tmp_path / (obj_name + ".fatbin")
    co = tmp_path / (obj_name + ".co")
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fb}", obj, str(tmp_path / "scratch.o")], check=True,
                   capture_output=True)
    subprocess.run([bundler, "--unbundle", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={fb}", f"--output={co}"], check=True, capture_output=True)
    notes = subprocess.run([readelf, "--notes", str(co)], check=True, capture_output=True, text=True).stdout
    out, cur = {}, {}
    for line in notes.splitlines():
        s = line.strip()
        if s.startswith("- ") and cur:  # a new kernel's map starts
            if "name" in cur:
                out[cur["name"]] = (cur.get("vgpr", 0), cur.get("agpr", 0), cur.get("priv", 0))
            cur = {}
        s = s[2:] if s.startswith("- ") else s
        key, _, val = s.partition(":")
        val = val.strip()
        if key == ".name":
            cur["name"] = val
        elif key == ".vgpr_count":
            cur["vgpr"] = int(val)
        elif key == ".agpr_count":
            cur["agpr"] = int(val)
        elif key == ".private_segment_fixed_size":
            cur["priv"] = int(val)
    if "name" in cur:
        out[cur["name"]] = (cur.get("vgpr", 0), cur.get("agpr", 0), cur.get("priv", 0))
    return out


def _alloc(vgprs: int) -> int:
    return -(-vgprs // GRANULE) * GRANULE


def _one(regs: dict, needle: str):
    hits = [v for k, v in regs.items() if needle in k]
    assert hits, f"no kernel matching {needle}"
    return hits[0]


def test_plan_kernels_fit_beside_attention_waves(tmp_path):
    dec = kernel_registers("paged_decode.o", tmp_path)
    pre = kernel_registers("paged_prefill.o", tmp_path)
    plan = _one(dec, "plan_kernelENS_6Params")
    pplan = _one(pre, "prefill_plan_kernel")
    decode = _one(dec, "decode_mfma_kernelILi1ELi128ELi4E")  # bf16, D = 128, G = 4: the mixed step's decode
    for name, (v, a, priv) in (("plan_kernel", plan), ("prefill_plan_kernel", pplan)):
        assert v + a <= 64, f"{name}: {v} VGPRs + {a} AGPRs a lane (at most 64)"
        assert priv == 0, f"{name} spills {priv} bytes a lane"
        # four of its waves on a SIMD beside one resident decode wave
        assert 4 * _alloc(v + a) + _alloc(decode[0] + decode[1]) <= SIMD_VGPRS


def test_attention_kernels_register_budgets(tmp_path):
    """The prefill kernel runs two waves a SIMD (two four-wave workgroups a
    CU), so a wave holds at most 256 registers; the decode kernel one wave a
    SIMD.  In a mixed step a prefill wave and a decode wave may share a SIMD.
    Neither kernel spills."""
    dec = kernel_registers("paged_decode.o", tmp_path)
    pre = kernel_registers("paged_prefill.o", tmp_path)
    decode = _one(dec, "decode_mfma_kernelILi1ELi128ELi4E")
    prefill = _one(pre, "prefill_mfma_kernelILi1ELi128ELi4E")
    assert _alloc(prefill[0] + prefill[1]) <= SIMD_VGPRS // 2
    assert _alloc(decode[0] + decode[1]) + _alloc(prefill[0] + prefill[1]) <= SIMD_VGPRS
    assert decode[2] == 0 and prefill[2] == 0, "attention kernels must not spill"
