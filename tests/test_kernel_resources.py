"""Register budget of the decode kernels, read from the gfx950 code object
metadata of a device-only compile (CPU only; hipcc cross-compiles).

The one-tensor automaton kernel keeps 4 workgroups of 512 lanes per CU,
i.e. 8 waves per SIMD, only while it stays within 64 VGPRs and 80 SGPRs
and spills nothing in its block loop: above that the hardware fits fewer
waves and the decode slows down.  A source change that crosses the budget
fails here, before any GPU run."""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)

pytestmark = pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc"), reason="no hipcc")


@pytest.fixture(scope="module")
def kernel_meta(tmp_path_factory):
    from ecf8_amd.build import ARCH, HIPCC

    out = tmp_path_factory.mktemp("asm") / "decode.s"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-mcode-object-version=5",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(REPO, "include"), "--cuda-device-only", "-S", "-o", str(out),
           os.path.join(REPO, "ecf8_amd", "csrc", "ecf8_decode.hip")]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    text = out.read_text()
    section = text[text.find("amdhsa.kernels"):]
    meta = {}
    for entry in re.split(r"\n  - ", section):
        m = re.search(r"\.name:\s+(\S+)", entry)
        if m:
            meta[m.group(1)] = {k: int(v) for k, v in re.findall(
                r"\.(vgpr_count|sgpr_count|vgpr_spill_count|sgpr_spill_count|"
                r"group_segment_fixed_size):\s+(\d+)", entry)}
    shutil.rmtree(out.parent, ignore_errors=True)
    return meta


def _find(meta, *parts):
    names = [n for n in meta if all(p in n for p in parts)]
    assert len(names) == 1, (parts, names)
    return meta[names[0]]


def test_one_tensor_kernel_fits_eight_waves_per_simd(kernel_meta):
    m = _find(kernel_meta, "decode_dfa_kernelILi512ELb0ELb0E")
    assert m["vgpr_count"] <= 64, m
    assert m["sgpr_count"] <= 80, m
    assert m["vgpr_spill_count"] == 0 and m["sgpr_spill_count"] == 0, m
    # static LDS: automaton (6152 dwords) + wave totals + edge slots
    assert m["group_segment_fixed_size"] <= 24_704, m


@pytest.mark.parametrize("select", ["Lb0E", "Lb1E"])
def test_batched_kernel_stays_within_the_same_budget(kernel_meta, select):
    """Both instances (whole launches; routed launches selecting in the
    kernel) keep eight waves per SIMD and four workgroups per CU: 64 VGPRs,
    80 SGPRs, and static LDS that leaves room for a staging buffer; the
    whole-launch instance carries no task table."""
    m = _find(kernel_meta, "decode_dfa_batched_kernelILi512E" + select)
    assert m["vgpr_count"] <= 64, m
    assert m["sgpr_count"] <= 80, m
    assert m["group_segment_fixed_size"] <= (24_704 if select == "Lb0E" else 25_760), m
