"""Code-generation checks of the candidate-buffer kernels, without a GPU: the
gfx950 assembly of csrc/stk_approx.hip, compiled here with the build's flags.

group_kernel keeps a whole tile of accumulators and eight sort keys per lane
in registers (8 waves per workgroup, so at most 256 VGPRs per lane): a spill
or an indexed key array would put the sort network in scratch memory.  Every
instantiation (dtype x row blocks x c) is checked.  The lane exchanges of the
full sort (c = 128) must stay DPP moves (fused into the min / max when the
compiler can) apart from the one stride that goes through ds_bpermute.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "streamtopk-sae_amd", "csrc", "stk_approx.hip")
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "stk_approx.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "--cuda-device-only", "-S", SRC, "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _kernel(asm, name):
    a = asm.index(name + ":")
    body = asm[a:asm.index(".Lfunc_end", a)]
    i = asm.index(".name:           " + name)
    start = asm.rindex(".agpr_count:", 0, i)
    end = asm.find(".agpr_count:", i)
    return body, asm[start:end if end > 0 else len(asm)]


def _group(dt, nb, c):
    return f"_ZN3stk12group_kernelILi{dt}ELi{nb}ELi{c}EEEvNS_9GroupArgsE"


GROUP = [_group(dt, nb, c) for dt in (0, 1, 2) for nb in (1, 2, 4) for c in (16, 32, 64, 128)]


@pytest.mark.parametrize("name", GROUP + ["_ZN3stk11cand_kernelENS_8CandArgsE"])
def test_no_scratch_no_spill(asm, name):
    body, meta = _kernel(asm, name)
    assert re.search(r"\.private_segment_fixed_size:\s+0\b", meta)
    assert re.search(r"\.vgpr_spill_count:\s+0\b", meta)
    assert not re.search(r"\bscratch_(load|store)", body)


@pytest.mark.parametrize("nb", [1, 2, 4])
def test_sort_exchanges(asm, nb):
    body, meta = _kernel(asm, _group(2, nb, 128))
    assert int(re.search(r"\.vgpr_count:\s+(\d+)", meta).group(1)) <= 256
    dpp = len(re.findall(r"\bv_\w+_dpp\b", body))
    # per sort: 9 of the 10 exchange stages are DPP (the flips of 16 .. 128
    # entries, the half-cleaners of strides 8 and 16); per 32-row block two
    # rounds of the 32-bit network (8 keys per lane) and two of the 64-bit one
    assert dpp >= nb * 2 * 9 * (8 + 16)
    for ctl in ("row_mirror", "row_half_mirror", "quad_perm:[3,2,1,0]", "quad_perm:[1,0,3,2]",
                "quad_perm:[2,3,0,1]"):
        assert ctl in body, ctl
    # stride 32 (one half-cleaner) of both networks, and the check's read of the next lane
    assert body.count("ds_bpermute_b32") == nb * 2 * (8 + 1 + 16)
