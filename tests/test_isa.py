"""Code-generation checks of the large-batch kernel, without a GPU: the gfx950
assembly of csrc/stk_large.hip, compiled here with the build's flags.

The d-step loop of mainl_kernel must hold no waterfall loop: a buffer
resource the compiler takes for divergent is read into scalar registers lane
by lane around every load (v_readfirstlane, s_and_saveexec, a branch back),
which splits the MFMA / load interleave and cost 7-10 % of the kernel.  The
kernel must also make no flat memory accesses (they count on the LDS counter,
so an LDS wait would also wait for them) and use no scratch memory.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "streamtopk-sae_amd", "csrc", "stk_large.hip")
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "stk_large.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "--cuda-device-only", "-S", SRC, "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _kernel(asm, dt, sample):
    name = f"_ZN3stk12mainl_kernelILi{dt}ELb{1 if sample else 0}EEEvNS_9MainLArgsE"
    a = asm.index(name + ":")
    body = asm[a:asm.index(".Lfunc_end", a)]
    # the kernel's metadata map: its keys are sorted, so it runs from the
    # .agpr_count before .name to the next kernel's (or the map's end)
    i = asm.index(".name:           " + name)
    start = asm.rindex(".agpr_count:", 0, i)
    end = asm.find(".agpr_count:", i)
    meta = asm[start:end if end > 0 else len(asm)]
    return body, meta


def _loop_blocks(body):
    """The d-steps: each basic block of the kernel that issues MFMAs, from its
    first MFMA to its last (the tile's last step shares its block with the
    start of the epilogue, whose branches are not part of the d-step)."""
    blocks = re.split(r"\n(?=\.LBB\d+_\d+:)", body)
    out = []
    for b in blocks:
        if "v_mfma" in b:
            out.append(b[b.index("v_mfma"):b.rindex("v_mfma")])
    return out


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("sample", [False, True])
def test_dstep_loop_has_no_waterfall(asm, dt, sample):
    body, _ = _kernel(asm, dt, sample)
    loop = _loop_blocks(body)
    assert loop, "no MFMA block found"
    for blk in loop:
        assert "s_and_saveexec" not in blk and "v_readfirstlane" not in blk, blk[:400]
        # one buffer load to LDS per 16-byte chunk of the step: 32 per two d-steps
        assert blk.count("buffer_load_dwordx4") <= 32


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("sample", [False, True])
def test_no_flat_access_no_scratch(asm, dt, sample):
    body, meta = _kernel(asm, dt, sample)
    assert not re.search(r"\bflat_(load|store|atomic)", body)
    assert re.search(r"\.private_segment_fixed_size:\s+0\b", meta)
    assert re.search(r"\.vgpr_spill_count:\s+0\b", meta)
