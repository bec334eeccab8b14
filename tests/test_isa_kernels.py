"""Code-generation checks of the exact path's kernels, without a GPU: the
gfx950 assembly of csrc/stk_kernels.hip, compiled here with the build's flags.

No kernel may use scratch memory (a register spill or an indexed register
array), including the 512-thread selection kernels (the merge's two threads
per segment, the large sample's threshold), whose thread count halves the
registers a lane may hold.  main_kernel (8 waves, two per SIMD) must stay
within 256 VGPRs per lane.  The merges after mainl_kernel (256 threads) must
leave room for four workgroups per CU -- at most 128 registers per lane and
40 KiB of LDS each -- so that a large batch's rows (1024 at config 4, four per
CU) are merged in one round.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "streamtopk-sae_amd", "csrc", "stk_kernels.hip")
HIPCC = "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa") / "stk_kernels.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "--cuda-device-only", "-S", SRC, "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _kernels(asm):
    return re.findall(r"^\s+\.name:\s+(_ZN3stk\w+)\s*$", asm, re.M)


def _meta(asm, name):
    i = asm.index(".name:           " + name)
    start = asm.rindex(".agpr_count:", 0, i)
    end = asm.find(".agpr_count:", i)
    return asm[start:end if end > 0 else len(asm)]


def test_every_kernel_without_scratch(asm):
    names = _kernels(asm)
    # main, sample, thr (two sizes), merge (dense and segmented), pack, probe
    for part in ("main_kernel", "sample_kernel", "thr_kernel", "merge_kernel", "merge_seg_kernel",
                 "pack_kernel", "read_probe_kernel"):
        assert any(part in n for n in names), part
    for n in names:
        meta = _meta(asm, n)
        assert re.search(r"\.private_segment_fixed_size:\s+0\b", meta), n
        assert re.search(r"\.vgpr_spill_count:\s+0\b", meta), n
        body = asm[asm.index(n + ":"):asm.index(".Lfunc_end", asm.index(n + ":"))]
        assert not re.search(r"\bscratch_(load|store)", body), n


def test_selection_kernels_at_512_threads(asm):
    names = _kernels(asm)
    wide = [n for n in names if ("merge_seg_kernel" in n or "thr_kernel" in n) and "Li512E" in n]
    # the four merge widths and the large sample's threshold
    assert len(wide) == 5, wide


def test_main_kernel_registers(asm):
    for n in _kernels(asm):
        if "main_kernel" in n:
            vgpr = int(re.search(r"\.vgpr_count:\s+(\d+)", _meta(asm, n)).group(1))
            assert vgpr <= 256, (n, vgpr)


def test_large_batch_merges_four_per_cu(asm):
    names = _kernels(asm)
    # merge_kernel<16, 0, 256, 4> (after the sample pass) and
    # merge_seg_kernel<16, 4, 256, 4, 4, false> (after the exchange)
    want = ("merge_kernelILi16ELi0ELi256ELi4E", "merge_seg_kernelILi16ELi4ELi256ELi4ELi4ELb0E")
    for w in want:
        hits = [n for n in names if w in n]
        assert len(hits) == 1, (w, hits)
        meta = _meta(asm, hits[0])
        vgpr = int(re.search(r"\.vgpr_count:\s+(\d+)", meta).group(1))
        agpr = int(re.search(r"\.agpr_count:\s+(\d+)", meta).group(1))
        lds = int(re.search(r"\.group_segment_fixed_size:\s+(\d+)", meta).group(1))
        assert vgpr + agpr <= 128, (w, vgpr, agpr)
        assert lds <= 40 * 1024, (w, lds)
