"""Code-generation checks of the large-batch kernel, without a GPU: the gfx950
assembly of csrc/stk_large.hip, compiled here with the build's flags.

The d-step loop of mainl_kernel must hold no waterfall loop: a buffer
resource the compiler takes for divergent is read into scalar registers lane
by lane around every load (v_readfirstlane, s_and_saveexec, a branch back),
which splits the MFMA / load interleave and cost 7-10 % of the kernel.  The
kernel must also make no flat memory accesses (they count on the LDS counter,
so an LDS wait would also wait for them) and use no scratch memory.

The kernel's MFMAs are inline asm, which the compiler's hazard checks do not
see into, so the required wait states are checked here on its output:
  - an MFMA result read by a VALU instruction (v_accvgpr_read/mov, or a store
    of AGPR data) at least 20 wait states after the last MFMA before it (the
    largest requirement on gfx950: passes + 4 for a 16-pass MFMA);
  - a VGPR written by a VALU instruction and read by an MFMA as an operand, or
    an AGPR written by v_accvgpr_write/mov and read as the accumulator, at
    least 2 wait states later;
  - the accumulators stay in place: no AGPR moves or copies inside the d-step
    loop (the pattern the builtin MFMAs fall into at this register pressure).
And one schedule property: after each d-step's barrier, the previous step's
16 deferred MFMAs issue before the first wait for an LDS read.
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


def _kernel(asm, dt, sample, tail=False):
    name = f"_ZN3stk12mainl_kernelILi{dt}ELb{1 if sample else 0}ELb{1 if tail else 0}EEEvNS_9MainLArgsE"
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
@pytest.mark.parametrize("tail", [False, True])
def test_dstep_loop_has_no_waterfall(asm, dt, sample, tail):
    body, _ = _kernel(asm, dt, sample, tail)
    loop = _loop_blocks(body)
    assert loop, "no MFMA block found"
    for blk in loop:
        assert "s_and_saveexec" not in blk and "v_readfirstlane" not in blk, blk[:400]
        # one buffer load to LDS per 16-byte chunk of the step: 32 per two d-steps
        assert blk.count("buffer_load_dwordx4") <= 32


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("sample", [False, True])
@pytest.mark.parametrize("tail", [False, True])
def test_deferred_mfmas_follow_each_barrier(asm, dt, sample, tail):
    """Each d-step's barrier is followed by the previous step's 16 deferred
    MFMAs before the first wait for an LDS read: the matrix cores work while
    the step's first operand reads land.  A wait hoisted above them would
    leave the results right and the d-steps ~2-3 % slower."""
    body, _ = _kernel(asm, dt, sample, tail)
    blocks = [b for b in re.split(r"\n(?=\.LBB\d+_\d+:)", body) if b.count("v_mfma") >= 256]
    assert len(blocks) == 1, "one block holds the two-step loop body"
    steps = blocks[0].split("s_barrier")[1:3]   # the loop body's two d-steps
    assert len(steps) == 2
    for st in steps:
        assert re.split(r"s_waitcnt[^\n]*lgkmcnt", st)[0].count("v_mfma") == 16


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("sample", [False, True])
@pytest.mark.parametrize("tail", [False, True])
def test_no_flat_access_no_scratch(asm, dt, sample, tail):
    body, meta = _kernel(asm, dt, sample, tail)
    assert not re.search(r"\bflat_(load|store|atomic)", body)
    assert re.search(r"\.private_segment_fixed_size:\s+0\b", meta)
    assert re.search(r"\.vgpr_spill_count:\s+0\b", meta)


def _cfg(body):
    """The kernel's basic blocks: a list of (instructions, successor indices),
    each instruction as (mnemonic, operand text); labels, directives and
    comments dropped."""
    blocks, labels = [[]], {}
    for line in body.split("\n"):
        t = line.split(";")[0].strip()
        if not t or t.startswith("."):
            if t.endswith(":") and t.startswith(".LBB"):
                if blocks[-1]:
                    blocks.append([])
                labels[t[:-1]] = len(blocks) - 1
            continue
        if t.endswith(":"):
            continue
        parts = t.split(None, 1)
        blocks[-1].append((parts[0], parts[1] if len(parts) > 1 else ""))
    out = []
    for i, ins in enumerate(blocks):
        succ, fall = [], True
        for op, args in ins:
            if op == "s_branch":
                succ.append(labels[args.strip()])
                fall = False
            elif op.startswith("s_cbranch"):
                succ.append(labels[args.strip()])
            elif op == "s_endpgm":
                fall = False
        if fall and i + 1 < len(blocks):
            succ.append(i + 1)
        out.append((ins, succ))
    return out


def _preds(cfg):
    preds = [[] for _ in cfg]
    for i, (_, succ) in enumerate(cfg):
        for j in succ:
            preds[j].append(i)
    return preds


def _regs(text, kind):
    """Register numbers of kind 'v' or 'a' named in an operand text."""
    regs = set()
    for lo, hi in re.findall(r"\b%s\[(\d+):(\d+)\]" % kind, text):
        regs.update(range(int(lo), int(hi) + 1))
    for r in re.findall(r"\b%s(\d+)\b" % kind, text):
        regs.add(int(r))
    return regs


def _wait_states(ins):
    return int(ins[1], 0) + 1 if ins[0] == "s_nop" else 1


def _walk_back(cfg, preds, b, i, limit, hit):
    """Every instruction on the paths that end just before instruction i of
    block b, nearest first, until limit wait states: calls hit(ins, ws) with
    the wait states between that instruction and the end; hit returns True to
    stop the path there."""
    stack, seen = [(b, i, 0)], set()
    while stack:
        b, i, ws = stack.pop()
        if (b, i, ws) in seen:
            continue
        seen.add((b, i, ws))
        ins = cfg[b][0]
        stopped = False
        for j in range(i - 1, -1, -1):
            if ws >= limit or hit(ins[j], ws):
                stopped = True
                break
            ws += _wait_states(ins[j])
        if not stopped and ws < limit:
            for p in preds[b]:
                stack.append((p, len(cfg[p][0]), ws))


def _is_acc_read(op, args):
    return (op.startswith(("v_accvgpr_read", "v_accvgpr_mov")) or
            (op.startswith(("global_store", "buffer_store", "ds_write")) and bool(_regs(args, "a"))))


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("sample", [False, True])
@pytest.mark.parametrize("tail", [False, True])
def test_mfma_result_reads_wait(asm, dt, sample, tail):
    """On every path into a VALU read of an AGPR, at least 20 wait states
    separate it from the last MFMA."""
    body, _ = _kernel(asm, dt, sample, tail)
    cfg = _cfg(body)
    preds = _preds(cfg)
    reads = 0
    for b, (ins, _) in enumerate(cfg):
        for i, (op, args) in enumerate(ins):
            if not _is_acc_read(op, args):
                continue
            reads += 1

            def hit(x, ws):
                assert not x[0].startswith("v_mfma"), f"{op} {args}: {ws} wait states after {x[0]} {x[1]}"
                return False
            _walk_back(cfg, preds, b, i, 20, hit)
    assert reads > 0


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("sample", [False, True])
@pytest.mark.parametrize("tail", [False, True])
def test_mfma_operands_not_fresh_from_valu(asm, dt, sample, tail):
    """On every path into an MFMA, no VALU instruction writes a VGPR it reads,
    and no v_accvgpr_write/mov an AGPR it reads, within 2 wait states."""
    body, _ = _kernel(asm, dt, sample, tail)
    cfg = _cfg(body)
    preds = _preds(cfg)
    nmfma = 0
    for b, (ins, _) in enumerate(cfg):
        for i, (op, args) in enumerate(ins):
            if not op.startswith("v_mfma"):
                continue
            nmfma += 1
            srcs = args.partition(",")[2]
            src_v, src_a = _regs(srcs, "v"), _regs(srcs, "a")

            def hit(x, ws):
                pop, pargs = x
                pdst = pargs.split(",")[0]
                if pop.startswith(("v_accvgpr_write", "v_accvgpr_mov")):
                    assert not (_regs(pdst, "a") & src_a), f"{op} {args} reads {pdst} of {pop} after {ws}"
                elif pop.startswith("v_") and not pop.startswith(("v_mfma", "v_readlane", "v_readfirstlane",
                                                                  "v_cmp")):
                    assert not (_regs(pdst, "v") & src_v), f"{op} {args} reads {pdst} of {pop} after {ws}"
                return False
            _walk_back(cfg, preds, b, i, 2, hit)
    assert nmfma > 0


@pytest.mark.parametrize("dt", [0, 1, 2])
@pytest.mark.parametrize("sample", [False, True])
@pytest.mark.parametrize("tail", [False, True])
def test_accumulators_stay_in_place(asm, dt, sample, tail):
    body, _ = _kernel(asm, dt, sample, tail)
    for blk in _loop_blocks(body):
        assert "v_accvgpr" not in blk
        for m in re.finditer(r"v_mfma\S*\s+(a\[\d+:\d+\]),[^\n]*,\s*(a\[\d+:\d+\])", blk):
            assert m.group(1) == m.group(2), m.group(0)


def test_hazard_walk_sees_across_blocks():
    """The checks' own test, on hand-written text: a read 3 wait states after
    an MFMA in the block before, and an MFMA operand written by the VALU just
    before it in the block before, are both found."""
    body = "\n".join([
        "k:",
        "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]",
        "\ts_cbranch_scc0 .LBB0_2",
        ".LBB0_1:",
        "\ts_nop 1",
        "\tv_accvgpr_read_b32 v8, a0",
        ".LBB0_2:",
        "\tv_mov_b32_e32 v5, 0",
        "\ts_branch .LBB0_3",
        ".LBB0_3:",
        "\tv_mfma_f32_16x16x32_bf16 a[4:7], v[0:3], v[4:7], a[4:7]",
        "\ts_endpgm",
    ])
    cfg = _cfg(body)
    preds = _preds(cfg)
    assert [s for _, s in cfg] == [[2, 1], [2], [3], []]
    found = []

    def hit(x, ws):
        if x[0].startswith("v_mfma"):
            found.append(("mfma", ws))
            return True
        return False
    _walk_back(cfg, preds, 1, 1, 20, hit)
    assert found == [("mfma", 3)]
    found.clear()

    def hit2(x, ws):
        if x[0].startswith("v_mov"):
            found.append(("valu", ws))
        return False
    _walk_back(cfg, preds, 3, 0, 2, hit2)
    assert found == [("valu", 1)]
