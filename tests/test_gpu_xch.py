"""GPU tests of the streaming kernels' threshold exchange.

Without a sample pass, every main_kernel workgroup publishes the largest score
of each row in its first tile (mainl_kernel, for 512 rows and more: one per 64
latents of it); the owner of a row takes the k-th largest of those maxima as
the row's threshold, and every workgroup reads its rows' thresholds before
its first epilogue filters anything.  Every shared word carries the call's
tag beside its data, and every poll is bounded: a poll that runs out leaves
threshold 0 (every score a candidate), so the result stays exact.

Checked here: which kernels a call launches (the exchange replaces the
sample and threshold passes when the grid has at least max(k, 16)
workgroups per row block, or, for 512 rows and more, 4 maxima per row and W
range reach k), exact results with every wait forced to run out after one poll or none
(the xch_wait test hook, read by the library at each call), back-to-back calls
on one cached workspace with different inputs and shapes (stale maxima and
thresholds of an earlier call must never be taken for this call's), and score
distributions that defeat the threshold (all scores equal, all the best
latents in one workgroup's range).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from hooks import hooks
from parity import check_against_scores, term_magnitudes, tol_of
from streamtopk_sae import _lib, make_inputs, topk_sae_cuda_exact

pytestmark = pytest.mark.gpu

DT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def _np(t):
    return t.detach().float().cpu().numpy()


def _check_out(V, I, X, W, b, k, dtype_name, name):
    S = oracle.scores_f64(_np(X), _np(W), _np(b))
    A = term_magnitudes(_np(X), _np(W), _np(b))
    check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, tol_of(dtype_name), name, A=A, d=X.shape[1])


def _check(X, W, b, k, dtype_name, name):
    V, I = topk_sae_cuda_exact(X, W, b, k)
    torch.cuda.synchronize()
    _check_out(V, I, X, W, b, k, dtype_name, name)
    return V, I


def _launches(fn):
    """Kernel launches of fn() by name, from the library's per-kernel event records."""
    lib = _lib.load()
    _lib.check(lib.stk_profile_enable(1))
    try:
        fn()
        torch.cuda.synchronize()
        out = {}
        for name in ("sample_kernel", "thr_kernel", "main_kernel", "merge_kernel"):
            tot = ctypes.c_double(0.0)
            n = ctypes.c_int64(0)
            _lib.check(lib.stk_profile_read(name.encode(), ctypes.byref(tot), ctypes.byref(n)))
            out[name] = n.value
        return out
    finally:
        _lib.check(lib.stk_profile_enable(0))


@pytest.mark.parametrize("B,F,k,xch", [
    (128, 65536, 32, True),      # config 1's shape: 256 workgroups
    (40, 16384 + 37, 64, True),  # 65 tiles, 65 workgroups >= k
    (40, 16384 + 37, 128, False),  # 65 workgroups < k: the sample pass seeds the thresholds
    (600, 65536, 64, True),      # large batch: mainl_kernel, 80 W ranges x 4 maxima per row
    (4096, 65536, 128, False),   # 16 W ranges x 4 maxima < k: mainl_kernel with a sample pass
    (512, 20000, 64, True),      # 79 tiles over 128 W ranges: the 79 that hold tiles exchange
    (2048, 65536, 32, True),     # eight row blocks of 32 W ranges; rows merged in two rounds
])
def test_exchange_replaces_threshold_passes(cuda_dev, B, F, k, xch):
    print(f"case launches B={B} F={F} k={k}", flush=True)
    X, W, b = make_inputs(B, 64 if B > 1024 else 128, F, torch.bfloat16, seed=11, device=cuda_dev)
    n = _launches(lambda: topk_sae_cuda_exact(X, W, b, k))
    assert n["main_kernel"] == 1 and n["merge_kernel"] == 1, n
    if xch:
        assert n["sample_kernel"] == 0 and n["thr_kernel"] == 0, n
    else:
        assert n["sample_kernel"] == 1 and n["thr_kernel"] == 1, n


@pytest.mark.parametrize("B,d,F,k,dtype_name", [
    (1, 64, 8192, 16, "bf16"),
    (64, 256, 65536, 64, "bf16"),
    (128, 128, 40000, 128, "fp16"),
    (300, 96, 30000, 32, "fp32"),   # three row blocks, each its own exchange
    (600, 128, 30000, 64, "bf16"),  # mainl_kernel, three row blocks
    (1024, 256, 65536, 128, "fp16"),
    (512, 64, 20000, 32, "bf16"),   # mainl_kernel with empty W ranges
    (2048, 64, 65536, 32, "bf16"),  # more rows than one round of the merge's workgroups
])
def test_exchange_waits_run_out(cuda_dev, B, d, F, k, dtype_name):
    """Exchange waits that run out: with no poll at all every threshold stays
    0; with a single poll an owner takes the k-th of the maxima that did
    arrive if at least k did, and a reader keeps every threshold that did.
    Either way the result is exact, and equal to the exchange's."""
    print(f"case xch timeout B={B} d={d} F={F} k={k} {dtype_name}", flush=True)
    X, W, b = make_inputs(B, d, F, DT[dtype_name], seed=12, device=cuda_dev)
    with hooks(xch_wait=-1):
        V0, I0 = _check(X, W, b, k, dtype_name, "no poll")
    with hooks(xch_wait=0):
        V2, I2 = _check(X, W, b, k, dtype_name, "one poll")
    V1, I1 = _check(X, W, b, k, dtype_name, "exchange")
    assert torch.equal(I0, I1) and torch.equal(V0, V1)
    assert torch.equal(I2, I1) and torch.equal(V2, V1)


def test_back_to_back_calls(cuda_dev):
    """Calls on one cached workspace, inputs and shapes changing from call to
    call with no synchronisation between them: each result matches its own
    inputs.  A stale maximum or threshold of an earlier call taken for this
    call's would raise a threshold above the row's k-th score and drop answers."""
    print("case back-to-back", flush=True)
    cases = []
    for i, (B, F, k) in enumerate([(128, 65536, 32), (128, 65536, 32), (96, 50000, 64),
                                   (128, 65536, 32), (33, 65536, 16), (128, 65536, 32)]):
        X, W, b = make_inputs(B, 128, F, torch.bfloat16, seed=100 + i, device=cuda_dev)
        if i == 3:
            # the previous maxima would now be far too high thresholds
            X = X * 1e-3
        cases.append((X, W, b, k))
    for i, (B, F, k) in enumerate([(600, 40000, 64), (1024, 65536, 128), (600, 40000, 64)]):
        X, W, b = make_inputs(B, 128, F, torch.bfloat16, seed=200 + i, device=cuda_dev)
        cases.append((X * (1e-3 if i == 2 else 1.0), W, b, k))
    outs = [topk_sae_cuda_exact(X, W, b, k) for X, W, b, k in cases]
    torch.cuda.synchronize()
    for i, ((X, W, b, k), (V, I)) in enumerate(zip(cases, outs)):
        S = oracle.scores_f64(_np(X), _np(W), _np(b))
        check_against_scores(V.cpu().numpy(), I.cpu().numpy(), S, k, tol_of("bf16"), f"call {i}")


def test_all_scores_equal(cuda_dev):
    """Every score equal: the threshold accepts every latent (ties at its
    value are candidates), and the lower index wins among equals."""
    print("case all-equal", flush=True)
    B, d, F, k = 64, 64, 65536, 64
    X = torch.zeros(B, d, dtype=torch.bfloat16, device=cuda_dev)
    W = torch.ones(F, d, dtype=torch.bfloat16, device=cuda_dev)
    b = torch.full((F,), 0.25, dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, k)
    assert torch.equal(I.cpu(), torch.arange(k, dtype=torch.int32).expand(B, k))
    assert bool((V == 0.25).all())


def test_all_scores_equal_large_batch(cuda_dev):
    """As test_all_scores_equal, through mainl_kernel's exchange."""
    print("case all-equal large", flush=True)
    B, d, F, k = 512, 64, 65536, 128
    X = torch.zeros(B, d, dtype=torch.bfloat16, device=cuda_dev)
    W = torch.ones(F, d, dtype=torch.bfloat16, device=cuda_dev)
    b = torch.full((F,), -1.5, dtype=torch.float32, device=cuda_dev)
    V, I = topk_sae_cuda_exact(X, W, b, k)
    assert torch.equal(I.cpu(), torch.arange(k, dtype=torch.int32).expand(B, k))
    assert bool((V == -1.5).all())


def test_best_latents_in_one_workgroup(cuda_dev):
    """All of a row's best latents inside one workgroup's range of tiles: the
    exchanged threshold is low for them and that workgroup's queues spill;
    the answer is still exact."""
    print("case clustered", flush=True)
    B, d, F, k = 128, 128, 262144, 128
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=13, device=cuda_dev)
    b = b.clone()
    b[5000:5000 + 2 * k] += 50.0
    _check(X, W, b, k, "bf16", "clustered")


def test_best_latents_in_one_w_range_large_batch(cuda_dev):
    """As test_best_latents_in_one_workgroup, through mainl_kernel's exchange."""
    print("case clustered large", flush=True)
    B, d, F, k = 512, 128, 131072, 128
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=14, device=cuda_dev)
    b = b.clone()
    b[70000:70000 + 2 * k] += 50.0
    _check(X, W, b, k, "bf16", "clustered large")


@pytest.mark.parametrize("B,d,F,k,dtype_name", [
    (128, 256, 65536, 64, "bf16"),
    (600, 128, 40000, 64, "bf16"),
    (1024, 128, 65536, 128, "fp16"),
])
def test_sample_pass_path(cuda_dev, B, d, F, k, dtype_name):
    """The sample and threshold passes (the path of grids too small for the
    exchange), forced with the no_xch test hook at shapes that would exchange:
    both paths exact against the oracle (the sampled latents' scores are
    summed in another order there, so values may differ in the last bit)."""
    print(f"case sample path B={B} d={d} F={F} k={k} {dtype_name}", flush=True)
    X, W, b = make_inputs(B, d, F, DT[dtype_name], seed=15, device=cuda_dev)
    with hooks(no_xch=1):
        n = _launches(lambda: topk_sae_cuda_exact(X, W, b, k))
        assert n["sample_kernel"] == 1 and n["thr_kernel"] == 1, n
        _check(X, W, b, k, dtype_name, "sample pass")
    _check(X, W, b, k, dtype_name, "exchange")


def _timeouts(X):
    """The exchange's count of polls that ran out, in the workspace the op
    keeps for X's device and current stream: the second 32-bit word of the
    workspace's control line (after the epoch)."""
    from streamtopk_sae import ops
    key = (X.device.index, int(torch.cuda.current_stream(X.device).cuda_stream))
    torch.cuda.synchronize()
    ws = ops._WS[key]
    return int(ws[4:8].cpu().view(torch.int32)[0])


@pytest.mark.parametrize("B,d,F,k,short_waits", [
    (128, 768, 65536, 32, True),      # config 1's shape
    (128, 2048, 262144, 64, False),   # config 2's shape
    (40, 256, 16384 + 37, 64, True),
    (300, 128, 100000, 64, False),
    (600, 128, 65536, 64, True),      # mainl_kernel
    (1024, 256, 262144, 128, False),  # mainl_kernel, config 4's grid
    (512, 64, 20000, 64, True),       # mainl_kernel, 79 of 128 W ranges hold tiles
    (2048, 768, 65536, 32, False),    # mainl_kernel, eight row blocks of 32 W ranges
])
def test_exchange_never_runs_out(cuda_dev, B, d, F, k, short_waits):
    """On an idle device every workgroup of the grid is resident, so no poll of
    the exchange runs out (one that did would leave thresholds at 0: exact but
    slow).  At the smaller shapes a wait of 1 tick makes them run out, which
    the count shows (the larger ones would take long with threshold 0)."""
    print(f"case xch no timeout B={B} d={d} F={F} k={k}", flush=True)
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=16, device=cuda_dev)
    topk_sae_cuda_exact(X, W, b, k)   # sizes the op's workspace
    before = _timeouts(X)
    for _ in range(5):
        topk_sae_cuda_exact(X, W, b, k)
    assert _timeouts(X) == before
    if short_waits:
        with hooks(xch_wait=1):
            _check(X, W, b, k, "bf16", "1-tick waits")
        assert _timeouts(X) > before


@pytest.mark.parametrize("B,d,F,k", [
    (128, 256, 65536, 32),      # main_kernel's exchange
    (600, 128, 81920, 64),      # mainl_kernel's
])
def test_graph_replays_with_new_inputs(cuda_dev, B, d, F, k):
    """The op captured in a graph and replayed with new inputs each time.
    A replay's kernel arguments never change, so the exchange's tag must not
    come from them: it is the workspace's epoch + 1, advanced by every call's
    merge.  Each replay is checked against the oracle and against an eager
    call on the same inputs (bit for bit), with eager work and
    synchronisations between the replays."""
    print(f"case graph replay B={B} d={d} F={F} k={k}", flush=True)
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=17, device=cuda_dev)
    s = torch.cuda.Stream(cuda_dev)
    s.wait_stream(torch.cuda.current_stream(cuda_dev))
    with torch.cuda.stream(s):
        for _ in range(2):
            topk_sae_cuda_exact(X, W, b, k)   # the op's workspace for s, outside the capture
    torch.cuda.current_stream(cuda_dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        V, I = topk_sae_cuda_exact(X, W, b, k)
    for i in range(4):
        Xn, _, _ = make_inputs(B, d, F, torch.bfloat16, seed=400 + i, device=cuda_dev)
        if i == 2:
            Xn = Xn * 1e-3   # thresholds far below the previous replay's
        X.copy_(Xn)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        Vg, Ig = V.clone(), I.clone()
        S = oracle.scores_f64(_np(X), _np(W), _np(b))
        check_against_scores(Vg.cpu().numpy(), Ig.cpu().numpy(), S, k, tol_of("bf16"), f"replay {i}")
        Ve, Ie = topk_sae_cuda_exact(X, W, b, k)
        torch.cuda.synchronize()
        assert torch.equal(Ve, Vg) and torch.equal(Ie, Ig), f"replay {i} differs from the eager call"


# ---------------------------------------------------------------------------
# The workspace's control line and the exchange's tags.
# ---------------------------------------------------------------------------
TAG_PERIOD = (1 << 22) - 1          # kTagPeriod: tags run 1 .. TAG_PERIOD
IMG_100 = 0xC2C80000                # ordered_u32(100.0f): a stale sort key's high word


def _ws(X):
    """The workspace the op keeps for X's device and current stream."""
    from streamtopk_sae import ops
    key = (X.device.index, int(torch.cuda.current_stream(X.device).cuda_stream))
    torch.cuda.synchronize()
    return ops._WS[key]


def _epoch(ws):
    torch.cuda.synchronize()
    return int(ws[0:4].cpu().view(torch.int32)[0]) & 0xFFFFFFFF


def _set_epoch(ws, e):
    ws[0:4].copy_(torch.tensor([e], dtype=torch.int64).view(torch.uint8)[:4].to(ws.device))
    torch.cuda.synchronize()


def _plant_stale_keys(ws):
    """Every word past the control line becomes a sort key of score 100 (what
    a candidate list of an earlier, larger call leaves): high word IMG_100,
    low word 0xFFFFFFFF - j."""
    n = (ws.numel() - 256) // 8
    j = np.arange(n, dtype=np.uint64)
    keys = (np.uint64(IMG_100) << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - (j & np.uint64(0xFFFFFFFF)))
    ws[256:256 + 8 * n].copy_(torch.from_numpy(keys.view(np.uint8)).to(ws.device))
    torch.cuda.synchronize()


XCH_SHAPES = [(128, 256, 65536, 32),    # main_kernel's exchange
              (600, 128, 81920, 64)]    # mainl_kernel's


@pytest.mark.parametrize("B,d,F,k", XCH_SHAPES)
def test_mixed_calls_share_workspace(cuda_dev, B, d, F, k):
    """The candidate-buffer path and the shard merge use the same cached
    workspace as the exact path on one stream; their buffers start past the
    control line, so exact calls interleaved with them, each on new inputs,
    stay exact, and only exact calls advance the epoch (a merge or candidate
    call that wrote into the control line would repeat exact calls' tags and
    let them take an earlier call's maxima for their own)."""
    from streamtopk_sae import merge_topk_shards, topk_sae_cuda_approx
    print(f"case mixed calls B={B} d={d} F={F} k={k}", flush=True)
    _, W, b = make_inputs(B, d, F, torch.bfloat16, seed=60, device=cuda_dev)
    Fc = 4096
    Wc, bc = W[:Fc].contiguous(), b[:Fc].contiguous()
    topk_sae_cuda_exact(torch.zeros(B, d, dtype=torch.bfloat16, device=cuda_dev), W, b, k)
    ws = _ws(W)
    e0 = _epoch(ws)
    for i in range(4):
        X, _, _ = make_inputs(B, d, F, torch.bfloat16, seed=600 + i, device=cuda_dev)
        if i % 2:
            X = X * 1e-3   # thresholds far below the previous call's
        # the candidate path and the merge first, on the same stream and workspace
        Xc = X[:64].contiguous()
        cb = torch.empty((64, Fc // 128, 32), dtype=torch.float32, device=cuda_dev)
        Va, Ia = topk_sae_cuda_approx(Xc, Wc, bc, 16, 32, candidate_buffer=cb)
        parts_v = torch.sort(torch.randn(3, B, k, device=cuda_dev), dim=2, descending=True).values
        parts_i = torch.randint(0, F, (3, B, k), dtype=torch.int32, device=cuda_dev)
        merge_topk_shards(parts_v, parts_i, k)
        assert _ws(W).data_ptr() == ws.data_ptr()
        V, I = topk_sae_cuda_exact(X, W, b, k)
        torch.cuda.synchronize()
        _check_out(V, I, X, W, b, k, "bf16", f"mixed call {i}")
        _check_out(Va, Ia, Xc, Wc, bc, 16, "bf16", f"mixed approx {i}")
        assert _epoch(ws) == e0 + i + 1, "only exact calls advance the epoch"


@pytest.mark.parametrize("B,d,F,k", XCH_SHAPES)
def test_preset_epoch_over_stale_keys(cuda_dev, B, d, F, k):
    """The workspace full of stale sort keys of score 100 and its epoch preset
    to one below their high word: a tag taken straight from that epoch would
    equal the keys' high word, and the exchange would read them as this
    call's maxima and thresholds (near +inf: answers dropped).  Tags are
    reduced modulo a period below every score image, so none matches; the
    result is exact and the epoch is back in range after the call."""
    print(f"case preset epoch B={B} d={d} F={F} k={k}", flush=True)
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=61, device=cuda_dev)
    topk_sae_cuda_exact(X, W, b, k)
    ws = _ws(X)
    for epoch in (IMG_100 - 1, 0xFFFFFFFE, TAG_PERIOD - 1):
        _plant_stale_keys(ws)
        _set_epoch(ws, epoch)
        Xn, _, _ = make_inputs(B, d, F, torch.bfloat16, seed=610 + epoch % 7, device=cuda_dev)
        _check(Xn, W, b, k, "bf16", f"preset epoch {epoch:#x}")
        assert _epoch(ws) < TAG_PERIOD
    _set_epoch(ws, TAG_PERIOD - 1)
    _check(X, W, b, k, "bf16", "last tag of the period")
    assert _epoch(ws) == 0, "the epoch wraps to 0 after the period's last tag"


@pytest.mark.parametrize("B,d,F,k", XCH_SHAPES)
def test_wrapped_tag_meets_zeroed_words(cuda_dev, B, d, F, k):
    """A tag that comes round again (the epoch set back to the first call's,
    as after kTagPeriod calls): the merge zeroed the words the first call
    tagged, so the second call, on inputs whose scores are 1000x smaller,
    cannot take the first call's maxima and thresholds for its own."""
    print(f"case wrapped tag B={B} d={d} F={F} k={k}", flush=True)
    X, W, b = make_inputs(B, d, F, torch.bfloat16, seed=62, device=cuda_dev)
    topk_sae_cuda_exact(X, W, b, k)
    ws = _ws(X)
    _set_epoch(ws, 5)
    _check(X, W, b, k, "bf16", "tag 6, first use")
    _set_epoch(ws, 5)
    _check(X * 1e-3, W, b, k, "bf16", "tag 6 again, scores 1000x smaller")
