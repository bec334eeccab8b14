"""stk_read_probe, the plain HBM read stream bench.py compares the streaming
kernels with: it must read every byte once, which its digest (the XOR of
all 32-bit words, XORed into the sink) shows."""
import ctypes

import numpy as np
import pytest
import torch

from streamtopk_sae import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, 10 * 2**20 + 16 * 7, 64 * 2**20])
def test_read_probe_digest(cuda_dev, nbytes):
    lib = _lib.load()
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).to(cuda_dev)
    sink = torch.full((1,), 0x5A5A5A5A, dtype=torch.int32, device=cuda_dev)
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.stk_read_probe(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()),
                            ctypes.c_void_p(st))
    _lib.check(rc)
    torch.cuda.synchronize()
    want = np.bitwise_xor.reduce(host) ^ np.uint32(0x5A5A5A5A)
    assert np.uint32(sink.cpu().numpy().view(np.uint32)[0]) == want


def test_read_probe_rejects_misaligned(cuda_dev):
    lib = _lib.load()
    buf = torch.zeros(64, dtype=torch.int32, device=cuda_dev)
    sink = torch.zeros(1, dtype=torch.int32, device=cuda_dev)
    rc = lib.stk_read_probe(ctypes.c_void_p(buf.data_ptr()), 20, ctypes.c_void_p(sink.data_ptr()), None)
    assert rc != 0
    assert "16-byte" in lib.stk_last_error().decode()
