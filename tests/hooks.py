"""Test-only library hooks (stk_test_set_hooks, exported by the library but not
declared in include/streamtopk.h), set for the duration of a with-block and
reset to the product's defaults afterwards.  The library reads them when a
call is made, so a with-block around the calls is enough; nothing in the
environment is read."""
import contextlib

from streamtopk_sae import _lib

# The exchange's default poll bound: 500 us of the 100 MHz real-time counter
# (kXchWaitTicks in csrc/stk_kernels.h).
XCH_WAIT_DEFAULT = 50000


@contextlib.contextmanager
def hooks(no_xch=0, max_rounds=-1, xch_wait=XCH_WAIT_DEFAULT):
    """no_xch: never take the threshold exchange; max_rounds >= 0: the
    streaming kernels' retry bound; xch_wait: the exchange's poll bound in
    ticks (0: one poll, < 0: none, so every threshold is 0)."""
    lib = _lib.load()
    _lib.check(lib.stk_test_set_hooks(int(no_xch), int(max_rounds), int(xch_wait)))
    try:
        yield
    finally:
        _lib.check(lib.stk_test_set_hooks(0, -1, XCH_WAIT_DEFAULT))
