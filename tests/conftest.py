import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# the directory the GPU runs bring back with their results
TIE_LOG_DIR = os.path.join(ROOT, "gpurun_out")
PKG_DIR = os.path.join(ROOT, "streamtopk-sae_amd")
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (PKG_DIR, ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")
    config.addinivalue_line("markers", "slow: full-size configurations")


@pytest.fixture(scope="session")
def cuda_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The parity checks' near-tie log (parity.TIE_LOG), kept short enough for
    the tail of a quiet run: one line per full-size configuration (its checks
    grouped), one per check with near-tie rows, and the totals; every check is
    also written to parity_ties.json in the output directory (TIE_LOG_DIR)."""
    try:
        import parity
    except ImportError:
        return
    log = parity.TIE_LOG
    if not log:
        return
    import json
    groups = {}
    for e in log:
        head = e["name"].split("/")[0].split(" ")[0]
        if head in ("headline", "config0", "config1", "config3", "config4", "B=2048"):
            g = groups.setdefault(head, [0, 0, 0, 0.0])
            g[0] += 1
            g[1] += e["rows"]
            g[2] += e["tie_rows"]
            g[3] = max(g[3], e["value_err_over_bound"] if e["bound"] == "fp32-sum" else 0.0)
    rows = sum(e["rows"] for e in log)
    ties = sum(e["tie_rows"] for e in log)
    bounded = [e for e in log if e["bound"] == "fp32-sum"]
    tr = terminalreporter
    tr.write_sep("-", "parity near-tie log")
    for head, (n, r, t, m) in groups.items():
        tr.write_line(f"  {head}: {n} checks, {t}/{r} rows with near-ties, value err/fp32-sum bound <= {m:.2g}")
    for e in log:
        if e["tie_rows"]:
            tr.write_line(f"  near-tie: {e['name']}: {e['tie_rows']}/{e['rows']} rows (k={e['k']})")
    tr.write_line(f"  all: {len(log)} checks, {ties}/{rows} rows with near-tie index differences "
                  f"({ties / max(rows, 1):.3%}); {len(bounded)} checks held to the fp32 sum bound, "
                  f"largest err/bound {max((e['value_err_over_bound'] for e in bounded), default=0.0):.2g}")
    try:
        out = TIE_LOG_DIR
        os.makedirs(out, exist_ok=True)
        with open(os.path.join(out, "parity_ties.json"), "w") as f:
            json.dump({"checks": log, "rows": rows, "tie_rows": ties}, f, indent=1)
    except OSError:
        pass
