import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "tests"), os.path.join(ROOT, "tests", "golden")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (runs the HIP library on cuda:0)")


@pytest.fixture(scope="session", autouse=True)
def _cache_dir(tmp_path_factory):
    """AUTO's measurements persist in the cache directory
    ($XDG_CACHE_HOME/janas): the session gets an empty one of its own, so
    no earlier run's file decides a test's way."""
    old = os.environ.get("XDG_CACHE_HOME")
    os.environ["XDG_CACHE_HOME"] = str(tmp_path_factory.mktemp("cache"))
    yield
    if old is None:
        os.environ.pop("XDG_CACHE_HOME", None)
    else:
        os.environ["XDG_CACHE_HOME"] = old


@pytest.fixture(scope="session", autouse=True)
def _float_unless_named():
    """Instances a test makes without naming a way compute FLOAT. AUTO's way
    is a measurement of both ways' speed on the device at the first call
    (the reference's rule, attention.c:1183-1247); where the two run within
    the measurement's noise of each other it can fall either way, and a test
    that compares with the FLOAT restatement, or a block with its tokens,
    needs one way. The tests of AUTO name it."""
    from janas_amd import attention as att
    defaults = att.Attention.__init__.__defaults__
    att.Attention.__init__.__defaults__ = (defaults[0], att.FLOAT)
    yield
    att.Attention.__init__.__defaults__ = defaults


@pytest.fixture(scope="session")
def gpu():
    """The GPU tests run where a GPU is: fail, never skip, without one."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    torch.cuda.init()
    return torch.device("cuda:0")


def pytest_sessionfinish(session, exitstatus):
    """With JANAS_PARITY_OUT set: every parity check's achieved error next
    to its bar, as a markdown table (attn_helpers.within records them)."""
    path = os.environ.get("JANAS_PARITY_OUT")
    if not path:
        return
    import attn_helpers
    rows = attn_helpers.MARGINS
    if not rows:
        return
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        f.write("| test | check | max error | bar | error / bar |\n")
        f.write("|---|---|---|---|---|\n")
        for test, what, err, bar in rows:
            f.write(f"| {test} | {what} | {err:.3e} | {bar:.1e} | "
                    f"{err / bar:.1%} |\n")
