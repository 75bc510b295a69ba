"""JANAS_ATTN_SKIPSTAT=1: the reference's statistic of the chunks a row
could have skipped (attention.c:841-869, :883-898), counted by the split
path's merge on the device and printed when the program ends.

The caches are built so that every chunk's largest score is known exactly:
with the query e_0 and scale 1, a chunk whose keys hold 20 in column 0
scores 20 everywhere, the others 0. So each (token, head) row has its
chunks 0 below the row's maximum of 20 - below max-8 and max-16, not below
max-32 - and the printed percentages follow from the chunk counts alone.
The statistic is process-wide and read at the first create, so the calls
run in a child process."""
import os
import re
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, ROOT)
import janas_amd as jm

dev = torch.device("cuda:0")
h, kvh, hd = 8, 2, 128
rng = np.random.default_rng(5)
# (cache type, positions, hot chunks)
for kv, L, hot in ((jm.KV_F16, 4096, (3, 9)), (jm.KV_I8, 20000, (0, 70))):
    if kv == jm.KV_F16:
        k = np.zeros((kvh, L, hd), np.float16)
        for c in hot:
            k[:, 256 * c:256 * (c + 1), 0] = 20.0
        v = rng.standard_normal((kvh, L, hd)).astype(np.float16)
        ks = vs = None
    else:
        k = np.zeros((kvh, L, hd), np.int8)
        for c in hot:
            k[:, 256 * c:256 * (c + 1), 0] = 127
        ks = np.full((kvh, L), 20.0 / 127.0, np.float32)
        v = rng.integers(-127, 128, (kvh, L, hd)).astype(np.int8)
        vs = np.full((kvh, L), 0.01, np.float32)
    q = np.zeros((1, h, hd), np.float32)
    q[:, :, 0] = 1.0
    t = lambda x: None if x is None else torch.from_numpy(x).to(dev)
    out = torch.zeros((1, h, hd), device=dev)
    with jm.Attention(h, kvh, hd, L, 1, jm.FLOAT) as a:
        a.set_scale(1.0)
        a.run_dev(kv, [dict(k=t(k), v=t(v), ks=t(ks), vs=t(vs), q=t(q),
                            out=out, cap=L, n=1, pos0=L - 1)])
        torch.cuda.synchronize()
    assert torch.isfinite(out).all()
print("child done", flush=True)
""".replace("ROOT", repr(ROOT))


def expected(rows):
    """(chunks, below 8, below 16, below 32) summed over the rows: each row
    (chunks, hot) counts all its chunks, the cold ones below 8 and 16."""
    n = sum(c for c, _ in rows)
    cold = sum(c - hot for c, hot in rows)
    return n, cold, cold, 0


def test_skipstat_counts(gpu):
    env = dict(os.environ, JANAS_ATTN_SKIPSTAT="1")
    p = subprocess.run([sys.executable, "-u", "-c", CHILD], env=env,
                       capture_output=True, text=True, timeout=300)
    print(p.stdout)
    print(p.stderr)
    assert p.returncode == 0, p.stderr
    lines = re.findall(r"attention skip ceiling, (.*?): (\d+) chunks; below "
                       r"max-8 ([\d.]+)%, max-16 ([\d.]+)%, max-32 ([\d.]+)%",
                       p.stderr)
    got = {w: tuple(float(x) for x in rest) for w, *rest in lines}
    # 8 heads; f16 call: 16 chunks, 2 hot; int8 call (past 16384): 79 chunks,
    # 2 hot
    rows_all = [(16, 2)] * 8 + [(79, 2)] * 8
    rows_late = [(79, 2)] * 8
    for what, rows in (("all rows", rows_all), ("rows past 16384", rows_late)):
        n, b8, b16, b32 = expected(rows)
        want = (n, round(100.0 * b8 / n, 1), round(100.0 * b16 / n, 1),
                round(100.0 * b32 / n, 1))
        assert what in got, p.stderr
        assert got[what] == want, (what, got[what], want)
