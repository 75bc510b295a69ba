"""bench.py's conventions on the CPU: the algorithmic work it divides by
(4 head_dim flops a (query, key) pair, causal; K/V bytes read once) at the
BASELINE configurations, the engine's quantization rule it fills int8 /
int16 caches with, and that more than one GPU is refused before anything
touches a device."""
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_prefill_flops_match_the_configs():
    # the 8k prompt, 32 / 8 / 128: P = 8192 * 8193 / 2 pairs a head
    assert bench.prefill_flops(128, 32, 0, 8192) == 549822922752.0
    # config 2: 1024 tokens
    assert bench.prefill_flops(128, 32, 0, 1024) == 4.0 * 128 * 32 * 1024 * 1025 / 2
    # a block of 64 at 4096: every token sees the prefix and its own rows
    n, p0 = 64, 4096
    assert bench.prefill_flops(128, 32, p0, n) == 4.0 * 128 * 32 * sum(p0 + j + 1 for j in range(n))


def test_config4_bytes():
    w = bench.decode_workload()
    assert w["k"].dtype == np.float16 and w["k"].shape == (2, 32768, 256)
    assert w["k"].nbytes + w["v"].nbytes == 67108864
    assert w["scale"] == 1.0 / 16.0


def test_quantized_rows_follow_the_cache_write():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 5, 16)).astype(np.float32)
    for dt, top in ((np.int8, 127), (np.int16, 32767)):
        q, s = bench.quantized(x, dt)
        assert q.dtype == dt and s.shape == (2, 5)
        # the row's largest magnitude becomes top; every number within half
        # a step of its own value
        assert np.all(np.abs(q).max(axis=2) == top)
        assert np.all(np.abs(q * s[..., None] - x) <= s[..., None] * 0.5 + 1e-7)


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr
    assert p.stdout == ""
