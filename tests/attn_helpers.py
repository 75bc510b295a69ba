"""Shared test helpers: the BASELINE configurations' seeded inputs, device
copies, and the comparison bars."""
import os

import numpy as np

from cases import normal, splitmix

KV_I8, KV_I16, KV_F16, KV_F32 = 0, 1, 2, 3

# parity bars (written here, used by every parity test)
TOL_F32_REL = 1e-5   # f32 decode: max |err| / max |ref|
TOL_F16_ABS = 2e-3   # f16 K/V paths: max |err| on softmax-normalised outputs
TOL_FLOAT_ABS = 1e-5  # int8 / int16 cache, FLOAT scores (test_attention.c:146)


# every parity check of the session: (test, what, achieved error, bar);
# conftest.py writes them out when JANAS_PARITY_OUT names a file
MARGINS = []


def within(err, bar, what=""):
    """Record a parity check's achieved error next to its bar (and print
    it); True when the error is within the bar."""
    test = os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]
    err, bar = float(err), float(bar)
    MARGINS.append((test, what, err, bar))
    print(f"{test} {what}: error {err:.3e}, bar {bar:.1e} "
          f"({err / bar:.1%} of it)")
    return err <= bar


def threads():
    return max(1, min(16, os.cpu_count() or 1))


def uniform_lens(seed, count, lo, hi):
    """count integers uniform in [lo, hi], from the counter generator."""
    z = splitmix(seed, count)
    return (lo + (z % np.uint64(hi - lo + 1))).astype(np.int64)


def cache(seed, n_kv, cap, hd, dtype):
    x = normal(seed, n_kv * cap * hd).reshape(n_kv, cap, hd)
    return x.astype(dtype)


def config(i, seed=20261201):
    """Inputs of BASELINE.json config i (1-based), as numpy arrays.
    Returns a dict: geometry, kv type, and a list of sequences."""
    if i == 1:
        h, kvh, hd, L = 32, 8, 128, 1024
        return dict(n_head=h, n_kv=kvh, hd=hd, kv=KV_F32, scale=None,
                    gate=None, seqs=[dict(
                        k=cache(seed + 1, kvh, L, hd, np.float32),
                        v=cache(seed + 2, kvh, L, hd, np.float32),
                        q=normal(seed + 3, h * hd).reshape(1, h, hd),
                        pos0=L - 1, n=1)])
    if i == 2:
        h, kvh, hd, L = 32, 8, 128, 1024
        return dict(n_head=h, n_kv=kvh, hd=hd, kv=KV_F16, scale=None,
                    gate=None, seqs=[dict(
                        k=cache(seed + 1, kvh, L, hd, np.float16),
                        v=cache(seed + 2, kvh, L, hd, np.float16),
                        q=normal(seed + 3, L * h * hd).reshape(L, h, hd),
                        pos0=0, n=L)])
    if i == 3:
        h, kvh, hd = 32, 8, 128
        lens = uniform_lens(seed, 8, 512, 8192)
        seqs = []
        for s, L in enumerate(lens):
            L = int(L)
            seqs.append(dict(k=cache(seed + 10 * s + 1, kvh, L, hd, np.float16),
                             v=cache(seed + 10 * s + 2, kvh, L, hd, np.float16),
                             q=normal(seed + 10 * s + 3, h * hd).reshape(1, h, hd),
                             pos0=L - 1, n=1))
        return dict(n_head=h, n_kv=kvh, hd=hd, kv=KV_F16, scale=None,
                    gate=None, seqs=seqs)
    if i == 4:
        h, kvh, hd, L = 16, 2, 256, 32768
        return dict(n_head=h, n_kv=kvh, hd=hd, kv=KV_F16,
                    scale=np.float32(1.0 / 16.0),
                    gate=normal(seed + 4, h * hd).reshape(1, h, hd),
                    seqs=[dict(k=cache(seed + 1, kvh, L, hd, np.float16),
                               v=cache(seed + 2, kvh, L, hd, np.float16),
                               q=normal(seed + 3, h * hd).reshape(1, h, hd),
                               pos0=L - 1, n=1)])
    if i == 5:
        # speculative verify: 8 drafts at 8192 .. 8199 over an 8192 cache
        h, kvh, hd, L, nd = 32, 8, 128, 8192, 8
        return dict(n_head=h, n_kv=kvh, hd=hd, kv=KV_F16, scale=None,
                    gate=None, seqs=[dict(
                        k=cache(seed + 1, kvh, L + nd, hd, np.float16),
                        v=cache(seed + 2, kvh, L + nd, hd, np.float16),
                        q=normal(seed + 3, nd * h * hd).reshape(nd, h, hd),
                        pos0=L, n=nd)])
    raise ValueError(i)


def oracle_out(orc, cfg, seq, block=64):
    """The restatement's output for one sequence of a config (gated)."""
    out = orc.run(np.ascontiguousarray(seq["q"], np.float32), seq["k"],
                  seq["v"], seq.get("ks"), seq.get("vs"), n_head=cfg["n_head"],
                  n_kv=cfg["n_kv"], hd=cfg["hd"], pos0=seq["pos0"],
                  kv=cfg["kv"], scale=cfg["scale"], threads=threads(),
                  block=block)
    if cfg.get("gate") is not None:
        orc.gate(out, cfg["gate"])
    return out


def rel_err(out, ref):
    return float(np.abs(out.astype(np.float64) - ref).max() /
                 max(np.abs(ref).max(), 1e-30))


def abs_err(out, ref):
    return float(np.abs(out.astype(np.float64) - ref).max())
