"""Seeded random geometries through janas_attn_run_dev against the CPU
restatement: element type, head size, GQA group, block length, position,
window, ring and output gate drawn from a fixed counter generator, on both
paths (split-KV for blocks of up to 64 tokens, the MFMA prefill for longer
ones). The cases are the same on every run; each prints its draw first.

Bars: the split path is float-accurate (f32 cache: max |err| / max |ref|
1e-5; int8 / int16 / f16: 1e-5 of max(1, max |ref|), the reference's FLOAT
bar, test_attention.c:146); so is the prefill path over int8 / int16 caches
up to head size 256 (the exact kernel); over f16 caches, and at head size
512, it computes in f16 (2e-3 abs).
"""
import numpy as np
import pytest
import torch

import janas_amd
from attn_helpers import (KV_F16, KV_F32, KV_I8, KV_I16, TOL_F16_ABS,
                          TOL_F32_REL, TOL_FLOAT_ABS, abs_err, cache, rel_err,
                          threads, within)
from cases import normal, splitmix
from janas_amd import Attention
from oracle import orc

pytestmark = pytest.mark.gpu

N_CASES = 48
CHUNK = 256


def draw(i):
    """Case i's geometry, from 12 draws of the counter generator."""
    z = [int(x) for x in splitmix(7100 + i, 12)]
    prefill = i % 3 == 2
    kinds = [KV_I8, KV_I16, KV_F16] if prefill else [KV_I8, KV_I16, KV_F16, KV_F32]
    kv = kinds[z[0] % len(kinds)]
    hds = [64, 96, 128] if kv == KV_F32 else [64, 96, 128, 200, 256, 320, 512]
    hd = hds[z[1] % len(hds)]
    group = [1, 2, 4, 8][z[2] % 4]
    n_kv = 1 + z[3] % 3
    n = 65 + z[4] % 300 if prefill else 1 + z[4] % 64
    pos0 = z[5] % 3000
    window = 0 if z[6] % 2 else 64 + z[7] % 1500
    ring = window > 0 and z[8] % 3 == 0
    gate = z[9] % 3  # 0 none, 1 per element, 2 per head
    if ring:
        # a ring of whole chunks that holds the call (attention.c:1281-1286)
        cap = CHUNK * ((window + n) // CHUNK + 3)
    else:
        cap = pos0 + n + z[10] % 200
    return dict(kv=kv, hd=hd, n_head=group * n_kv, n_kv=n_kv, n=n, pos0=pos0,
                window=window, ring=ring, gate=gate, cap=cap,
                path="prefill" if prefill else "split", seed=9100 + 10 * i)


def inputs(g):
    """K / V in the cache's element type (int8 / int16 as the engine writes
    them: each row's largest magnitude at the top code, scale max / top),
    q, and the gate."""
    n_kv, cap, hd, s = g["n_kv"], g["cap"], g["hd"], g["seed"]
    ks = vs = None
    if g["kv"] in (KV_I8, KV_I16):
        top = np.float32(127.0 if g["kv"] == KV_I8 else 32767.0)
        dt = np.int8 if g["kv"] == KV_I8 else np.int16
        out = []
        for j in (1, 2):
            x = cache(s + j, n_kv, cap, hd, np.float32)
            m = np.maximum(np.abs(x).max(axis=2), np.float32(1e-20))
            out.append((np.rint(x * (top / m)[..., None]).astype(dt),
                        (m / top).astype(np.float32)))
        (k, ks), (v, vs) = out
    else:
        dt = np.float16 if g["kv"] == KV_F16 else np.float32
        k = cache(s + 1, n_kv, cap, hd, dt)
        v = cache(s + 2, n_kv, cap, hd, dt)
    q = normal(s + 3, g["n"] * g["n_head"] * hd).reshape(g["n"], g["n_head"], hd)
    gate = None
    if g["gate"] == 1:
        gate = normal(s + 4, g["n"] * g["n_head"] * hd).reshape(g["n"], g["n_head"], hd)
    elif g["gate"] == 2:
        gate = normal(s + 4, g["n"] * g["n_head"]).reshape(g["n"], g["n_head"])
    return k, v, ks, vs, q, gate


def to_dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_geometry(gpu, i):
    g = draw(i)
    print(f"case {i}: {g}", flush=True)
    k, v, ks, vs, q, gate = inputs(g)
    n, h, hd = g["n"], g["n_head"], g["hd"]
    d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), q=to_dev(q, gpu),
             out=torch.full((n, h, hd), float("nan"), device=gpu),
             cap=g["cap"], n=n, pos0=g["pos0"])
    if ks is not None:
        d["ks"], d["vs"] = to_dev(ks, gpu), to_dev(vs, gpu)
    gate_mode = 0
    if gate is not None:
        d["gate"] = to_dev(gate, gpu)
        gate_mode = janas_amd.GATE_ELEM if g["gate"] == 1 else janas_amd.GATE_HEAD
    with Attention(h, g["n_kv"], hd, g["cap"]) as a:
        if g["window"]:
            a.set_window(g["window"])
        if g["ring"]:
            a.set_ring(True)
        a.run_dev(g["kv"], [d], gate_mode=gate_mode, path=g["path"])
        torch.cuda.synchronize()
    out = d["out"].cpu().numpy()
    ref = orc.run(np.ascontiguousarray(q, np.float32), k, v, ks, vs,
                  n_head=h, n_kv=g["n_kv"], hd=hd, pos0=g["pos0"], kv=g["kv"],
                  window=g["window"], ring=g["ring"], threads=threads(),
                  block=64)
    if gate is not None:
        orc.gate(ref, gate, per_head=g["gate"] == 2)
    assert np.isfinite(out).all()
    exact = g["kv"] in (KV_I8, KV_I16) and hd <= 256
    if g["path"] == "prefill" and not exact:
        err, bar = abs_err(out, ref), TOL_F16_ABS
    elif g["kv"] == KV_F32:
        err, bar = rel_err(out, ref), TOL_F32_REL
    else:
        err = abs_err(out, ref)
        bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
    print(f"case {i}: max err {err:.2e} (bar {bar:.1e})")
    assert within(err, bar, "vs oracle")


N_INT16 = 24


@pytest.mark.parametrize("i", range(N_INT16))
def test_random_geometry_int16(gpu, i):
    """The INT16 way over int8 caches (blocks of up to 64 tokens, split-KV;
    head sizes 64 to 512: the f16 planes' products at 64, the integer key
    products from 128, the wide kernel at 512) against the restatement's
    INT16 way, whose scores, weights and quantized weights are the
    reference's bits: within the FLOAT bar (the sums differ only in order)."""
    z = [int(x) for x in splitmix(7500 + i, 10)]
    hd = [64, 128, 256, 512][z[0] % 4]
    group = [1, 2, 4, 8][z[1] % 4]
    n_kv = 1 + z[2] % 3
    n = 1 + z[3] % 64
    pos0 = z[4] % 3000
    window = 0 if z[5] % 2 else 64 + z[6] % 1500
    ring = window > 0 and z[7] % 3 == 0
    cap = CHUNK * ((window + n) // CHUNK + 3) if ring else pos0 + n + z[8] % 200
    g = dict(kv=KV_I8, hd=hd, n_head=group * n_kv, n_kv=n_kv, n=n, pos0=pos0,
             window=window, ring=ring, gate=z[9] % 3, cap=cap, path="split",
             seed=9700 + 10 * i)
    print(f"case {i}: {g}", flush=True)
    k, v, ks, vs, q, gate = inputs(g)
    h = g["n_head"]
    d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), ks=to_dev(ks, gpu), vs=to_dev(vs, gpu),
             q=to_dev(q, gpu), out=torch.full((n, h, hd), float("nan"), device=gpu),
             cap=cap, n=n, pos0=pos0)
    gate_mode = 0
    if gate is not None:
        d["gate"] = to_dev(gate, gpu)
        gate_mode = janas_amd.GATE_ELEM if g["gate"] == 1 else janas_amd.GATE_HEAD
    with Attention(h, n_kv, hd, cap, 1, janas_amd.INT16) as a:
        if window:
            a.set_window(window)
        if ring:
            a.set_ring(True)
        a.run_dev(KV_I8, [d], gate_mode=gate_mode, path="split")
        torch.cuda.synchronize()
    out = d["out"].cpu().numpy()
    ref = orc.run(np.ascontiguousarray(q, np.float32), k, v, ks, vs, n_head=h,
                  n_kv=n_kv, hd=hd, pos0=pos0, kv=KV_I8, window=window, ring=ring,
                  threads=threads(), block=64, int16=True)
    if gate is not None:
        orc.gate(ref, gate, per_head=g["gate"] == 2)
    assert np.isfinite(out).all()
    err = abs_err(out, ref)
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
    print(f"case {i}: max err {err:.2e} (bar {bar:.1e})")
    assert within(err, bar, "INT16 vs oracle")


@pytest.mark.parametrize("path", ["split", "prefill"])
def test_random_many_sequences(gpu, path):
    """19 sequences of random lengths and offsets in one call: the library
    launches them 16 at a time, and each workgroup finds its sequence among
    the launch's; every sequence must equal its own restatement."""
    h, kvh, hd = 8, 2, 128
    z = [int(x) for x in splitmix(7300 + (path == "prefill"), 3 * 19)]
    seqs, dev = [], []
    for i in range(19):
        n = 1 + z[3 * i] % 40 if path == "split" else 65 + z[3 * i] % 150
        pos0 = z[3 * i + 1] % 1500
        cap = pos0 + n + z[3 * i + 2] % 100
        s = dict(k=cache(7400 + 4 * i, kvh, cap, hd, np.float16),
                 v=cache(7401 + 4 * i, kvh, cap, hd, np.float16),
                 q=normal(7402 + 4 * i, n * h * hd).reshape(n, h, hd),
                 pos0=pos0, n=n)
        seqs.append(s)
        dev.append(dict(k=to_dev(s["k"], gpu), v=to_dev(s["v"], gpu),
                        q=to_dev(s["q"], gpu),
                        out=torch.full((n, h, hd), float("nan"), device=gpu),
                        cap=cap, n=n, pos0=pos0))
    print(f"{path}: lengths {[s['n'] for s in seqs]}", flush=True)
    with Attention(h, kvh, hd, 4096) as a:
        a.run_dev(KV_F16, dev, path=path)
        torch.cuda.synchronize()
    worst = 0.0
    for s, d in zip(seqs, dev):
        ref = orc.run(np.ascontiguousarray(s["q"], np.float32), s["k"], s["v"],
                      n_head=h, n_kv=kvh, hd=hd, pos0=s["pos0"], kv=KV_F16,
                      threads=threads(), block=64)
        out = d["out"].cpu().numpy()
        assert np.isfinite(out).all()
        err = abs_err(out, ref)
        worst = max(worst, err if path == "prefill" else
                    err / max(1.0, float(np.abs(ref).max())))
    bar = TOL_F16_ABS if path == "prefill" else TOL_FLOAT_ABS
    print(f"{path}: worst err {worst:.2e} (bar {bar:.0e})")
    assert within(worst, bar, "worst vs oracle")


def draw_exact(i):
    """Case i of the exact kernel's geometries: int8 or int16, head sizes up
    to 256 (padded ones too), any group, windows, rings, gates, prompts of
    65 to 700 tokens."""
    z = [int(x) for x in splitmix(7500 + i, 12)]
    kv = [KV_I8, KV_I16][z[0] % 2]
    hd = [40, 64, 96, 128, 200, 256][z[1] % 6]
    group = [1, 2, 3, 4, 8][z[2] % 5]
    n_kv = 1 + z[3] % 3
    n = 65 + z[4] % 636
    pos0 = z[5] % 2000
    window = 0 if z[6] % 2 else 64 + z[7] % 1200
    ring = window > 0 and z[8] % 3 == 0
    gate = z[9] % 3
    cap = CHUNK * ((window + n) // CHUNK + 3) if ring else pos0 + n + z[10] % 200
    return dict(kv=kv, hd=hd, n_head=group * n_kv, n_kv=n_kv, n=n, pos0=pos0,
                window=window, ring=ring, gate=gate, cap=cap, path="prefill",
                seed=9600 + 10 * i)


@pytest.mark.parametrize("i", range(32))
def test_random_exact_prefill(gpu, i):
    """The exact kernel on seeded random geometries, two sequences a launch
    (the second a shorter, later call over the same cache, so their copies
    sit at different offsets), each within the FLOAT bar of the
    restatement."""
    g = draw_exact(i)
    print(f"case {i}: {g}", flush=True)
    k, v, ks, vs, q, gate = inputs(g)
    n, h, hd = g["n"], g["n_head"], g["hd"]
    n2 = max(1, n // 3)
    p2 = g["pos0"] + n - n2
    calls = [(q, g["pos0"], n, gate), (q[-n2:], p2, n2,
                                       None if gate is None else gate[-n2:])]
    gate_mode = 0 if gate is None else (janas_amd.GATE_ELEM if g["gate"] == 1
                                        else janas_amd.GATE_HEAD)
    dev = []
    for qq, p, m, gg in calls:
        d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), ks=to_dev(ks, gpu),
                 vs=to_dev(vs, gpu), q=to_dev(qq, gpu),
                 out=torch.full((m, h, hd), float("nan"), device=gpu),
                 cap=g["cap"], n=m, pos0=p)
        if gg is not None:
            d["gate"] = to_dev(gg, gpu)
        dev.append(d)
    with Attention(h, g["n_kv"], hd, g["cap"]) as a:
        if g["window"]:
            a.set_window(g["window"])
        if g["ring"]:
            a.set_ring(True)
        a.prof_enable(True)
        a.run_dev(g["kv"], dev, gate_mode=gate_mode, path="prefill")
        torch.cuda.synchronize()
        assert a.prof_read()["split"][0] == 0
    worst = 0.0
    for (qq, p, m, gg), d in zip(calls, dev):
        ref = orc.run(np.ascontiguousarray(qq, np.float32), k, v, ks, vs,
                      n_head=h, n_kv=g["n_kv"], hd=hd, pos0=p, kv=g["kv"],
                      window=g["window"], ring=g["ring"], threads=threads(),
                      block=64)
        if gg is not None:
            orc.gate(ref, gg, per_head=g["gate"] == 2)
        out = d["out"].cpu().numpy()
        assert np.isfinite(out).all()
        worst = max(worst, abs_err(out, ref) / max(1.0, float(np.abs(ref).max())))
    print(f"case {i}: worst err {worst:.2e}")
    assert within(worst, TOL_FLOAT_ABS, "exact prefill vs oracle")
