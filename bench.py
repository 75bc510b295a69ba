"""Benchmark of the KV-cache attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                    [--only decode|prefill|wide|copy|gemm|configs]

Headline (BASELINE.json metric): decode attention KV GB/s at 32k context on
BASELINE config 4 - 16 query / 2 KV heads, head_dim 256, 32,768 positions,
f16 K/V, f32 query, gate sigmoid(g) fused - and causal prefill TFLOPS at 8k
(32 / 8 / 128, 8,192 tokens). A step is one attention call over the resident
cache (the split kernel and the merge). Inputs are synthetic N(0, 1), drawn
from a fixed seed, resident in HBM before timing starts. The prefill figure
rides along in the same line under "prefill": one causal call over an
8,192-token prompt, its algorithmic flops (4 x head_dim per visible
(token, head, position)) over the launch time. Under "wide": Gemma 4's
head size - a decode step at 32k over an int16 cache with head_dim 512
(16 / 2 heads, the reference test's score scale 0.02), the wide kernel's
KV bytes (and scales) over its launch time. Beside the prefill, under
"reference_gemm": a plain f16 GEMM through the vendor library (torch.matmul,
8192^3, N(0, 1) operands) on the same box - the practical MFMA rate that
random data allows (the clock falls well below its 2.4 GHz peak under
random operands), as a yardstick for the prefill's fraction of 2.5 PFLOP/s.
Under "configs": the other BASELINE configurations, each timed as the
calls the engine makes, through the library's own routing
(janas_attn_run_dev): 1 (f32 decode at 1k, launch-bound), 2 (causal prefill
of 1,024 tokens), 3 (ragged decode of 8 sequences), 5a (verify of 8 drafts
at 8k) and 5b (an 8k prompt as 16 chunks of 512).

Prints one JSON line. ``roofline`` is the split kernel's: its algorithmic
bytes (every K/V element of the visible positions once) over its average
launch time, measured with HIP events on the stream it runs on, against the
8 TB/s HBM peak. ``cpu_baseline`` times this repo's C restatement of the
reference's CPU attention (oracle/, pthreads over the host's cores) on a
bounded sample of the same workload.
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = ("decode attn KV GB/s (% HBM peak) @32k ctx; "
          "prefill attn TFLOPS (% MFMA peak) @8k")
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
SEED = 20261201


def normal(rng, shape, dtype):
    return rng.standard_normal(shape, dtype=np.float32).astype(dtype)


def decode_workload():
    """BASELINE config 4."""
    h, kvh, hd, L = 16, 2, 256, 32768
    rng = np.random.default_rng(SEED)
    return dict(h=h, kvh=kvh, hd=hd, L=L, scale=1.0 / 16.0,
                k=normal(rng, (kvh, L, hd), np.float16),
                v=normal(rng, (kvh, L, hd), np.float16),
                q=normal(rng, (1, h, hd), np.float32),
                g=normal(rng, (1, h, hd), np.float32))


def quantized(x, dtype):
    """Rows of x (n_kv, L, hd) quantized as the engine's cache write does
    (model_attn.c:126-145): the row's largest magnitude becomes 127 or
    32767, one float scale a row."""
    top = 127 if dtype == np.int8 else 32767
    xf = x.astype(np.float32)
    mx = np.abs(xf).max(axis=2, keepdims=True)
    mx[mx == 0] = 1.0
    q = np.rint(xf * (top / mx)).astype(dtype)
    return q, (mx[..., 0] / top).astype(np.float32)


def int_decode_workload(dtype):
    """BASELINE config 4's shape over the engine's own cache formats: the
    same N(0, 1) keys and values as int8 or int16 with per-row scales."""
    w = decode_workload()
    k, ks = quantized(w["k"], dtype)
    v, vs = quantized(w["v"], dtype)
    return dict(w, k=k, v=v, ks=ks, vs=vs)


def wide_workload():
    """head_dim 512 over an int16 cache (Gemma 4's full-attention layers):
    keys and values uniform int16, scales U(0.001, 0.02) / 258 as the
    reference's test draws them (test_attention.c:270-279)."""
    h, kvh, hd, L = 16, 2, 512, 32768
    rng = np.random.default_rng(SEED + 4)
    ints = lambda: rng.integers(-32767, 32768, (kvh, L, hd), dtype=np.int16)
    scl = lambda: (rng.uniform(0.001, 0.02, (kvh, L)) / 258.0).astype(np.float32)
    return dict(h=h, kvh=kvh, hd=hd, L=L, scale=0.02, k=ints(), v=ints(),
                ks=scl(), vs=scl(), q=normal(rng, (1, h, hd), np.float32))


def prefill_workload():
    """The 8k causal prefill: BASELINE config 2's heads at 8,192 tokens."""
    h, kvh, hd, L = 32, 8, 128, 8192
    rng = np.random.default_rng(SEED + 2)
    return dict(h=h, kvh=kvh, hd=hd, L=L, scale=1.0 / np.sqrt(hd),
                k=normal(rng, (kvh, L, hd), np.float16),
                v=normal(rng, (kvh, L, hd), np.float16),
                q=normal(rng, (L, h, hd), np.float32))


def prefill_flops(hd, h, pos0, n):
    """4 x head_dim flops per (token, head, visible position): the score
    and the value product, causal."""
    seen = n * pos0 + n * (n + 1) / 2
    return 4.0 * hd * h * seen


def traffic_from_profiles(kernel):
    """HBM bytes a launch from profiles/<kernel>_traffic.md (the PMC runs'
    summary), or None."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_traffic.md")
    try:
        text = open(path).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    return float(m.group(1)) if m else None


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform's."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_cores():
    """Every core the host gives this process: the CPU baseline runs the
    restatement on all of them."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:
        return max(1, os.cpu_count() or 1)


def cpu_decode_baseline(w, budget_s=10.0):
    """The restatement on the host's cores over the same config-4 call."""
    from oracle import orc
    cores = cpu_cores()
    args = dict(n_head=w["h"], n_kv=w["kvh"], hd=w["hd"], pos0=w["L"] - 1,
                kv=orc.KV_F16, scale=w["scale"], threads=cores)
    orc.run(w["q"], w["k"], w["v"], **args)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        out = orc.run(w["q"], w["k"], w["v"], **args)
        orc.gate(out, w["g"])
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    kv_bytes = 2 * w["kvh"] * w["L"] * w["hd"] * 2
    return {"value": round(kv_bytes / t / 1e9, 3), "unit": "GB/s",
            "cores": cores, "cpu": cpu_model(), "kind": "port",
            "sample": f"config 4 decode call (32768 positions), median of "
                      f"{len(times)} calls, {t * 1e3:.1f} ms each"}


def cpu_prefill_baseline(w, block=64, every=8):
    """The restatement on the host's cores over the 8k prompt as the engine
    makes it: 128 calls of 64 tokens (model_attn.c:343-353). Every
    every-th call is timed (one each, after one warm-up call) and the
    prompt's time is their sum times every - a bounded sample: a block's
    cost grows linearly with its position, so the sampled blocks (positions
    0, 512, 1024, ...) stand for the 8 blocks after each of them up to half
    a block's growth, which the report's figure includes."""
    from oracle import orc
    cores = cpu_cores()
    L = w["L"]
    args = dict(n_head=w["h"], n_kv=w["kvh"], hd=w["hd"], kv=orc.KV_F16,
                scale=float(w["scale"]), threads=cores)
    q0 = np.ascontiguousarray(w["q"][:block])
    orc.run(q0, w["k"], w["v"], pos0=0, **args)  # warm-up
    starts = list(range(0, L, block * every))
    t = 0.0
    for p in starts:
        q = np.ascontiguousarray(w["q"][p:p + block])
        t0 = time.perf_counter()
        orc.run(q, w["k"], w["v"], pos0=p, **args)
        t += time.perf_counter() - t0
    # the sampled block stands for itself and the every - 1 after it; their
    # work grows by a block each, so scale by the ratio of the work
    sampled = sum(prefill_flops(w["hd"], w["h"], p, block) for p in starts)
    t_prompt = t * prefill_flops(w["hd"], w["h"], 0, L) / sampled
    fl = prefill_flops(w["hd"], w["h"], 0, L)
    return {"value": round(fl / t_prompt / 1e12, 4), "unit": "TFLOP/s",
            "cores": cores, "cpu": cpu_model(), "kind": "port",
            "sample": f"the {L}-token prompt as {L // block} calls of {block} "
                      f"tokens; {len(starts)} of them timed (every {every}th, "
                      f"{t:.2f} s) and the prompt's time scaled from them by "
                      f"the work (flops) of the calls: {t_prompt:.2f} s"}


NCOPY = 9  # 9 caches of 67 MB: more than twice the 256 MB infinity cache
# the 64-token block lines: 4160 positions over 8 KV heads of 128 (int8
# 8.5 MB with scales, f16 17 MB a copy), over 512 MB either way
NCOPY_BLOCK8 = 64
NCOPY_BLOCK16 = 32


def bench_decode(torch, jm, w, steps, warmup, kv=None, ncopy=NCOPY,
                 scores=None):
    """Decode steps (split + merge kernels) launched back to back on one
    stream, each over the next of ncopy copies of the cache - a real decode
    reads another layer's cache each call, so none stays in the 256 MB
    infinity cache. Then each kernel's average launch time: a batch of its
    launches alone, bracketed by HIP events on the same stream."""
    dev = torch.device("cuda:0")
    kv = jm.KV_F16 if kv is None else kv
    k0 = torch.from_numpy(w["k"]).to(dev)
    v0 = torch.from_numpy(w["v"]).to(dev)
    ks = [k0] + [k0.clone() for _ in range(ncopy - 1)]
    vs = [v0] + [v0.clone() for _ in range(ncopy - 1)]
    kz = torch.from_numpy(w["ks"]).to(dev) if "ks" in w else None
    vz = torch.from_numpy(w["vs"]).to(dev) if "vs" in w else None
    q = torch.from_numpy(w["q"]).to(dev)
    g = torch.from_numpy(w["g"]).to(dev) if "g" in w else None
    out = torch.empty_like(q)
    a = jm.Attention(w["h"], w["kvh"], w["hd"], w["L"], 1,
                     jm.FLOAT if scores is None else scores)
    a.set_scale(w["scale"])
    # a stream of its own: the legacy default stream's handle is 0, which
    # the library reads as "the instance's stream" - the events must be on
    # the stream the kernels run on
    stream = torch.cuda.Stream()

    def calls(path):
        return [a.prepare(kv, [dict(k=ks[i], v=vs[i], ks=kz, vs=vz, q=q,
                                    out=out, gate=g, cap=w["L"], n=1,
                                    pos0=w["L"] - 1)],
                          gate_mode=jm.GATE_ELEM if g is not None else
                          jm.GATE_NONE, stream=stream.cuda_stream,
                          path=path) for i in range(ncopy)]

    def timed(fns, n):
        assert stream.cuda_stream != 0
        for i in range(warmup):
            fns[i % ncopy]()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
            enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(n):
            fns[i % ncopy]()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n, time.perf_counter() - t0

    ms, wall = timed(calls("split"), steps)
    # each kernel alone: at least 500 launches (a 4 us kernel timed over a
    # handful of launches is mostly the events' own granularity)
    split_ms, _ = timed(calls("split-kernel"), max(steps, 500))
    merge_ms, _ = timed(calls("merge-kernel"), max(steps, 500))
    a.close()
    return ms, wall, split_ms, merge_ms


def bench_prefill(torch, jm, w, steps, warmup, kv=None):
    """One causal prefill call of the whole prompt, launches back to back on
    a stream of its own, HIP events around them on that stream. kv: the
    cache's element type (f16 by default; int8 / int16 with w's scales)."""
    dev = torch.device("cuda:0")
    k = torch.from_numpy(w["k"]).to(dev)
    v = torch.from_numpy(w["v"]).to(dev)
    q = torch.from_numpy(w["q"]).to(dev)
    kz = torch.from_numpy(w["ks"]).to(dev) if "ks" in w else None
    vz = torch.from_numpy(w["vs"]).to(dev) if "vs" in w else None
    out = torch.empty_like(q)
    stream = torch.cuda.Stream()
    assert stream.cuda_stream != 0
    with jm.Attention(w["h"], w["kvh"], w["hd"], w["L"]) as a:
        call = a.prepare(jm.KV_F16 if kv is None else kv,
                         [dict(k=k, v=v, ks=kz, vs=vz, q=q, out=out,
                               cap=w["L"], n=w["L"], pos0=0)],
                         stream=stream.cuda_stream, path="prefill")
        for _ in range(warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
            enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_gemm(torch, n=8192, steps=10, warmup=3):
    """f16 GEMM of two random N(0, 1) n x n matrices through torch.matmul
    (the vendor library): TFLOP/s over launches timed with HIP events on
    torch's current stream, where they run."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(SEED + 9)
    a = torch.randn(n, n, generator=g, device=dev, dtype=torch.float32).half()
    b = torch.randn(n, n, generator=g, device=dev, dtype=torch.float32).half()
    for _ in range(warmup):
        c = torch.matmul(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
        enable_timing=True)
    e0.record()
    for _ in range(steps):
        c = torch.matmul(a, b)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    del a, b, c
    return {"what": f"torch.matmul f16 {n}x{n}x{n}, N(0,1) operands",
            "value": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1),
            "unit": "TFLOP/s", "ms": round(ms, 4)}


def _timed(torch, fns, steps, warmup, stream):
    """ms per call of fns (rotating), HIP events on the calls' stream."""
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(
        enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        fns[i % len(fns)]()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def configs_leg(torch, jm, steps=200, warmup=20):
    """BASELINE configs 1, 2, 3, 5a and 5b (synthetic N(0, 1), seeded):
    one call (5b: the 16 chunk calls) through janas_attn_run_dev, on a
    stream of its own. Decode-like configs rotate over enough cache copies
    to exceed twice the 256 MB infinity cache (config 1's 8 MB is
    launch-bound by design and is not rotated). Also the drop-in's own
    prefill shape: a 64-token block at 4096 positions, the calls
    model_attn.c:343-353 makes, through janas_attn_run over an int8 cache
    and through janas_attn_run_dev over f16."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream()
    h, kvh, hd = 32, 8, 128
    res = {}

    def dev_t(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(dev)

    def decode_like(name, rng, kv, dtype, lens, n, ncopy, workload):
        cap = max(lens)
        seqs_np = [dict(k=normal(rng, (kvh, L, hd), dtype),
                        v=normal(rng, (kvh, L, hd), dtype),
                        q=normal(rng, (n, h, hd), np.float32), L=L)
                   for L in lens]
        copies = []
        for _ in range(ncopy):
            copies.append([dict(k=dev_t(x["k"]), v=dev_t(x["v"]),
                                q=dev_t(x["q"]),
                                out=torch.empty((n, h, hd), device=dev),
                                cap=x["L"], n=n, pos0=x["L"] - n)
                           for x in seqs_np])
        a = jm.Attention(h, kvh, hd, cap)
        fns = [a.prepare(kv, c, stream=stream.cuda_stream) for c in copies]
        ms = _timed(torch, fns, steps, warmup, stream)
        a.close()
        esz = np.dtype(dtype).itemsize
        kv_bytes = sum(2 * kvh * L * hd * esz for L in lens)
        gbs = kv_bytes / (ms * 1e-3) / 1e9
        res[name] = {"workload": workload, "ms": round(ms, 5),
                     "value": round(gbs, 1), "unit": "GB/s",
                     "kv_bytes": kv_bytes, "bound": "hbm",
                     "frac": round(gbs / HBM_PEAK_GBS, 4)}

    rng = np.random.default_rng(SEED + 21)
    decode_like("1", rng, jm.KV_F32, np.float32, [1024], 1, 1,
                "decode, 32 Q / 8 KV heads, head_dim 128, 1024 positions, "
                "f32 K/V and q (launch-bound)")
    rng = np.random.default_rng(SEED + 23)
    lens = [int(x) for x in rng.integers(512, 8193, 8)]
    decode_like("3", rng, jm.KV_F16, np.float16, lens, 1, 5,
                f"ragged decode, 8 sequences of {lens} positions, 32 / 8 "
                "heads, head_dim 128, f16 K/V, f32 q, one call")
    rng = np.random.default_rng(SEED + 25)
    decode_like("5a", rng, jm.KV_F16, np.float16, [8200], 8, 16,
                "verify: 8 drafts at positions 8192..8199 over the cache, "
                "32 / 8 heads, head_dim 128, f16 K/V, f32 q")

    def prefill_like(name, rng, L, chunk, reps, workload):
        k = dev_t(normal(rng, (kvh, L, hd), np.float16))
        v = dev_t(normal(rng, (kvh, L, hd), np.float16))
        q = dev_t(normal(rng, (L, h, hd), np.float32))
        out = torch.empty_like(q)
        a = jm.Attention(h, kvh, hd, L)
        fns = [a.prepare(jm.KV_F16, [dict(
            k=k, v=v, q=q[c:c + chunk], out=out[c:c + chunk], cap=L,
            n=chunk, pos0=c)], stream=stream.cuda_stream)
            for c in range(0, L, chunk)]
        ncall = len(fns)
        ms = _timed(torch, fns, reps * ncall, 2 * ncall, stream) * ncall
        a.close()
        fl = prefill_flops(hd, h, 0, L)
        tf = fl / (ms * 1e-3) / 1e12
        res[name] = {"workload": workload, "ms": round(ms, 5),
                     "value": round(tf, 2), "unit": "TFLOP/s", "flops": fl,
                     "bound": "mfma", "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}

    prefill_like("2", np.random.default_rng(SEED + 22), 1024, 1024, 50,
                 "causal prefill, 1024 tokens, 32 / 8 heads, head_dim 128, "
                 "f16 K/V, f32 q")
    prefill_like("5b", np.random.default_rng(SEED + 26), 8192, 512, 10,
                 "chunked prefill: an 8192-token prompt as 16 calls of 512 "
                 "(pos0 = 512 c) over the growing cache, 32 / 8 heads, "
                 "head_dim 128, f16 K/V, f32 q")

    # the drop-in's prefill: one 64-token block at positions 4096..4159,
    # each call over the next of enough cache copies to exceed twice the
    # infinity cache (an engine's layers each have their own cache)
    L, n, p0 = 4160, 64, 4096
    rng = np.random.default_rng(SEED + 27)
    kf = normal(rng, (kvh, L, hd), np.float32)
    vf = normal(rng, (kvh, L, hd), np.float32)
    q = dev_t(normal(rng, (n, h, hd), np.float32))
    out = torch.empty_like(q)
    fl = prefill_flops(hd, h, p0, n)
    k8, ks8 = quantized(kf, np.int8)
    v8, vs8 = quantized(vf, np.int8)
    k8, ks8, v8, vs8 = (dev_t(x) for x in (k8, ks8, v8, vs8))
    c8 = [(k8, ks8, v8, vs8)] + [tuple(x.clone() for x in (k8, ks8, v8, vs8))
                                  for _ in range(NCOPY_BLOCK8 - 1)]
    a = jm.Attention(h, kvh, hd, L, 1, jm.FLOAT)
    # janas_attn_run is synchronous on the instance's own stream: the time
    # a caller waits, by the host clock, over back-to-back calls
    for i in range(warmup):
        kk, kz, vv, vz = c8[i % len(c8)]
        a.run(q, kk, kz, vv, vz, n, p0, out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        kk, kz, vv, vz = c8[i % len(c8)]
        a.run(q, kk, kz, vv, vz, n, p0, out)
    ms = (time.perf_counter() - t0) * 1e3 / steps
    a.close()
    del c8
    res["block64-dropin-int8"] = {
        "workload": "janas_attn_run (the drop-in), 64 tokens at positions "
                    "4096..4159, 32 / 8 heads, head_dim 128, int8 K/V with "
                    "per-row scales, FLOAT scores, device pointers, "
                    f"{NCOPY_BLOCK8} cache copies in turn; host clock around "
                    "each synchronous call",
        "ms": round(ms, 5), "value": round(fl / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s", "flops": fl, "bound": "mfma",
        "frac": round(fl / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    k16, v16 = dev_t(kf.astype(np.float16)), dev_t(vf.astype(np.float16))
    c16 = [(k16, v16)] + [(k16.clone(), v16.clone())
                          for _ in range(NCOPY_BLOCK16 - 1)]
    a = jm.Attention(h, kvh, hd, L)
    fns = [a.prepare(jm.KV_F16, [dict(k=kk, v=vv, q=q, out=out, cap=L, n=n,
                                      pos0=p0)], stream=stream.cuda_stream)
           for kk, vv in c16]
    ms = _timed(torch, fns, steps, warmup, stream)
    a.close()
    del c16
    res["block64-f16"] = {
        "workload": "janas_attn_run_dev, one 64-token block at positions "
                    "4096..4159 (split path: a block equals its tokens), "
                    "32 / 8 heads, head_dim 128, f16 K/V, f32 q, "
                    f"{NCOPY_BLOCK16} cache copies in turn",
        "ms": round(ms, 5), "value": round(fl / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s", "flops": fl, "bound": "mfma",
        "frac": round(fl / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)}
    res.update(host_leg(torch, jm))
    return res


def host_leg(torch, jm, steps=40, warmup=5):
    """janas_attn_run with everything in host memory, as an engine linked
    unchanged calls it: the cache staged through the device at every call,
    and the same calls after janas_attn_import of the cache (only the rows
    of the call's positions cross PCIe). Host clock around each synchronous
    call; q and out cross PCIe either way."""
    res = {}

    def timed(a, args):
        for _ in range(warmup):
            a.run(*args)
        t0 = time.perf_counter()
        for _ in range(steps):
            a.run(*args)
        return (time.perf_counter() - t0) * 1e3 / steps

    cases = (
        ("block64", 32, 8, 128, 4160, 64, 4096),
        ("decode4", 16, 2, 256, 32768, 1, 32767),
    )
    for name, h, kvh, hd, L, n, p0 in cases:
        rng = np.random.default_rng(SEED + 29)
        k8, ks8 = quantized(normal(rng, (kvh, L, hd), np.float32), np.int8)
        v8, vs8 = quantized(normal(rng, (kvh, L, hd), np.float32), np.int8)
        q = normal(rng, (n, h, hd), np.float32)
        out = np.zeros_like(q)
        args = (q, k8, ks8, v8, vs8, n, p0, out)
        a = jm.Attention(h, kvh, hd, L, 1, jm.FLOAT)
        if hd == 256:
            a.set_scale(1.0 / 16.0)
        staged_ms = timed(a, args)
        for x in (k8, ks8, v8, vs8):
            assert a.import_host(x) == 0
        imported_ms = timed(a, args)
        a.close()
        fl = prefill_flops(hd, h, p0, n)
        kv_bytes = 2 * kvh * L * (hd + 4)
        res[f"dropin-host-{name}-int8"] = {
            "workload": f"janas_attn_run, host pointers, {n} token(s) at "
                        f"positions {p0}..{p0 + n - 1}, {h} / {kvh} heads, "
                        f"head_dim {hd}, int8 K/V with per-row scales, FLOAT "
                        "scores; host clock; staged: the cache copied to the "
                        "device at every call; imported: janas_attn_import "
                        "once, the call's rows copied",
            "staged_ms": round(staged_ms, 4), "imported_ms": round(imported_ms, 4),
            "unit": "ms", "kv_bytes": kv_bytes, "flops": fl}
    return res


def bench_copy(torch, steps):
    """A plain 64 MiB device copy: the known-size kernel that scales the
    HBM byte counters (FETCH_SIZE, WRITE_SIZE) of a profile."""
    dev = torch.device("cuda:0")
    src = torch.ones(16 << 20, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": src.numel() * 4,
                      "copy_bytes_written": dst.numel() * 4}), flush=True)


def wide_leg(torch, jm, steps, warmup):
    """The head_dim 512 int16 decode (wide kernel + merge), 5 cache copies
    of 134 MB so none stays in the infinity cache."""
    w = wide_workload()
    ms, _, split_ms, merge_ms = bench_decode(torch, jm, w, steps, warmup,
                                             kv=jm.KV_I16, ncopy=5)
    kv_bytes = 2 * w["kvh"] * w["L"] * w["hd"] * 2 + 2 * w["kvh"] * w["L"] * 4
    achieved = kv_bytes / (split_ms * 1e-3) / 1e9
    return {
        "metric": "hd-512 int16 decode attn KV GB/s @32k",
        "value": round(kv_bytes / (ms * 1e-3) / 1e9, 2), "unit": "GB/s",
        "ms": round(ms, 5),
        "config": {"workload": "decode, 16 Q / 2 KV heads, head_dim 512, "
                               "32768 positions, int16 K/V with per-row "
                               "scales, f32 q, score scale 0.02",
                   "kv_bytes": kv_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("wide_kernel_hd512"),
                     "kernel": "wide_kernel<i16, 512, 2>",
                     "kernel_us": round(split_ms * 1e3, 3),
                     "merge_us": round(merge_ms * 1e3, 3)},
    }


def int_leg(torch, jm, steps, warmup, prefill_steps=5):
    """The engine's own cache formats. Config 4's decode over int8 and int16
    caches: the step (split + merge), with the split kernel's own time and
    HBM rate; bytes: keys, values and their scales once. int8 twice: the
    FLOAT scores way, and the INT16 way (which AUTO resolves to at this
    context, as the reference's). Then the 8k prefill over the same prompt's
    rows quantized to int8 and to int16."""
    res = {}
    for name, dtype, kv, ncopy, scores in (
            ("4-int8", np.int8, jm.KV_I8, 16, jm.FLOAT),
            ("4-int8-int16", np.int8, jm.KV_I8, 16, jm.INT16),
            ("4-int16", np.int16, jm.KV_I16, 8, jm.FLOAT)):
        w = int_decode_workload(dtype)
        ms, _, split_ms, merge_ms = bench_decode(torch, jm, w, steps, warmup,
                                                 kv=kv, ncopy=ncopy,
                                                 scores=scores)
        b = 2 * w["k"].nbytes + 2 * w["ks"].nbytes
        way = "INT16" if scores == jm.INT16 else "FLOAT"
        res[name] = {"workload": "decode, 16 Q / 2 KV heads, head_dim 256, "
                                 f"32768 positions, {np.dtype(dtype).name} "
                                 "K/V with per-row scales, f32 q, gated, "
                                 f"{way} scores",
                     "ms": round(ms, 5), "value": round(b / (ms * 1e-3) / 1e9, 1),
                     "unit": "GB/s", "kv_bytes": b, "bound": "hbm",
                     "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "split_us": round(split_ms * 1e3, 3),
                     "split_frac": round(b / (split_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "merge_us": round(merge_ms * 1e3, 3)}
    w = prefill_workload()
    fl = prefill_flops(w["hd"], w["h"], 0, w["L"])
    for name, dtype, kv in (("8k-prefill-int8", np.int8, jm.KV_I8),
                            ("8k-prefill-int16", np.int16, jm.KV_I16)):
        k, ks = quantized(w["k"], dtype)
        v, vs = quantized(w["v"], dtype)
        ms = bench_prefill(torch, jm, dict(w, k=k, v=v, ks=ks, vs=vs),
                           prefill_steps, 2, kv=kv)
        tf = fl / (ms * 1e-3) / 1e12
        res[name] = {"workload": "causal prefill, 32 Q / 8 KV heads, head_dim "
                                 f"128, 8192 tokens, {np.dtype(dtype).name} K/V "
                                 "with per-row scales (the f16 prompt's rows "
                                 "quantized), f32 q",
                     "ms": round(ms, 4), "value": round(tf, 2),
                     "unit": "TFLOP/s", "flops": fl, "bound": "mfma",
                     "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline leg")
    ap.add_argument("--only", choices=("decode", "prefill", "wide", "copy",
                                       "gemm", "configs", "int"),
                    help="run one leg alone (profiling)")
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--kv", choices=("f16", "int8", "int16"), default="f16",
                    help="--only prefill: the cache's element type (int8 / "
                         "int16: the prompt's rows quantized, per-row scales)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is "
              "not supported (the path's multi-GPU sharding is design only)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import janas_amd as jm
    jm.lib()
    assert torch.cuda.is_available(), "bench.py needs the GPU"

    if args.only == "copy":
        bench_copy(torch, args.steps)
        return
    if args.only == "gemm":
        print(json.dumps(bench_gemm(torch)), flush=True)
        return
    if args.only == "configs":
        print(json.dumps(configs_leg(torch, jm)), flush=True)
        return
    if args.only == "int":
        print(json.dumps(int_leg(torch, jm, args.steps, args.warmup)),
              flush=True)
        return
    if args.only == "prefill":
        wp = prefill_workload()
        kv = None
        if args.kv != "f16":
            dt = np.int8 if args.kv == "int8" else np.int16
            k, ks = quantized(wp["k"], dt)
            v, vs = quantized(wp["v"], dt)
            wp = dict(wp, k=k, v=v, ks=ks, vs=vs)
            kv = jm.KV_I8 if args.kv == "int8" else jm.KV_I16
        pms = bench_prefill(torch, jm, wp, args.prefill_steps, 3, kv=kv)
        print(json.dumps({"prefill_ms": pms, "kv": args.kv}), flush=True)
        return
    if args.only == "wide":
        print(json.dumps(wide_leg(torch, jm, args.steps, args.warmup)),
              flush=True)
        return
    w = decode_workload()
    ms, wall, split_ms, merge_ms = bench_decode(torch, jm, w, args.steps,
                                                args.warmup)
    if args.only == "decode":
        print(json.dumps({"decode_ms": ms, "split_ms": split_ms,
                          "merge_ms": merge_ms}), flush=True)
        return
    kv_bytes = 2 * w["kvh"] * w["L"] * w["hd"] * 2
    value = kv_bytes / (ms * 1e-3) / 1e9
    split_us = split_ms * 1e3
    achieved = kv_bytes / (split_us * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic N(0,1), seeded",
        "config": {"workload": "BASELINE config 4: gated decode, 16 Q / 2 KV "
                               "heads, head_dim 256, 32768 positions, f16 K/V, "
                               "f32 q, element-wise gate",
                   "kv_bytes": kv_bytes, "hbm_peak_fraction": round(
                       value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles("split_kernel_cfg4"),
                     "kernel": "split_kernel<f16, 256>",
                     "kernel_us": round(split_us, 3),
                     "merge_us": round(merge_ms * 1e3, 3)},
    }
    wp = prefill_workload()
    pms = bench_prefill(torch, jm, wp, args.prefill_steps, 3)
    fl = prefill_flops(wp["hd"], wp["h"], 0, wp["L"])
    tf = fl / (pms * 1e-3) / 1e12
    line["prefill"] = {
        "metric": "causal prefill attn TFLOP/s @8k",
        "value": round(tf, 2), "unit": "TFLOP/s", "ms": round(pms, 4),
        "config": {"workload": "causal prefill, 32 Q / 8 KV heads, head_dim "
                               "128, 8192 tokens, f16 K/V, f32 q",
                   "flops": fl},
        "roofline": {"bound": "mfma", "achieved": round(tf, 2),
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                     "traffic": traffic_from_profiles("prefill_dma_kernel_8k"),
                     "kernel": "prefill_dma_kernel<128>"},
    }
    gemm = bench_gemm(torch)
    gemm["prefill_over_gemm"] = round(tf / gemm["value"], 4)
    line["prefill"]["reference_gemm"] = gemm
    line["wide"] = wide_leg(torch, jm, max(1, args.steps // 4),
                            min(args.warmup, 20))
    line["configs"] = configs_leg(torch, jm)
    line["configs"].update(int_leg(torch, jm, max(1, args.steps // 2),
                                          min(args.warmup, 20)))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_decode_baseline(w)
        line["prefill"]["cpu_baseline"] = cpu_prefill_baseline(wp)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
