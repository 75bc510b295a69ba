"""MFMA prefill path on the GPU against the CPU restatement of the
reference's attention: BASELINE config 2 (1024-token causal prefill), config
5's chunked prefill (8192 tokens in calls of 512 over the growing cache),
and the shapes the engine's callers make (model_attn.c:284-294) - ragged
lengths, GQA groups that do not divide the tile, padded head sizes, sliding
windows, a ring cache, set_last spans, the fused gate and several sequences
a call. The prefill path computes the query and the weights in f16, so the
bar is the f16 one (max abs error 2e-3 on the normalised outputs).

A call whose row blocks would leave compute units idle splits each block's
key tiles into segments merged in order afterwards; most of the small shapes
below take that route, the 8k prompt and the larger calls do not.
"""
import numpy as np
import pytest
import torch

import janas_amd
from attn_helpers import (KV_F16, KV_F32, TOL_F16_ABS, TOL_F32_REL,
                          TOL_FLOAT_ABS, abs_err, cache, config, oracle_out,
                          rel_err, threads, within)
from cases import normal
from janas_amd import Attention
from oracle import orc

pytestmark = pytest.mark.gpu


def to_dev(x, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def prefill_launches(a):
    return a.prof_read()["prefill"][0]


def run_prefill(a, seqs, gpu, gate_mode=0, path="prefill"):
    """seqs: numpy dicts (k, v, q, pos0, n, optional gate / last); returns
    the outputs as numpy arrays."""
    dev = []
    for s in seqs:
        d = dict(k=to_dev(s["k"], gpu), v=to_dev(s["v"], gpu),
                 q=to_dev(np.ascontiguousarray(s["q"], np.float32), gpu),
                 cap=s["k"].shape[1], n=s["n"], pos0=s["pos0"])
        d["out"] = torch.full(d["q"].shape, float("nan"), device=gpu)
        if s.get("gate") is not None:
            d["gate"] = to_dev(s["gate"], gpu)
        if s.get("last") is not None:
            d["last"] = to_dev(s["last"].astype(np.uint32).view(np.int32), gpu)
            d["last_max"] = int(s["last"].max())
        dev.append(d)
    a.run_dev(KV_F16, dev, gate_mode=gate_mode, path=path)
    torch.cuda.synchronize()
    return [d["out"].cpu().numpy() for d in dev]


def oracle(geom, s, gate_mode=0):
    out = orc.run(np.ascontiguousarray(s["q"], np.float32), s["k"], s["v"],
                  n_head=geom["n_head"], n_kv=geom["n_kv"], hd=geom["hd"],
                  pos0=s["pos0"], kv=KV_F16, scale=geom.get("scale"),
                  window=geom.get("window", 0), ring=geom.get("ring", False),
                  last=s.get("last"), threads=threads(), block=64)
    if gate_mode:
        orc.gate(out, s["gate"], per_head=gate_mode == janas_amd.GATE_HEAD)
    return out


def test_config2_causal_prefill(gpu):
    cfg = config(2)
    s = cfg["seqs"][0]
    with Attention(cfg["n_head"], cfg["n_kv"], cfg["hd"], s["k"].shape[1]) as a:
        a.prof_enable(True)
        (out,) = run_prefill(a, [s], gpu, path="auto")
        assert prefill_launches(a) == 1, "n > 64 must take the prefill path"
    ref = oracle_out(orc, cfg, s)
    err = abs_err(out, ref)
    print(f"config 2: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


def test_config5_chunked_prefill(gpu):
    """An 8192-token prompt in calls of 512 over the cache the earlier calls
    filled, and the same prompt in one call (the prefill headline): both
    checked directly against the restatement over row blocks of 512 tokens
    at the start, the middle and the end, and against each other within
    the f16 bar (a 512-token chunk splits its key range into segments, the
    whole prompt does not, so the two sum in a different order)."""
    h, kvh, hd, L, step = 32, 8, 128, 8192, 512
    seed = 20261201
    k = cache(seed + 11, kvh, L, hd, np.float16)
    v = cache(seed + 12, kvh, L, hd, np.float16)
    q = normal(seed + 13, L * h * hd).reshape(L, h, hd)
    kd, vd, qd = to_dev(k, gpu), to_dev(v, gpu), to_dev(q, gpu)
    chunked = torch.full(qd.shape, float("nan"), device=gpu)
    whole = torch.full(qd.shape, float("nan"), device=gpu)
    with Attention(h, kvh, hd, L) as a:
        a.prof_enable(True)
        for p0 in range(0, L, step):
            a.run_dev(KV_F16, [dict(k=kd, v=vd, q=qd[p0:p0 + step],
                                    out=chunked[p0:p0 + step], cap=L,
                                    n=step, pos0=p0)])
        a.run_dev(KV_F16, [dict(k=kd, v=vd, q=qd, out=whole, cap=L, n=L,
                                pos0=0)])
        torch.cuda.synchronize()
        assert prefill_launches(a) == L // step + 1
    out = chunked.cpu().numpy()
    wout = whole.cpu().numpy()
    diff = abs_err(out, wout)
    assert within(diff, TOL_F16_ABS, "chunked vs whole prompt")
    geom = dict(n_head=h, n_kv=kvh, hd=hd)
    worst, wworst = 0.0, 0.0
    for c in (0, 1, 8, 15):
        p0 = c * step
        ref = oracle(geom, dict(k=k, v=v, q=q[p0:p0 + step], pos0=p0))
        worst = max(worst, abs_err(out[p0:p0 + step], ref))
        wworst = max(wworst, abs_err(wout[p0:p0 + step], ref))
    assert within(worst, TOL_F16_ABS, "chunked, blocks 0 1 8 15 vs oracle")
    assert within(wworst, TOL_F16_ABS, "whole prompt, blocks 0 1 8 15 vs oracle")


# (n_head, n_kv, hd, cap, n, pos0, window, scale)
SHAPES = {
    "g4_hd128_ragged": (8, 2, 128, 512, 200, 37, 0, None),
    "g3_hd64": (6, 2, 64, 400, 300, 0, 0, None),
    "g1_hd96_late": (4, 4, 96, 1400, 129, 1000, 0, None),
    "g8_hd128_window": (8, 1, 128, 1024, 333, 50, 100, None),
    "g2_hd40_window_long": (4, 2, 40, 2048, 700, 1200, 513, 0.3),
    "g5_hd120_n65": (10, 2, 120, 300, 65, 200, 0, None),
    "g16_hd64": (16, 1, 64, 600, 257, 300, 0, None),
    # head size 256 (4 waves, 64-position tiles): config 4's heads, a
    # window, and 200 columns (the last tiles partly past the row)
    "g8_hd256_cfg4": (16, 2, 256, 1100, 700, 300, 0, 1.0 / 16),
    "g4_hd256_window": (8, 2, 256, 900, 257, 600, 300, None),
    "g3_hd200": (6, 2, 200, 500, 130, 100, 0, None),
    # head size 512 (Gemma 4's global layers): each row split into two
    # column halves whose partial scores meet in LDS; 384 and 264 leave the
    # second half partly or almost wholly past the row
    "g8_hd512_scale": (16, 2, 512, 900, 300, 400, 0, 0.02),
    "g4_hd384_window": (8, 2, 384, 800, 200, 500, 256, None),
    "g2_hd264": (4, 2, 264, 500, 130, 100, 0, None),
}


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_prefill_shapes(name, gpu):
    h, kvh, hd, cap, n, pos0, window, scale = SHAPES[name]
    seed = 7000 + sorted(SHAPES).index(name)
    s = dict(k=cache(seed, kvh, cap, hd, np.float16),
             v=cache(seed + 1, kvh, cap, hd, np.float16),
             q=normal(seed + 2, n * h * hd).reshape(n, h, hd), pos0=pos0, n=n)
    geom = dict(n_head=h, n_kv=kvh, hd=hd, scale=scale, window=window)
    with Attention(h, kvh, hd, cap) as a:
        if scale is not None:
            a.set_scale(scale)
        if window:
            a.set_window(window)
        (out,) = run_prefill(a, [s], gpu)
    ref = oracle(geom, s)
    err = abs_err(out, ref)
    print(f"{name}: max abs err {err:.2e}")
    assert np.isfinite(out).all()
    assert within(err, TOL_F16_ABS, "vs oracle")


@pytest.mark.parametrize("gate_mode", [janas_amd.GATE_ELEM,
                                       janas_amd.GATE_HEAD])
def test_prefill_gate(gate_mode, gpu):
    h, kvh, hd, cap, n = 16, 2, 128, 700, 300
    g_shape = (n, h, hd) if gate_mode == janas_amd.GATE_ELEM else (n, h)
    s = dict(k=cache(81, kvh, cap, hd, np.float16),
             v=cache(82, kvh, cap, hd, np.float16),
             q=normal(83, n * h * hd).reshape(n, h, hd), pos0=100, n=n,
             gate=normal(84, int(np.prod(g_shape))).reshape(g_shape))
    geom = dict(n_head=h, n_kv=kvh, hd=hd, scale=1.0 / 16)
    with Attention(h, kvh, hd, cap) as a:
        a.set_scale(1.0 / 16)
        (out,) = run_prefill(a, [s], gpu, gate_mode=gate_mode)
    err = abs_err(out, oracle(geom, s, gate_mode))
    print(f"gate {gate_mode}: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


def test_prefill_set_last_span(gpu):
    """A picture's tokens attend both ways within their span
    (attention.h:89-97)."""
    h, kvh, hd, cap, n, pos0 = 8, 2, 128, 600, 200, 150
    p = pos0 + np.arange(n)
    lo, hi = 230, 290
    last = np.where((p >= lo) & (p < hi), hi - 1, p).astype(np.uint32)
    s = dict(k=cache(91, kvh, cap, hd, np.float16),
             v=cache(92, kvh, cap, hd, np.float16),
             q=normal(93, n * h * hd).reshape(n, h, hd), pos0=pos0, n=n,
             last=last)
    geom = dict(n_head=h, n_kv=kvh, hd=hd)
    with Attention(h, kvh, hd, cap) as a:
        (out,) = run_prefill(a, [s], gpu)
    err = abs_err(out, oracle(geom, s))
    print(f"set_last span: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


def test_prefill_ring(gpu):
    """A sliding-window layer on a ring: position p in row p mod cap."""
    h, kvh, hd, cap, window, n, pos0 = 8, 2, 128, 1024, 256, 200, 3000
    s = dict(k=cache(101, kvh, cap, hd, np.float16),
             v=cache(102, kvh, cap, hd, np.float16),
             q=normal(103, n * h * hd).reshape(n, h, hd), pos0=pos0, n=n)
    geom = dict(n_head=h, n_kv=kvh, hd=hd, window=window, ring=True)
    with Attention(h, kvh, hd, cap) as a:
        a.set_window(window)
        a.set_ring(True)
        (out,) = run_prefill(a, [s], gpu)
    err = abs_err(out, oracle(geom, s))
    print(f"ring: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


def test_prefill_several_sequences(gpu):
    """Sequences of different lengths and offsets in one launch, each its
    own cache; each equals its own call bit for bit."""
    h, kvh, hd = 8, 2, 128
    seqs = []
    for i, (cap, n, pos0) in enumerate([(400, 100, 0), (900, 257, 640),
                                        (300, 70, 1), (2000, 512, 1488)]):
        seqs.append(dict(k=cache(200 + 3 * i, kvh, cap, hd, np.float16),
                         v=cache(201 + 3 * i, kvh, cap, hd, np.float16),
                         q=normal(202 + 3 * i, n * h * hd).reshape(n, h, hd),
                         pos0=pos0, n=n))
    geom = dict(n_head=h, n_kv=kvh, hd=hd)
    with Attention(h, kvh, hd, 2000) as a:
        outs = run_prefill(a, seqs, gpu)
        for s, out in zip(seqs, outs):
            (alone,) = run_prefill(a, [s], gpu)
            assert np.array_equal(out.view(np.int32), alone.view(np.int32))
            err = abs_err(out, oracle(geom, s))
            print(f"n {s['n']} pos0 {s['pos0']}: max abs err {err:.2e}")
            assert within(err, TOL_F16_ABS, "vs oracle")


# (n_head, n_kv, hd, cap, n, pos0, window): calls small enough to split
# their key range (a few row blocks over thousands of positions)
SPLITS = {
    "hd128_n65_late": (8, 2, 128, 3100, 65, 3000, 0),
    "hd128_g8_n100": (16, 2, 128, 5000, 100, 4800, 0),
    "hd96_window": (8, 2, 96, 4000, 90, 3500, 2000),
    "hd256_n100": (16, 2, 256, 2200, 100, 2000, 0),
    "hd512_n80": (8, 2, 512, 2100, 80, 2000, 0),
    # from position 0: the first row block has one tile for two segments
    # (an empty segment, merged as no weight)
    "hd64_n1536_start": (8, 2, 64, 1600, 1536, 0, 0),
}


@pytest.mark.parametrize("name", sorted(SPLITS))
def test_prefill_split_key_range(name, gpu):
    """Split calls against the restatement; the same call twice is bitwise
    the same."""
    h, kvh, hd, cap, n, pos0, window = SPLITS[name]
    sd = 7000 + hd + n
    s = dict(k=cache(sd, kvh, cap, hd, np.float16),
             v=cache(sd + 1, kvh, cap, hd, np.float16),
             q=normal(sd + 2, n * h * hd).reshape(n, h, hd), pos0=pos0, n=n)
    geom = dict(n_head=h, n_kv=kvh, hd=hd, window=window)
    with Attention(h, kvh, hd, cap) as a:
        if window:
            a.set_window(window)
        (out,) = run_prefill(a, [s], gpu)
        (again,) = run_prefill(a, [s], gpu)
    assert np.array_equal(out.view(np.int32), again.view(np.int32))
    err = abs_err(out, oracle(geom, s))
    print(f"{name}: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


# (n_head, n_kv, hd, cap, n, pos0, window, ring, span, gate): f16 calls
# whose DMA-kernel workgroups would leave compute units idle, which take
# the two-halves kernel (two key groups of 4 waves over 128 rows)
HALVES = {
    # 2 key tiles of 64 for the latest block: one a group
    "tiny_start": (8, 2, 128, 200, 100, 0, 0, False, False, 0),
    # an odd tile count (19): group 1's last step is masked
    "odd_tiles_hd96": (8, 2, 96, 1300, 200, 1000, 0, False, False, 0),
    # 48 tiles for a few blocks: key segments too, merged afterwards
    "segments": (8, 2, 128, 3100, 64, 3000, 0, False, False, 0),
    "window_ring": (8, 2, 128, 1024, 150, 2900, 300, True, False, 0),
    "span_gate": (16, 2, 128, 900, 200, 300, 0, False, True,
                  janas_amd.GATE_ELEM),
    "g3_hd80": (6, 2, 80, 700, 333, 200, 0, False, False, janas_amd.GATE_HEAD),
}


@pytest.mark.parametrize("name", sorted(HALVES))
def test_prefill_halves(name, gpu):
    """The two-halves kernel against the restatement; the same call twice is
    bitwise the same."""
    h, kvh, hd, cap, n, pos0, window, ring, span, gate = HALVES[name]
    sd = 7700 + sorted(HALVES).index(name) * 10
    s = dict(k=cache(sd, kvh, cap, hd, np.float16),
             v=cache(sd + 1, kvh, cap, hd, np.float16),
             q=normal(sd + 2, n * h * hd).reshape(n, h, hd), pos0=pos0, n=n)
    if span:
        p = pos0 + np.arange(n)
        s["last"] = np.where((p >= pos0 + 40) & (p < pos0 + 90), pos0 + 89,
                             p).astype(np.uint32)
    if gate:
        g_shape = (n, h, hd) if gate == janas_amd.GATE_ELEM else (n, h)
        s["gate"] = normal(sd + 3, int(np.prod(g_shape))).reshape(g_shape)
    geom = dict(n_head=h, n_kv=kvh, hd=hd, window=window, ring=ring)
    with Attention(h, kvh, hd, cap) as a:
        if window:
            a.set_window(window)
        if ring:
            a.set_ring(True)
        (out,) = run_prefill(a, [s], gpu, gate_mode=gate)
        (again,) = run_prefill(a, [s], gpu, gate_mode=gate)
    assert np.array_equal(out.view(np.int32), again.view(np.int32))
    err = abs_err(out, oracle(geom, s, gate))
    print(f"halves {name}: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


@pytest.mark.parametrize("n_kv,G,n,pos0", [(3, 2, 300, 900), (6, 2, 700, 0),
                                            (12, 2, 1100, 200)])
def test_prefill_kv_head_counts(n_kv, G, n, pos0, gpu):
    """KV head counts whose row blocks are dealt to groups of 8, 4 and 2
    XCDs (8 / gcd(n_kv, 8)): every workgroup runs once, against the
    restatement."""
    h, hd = n_kv * G, 128
    cap = pos0 + n
    sd = 7900 + n_kv
    s = dict(k=cache(sd, n_kv, cap, hd, np.float16),
             v=cache(sd + 1, n_kv, cap, hd, np.float16),
             q=normal(sd + 2, n * h * hd).reshape(n, h, hd), pos0=pos0, n=n)
    geom = dict(n_head=h, n_kv=n_kv, hd=hd)
    with Attention(h, n_kv, hd, cap) as a:
        (out,) = run_prefill(a, [s], gpu)
    err = abs_err(out, oracle(geom, s))
    print(f"n_kv {n_kv}: max abs err {err:.2e}")
    assert np.isfinite(out).all()
    assert within(err, TOL_F16_ABS, "vs oracle")


def test_prefill_halves_beside_dma_kernel(gpu):
    """A launch with sequences for both kernels (a 2048-token chunk fills
    the GPU with the DMA kernel's segments; the others take the halves):
    each sequence equals its own call bit for bit."""
    h, kvh, hd = 8, 2, 128
    seqs = []
    for i, (cap, n, pos0) in enumerate([(4096, 2048, 2048), (900, 257, 640),
                                        (300, 70, 1)]):
        seqs.append(dict(k=cache(240 + 3 * i, kvh, cap, hd, np.float16),
                         v=cache(241 + 3 * i, kvh, cap, hd, np.float16),
                         q=normal(242 + 3 * i, n * h * hd).reshape(n, h, hd),
                         pos0=pos0, n=n))
    geom = dict(n_head=h, n_kv=kvh, hd=hd)
    with Attention(h, kvh, hd, 4096) as a:
        outs = run_prefill(a, seqs, gpu)
        for s, out in zip(seqs, outs):
            (alone,) = run_prefill(a, [s], gpu)
            assert np.array_equal(out.view(np.int32), alone.view(np.int32))
            err = abs_err(out, oracle(geom, s))
            print(f"mixed launch n {s['n']} pos0 {s['pos0']}: max abs err {err:.2e}")
            assert within(err, TOL_F16_ABS, "vs oracle")


def quantized(seed, n_kv, cap, hd, wide):
    """A cache as the engine writes it (model_attn.c:115-145): each row's
    largest magnitude at 127 (32767), its scale max / 127."""
    x = cache(seed, n_kv, cap, hd, np.float32)
    top = np.float32(32767.0 if wide else 127.0)
    m = np.abs(x).max(axis=2)
    z = (m / top).astype(np.float32)
    q = np.rint(x * (top / m)[..., None]).astype(np.int16 if wide else np.int8)
    return q, z


def quantized_bar(hd):
    """int8 / int16 caches up to head size 256 take the exact kernel (the
    cached integers exact, the query and the weights as two f16 planes):
    the reference's own FLOAT bar (test_attention.c:146). Above 256 the
    register-staged kernel dequantizes rows into f16: the f16 bar."""
    return TOL_FLOAT_ABS if hd <= 256 else TOL_F16_ABS


@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("geom", [dict(n_head=32, n_kv=8, hd=128, cap=1024,
                                       n=1024, pos0=0),
                                  dict(n_head=12, n_kv=4, hd=64, cap=900,
                                       n=333, pos0=500, window=300),
                                  dict(n_head=8, n_kv=1, hd=96, cap=768,
                                       n=200, pos0=600, window=200,
                                       ring=True),
                                  dict(n_head=16, n_kv=2, hd=256, cap=800,
                                       n=500, pos0=100),
                                  dict(n_head=6, n_kv=3, hd=200, cap=700,
                                       n=90, pos0=0),
                                  dict(n_head=16, n_kv=2, hd=512, cap=900,
                                       n=300, pos0=400, window=1024)])
def test_prefill_quantized_cache(gpu, wide, geom):
    """int8 / int16 caches with their scales (the engine's own format) on
    the MFMA path: up to head size 256 the exact kernel over a copy of the
    visible rows as f16 planes, within the reference's FLOAT bar; at 512
    the rows dequantized into f16 as tiles are staged, within the f16 bar."""
    h, kvh, hd, cap = geom["n_head"], geom["n_kv"], geom["hd"], geom["cap"]
    n, pos0 = geom["n"], geom["pos0"]
    k, ks = quantized(400 + hd, kvh, cap, hd, wide)
    v, vs = quantized(401 + hd, kvh, cap, hd, wide)
    q = normal(402 + hd, n * h * hd).reshape(n, h, hd)
    kv = janas_amd.KV_I16 if wide else janas_amd.KV_I8
    out = torch.full((n, h, hd), float("nan"), device=gpu)
    with Attention(h, kvh, hd, cap) as a:
        if geom.get("window"):
            a.set_window(geom["window"])
        if geom.get("ring"):
            a.set_ring(True)
        a.prof_enable(True)
        a.run_dev(kv, [dict(k=to_dev(k, gpu), v=to_dev(v, gpu),
                            ks=to_dev(ks, gpu), vs=to_dev(vs, gpu),
                            q=to_dev(q, gpu), out=out, cap=cap, n=n,
                            pos0=pos0)], path="prefill")
        torch.cuda.synchronize()
        # the prefill path (and, up to head size 256, its copy pass), not
        # the split path
        prof = a.prof_read()
        assert prof["prefill"][0] >= 1 and prof["split"][0] == 0
    ref = orc.run(q, k, v, ks, vs, n_head=h, n_kv=kvh, hd=hd, pos0=pos0,
                  kv=kv, window=geom.get("window", 0),
                  ring=geom.get("ring", False), threads=threads(), block=64)
    err = abs_err(out.cpu().numpy(), ref)
    print(f"{geom} wide={wide}: max abs err {err:.2e}")
    assert within(err, quantized_bar(hd), "vs oracle")


@pytest.mark.parametrize("hd", [128, 64, 256])
@pytest.mark.parametrize("wide", [False, True])
def test_prefill_quantized_long_prompt_exact(gpu, wide, hd):
    """A long int8 / int16 prompt through janas_attn_run_dev (the engine's
    route for calls of more than 64 tokens) takes the exact kernel over a
    copy of its rows; the allocation-free entry point, whose copy and
    partials sit in the device's fixed array, gives the same bits. Both
    within the reference's FLOAT bar of the restatement."""
    h, kvh, n, pos0 = (32, 8, 2048, 0) if hd <= 128 else (16, 2, 1536, 0)
    k, ks = quantized(9100 + wide, kvh, n, hd, wide)
    v, vs = quantized(9102 + wide, kvh, n, hd, wide)
    q = normal(9104, n * h * hd).reshape(n, h, hd)
    kv = janas_amd.KV_I16 if wide else janas_amd.KV_I8
    d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), ks=to_dev(ks, gpu),
             vs=to_dev(vs, gpu), q=to_dev(q, gpu), cap=n, n=n, pos0=pos0)
    outs = []
    with Attention(h, kvh, hd, n, 1, janas_amd.FLOAT) as a:
        for path in ("auto", "noalloc"):
            dd = dict(d, out=torch.full(d["q"].shape, float("nan"), device=gpu))
            a.prof_enable(True)
            a.run_dev(kv, [dd], path=path)
            torch.cuda.synchronize()
            prof = a.prof_read()
            if path == "auto":
                assert prof["prefill"][0] >= 1 and prof["split"][0] == 0
            outs.append(dd["out"].cpu().numpy())
    assert np.array_equal(outs[0].view(np.int32), outs[1].view(np.int32))
    ref = orc.run(q.astype(np.float32), k, v, ks, vs, n_head=h, n_kv=kvh,
                  hd=hd, pos0=pos0, kv=kv, threads=threads(), block=64)
    err = abs_err(outs[0], ref)
    print(f"exact {'int16' if wide else 'int8'} hd {hd}: max abs err {err:.2e}")
    assert within(err, TOL_FLOAT_ABS, "vs oracle")


@pytest.mark.parametrize("wide", [False, True])
def test_prefill_quantized_8k(gpu, wide):
    """The benched 8k prompt (32 / 8 / 128, one call) over the engine's own
    int8 / int16 cache, checked against the restatement over row blocks of
    512 tokens at the start, the middle and the end, at the reference's
    FLOAT bar."""
    h, kvh, hd, L, step = 32, 8, 128, 8192, 512
    k, ks = quantized(9200 + wide, kvh, L, hd, wide)
    v, vs = quantized(9202 + wide, kvh, L, hd, wide)
    q = normal(9204, L * h * hd).reshape(L, h, hd)
    kv = janas_amd.KV_I16 if wide else janas_amd.KV_I8
    out = torch.full((L, h, hd), float("nan"), device=gpu)
    with Attention(h, kvh, hd, L, 1, janas_amd.FLOAT) as a:
        a.prof_enable(True)
        a.run_dev(kv, [dict(k=to_dev(k, gpu), v=to_dev(v, gpu),
                            ks=to_dev(ks, gpu), vs=to_dev(vs, gpu),
                            q=to_dev(q, gpu), out=out, cap=L, n=L, pos0=0)])
        torch.cuda.synchronize()
        prof = a.prof_read()
        assert prof["prefill"][0] >= 1 and prof["split"][0] == 0
    o = out.cpu().numpy()
    worst = 0.0
    for c in (0, 1, 8, 15):
        p0 = c * step
        ref = orc.run(q[p0:p0 + step], k, v, ks, vs, n_head=h, n_kv=kvh,
                      hd=hd, pos0=p0, kv=kv, threads=threads(), block=64)
        worst = max(worst, abs_err(o[p0:p0 + step], ref))
    print(f"8k {'int16' if wide else 'int8'}: max abs err {worst:.2e}")
    assert within(worst, TOL_FLOAT_ABS, "blocks 0 1 8 15 vs oracle")


def test_prefill_refuses_what_it_has_no_kernel_for(gpu):
    """f32 caches have no prefill kernel: janas_attn_run_dev_prefill says
    ENOTSUP, janas_attn_run_dev takes the split path (float-accurate)."""
    h, kvh, hd, cap, n = 4, 2, 128, 300, 100
    k = cache(301, kvh, cap, hd, np.float32)
    v = cache(302, kvh, cap, hd, np.float32)
    q = normal(303, n * h * hd).reshape(n, h, hd)
    d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), q=to_dev(q, gpu),
             out=torch.full((n, h, hd), float("nan"), device=gpu),
             cap=cap, n=n, pos0=0)
    with Attention(h, kvh, hd, cap) as a:
        with pytest.raises(janas_amd.AttnError) as e:
            a.run_dev(KV_F32, [d], path="prefill")
        assert e.value.code == -5
        a.prof_enable(True)
        a.run_dev(KV_F32, [d], path="auto")
        torch.cuda.synchronize()
        assert prefill_launches(a) == 0
    ref = orc.run(q, k, v, None, None, n_head=h, n_kv=kvh, hd=hd, pos0=0,
                  kv=KV_F32, threads=threads(), block=64)
    assert within(rel_err(d["out"].cpu().numpy(), ref), TOL_F32_REL, "rel_err(d['out'].cpu().numpy(), ref)")


@pytest.mark.parametrize("kv", [KV_F16, janas_amd.KV_I8])
@pytest.mark.parametrize("path,n", [("split", 40), ("prefill", 200)])
def test_last_past_last_max_is_clamped(gpu, kv, path, n):
    """set_last entries past the call's last_max see up to last_max, on the
    split path and on the prefill path (f16 and the exact int8 kernel)
    alike: the same bits as the call with those entries clamped, and within
    the bar of the restatement given the clamped entries."""
    h, kvh, hd, cap, pos0 = 8, 2, 128, 600, 150
    last_max = pos0 + n - 1 + 20
    last = np.arange(pos0, pos0 + n, dtype=np.int64)
    last[n // 3: 2 * n // 3] = pos0 + n - 1 + 15      # a span, inside
    last[2 * n // 3:] = last_max + 37                  # past last_max
    clamped = np.minimum(last, last_max)
    if kv == KV_F16:
        k = cache(321, kvh, cap, hd, np.float16)
        v = cache(322, kvh, cap, hd, np.float16)
        ks = vs = None
    else:
        k, ks = quantized(321, kvh, cap, hd, False)
        v, vs = quantized(322, kvh, cap, hd, False)
    q = normal(323, n * h * hd).reshape(n, h, hd)
    outs = []
    with Attention(h, kvh, hd, cap, 1, janas_amd.FLOAT) as a:
        for lst in (last, clamped):
            d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), q=to_dev(q, gpu),
                     out=torch.full((n, h, hd), float("nan"), device=gpu),
                     cap=cap, n=n, pos0=pos0, last_max=last_max,
                     last=to_dev(lst.astype(np.uint32).view(np.int32), gpu))
            if ks is not None:
                d.update(ks=to_dev(ks, gpu), vs=to_dev(vs, gpu))
            a.run_dev(kv, [d], path=path)
            torch.cuda.synchronize()
            outs.append(d["out"].cpu().numpy())
    assert np.array_equal(outs[0].view(np.int32), outs[1].view(np.int32))
    ref = orc.run(q, k, v, ks, vs, n_head=h, n_kv=kvh, hd=hd, pos0=pos0,
                  kv=kv, last=clamped.astype(np.uint32), threads=threads(),
                  block=64)
    bar = TOL_F16_ABS if (kv == KV_F16 and path == "prefill") else TOL_FLOAT_ABS
    assert within(abs_err(outs[0], ref), bar, f"{path} clamped last[]")
