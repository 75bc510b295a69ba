"""Split-KV path on the GPU against the CPU restatement and the reference's
golden outputs: the drop-in janas_attn_run (host and device pointers), the
device extension on BASELINE configs 1, 3, 4 and 5 (verify), and the
block-versus-token bit identity the reference promises (attention.h:13-16).
"""
import numpy as np
import pytest
import torch

import janas_amd
from attn_helpers import (KV_F16, KV_F32, KV_I8, TOL_F16_ABS, TOL_F32_REL,
                          TOL_FLOAT_ABS, abs_err, config, oracle_out, rel_err, within)
from cases import CASES, KV_I16, call_kwargs, make_inputs
from janas_amd import Attention
from oracle import orc

pytestmark = pytest.mark.gpu

MAX_BLOCK = janas_amd.MAX_BLOCK
# every golden case, Gemma 4's head_dim 512 included (the wide kernel)
SUPPORTED = sorted(CASES)


def to_dev(x, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def make_attn(name):
    c = CASES[name]
    a = Attention(c["n_head"], c["n_kv"], c["hd"], c["n_ctx"], 1,
                  janas_amd.FLOAT)
    if c["kv"] == KV_I16:
        a.set_kv16(True)
    if c.get("window"):
        a.set_window(c["window"])
    if c.get("ring"):
        a.set_ring(True)
    if c.get("scale") is not None:
        a.set_scale(c["scale"])
    return a


def run_dropin(name, inp, device=None):
    """janas_attn_run in calls of at most 64 tokens, as the engine makes
    them (model_attn.c:284-294); host arrays, or device tensors."""
    c = CASES[name]
    n, pos0 = c["n"], c["pos0"]
    q, k, v, ks, vs, last = (inp[x] for x in ("q", "k", "v", "ks", "vs",
                                              "last"))
    out = np.zeros_like(q)
    if device is not None:
        q, k, v, ks, vs = (to_dev(x, device) for x in (q, k, v, ks, vs))
        outd = torch.zeros(out.shape, dtype=torch.float32, device=device)
    with make_attn(name) as a:
        for s in range(0, n, MAX_BLOCK):
            m = min(MAX_BLOCK, n - s)
            if last is not None:
                a.set_last(np.ascontiguousarray(last[s:s + m]))
            if device is None:
                o = np.zeros((m,) + q.shape[1:], np.float32)
                a.run(np.ascontiguousarray(q[s:s + m]), k, ks, v, vs, m,
                      pos0 + s, o)
                out[s:s + m] = o
            else:
                a.run(q[s:s + m], k, ks, v, vs, m, pos0 + s, outd[s:s + m])
    if device is not None:
        out = outd.cpu().numpy()
    return out


@pytest.mark.parametrize("name", SUPPORTED)
def test_dropin_host_matches_reference(name, gpu):
    inp = make_inputs(name)
    ref = np.load(f"tests/golden/{name}.npz")["out"]
    out = run_dropin(name, inp)
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
    err = abs_err(out, ref)
    print(f"{name}: |gpu - reference| = {err:.2e} (bar {bar:.1e})")
    assert within(err, bar, "vs oracle")


@pytest.mark.parametrize("name", SUPPORTED)
def test_dropin_device_matches_closed_form(name, gpu):
    inp = make_inputs(name)
    ex = orc.exact(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                   last=inp["last"], **call_kwargs(name))
    out = run_dropin(name, inp, device=gpu)
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ex).max()))
    err = abs_err(out, ex)
    print(f"{name}: |gpu - exact| = {err:.2e} (bar {bar:.1e})")
    assert within(err, bar, "vs oracle")


@pytest.mark.parametrize("name", ["i8_8x1x128_p250_n17", "i8_4x2x64_p0_n64",
                                  "i16_4x1x64_p1030_n5_w64_ring",
                                  "i8_4x1x64_p600_n8_w300",
                                  "i16_2x1x512_p100_n3"])
def test_dropin_block_equals_tokens(name, gpu):
    """A token's result does not depend on the block it runs in."""
    c = CASES[name]
    inp = make_inputs(name)
    q, k, v, ks, vs = (to_dev(inp[x], gpu) for x in ("q", "k", "v", "ks", "vs"))
    n, pos0 = c["n"], c["pos0"]
    blk = torch.zeros(q.shape, dtype=torch.float32, device=gpu)
    one = torch.zeros(q.shape, dtype=torch.float32, device=gpu)
    with make_attn(name) as a:
        a.run(q, k, ks, v, vs, n, pos0, blk)
        for j in range(n):
            a.run(q[j:j + 1], k, ks, v, vs, 1, pos0 + j, one[j:j + 1])
    assert torch.equal(blk.view(torch.int32), one.view(torch.int32))


def seq_dev(cfg, s, gpu):
    d = dict(k=to_dev(s["k"], gpu), v=to_dev(s["v"], gpu),
             q=to_dev(np.ascontiguousarray(s["q"], np.float32), gpu),
             cap=s["k"].shape[1], n=s["n"], pos0=s["pos0"])
    d["out"] = torch.zeros(d["q"].shape, dtype=torch.float32, device=gpu)
    if cfg.get("gate") is not None:
        d["gate"] = to_dev(cfg["gate"], gpu)
    return d


def run_cfg(cfg, gpu, path="split"):
    seqs = [seq_dev(cfg, s, gpu) for s in cfg["seqs"]]
    cap = max(s["cap"] for s in seqs)
    with Attention(cfg["n_head"], cfg["n_kv"], cfg["hd"], cap) as a:
        if cfg["scale"] is not None:
            a.set_scale(float(cfg["scale"]))
        gate = janas_amd.GATE_ELEM if cfg.get("gate") is not None else 0
        a.run_dev(cfg["kv"], seqs, gate_mode=gate, path=path)
        torch.cuda.synchronize()
    return [s["out"].cpu().numpy() for s in seqs]


def test_config1_f32_decode(gpu):
    cfg = config(1)
    (out,) = run_cfg(cfg, gpu)
    ref = oracle_out(orc, cfg, cfg["seqs"][0])
    err = rel_err(out, ref)
    print(f"config 1: max rel err {err:.2e}")
    assert within(err, TOL_F32_REL, "vs oracle")


def test_config3_ragged_decode(gpu):
    cfg = config(3)
    outs = run_cfg(cfg, gpu)
    worst = 0.0
    for s, out in zip(cfg["seqs"], outs):
        worst = max(worst, abs_err(out, oracle_out(orc, cfg, s)))
    print(f"config 3: lens {[s['pos0'] + 1 for s in cfg['seqs']]}, "
          f"max abs err {worst:.2e}")
    assert within(worst, TOL_F16_ABS, "worst vs oracle")


def test_config4_gated_long_decode(gpu):
    cfg = config(4)
    (out,) = run_cfg(cfg, gpu)
    ref = oracle_out(orc, cfg, cfg["seqs"][0])
    err = abs_err(out, ref)
    print(f"config 4: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


def test_config5_verify(gpu):
    cfg = config(5)
    (out,) = run_cfg(cfg, gpu)
    ref = oracle_out(orc, cfg, cfg["seqs"][0])
    err = abs_err(out, ref)
    print(f"config 5 verify: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "vs oracle")


def test_config5_verify_equals_tokens(gpu):
    """8 drafts in one call equal 8 one-token calls bit for bit."""
    cfg = config(5)
    s = cfg["seqs"][0]
    d = seq_dev(cfg, s, gpu)
    with Attention(cfg["n_head"], cfg["n_kv"], cfg["hd"], d["cap"]) as a:
        a.run_dev(KV_F16, [d], path="split")
        one = torch.zeros_like(d["out"])
        for j in range(s["n"]):
            dj = dict(d, q=d["q"][j:j + 1], out=one[j:j + 1], n=1,
                      pos0=s["pos0"] + j)
            a.run_dev(KV_F16, [dj], path="split")
        torch.cuda.synchronize()
    assert torch.equal(d["out"].view(torch.int32), one.view(torch.int32))


def test_f32_cache_equals_int8_unit_scales(gpu):
    """An f32 cache holding the int8 numbers with unit scales gives the
    reference's int8 result (both within the FLOAT bar of it)."""
    name = "i8unit_8x2x128_p300_n4"
    c = CASES[name]
    inp = make_inputs(name)
    ref = np.load(f"tests/golden/{name}.npz")["out"]
    for kv, dt in ((KV_F32, np.float32), (KV_F16, np.float16)):
        cfg = dict(n_head=c["n_head"], n_kv=c["n_kv"], hd=c["hd"], kv=kv,
                   scale=None, gate=None,
                   seqs=[dict(k=inp["k"].astype(dt), v=inp["v"].astype(dt),
                              q=inp["q"], pos0=c["pos0"], n=c["n"])])
        (out,) = run_cfg(cfg, gpu)
        err = abs_err(out, ref)
        print(f"kv {kv}: |gpu - reference int8| = {err:.2e}")
        assert within(err, TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max())), "vs oracle")


@pytest.mark.parametrize("hd", [72, 200])
def test_int8_rows_of_8_mod_16_bytes(hd, gpu):
    """int8 rows whose length is 8 mod 16 bytes: the last 16-byte unit of a
    row is read 8 bytes early (never past the buffer at the cache's last
    row) and its halves put back; decode at the cache's last position."""
    from cases import uniform
    h, kvh, cap = 8, 2, 777
    cells, rows = kvh * cap * hd, kvh * cap
    k = uniform(7001 + hd, cells, -127, 127).astype(np.int32).astype(np.int8)
    v = uniform(7002 + hd, cells, -127, 127).astype(np.int32).astype(np.int8)
    ks = uniform(7003 + hd, rows, 0.001, 0.02).reshape(kvh, cap)
    vs = uniform(7004 + hd, rows, 0.001, 0.02).reshape(kvh, cap)
    q = uniform(7005 + hd, 2 * h * hd, -3, 3).reshape(2, h, hd)
    k, v = k.reshape(kvh, cap, hd), v.reshape(kvh, cap, hd)
    ref = orc.run(q, k, v, ks, vs, n_head=h, n_kv=kvh, hd=hd, pos0=cap - 2,
                  kv=KV_I8, threads=4)
    d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), ks=to_dev(ks, gpu),
             vs=to_dev(vs, gpu), q=to_dev(q, gpu), cap=cap, n=2, pos0=cap - 2)
    d["out"] = torch.zeros(d["q"].shape, dtype=torch.float32, device=gpu)
    with Attention(h, kvh, hd, cap) as a:
        a.run_dev(KV_I8, [d], path="split")
        torch.cuda.synchronize()
    err = abs_err(d["out"].cpu().numpy(), ref)
    print(f"int8 hd {hd}: max abs err {err:.2e}")
    assert within(err, TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max())), "vs oracle")


def block_case(kv, n_kv=8, h=32, hd=128, L=4096, n=64, seed=8100):
    """A 64-token block at the cache's end over 8 KV heads and 16 chunks:
    16 row tiles read each chunk (plain loads, kept in L2) and the merge
    takes 128 columns a workgroup."""
    from cases import uniform
    cells, rows = n_kv * L * hd, n_kv * L
    if kv == KV_F16:
        k = normal_cache(seed + 1, cells).astype(np.float16)
        v = normal_cache(seed + 2, cells).astype(np.float16)
        ks = vs = None
    else:
        lim = 127 if kv == KV_I8 else 32767
        dt = np.int8 if kv == KV_I8 else np.int16
        k = uniform(seed + 1, cells, -lim, lim).astype(np.int32).astype(dt)
        v = uniform(seed + 2, cells, -lim, lim).astype(np.int32).astype(dt)
        div = np.float32(1.0 if kv == KV_I8 else 258.0)
        ks = (uniform(seed + 3, rows, 0.001, 0.02) / div).reshape(n_kv, L)
        vs = (uniform(seed + 4, rows, 0.001, 0.02) / div).reshape(n_kv, L)
    q = uniform(seed + 5, n * h * hd, -3, 3).reshape(n, h, hd)
    return dict(k=k.reshape(n_kv, L, hd), v=v.reshape(n_kv, L, hd), ks=ks,
                vs=vs, q=q, n_kv=n_kv, h=h, hd=hd, L=L, n=n)


def normal_cache(seed, count):
    from cases import normal
    return normal(seed, count)


def run_block(c, kv, gpu, pos0, window=0, last=None, per_token=False,
              scores=janas_amd.FLOAT):
    d = dict(k=to_dev(c["k"], gpu), v=to_dev(c["v"], gpu),
             q=to_dev(c["q"], gpu), cap=c["L"], n=c["n"], pos0=pos0)
    if c["ks"] is not None:
        d["ks"], d["vs"] = to_dev(c["ks"], gpu), to_dev(c["vs"], gpu)
    d["out"] = torch.zeros(d["q"].shape, dtype=torch.float32, device=gpu)
    with Attention(c["h"], c["n_kv"], c["hd"], c["L"], 1, scores) as a:
        if window:
            a.set_window(window)
        if not per_token:
            if last is not None:
                d["last"] = to_dev(last, gpu)
                d["last_max"] = int(last.max())
            a.run_dev(kv, [d], path="split")
        else:
            for j in range(c["n"]):
                dj = dict(d, q=d["q"][j:j + 1], out=d["out"][j:j + 1], n=1,
                          pos0=pos0 + j)
                if last is not None:
                    dj["last"] = to_dev(last[j:j + 1], gpu)
                    dj["last_max"] = int(last[j])
                a.run_dev(kv, [dj], path="split")
        torch.cuda.synchronize()
    return d["out"].cpu().numpy()


@pytest.mark.parametrize("kv", [KV_F16, KV_I8, KV_I16])
def test_large_block_equals_tokens(kv, gpu):
    """A 64-token block over a 4096-position cache equals 64 one-token calls
    bit for bit (their chunks are loaded nontemporally, the block's are
    not), and the restatement within the bar."""
    c = block_case(kv)
    pos0 = c["L"] - c["n"]
    blk = run_block(c, kv, gpu, pos0)
    one = run_block(c, kv, gpu, pos0, per_token=True)
    assert np.array_equal(blk.view(np.int32), one.view(np.int32))
    ref = orc.run(c["q"], c["k"], c["v"], c["ks"], c["vs"], n_head=c["h"],
                  n_kv=c["n_kv"], hd=c["hd"], pos0=pos0, kv=kv, threads=16)
    err = abs_err(blk, ref)
    bar = TOL_F16_ABS if kv == KV_F16 else TOL_FLOAT_ABS * max(
        1.0, float(np.abs(ref).max()))
    print(f"kv {kv}: large block max abs err {err:.2e} (bar {bar:.1e})")
    assert within(err, bar, "vs oracle")


@pytest.mark.parametrize("L,pos0", [(4160, 4088), (16448, 16376)])
def test_block_across_merge_batch_sizes_equals_tokens(L, pos0, gpu):
    """The merge loads a group's chunks in batches of 2, 8 or 16 by the
    launch's longest span (up to 16, 64 chunks). A block at positions
    4088..4103 spans 17 chunks (batches of 8) while its first tokens alone
    span 16 (batches of 2); one at 16376..16391 spans 65 (16) against 64
    (8). Chunks past a row's range enter with weight 0, so the block
    equals its tokens bit for bit all the same."""
    c = block_case(KV_F16, L=L, n=16, seed=8700 + L)
    blk = run_block(c, KV_F16, gpu, pos0)
    one = run_block(c, KV_F16, gpu, pos0, per_token=True)
    assert np.array_equal(blk.view(np.int32), one.view(np.int32))
    ref = orc.run(c["q"], c["k"], c["v"], None, None, n_head=c["h"],
                  n_kv=c["n_kv"], hd=c["hd"], pos0=pos0, kv=KV_F16, threads=16)
    err = abs_err(blk, ref)
    print(f"block at {pos0}: max abs err {err:.2e}")
    assert within(err, TOL_F16_ABS, "block vs oracle")


# (cache, heads, KV heads, head size, tokens, scores): a KV head's rows fill
# two 8-row tiles only in part (15, 12, 9 and 16 rows), so one workgroup
# takes both, while a token alone (at most 8 rows) takes one tile a
# workgroup
TWO_TILES = [(KV_F16, 6, 2, 64, 5, janas_amd.FLOAT),
             (KV_F16, 4, 4, 128, 12, janas_amd.FLOAT),
             (KV_I8, 12, 4, 128, 3, janas_amd.FLOAT),
             (KV_I16, 16, 2, 64, 2, janas_amd.FLOAT),
             (KV_I8, 6, 2, 128, 5, janas_amd.INT16),
             (KV_I8, 8, 1, 64, 2, janas_amd.INT16)]


@pytest.mark.parametrize("kv,h,n_kv,hd,n,scores", TWO_TILES)
def test_two_tile_workgroups_equal_tokens(kv, h, n_kv, hd, n, scores, gpu):
    """Blocks whose rows take the two-tile workgroups, the second tile only
    partly filled, equal their tokens run one at a time (one-tile
    workgroups) bit for bit; FLOAT blocks against the restatement too."""
    c = block_case(kv, n_kv=n_kv, h=h, hd=hd, L=1000, n=n, seed=8400 + h + hd + n)
    pos0 = c["L"] - n
    blk = run_block(c, kv, gpu, pos0, scores=scores)
    one = run_block(c, kv, gpu, pos0, per_token=True, scores=scores)
    assert np.array_equal(blk.view(np.int32), one.view(np.int32))
    ref = orc.run(c["q"], c["k"], c["v"], c["ks"], c["vs"], n_head=h,
                  n_kv=n_kv, hd=hd, pos0=pos0, kv=kv, threads=16,
                  int16=scores == janas_amd.INT16)
    err = abs_err(blk, ref)
    bar = TOL_F16_ABS if kv == KV_F16 else TOL_FLOAT_ABS * max(
        1.0, float(np.abs(ref).max()))
    print(f"two tiles kv {kv} {h}/{n_kv}/{hd} n {n} scores {scores}: max abs err {err:.2e}")
    assert within(err, bar, "two-tile block vs oracle")


def test_large_block_window_and_last(gpu):
    """Row tiles of the block see different chunks: a window of 700 and a
    span that sees past itself."""
    c = block_case(KV_I8, seed=8200)
    pos0 = c["L"] - c["n"] - 500
    p = pos0 + np.arange(c["n"])
    last = np.where((p >= pos0 + 10) & (p < pos0 + 30), pos0 + 29, p).astype(
        np.uint32)
    blk = run_block(c, KV_I8, gpu, pos0, window=700, last=last)
    one = run_block(c, KV_I8, gpu, pos0, window=700, last=last, per_token=True)
    assert np.array_equal(blk.view(np.int32), one.view(np.int32))
    ref = orc.run(c["q"], c["k"], c["v"], c["ks"], c["vs"], n_head=c["h"],
                  n_kv=c["n_kv"], hd=c["hd"], pos0=pos0, kv=KV_I8, window=700,
                  last=last, threads=16)
    err = abs_err(blk, ref)
    print(f"large block, window + last: max abs err {err:.2e}")
    assert within(err, TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max())), "vs oracle")


def test_large_block_ragged_sequences(gpu):
    """Three sequences in one launch (64, 37 and 1 tokens): each equals its
    own one-token calls bit for bit."""
    cs = [block_case(KV_F16, seed=8300 + i) for i in range(3)]
    ns, pos = [64, 37, 1], [4032, 3000, 4095]
    seqs = []
    for c, n, p0 in zip(cs, ns, pos):
        d = dict(k=to_dev(c["k"], gpu), v=to_dev(c["v"], gpu),
                 q=to_dev(c["q"][:n], gpu), cap=c["L"], n=n, pos0=p0)
        d["out"] = torch.zeros(d["q"].shape, dtype=torch.float32, device=gpu)
        seqs.append(d)
    with Attention(32, 8, 128, 4096) as a:
        a.run_dev(KV_F16, seqs, path="split")
        torch.cuda.synchronize()
        for d, n, p0 in zip(seqs, ns, pos):
            one = torch.zeros_like(d["out"])
            for j in range(n):
                a.run_dev(KV_F16, [dict(d, q=d["q"][j:j + 1], out=one[j:j + 1],
                                        n=1, pos0=p0 + j)], path="split")
            torch.cuda.synchronize()
            assert torch.equal(d["out"].view(torch.int32), one.view(torch.int32))
