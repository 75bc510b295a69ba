"""Head sizes above 256 (Gemma 4's 512) on the GPU: the wide split kernel
against the CPU restatement, at the reference's sixteen-bit test shapes
(test_attention.c:253-338: int16 keys and values, windows 0, 256 and 1024,
score scale 0.02, hd 512), with int8 and f16 caches, a head size that is not
a whole tile (384), spans that see past themselves, a ring, and the block
versus token-by-token bit identity.
"""
import numpy as np
import pytest
import torch

import janas_amd
from attn_helpers import (KV_F16, KV_I8, KV_I16, TOL_F16_ABS, TOL_FLOAT_ABS,
                          abs_err, threads, within)
from cases import normal, uniform
from janas_amd import Attention
from oracle import orc

pytestmark = pytest.mark.gpu


def to_dev(x, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def wide_inputs(kv, n_head, n_kv, hd, cap, n, seed):
    """The reference test's distributions (test_attention.c:270-279) for
    int8 / int16; N(0, 1) for f16."""
    cells, rows = n_kv * cap * hd, n_kv * cap
    if kv == KV_I16:
        k = uniform(seed + 1, cells, -32767, 32767).astype(np.int32).astype(np.int16)
        v = uniform(seed + 2, cells, -32767, 32767).astype(np.int32).astype(np.int16)
        ks = uniform(seed + 3, rows, 0.001, 0.02) / np.float32(258.0)
        vs = uniform(seed + 4, rows, 0.001, 0.02) / np.float32(258.0)
    elif kv == KV_I8:
        k = uniform(seed + 1, cells, -127, 127).astype(np.int32).astype(np.int8)
        v = uniform(seed + 2, cells, -127, 127).astype(np.int32).astype(np.int8)
        ks = uniform(seed + 3, rows, 0.001, 0.02)
        vs = uniform(seed + 4, rows, 0.001, 0.02)
    else:
        k = normal(seed + 1, cells).astype(np.float16)
        v = normal(seed + 2, cells).astype(np.float16)
        ks = vs = None
    if kv == KV_F16:
        q = normal(seed + 5, n * n_head * hd)
    else:
        q = uniform(seed + 5, n * n_head * hd, -3, 3)
    shape = (n_kv, cap, hd)
    return dict(q=q.reshape(n, n_head, hd).astype(np.float32),
                k=k.reshape(shape), v=v.reshape(shape),
                ks=None if ks is None else ks.reshape(n_kv, cap).astype(np.float32),
                vs=None if vs is None else vs.reshape(n_kv, cap).astype(np.float32))


def run_wide(inp, kv, n_head, n_kv, hd, cap, pos0, gpu, scale=None, window=0,
             ring=False, last=None, path="split"):
    q = to_dev(inp["q"], gpu)
    d = dict(k=to_dev(inp["k"], gpu), v=to_dev(inp["v"], gpu), q=q,
             out=torch.zeros(q.shape, dtype=torch.float32, device=gpu),
             cap=cap, n=q.shape[0], pos0=pos0)
    if inp["ks"] is not None:
        d["ks"] = to_dev(inp["ks"], gpu)
        d["vs"] = to_dev(inp["vs"], gpu)
    if last is not None:
        d["last"] = to_dev(np.ascontiguousarray(last, np.uint32), gpu)
        d["last_max"] = int(last.max())
    with Attention(n_head, n_kv, hd, cap) as a:
        if scale is not None:
            a.set_scale(scale)
        if window:
            a.set_window(window)
        if ring:
            a.set_ring(True)
        a.run_dev(kv, [d], path=path)
        torch.cuda.synchronize()
    return d["out"].cpu().numpy()


def oracle(inp, kv, n_head, n_kv, hd, pos0, scale=None, window=0, ring=False,
           last=None):
    return orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                   n_head=n_head, n_kv=n_kv, hd=hd, pos0=pos0, kv=kv,
                   scale=scale, window=window, ring=ring, last=last,
                   threads=threads(), block=64)


def bar(kv, ref):
    if kv == KV_F16:
        return TOL_F16_ABS
    return TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))


@pytest.mark.parametrize("window", [0, 256, 1024])
@pytest.mark.parametrize("n", [1, 8])
def test_gemma4_int16_hd512(window, n, gpu):
    """int16 K/V, 16 query heads over 2 KV heads (groups of 8), score scale
    0.02, 3000 positions: decode and an 8-token block."""
    h, kvh, hd, cap = 16, 2, 512, 3000
    pos0 = cap - n
    inp = wide_inputs(KV_I16, h, kvh, hd, cap, n, seed=4000 + window + n)
    out = run_wide(inp, KV_I16, h, kvh, hd, cap, pos0, gpu, scale=0.02,
                   window=window)
    ref = oracle(inp, KV_I16, h, kvh, hd, pos0, scale=0.02, window=window)
    err = abs_err(out, ref)
    print(f"int16 hd 512 window {window} n {n}: max abs err {err:.2e} "
          f"(bar {bar(KV_I16, ref):.1e})")
    assert within(err, bar(KV_I16, ref), "vs oracle")


@pytest.mark.parametrize("kv", [KV_I8, KV_F16])
@pytest.mark.parametrize("hd", [512, 384, 264])
def test_wide_other_types_and_sizes(kv, hd, gpu):
    """int8 and f16 caches; 384 and 264 leave the last column tiles
    partly or wholly outside the row."""
    h, kvh, cap, n = 8, 2, 1300, 3
    pos0 = cap - n
    inp = wide_inputs(kv, h, kvh, hd, cap, n, seed=5000 + hd + kv)
    out = run_wide(inp, kv, h, kvh, hd, cap, pos0, gpu)
    ref = oracle(inp, kv, h, kvh, hd, pos0)
    err = abs_err(out, ref)
    print(f"kv {kv} hd {hd}: max abs err {err:.2e} (bar {bar(kv, ref):.1e})")
    assert within(err, bar(kv, ref), "vs oracle")


def test_wide_sees_past_itself(gpu):
    """set_last: tokens 0..5 of a 12-token block see up to the block's
    sixth position, across a chunk boundary (test_attention.c:358)."""
    h, kvh, hd, cap, n = 8, 1, 512, 700, 12
    pos0 = 250
    inp = wide_inputs(KV_I16, h, kvh, hd, cap, n, seed=6100)
    p = pos0 + np.arange(n)
    last = np.where(p < pos0 + 6, pos0 + 5, p).astype(np.uint32)
    out = run_wide(inp, KV_I16, h, kvh, hd, cap, pos0, gpu, scale=0.02,
                   last=last)
    ref = oracle(inp, KV_I16, h, kvh, hd, pos0, scale=0.02, last=last)
    err = abs_err(out, ref)
    print(f"last: max abs err {err:.2e}")
    assert within(err, bar(KV_I16, ref), "vs oracle")


def test_wide_ring(gpu):
    """A ring of 1024 positions holding a window of 300 at position 5000."""
    h, kvh, hd, n, window = 4, 1, 512, 5, 300
    cap = janas_amd.ring_positions(window, 64)
    pos0 = 5000
    inp = wide_inputs(KV_I16, h, kvh, hd, cap, n, seed=6200)
    out = run_wide(inp, KV_I16, h, kvh, hd, cap, pos0, gpu, scale=0.02,
                   window=window, ring=True)
    ref = oracle(inp, KV_I16, h, kvh, hd, pos0, scale=0.02, window=window,
                 ring=True)
    err = abs_err(out, ref)
    print(f"ring cap {cap}: max abs err {err:.2e}")
    assert within(err, bar(KV_I16, ref), "vs oracle")


@pytest.mark.parametrize("kv", [KV_I16, KV_I8])
def test_wide_block_equals_tokens(kv, gpu):
    """A token's result does not depend on the block it runs in."""
    h, kvh, hd, cap, n = 8, 2, 512, 900, 10
    pos0 = cap - n
    inp = wide_inputs(kv, h, kvh, hd, cap, n, seed=6300 + kv)
    blk = run_wide(inp, kv, h, kvh, hd, cap, pos0, gpu, window=400)
    for j in range(n):
        one = dict(inp, q=inp["q"][j:j + 1])
        o = run_wide(one, kv, h, kvh, hd, cap, pos0 + j, gpu, window=400)
        assert np.array_equal(o.view(np.int32), blk[j:j + 1].view(np.int32)), j


def test_wide_dropin_host(gpu):
    """janas_attn_run (host arrays, int16 cache) at hd 512, two calls of a
    64-token engine block and a decode."""
    h, kvh, hd, cap = 8, 1, 512, 400
    inp = wide_inputs(KV_I16, h, kvh, hd, cap, 130, seed=6400)
    ref = oracle(inp, KV_I16, h, kvh, hd, 270, scale=0.02)
    out = np.zeros_like(inp["q"])
    with Attention(h, kvh, hd, cap, 1, janas_amd.FLOAT) as a:
        a.set_kv16(True)
        a.set_scale(0.02)
        for s in range(0, 130, 64):
            m = min(64, 130 - s)
            o = np.zeros((m, h, hd), np.float32)
            a.run(np.ascontiguousarray(inp["q"][s:s + m]), inp["k"], inp["ks"],
                  inp["v"], inp["vs"], m, 270 + s, o)
            out[s:s + m] = o
    err = abs_err(out, ref)
    print(f"drop-in hd 512: max abs err {err:.2e}")
    assert within(err, bar(KV_I16, ref), "vs oracle")


@pytest.mark.parametrize("hd", [520, 100])
def test_head_dim_refused(hd, gpu):
    """attention.c:998-1000: head_dim above 512 or not a multiple of 8."""
    with pytest.raises(ValueError):
        Attention(8, 2, hd, 1000)
