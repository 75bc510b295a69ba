"""The reference's INT16 scores way on the GPU (int8 caches, head size a
multiple of 16): the quantized query, exact integer scores, weights
quantized per (chunk, token, head) and exact integer value sums
(attention.c:158-193, :820-839, attention_scores.h).

* janas_attn_create resolves the asked way as the reference's scores_choice
  does (attention.c:960-982), set_kv16 takes INT16 back to FLOAT
  (:1061-1066), and janas_attn_scores_mode reports it;
* the drop-in's outputs against the reference's own INT16 outputs (golden
  fixtures from its compiled attention) at the FLOAT bar - the scores,
  weights and chunk sums are the reference's bit for bit, so only the
  merge's float rounding differs - and against the double-precision
  closed form at the reference's INT16 bar (test_attention.c:143-148);
* a block equals its tokens one by one, bit for bit;
* config 4's geometry at 32k positions, the wide kernel's head sizes,
  windows, rings and last[], against the restatement's INT16 way;
* AUTO: resolved at create as scores_choice does, then per call by the
  positions measured on the device at the first call (attn_calibrate,
  attention.c:1183-1262): a call's output is the chosen way's, bit for bit.
"""
import numpy as np
import pytest
import torch

import janas_amd
from attn_helpers import TOL_FLOAT_ABS, abs_err, threads, within
from cases import CASES, call_kwargs, int16_case, make_inputs, normal, splitmix
from janas_amd import Attention
from oracle import orc

pytestmark = pytest.mark.gpu

MAX_BLOCK = janas_amd.MAX_BLOCK
INT16_CASES = sorted(n for n in CASES if int16_case(n))
# the reference's bar for its INT16 way against the closed form, absolute on
# outputs of order one (test_attention.c:143-148)
TOL_INT16_EXACT = 1e-3


def to_dev(x, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def make_attn(name, scores=janas_amd.INT16):
    c = CASES[name]
    a = Attention(c["n_head"], c["n_kv"], c["hd"], c["n_ctx"], 1, scores)
    if c.get("window"):
        a.set_window(c["window"])
    if c.get("ring"):
        a.set_ring(True)
    if c.get("scale") is not None:
        a.set_scale(c["scale"])
    return a


def run_dropin(name, inp, device=None):
    """janas_attn_run under INT16 in calls of at most 64 tokens, as the
    engine makes them; host arrays, or device tensors."""
    c = CASES[name]
    n, pos0 = c["n"], c["pos0"]
    q, k, v, ks, vs, last = (inp[x] for x in ("q", "k", "v", "ks", "vs",
                                              "last"))
    out = np.zeros_like(q)
    if device is not None:
        q, k, v, ks, vs = (to_dev(x, device) for x in (q, k, v, ks, vs))
        outd = torch.zeros(out.shape, dtype=torch.float32, device=device)
    with make_attn(name) as a:
        assert a.scores_mode() == janas_amd.INT16
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
        assert a.status() == 0
    if device is not None:
        out = outd.cpu().numpy()
    return out


def test_scores_mode_resolution(gpu, monkeypatch):
    """scores_choice (attention.c:960-982): FLOAT and INT16 as asked, AUTO
    INT16 past 16384 positions, FLOAT for head sizes not a multiple of 16;
    the environment variable first; set_kv16 (attention.c:1061-1066)."""
    monkeypatch.delenv("JANAS_ATTN", raising=False)
    F, I, A = janas_amd.FLOAT, janas_amd.INT16, janas_amd.AUTO
    # (asked, head_dim, n_ctx) -> (scores_mode, scores_auto); an unknown
    # value takes AUTO's rule without being AUTO, as in the reference
    want = [((F, 128, 1024), (F, 0)), ((I, 128, 1024), (I, 0)),
            ((A, 128, 16384), (F, 1)), ((A, 128, 16385), (I, 1)),
            ((I, 40, 1024), (F, 0)), ((A, 40, 32768), (F, 1)),
            ((I, 512, 1024), (I, 0)), ((7, 128, 32768), (I, 0))]
    for (scores, hd, n_ctx), got in want:
        with Attention(4, 2, hd, n_ctx, 1, scores) as a:
            assert (a.scores_mode(), a.scores_auto()) == got, (scores, hd, n_ctx)
    with Attention(4, 2, 128, 1024, 1, I) as a:
        a.set_kv16(True)
        assert a.scores_mode() == F
        a.set_kv16(False)
        assert a.scores_mode() == F   # as the reference: it stays FLOAT
    monkeypatch.setenv("JANAS_ATTN", "int16")
    with Attention(4, 2, 128, 1024, 1, F) as a:
        assert (a.scores_mode(), a.scores_auto()) == (I, 0)
    monkeypatch.setenv("JANAS_ATTN", "auto")
    with Attention(4, 2, 128, 32768, 1, F) as a:
        assert (a.scores_mode(), a.scores_auto()) == (I, 1)
    monkeypatch.setenv("JANAS_ATTN", "float")
    with Attention(4, 2, 128, 32768, 1, I) as a:
        assert (a.scores_mode(), a.scores_auto()) == (F, 0)


@pytest.mark.parametrize("name", INT16_CASES)
def test_int16_dropin_matches_reference(name, gpu):
    """Host pointers: the reference's own INT16 outputs within the FLOAT
    bar, the closed form within the reference's INT16 bar."""
    inp = make_inputs(name)
    ref = np.load(f"tests/golden/{name}.npz")["out_int16"]
    out = run_dropin(name, inp)
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
    assert within(abs_err(out, ref), bar, f"{name} int16 vs reference int16")
    ex = orc.exact(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                   last=inp["last"], **call_kwargs(name))
    bar = TOL_INT16_EXACT * max(1.0, float(np.abs(ex).max()))
    assert within(abs_err(out, ex), bar, f"{name} int16 vs closed form")


@pytest.mark.parametrize("name", ["i8_8x1x128_p250_n17", "i8_4x2x64_p0_n64",
                                  "i8_4x1x64_p600_n8_w300",
                                  "i8_16x2x256_p254_n5", "i8_2x1x512_p300_n3"])
def test_int16_dropin_device_block_equals_tokens(name, gpu):
    """Device pointers; a block equals its tokens one by one, bit for bit,
    and the reference's INT16 outputs within the FLOAT bar."""
    c = CASES[name]
    inp = make_inputs(name)
    ref = np.load(f"tests/golden/{name}.npz")["out_int16"]
    out = run_dropin(name, inp, device=gpu)
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
    assert within(abs_err(out, ref), bar, f"{name} int16 device")
    q, k, v, ks, vs = (to_dev(inp[x], gpu) for x in ("q", "k", "v", "ks", "vs"))
    n, pos0 = c["n"], c["pos0"]
    blk = torch.zeros(q.shape, dtype=torch.float32, device=gpu)
    one = torch.zeros(q.shape, dtype=torch.float32, device=gpu)
    with make_attn(name) as a:
        for s in range(0, n, MAX_BLOCK):
            m = min(MAX_BLOCK, n - s)
            a.run(q[s:s + m], k, ks, v, vs, m, pos0 + s, blk[s:s + m])
        for j in range(n):
            a.run(q[j:j + 1], k, ks, v, vs, 1, pos0 + j, one[j:j + 1])
    assert torch.equal(blk.view(torch.int32), one.view(torch.int32))


def int8_cache(seed, n_kv, cap, hd):
    """Rows of N(0, 1) numbers quantized as the engine writes them (the
    largest magnitude of a row to 127, model_attn.c:126-145)."""
    x = normal(seed, n_kv * cap * hd).reshape(n_kv, cap, hd)
    mx = np.abs(x).max(axis=2, keepdims=True)
    return (np.rint(x * (127.0 / mx)).astype(np.int8),
            (mx[..., 0] / 127.0).astype(np.float32))


def test_int16_config4_geometry_at_32k(gpu):
    """16/2/256 over 32768 int8 positions under INT16: one decode token and
    a 5-token block against the restatement's INT16 way."""
    h, kvh, hd, L = 16, 2, 256, 32768
    k, ks = int8_cache(501, kvh, L, hd)
    v, vs = int8_cache(502, kvh, L, hd)
    q = normal(503, 5 * h * hd).reshape(5, h, hd)
    kd, vd, ksd, vsd = (to_dev(x, gpu) for x in (k, v, ks, vs))
    with Attention(h, kvh, hd, L, 1, janas_amd.INT16) as a:
        assert a.scores_mode() == janas_amd.INT16
        a.set_scale(1.0 / 16.0)
        for n in (1, 5):
            pos0 = L - n
            qd = to_dev(q[:n], gpu)
            out = torch.zeros(qd.shape, dtype=torch.float32, device=gpu)
            a.run(qd, kd, ksd, vd, vsd, n, pos0, out)
            ref = orc.run(np.ascontiguousarray(q[:n]), k, v, ks, vs,
                          n_head=h, n_kv=kvh, hd=hd, pos0=pos0, kv=orc.KV_I8,
                          scale=np.float32(1.0 / 16.0), int16=True,
                          threads=threads())
            bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
            assert within(abs_err(out.cpu().numpy(), ref), bar,
                          f"32k n={n} int16")


def draw(i):
    """Case i's geometry, from the counter generator: head sizes of both
    kernels (the split kernel to 256, the wide one above), windows, rings,
    spans that see past themselves."""
    z = [int(x) for x in splitmix(9300 + i, 12)]
    hd = [16, 64, 96, 128, 192, 256, 320, 512][z[0] % 8]
    group = [1, 2, 3, 4, 8][z[1] % 5]
    n_kv = 1 + z[2] % 2
    n = 1 + z[3] % 64
    pos0 = z[4] % 2500
    window = 0 if z[5] % 2 else 64 + z[6] % 1200
    ring = window > 0 and z[7] % 3 == 0
    picture = z[8] % 4 == 0 and n > 4
    cap = (256 * ((window + n) // 256 + 3) if ring else pos0 + n + z[9] % 300)
    return dict(hd=hd, n_head=group * n_kv, n_kv=n_kv, n=n, pos0=pos0,
                window=window, ring=ring, picture=picture, cap=cap,
                seed=9400 + 10 * i)


@pytest.mark.parametrize("i", range(16))
def test_int16_random_geometries(i, gpu):
    g = draw(i)
    h, kvh, hd, cap, n, pos0 = (g[x] for x in ("n_head", "n_kv", "hd", "cap",
                                               "n", "pos0"))
    k, ks = int8_cache(g["seed"] + 1, kvh, cap, hd)
    v, vs = int8_cache(g["seed"] + 2, kvh, cap, hd)
    q = normal(g["seed"] + 3, n * h * hd).reshape(n, h, hd)
    last = None
    if g["picture"]:
        p = pos0 + np.arange(n)
        a0, a1 = pos0 + 1, pos0 + n // 2
        last = np.where((p >= a0) & (p < a1), a1 - 1, p).astype(np.uint32)
    print(f"case {i}: {g}", flush=True)
    out = np.zeros_like(q)
    with Attention(h, kvh, hd, cap, 1, janas_amd.INT16) as a:
        assert a.scores_mode() == janas_amd.INT16
        if g["window"]:
            a.set_window(g["window"])
        if g["ring"]:
            a.set_ring(True)
        if last is not None:
            a.set_last(last)
        a.run(q, k, ks, v, vs, n, pos0, out)
        assert a.status() == 0
    ref = orc.run(q, k, v, ks, vs, n_head=h, n_kv=kvh, hd=hd, pos0=pos0,
                  kv=orc.KV_I8, window=g["window"], ring=g["ring"], last=last,
                  int16=True, threads=threads())
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
    assert within(abs_err(out, ref), bar, f"random {i} int16")


def test_int16_run_dev_long_prompt_stays_split(gpu):
    """run_dev with an int8 cache under INT16: a 200-token prompt stays on
    the split-KV path (the INT16 way is its alone) - equal to
    run_dev_split bit for bit - and within the FLOAT bar of the
    restatement's INT16 way."""
    h, kvh, hd, cap, n = 8, 2, 128, 1200, 200
    k, ks = int8_cache(601, kvh, cap, hd)
    v, vs = int8_cache(602, kvh, cap, hd)
    q = normal(603, n * h * hd).reshape(n, h, hd)
    d = dict(k=to_dev(k, gpu), v=to_dev(v, gpu), ks=to_dev(ks, gpu),
             vs=to_dev(vs, gpu), q=to_dev(q, gpu), cap=cap, n=n, pos0=900)
    auto = torch.zeros(d["q"].shape, dtype=torch.float32, device=gpu)
    split = torch.zeros_like(auto)
    with Attention(h, kvh, hd, cap, 1, janas_amd.INT16) as a:
        a.run_dev(janas_amd.KV_I8, [dict(d, out=auto)])
        a.run_dev(janas_amd.KV_I8, [dict(d, out=split)], path="split")
        torch.cuda.synchronize()
    assert torch.equal(auto.view(torch.int32), split.view(torch.int32))
    ref = orc.run(q, k, v, ks, vs, n_head=h, n_kv=kvh, hd=hd, pos0=900,
                  kv=orc.KV_I8, int16=True, threads=threads())
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
    assert within(abs_err(auto.cpu().numpy(), ref), bar, "200-token int16")


def test_int16_noalloc_and_q8k(gpu):
    """The INT16 way through run_dev and run_dev_noalloc with the Q8_K
    output fused into the merge, two sequences a launch: outputs and blocks
    equal bit for bit, the blocks the restatement's quantization of the
    output, the output the restatement's INT16 way within the FLOAT bar."""
    h, kvh, hd, L = 16, 2, 256, 4096
    k, ks = int8_cache(701, kvh, L, hd)
    v, vs = int8_cache(702, kvh, L, hd)
    qs = [normal(703, 3 * h * hd).reshape(3, h, hd),
          normal(704, 1 * h * hd).reshape(1, h, hd)]
    pos = [L - 3, 1500]
    kd, vd, ksd, vsd = (to_dev(x, gpu) for x in (k, v, ks, vs))
    nb = h * hd // 256

    def seqs(outs, blocks):
        return [dict(k=kd, v=vd, ks=ksd, vs=vsd, q=to_dev(q, gpu), out=o,
                     out_q8k=b, cap=L, n=q.shape[0], pos0=p)
                for q, o, b, p in zip(qs, outs, blocks, pos)]

    res = []
    with Attention(h, kvh, hd, L, 1, janas_amd.INT16) as a:
        for path in ("auto", "noalloc"):
            outs = [torch.full((q.shape[0], h, hd), float("nan"), device=gpu)
                    for q in qs]
            blocks = [torch.zeros((q.shape[0], nb, janas_amd.attention.Q8K_BYTES),
                                  dtype=torch.uint8, device=gpu) for q in qs]
            a.run_dev(janas_amd.KV_I8, seqs(outs, blocks), path=path)
            torch.cuda.synchronize()
            res.append(([o.cpu().numpy() for o in outs],
                        [b.cpu().numpy() for b in blocks]))
        assert a.status() == 0
    (o1, b1), (o2, b2) = res
    for x, y in zip(o1, o2):
        assert np.array_equal(x.view(np.int32), y.view(np.int32))
    for x, y in zip(b1, b2):
        assert x.tobytes() == y.tobytes()
    for q, o, b, p in zip(qs, o1, b1, pos):
        n = q.shape[0]
        assert b.tobytes() == orc.q8k_quantize(o.reshape(n, h * hd)).tobytes()
        ref = orc.run(q, k, v, ks, vs, n_head=h, n_kv=kvh, hd=hd, pos0=p,
                      kv=orc.KV_I8, int16=True, threads=threads())
        bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ref).max()))
        assert within(abs_err(o, ref), bar, f"int16 noalloc q8k n={n}")


def test_auto_measured_way(gpu, monkeypatch):
    """AUTO over an int8 cache: INT16 at create past 16384 positions (the
    reference's scores_choice), then per call the way measured on the device
    at the first call - janas_attn_scores_mode reports it, and the output is
    that way's bit for bit, through the drop-in and through Part 2. The same
    instance geometry later reuses the measurement. Under set_kv16 AUTO
    stays FLOAT without measuring."""
    monkeypatch.delenv("JANAS_ATTN", raising=False)
    h, kvh, hd, L = 16, 2, 256, 20000
    k, ks = int8_cache(601, kvh, L, hd)
    v, vs = int8_cache(602, kvh, L, hd)
    q = normal(603, 4 * h * hd).reshape(4, h, hd)
    kd, vd, ksd, vsd, qd = (to_dev(x, gpu) for x in (k, v, ks, vs, q))
    for n, pos0 in ((1, L - 1), (4, 17000), (1, 1500)):
        outs = {}
        for scores in (janas_amd.AUTO, janas_amd.FLOAT, janas_amd.INT16):
            out = torch.zeros((n, h, hd), dtype=torch.float32, device=gpu)
            with Attention(h, kvh, hd, L, 1, scores) as a:
                if scores == janas_amd.AUTO:
                    assert a.scores_mode() == janas_amd.INT16
                a.run(qd[:n], kd, ksd, vd, vsd, n, pos0, out)
                torch.cuda.synchronize()
                outs[scores] = (a.scores_mode(), out.cpu().numpy())
        way, got = outs[janas_amd.AUTO]
        assert way in (janas_amd.FLOAT, janas_amd.INT16)
        print(f"n={n} pos0={pos0}: AUTO measured "
              f"{'INT16' if way == janas_amd.INT16 else 'FLOAT'}")
        assert np.array_equal(got.view(np.uint32), outs[way][1].view(np.uint32))
        # Part 2, one sequence on the split path: the same choice
        out = torch.zeros((n, h, hd), dtype=torch.float32, device=gpu)
        with Attention(h, kvh, hd, L, 1, janas_amd.AUTO) as a:
            a.run_dev(janas_amd.KV_I8, [dict(k=kd, v=vd, ks=ksd, vs=vsd,
                                              q=qd[:n], out=out, cap=L, n=n,
                                              pos0=pos0)])
            torch.cuda.synchronize()
            assert a.scores_mode() == way
        assert np.array_equal(out.cpu().numpy().view(np.uint32),
                              got.view(np.uint32))
    with Attention(h, kvh, 128, L, 1, janas_amd.AUTO) as a:
        a.set_kv16(True)
        assert a.scores_mode() == janas_amd.FLOAT


@pytest.mark.parametrize("n_ctx,n", [(32768, 2048), (20000, 512)])
def test_auto_long_prompt_first_call(gpu, monkeypatch, n_ctx, n):
    """A fresh AUTO instance over an int8 cache past 16384 positions (INT16
    at create, as the reference's scores_choice) whose first call is a long
    prompt through janas_attn_run_dev: the call measures the way first and
    follows the reference's block rule (INT16 only from from16[1], which
    the device never measures below FLOAT's time), so the prompt takes the
    exact prefill kernel, bit for bit the explicit prefill path's output,
    and the allocation-free entry point on a fresh instance (which never
    measures and computes FLOAT until measured) gives the same bits. The
    output is within the reference's FLOAT bar of the restatement."""
    monkeypatch.delenv("JANAS_ATTN", raising=False)
    h, kvh, hd = 32, 8, 128
    k, ks = int8_cache(611, kvh, n, hd)
    v, vs = int8_cache(612, kvh, n, hd)
    q = normal(613, n * h * hd).reshape(n, h, hd)
    kd, vd, ksd, vsd, qd = (to_dev(x, gpu) for x in (k, v, ks, vs, q))

    def call(path, scores=janas_amd.AUTO, prof=False):
        out = torch.full((n, h, hd), float("nan"), device=gpu)
        with Attention(h, kvh, hd, n_ctx, 1, scores) as a:
            assert scores != janas_amd.AUTO or a.scores_mode() == janas_amd.INT16
            a.prof_enable(prof)
            a.run_dev(janas_amd.KV_I8, [dict(k=kd, v=vd, ks=ksd, vs=vsd, q=qd,
                                              out=out, cap=n, n=n, pos0=0)],
                      path=path)
            torch.cuda.synchronize()
            p = a.prof_read() if prof else None
            assert a.status() == 0
        return out.cpu().numpy(), p

    first, prof = call("auto", prof=True)
    assert prof["prefill"][0] >= 1 and prof["split"][0] == 0, prof
    explicit, _ = call("prefill", janas_amd.FLOAT)
    noalloc, _ = call("noalloc")
    assert np.array_equal(first.view(np.int32), explicit.view(np.int32))
    assert np.array_equal(first.view(np.int32), noalloc.view(np.int32))
    ref = orc.run(q, k, v, ks, vs, n_head=h, n_kv=kvh, hd=hd, pos0=0,
                  kv=orc.KV_I8, threads=threads(), block=64)
    assert within(abs_err(first, ref), TOL_FLOAT_ABS,
                  f"AUTO first call, {n} tokens")


def test_auto_measurement_persists(gpu, monkeypatch, tmp_path):
    """AUTO's measurement is kept in attn_gpu.txt under the cache directory
    ($XDG_CACHE_HOME/janas, as the reference keeps attn.txt,
    attention.c:1118-1164), one line "key from16[0] from16[1]" keyed by
    device and geometry; a geometry found there is taken without measuring.
    A line saying INT16 from 2048 (one token) makes a call at 4000 the
    INT16 way's bits and a call at 1500 the FLOAT way's."""
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path))
    monkeypatch.delenv("JANAS_ATTN", raising=False)
    h, kvh, hd, cap = 8, 2, 128, 4400
    k, ks = int8_cache(621, kvh, cap, hd)
    v, vs = int8_cache(622, kvh, cap, hd)
    q = normal(623, h * hd).reshape(1, h, hd)
    kd, vd, ksd, vsd, qd = (to_dev(x, gpu) for x in (k, v, ks, vs, q))

    def call(n_ctx, scores, pos0):
        out = torch.zeros((1, h, hd), dtype=torch.float32, device=gpu)
        with Attention(h, kvh, hd, n_ctx, 1, scores) as a:
            a.run_dev(janas_amd.KV_I8, [dict(k=kd, v=vd, ks=ksd, vs=vsd, q=qd,
                                              out=out, cap=cap, n=1,
                                              pos0=pos0)])
            torch.cuda.synchronize()
            way = a.scores_mode()
        return way, out.cpu().numpy()

    # a fresh geometry is measured, and its line written
    call(4321, janas_amd.AUTO, 4000)
    path = tmp_path / "janas" / "attn_gpu.txt"
    lines = [l for l in path.read_text().splitlines() if l.strip()]
    key, f0, f1 = lines[-1].split()
    assert key.endswith("|0|8/2/128|0|4321"), key
    assert int(f0) >= 1024 and int(f1) >= 1024
    # another geometry's line, as if an earlier process had measured INT16
    key2 = key[:-len("4321")] + "4322"
    with open(path, "a") as f:
        f.write(f"{key2} 2048 1024\n")
    for pos0, want in ((4000, janas_amd.INT16), (1500, janas_amd.FLOAT)):
        way, got = call(4322, janas_amd.AUTO, pos0)
        assert way == want
        _, ref = call(4322, want, pos0)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
