"""The CPU restatement pinned: against the reference's compiled attention
(golden fixtures, bit for bit), against the closed form in double precision,
against the reference's invariants, and against mistakes planted in it.
CPU only."""
import math

import numpy as np
import pytest

from attn_helpers import TOL_FLOAT_ABS
from cases import (CASES, KV_F16, KV_F32, KV_I8, call_kwargs, digest,
                   int16_case, make_inputs, normal)
from oracle import orc


def golden(name):
    z = np.load(f"tests/golden/{name}.npz")
    return z["out"], str(z["digest"])


INT16_CASES = sorted(n for n in CASES if int16_case(n))
# the reference's bar for its INT16 way against the closed form, absolute
# on outputs of order one (test_attention.c:143-148)
TOL_INT16_EXACT = 1e-3


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_inputs_rebuild(name):
    """The generator still draws the inputs the fixture was made from."""
    _, dg = golden(name)
    assert digest(make_inputs(name)) == dg


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_bit_exact_vs_reference(name):
    inp = make_inputs(name)
    ref, _ = golden(name)
    out = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                  last=inp["last"], threads=4, block=64, **call_kwargs(name))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_vs_closed_form(name):
    inp = make_inputs(name)
    kw = call_kwargs(name)
    out = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                  last=inp["last"], threads=4, block=64, **kw)
    ex = orc.exact(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                   last=inp["last"], **kw)
    bar = TOL_FLOAT_ABS * max(1.0, float(np.abs(ex).max()))
    assert np.abs(out - ex).max() <= bar


@pytest.mark.parametrize("name", INT16_CASES)
def test_oracle_int16_bit_exact_vs_reference(name):
    """The INT16 way (quantized query, exact integer scores, weights
    quantized to 16 bits, exact integer value sums) against the reference's
    compiled INT16 path."""
    inp = make_inputs(name)
    ref = np.load(f"tests/golden/{name}.npz")["out_int16"]
    out = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                  last=inp["last"], threads=4, block=64, int16=True,
                  **call_kwargs(name))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", INT16_CASES)
def test_oracle_int16_vs_closed_form(name):
    """Within the reference's INT16 bar of the double-precision softmax,
    and not equal to the FLOAT way (the quantization is there)."""
    inp = make_inputs(name)
    kw = call_kwargs(name)
    out = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                  last=inp["last"], threads=4, block=64, int16=True, **kw)
    ex = orc.exact(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                   last=inp["last"], **kw)
    bar = TOL_INT16_EXACT * max(1.0, float(np.abs(ex).max()))
    assert np.abs(out - ex).max() <= bar
    flt, _ = golden(name)
    assert not np.array_equal(out, flt)


def test_int16_only_for_int8_and_sixteen():
    """An int16 cache, or a head size not a multiple of 16, keeps the FLOAT
    way (attention.c:975-977, :1061-1066)."""
    for name in ("i16_4x1x64_p1030_n5_w64_ring",):
        inp = make_inputs(name)
        kw = call_kwargs(name)
        a = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                    threads=2, block=64, **kw)
        b = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                    threads=2, block=64, int16=True, **kw)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    h, hd, cap = 2, 40, 300
    k = (normal(3, cap * hd) * 40).astype(np.int8).reshape(1, cap, hd)
    v = (normal(4, cap * hd) * 40).astype(np.int8).reshape(1, cap, hd)
    ks = np.full((1, cap), 0.01, np.float32)
    q = normal(5, 2 * h * hd).reshape(2, h, hd)
    kw = dict(n_head=h, n_kv=1, hd=hd, pos0=cap - 2, kv=KV_I8)
    a = orc.run(q, k, v, ks, ks, threads=2, **kw)
    b = orc.run(q, k, v, ks, ks, threads=2, int16=True, **kw)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("name", ["i8_8x1x128_p250_n17", "i8_4x2x64_p0_n64",
                                  "i16_4x1x64_p1030_n5_w64_ring"])
def test_block_equals_token_by_token(name):
    """attention.h:13-16: a token's result does not depend on its block."""
    c = CASES[name]
    inp = make_inputs(name)
    kw = call_kwargs(name)
    blk = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                  threads=3, **kw)
    for j in range(c["n"]):
        kw1 = dict(kw, pos0=c["pos0"] + j)
        one = orc.run(np.ascontiguousarray(inp["q"][j:j + 1]), inp["k"],
                      inp["v"], inp["ks"], inp["vs"], threads=2, **kw1)
        assert np.array_equal(one.view(np.uint32), blk[j:j + 1].view(np.uint32))


@pytest.mark.parametrize("name", ["i8_8x1x128_p250_n17",
                                  "i8_4x1x64_p600_n8_w300"])
def test_int16_block_equals_token_by_token(name):
    """The INT16 way keeps the promise too: a query's scale is its own row's
    and a weight's scale its own (chunk, token, head) row's."""
    c = CASES[name]
    inp = make_inputs(name)
    kw = dict(call_kwargs(name), int16=True)
    blk = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                  threads=3, **kw)
    for j in range(c["n"]):
        kw1 = dict(kw, pos0=c["pos0"] + j)
        one = orc.run(np.ascontiguousarray(inp["q"][j:j + 1]), inp["k"],
                      inp["v"], inp["ks"], inp["vs"], threads=2, **kw1)
        assert np.array_equal(one.view(np.uint32), blk[j:j + 1].view(np.uint32))


def test_float_element_types_equal_int8_unit_scales():
    """f16 / f32 caches holding the int8 numbers, with unit scales, give the
    reference's int8 result bit for bit: the float element types follow the
    same arithmetic with scale 1."""
    name = "i8unit_8x2x128_p300_n4"
    inp = make_inputs(name)
    ref, _ = golden(name)
    kw = call_kwargs(name)
    for kv, dt in ((KV_F16, np.float16), (KV_F32, np.float32)):
        kw2 = dict(kw, kv=kv)
        out = orc.run(inp["q"], inp["k"].astype(dt), inp["v"].astype(dt),
                      threads=4, **kw2)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kv,dt", [(KV_F16, np.float16), (KV_F32, np.float32)])
def test_float_caches_vs_closed_form(kv, dt):
    """N(0,1) caches (the BASELINE configs' distribution), GQA 8 across
    chunk boundaries, a window: the restatement within float error."""
    h, kvh, hd, cap, n, pos0 = 16, 2, 128, 700, 5, 600
    k = normal(11, kvh * cap * hd).reshape(kvh, cap, hd).astype(dt)
    v = normal(12, kvh * cap * hd).reshape(kvh, cap, hd).astype(dt)
    q = normal(13, n * h * hd).reshape(n, h, hd)
    for window in (0, 300):
        kw = dict(n_head=h, n_kv=kvh, hd=hd, pos0=pos0, kv=kv, window=window)
        out = orc.run(q, k, v, threads=4, **kw)
        ex = orc.exact(q, k, v, **kw)
        assert np.abs(out - ex).max() <= 2e-6


def test_exp_det_is_an_exp():
    """janas_exp_det (vmath.h:36-52) against libm over the range the weights
    use, and its exact points."""
    xs = np.linspace(-80.0, 0.0, 20001, dtype=np.float32)
    worst = max(abs(orc.exp_det(x) - math.exp(float(x))) / math.exp(float(x))
                for x in xs)
    assert worst < 4e-7
    assert orc.exp_det(0.0) == 1.0


def test_gate_is_sigmoid():
    out = np.ones((2, 3, 8), np.float32)
    g = np.array([[-1.0, 0.0, 2.0], [5.0, -5.0, 0.5]], np.float32)
    orc.gate(out, g, per_head=True)
    want = 1.0 / (1.0 + np.exp(-g.astype(np.float64)))
    assert np.allclose(out, want[:, :, None], rtol=1e-6, atol=0)


def test_ring_positions_closed_form():
    # attention.c:1048-1054: window + n + one chunk, rounded up to chunks
    for w, n in ((0, 1), (64, 5), (256, 64), (1000, 17)):
        need = w + n + 256
        assert orc.ring_positions(w, n) == (need + 255) // 256 * 256


# ---- planted mistakes: each must be caught by the pins above -----------


def _perturbed(name, mutate, int16=False):
    inp = make_inputs(name)
    mutate(inp)
    out = orc.run(inp["q"], inp["k"], inp["v"], inp["ks"], inp["vs"],
                  last=inp["last"], threads=2, block=64, int16=int16,
                  **call_kwargs(name))
    return out


@pytest.mark.parametrize("int16", [False, True])
@pytest.mark.parametrize("mutation", ["key_scale_dropped", "transposed_q",
                                      "off_by_one_position", "sign"])
def test_planted_mistakes_are_caught(mutation, int16):
    name = "i8_8x1x128_p250_n17"
    z = np.load(f"tests/golden/{name}.npz")
    ref = z["out_int16"] if int16 else z["out"]

    def mutate(inp):
        if mutation == "key_scale_dropped":
            inp["ks"][:] = 1.0
        elif mutation == "transposed_q":
            n, h, d = inp["q"].shape
            inp["q"] = np.ascontiguousarray(
                inp["q"].reshape(n, d, h).transpose(0, 2, 1))
        elif mutation == "off_by_one_position":
            inp["k"] = np.ascontiguousarray(np.roll(inp["k"], 1, axis=1))
        elif mutation == "sign":
            inp["v"] = np.ascontiguousarray(-inp["v"])
    out = _perturbed(name, mutate, int16)
    assert np.abs(out - ref).max() > 1e-3
