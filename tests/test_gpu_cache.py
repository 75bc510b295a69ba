"""The cache around the attention on the GPU (include/janas_attn.h Part 3
and the Q8_K output), against the CPU restatement of the reference's rules
(oracle/cache_oracle.c, pinned in tests/test_cache_oracle.py):

* janas_attn_cache_write: int8 / int16 rows and scales bit for bit equal to
  qkv_item's (model_attn.c:75-146) - with and without norms, with a partial
  rotation, a ring, several tokens and heads; f16 / f32 caches hold the
  restatement's normalized, turned rows;
* janas_attn_q_prep: the queries bit for bit;
* janas_attn_cache_shift: the cache after a shift bit for bit equal to
  model.c:304-377's, plain and ring, int8 and int16;
* janas_attn_cache_copy: the state rows in copy_kv's packing
  (model_state.c:175-218), and back;
* the Q8_K output: bit for bit the restatement of janas_q8k_quantize applied
  to the device's own float output, on the split and the prefill path;
* end to end: a cache written on the device, then attended, matches the
  restatement's cache attended on the CPU.
"""
import numpy as np
import pytest
import torch

import janas_amd as jm
from attn_helpers import KV_F16, TOL_F16_ABS, TOL_FLOAT_ABS, abs_err, threads, within
from oracle import orc

pytestmark = pytest.mark.gpu

KV_I8, KV_I16, KV_F32 = jm.KV_I8, jm.KV_I16, jm.KV_F32


def dev(x, gpu):
    return torch.from_numpy(np.ascontiguousarray(x)).to(gpu)


def rope_tables(positions, n_rot, base=1000000.0):
    half = n_rot // 2
    inv = base ** (-2.0 * np.arange(half) / n_rot)
    ang = np.outer(np.asarray(positions, np.float64), inv)
    return (np.cos(ang).astype(np.float32).reshape(len(positions), half),
            np.sin(ang).astype(np.float32).reshape(len(positions), half))


def device_cache(gpu, n_kv, cap, hd, kv, ring=False, fill=0):
    dt = {KV_I8: torch.int8, KV_I16: torch.int16, KV_F16: torch.float16,
          KV_F32: torch.float32}[kv]
    k = torch.full((n_kv, cap, hd), fill, dtype=dt, device=gpu)
    v = torch.full((n_kv, cap, hd), fill, dtype=dt, device=gpu)
    ks = torch.zeros((n_kv, cap), dtype=torch.float32, device=gpu)
    vs = torch.zeros((n_kv, cap), dtype=torch.float32, device=gpu)
    c = jm.attention.cache(k, v, ks, vs, kv_type=kv, ring=ring)
    return c, (k, v, ks, vs)


WRITE_CASES = [
    # n, n_kv, hd, n_rot, k_norm, v_norm, ring, pos0, cap
    (1, 8, 128, 128, True, False, False, 1023, 1024),
    (5, 2, 256, 256, True, False, False, 100, 512),
    (17, 4, 64, 32, False, False, False, 0, 64),
    (3, 1, 512, 512, True, True, False, 7, 16),
    (6, 2, 128, 128, True, False, True, 509, 512),
    (2, 3, 96, 0, False, True, False, 4, 8),
]


@pytest.mark.parametrize("kv", [KV_I8, KV_I16])
@pytest.mark.parametrize("case", range(len(WRITE_CASES)))
def test_cache_write_bitwise(gpu, kv, case):
    n, n_kv, hd, n_rot, use_kn, v_norm, ring, pos0, cap = WRITE_CASES[case]
    rng = np.random.default_rng(100 + case)
    k = (2.0 * rng.standard_normal((n, n_kv, hd))).astype(np.float32)
    v = rng.standard_normal((n, n_kv, hd)).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32) if use_kn else None
    cs, sn = rope_tables(range(pos0, pos0 + n), n_rot)
    wide = kv == KV_I16
    dt = np.int16 if wide else np.int8
    kc = np.zeros((n_kv, cap, hd), dt)
    vc, kz, vz = np.zeros_like(kc), np.zeros((n_kv, cap), np.float32), \
        np.zeros((n_kv, cap), np.float32)
    orc.cache_write(k.copy(), v.copy(), cs=cs, sn=sn, n_rot=n_rot, pos0=pos0,
                    kc=kc, vc=vc, kz=kz, vz=vz, k_norm=kn, v_norm=v_norm,
                    ring=ring, eps=1e-6)
    print(f"case {case} kv {kv}: n={n} n_kv={n_kv} hd={hd} n_rot={n_rot}",
          flush=True)
    c, (gk, gv, gks, gvs) = device_cache(gpu, n_kv, cap, hd, kv, ring)
    kd = dev(k, gpu)
    jm.attention.cache_write(c, kd, dev(v, gpu),
                             cs=dev(cs, gpu) if n_rot else None,
                             sn=dev(sn, gpu) if n_rot else None,
                             n_rot=n_rot, pos0=pos0,
                             k_norm=None if kn is None else dev(kn, gpu),
                             eps=1e-6, v_norm=v_norm)
    torch.cuda.synchronize()
    assert np.array_equal(gk.cpu().numpy(), kc)
    assert np.array_equal(gv.cpu().numpy(), vc)
    assert gks.cpu().numpy().tobytes() == kz.tobytes()
    assert gvs.cpu().numpy().tobytes() == vz.tobytes()
    assert np.array_equal(kd.cpu().numpy(), k)  # inputs left as they were


@pytest.mark.parametrize("kv", [KV_F16, KV_F32])
def test_cache_write_float_caches(gpu, kv):
    n, n_kv, hd, n_rot, pos0, cap = 4, 2, 128, 64, 30, 64
    rng = np.random.default_rng(9)
    k = rng.standard_normal((n, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((n, n_kv, hd)).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    cs, sn = rope_tables(range(pos0, pos0 + n), n_rot)
    want_k = k.copy()
    orc.q_prep(want_k, cs=cs, sn=sn, n_rot=n_rot, q_norm=kn, eps=1e-6)
    c, (gk, gv, _, _) = device_cache(gpu, n_kv, cap, hd, kv)
    jm.attention.cache_write(c, dev(k, gpu), dev(v, gpu), cs=dev(cs, gpu),
                             sn=dev(sn, gpu), n_rot=n_rot, pos0=pos0,
                             k_norm=dev(kn, gpu), eps=1e-6)
    torch.cuda.synchronize()
    dt = np.float16 if kv == KV_F16 else np.float32
    got_k = gk.cpu().numpy()[:, pos0:pos0 + n].transpose(1, 0, 2)
    got_v = gv.cpu().numpy()[:, pos0:pos0 + n].transpose(1, 0, 2)
    assert np.array_equal(got_k, want_k.astype(dt))
    assert np.array_equal(got_v, v.astype(dt))


def test_q_prep_bitwise(gpu):
    n, n_head, hd, n_rot = 9, 16, 128, 128
    rng = np.random.default_rng(5)
    q = rng.standard_normal((n, n_head, hd)).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    cs, sn = rope_tables(range(40, 40 + n), n_rot)
    want = q.copy()
    orc.q_prep(want, cs=cs, sn=sn, n_rot=n_rot, q_norm=qn, eps=1e-6)
    qd = dev(q, gpu)
    jm.attention.q_prep(qd, cs=dev(cs, gpu), sn=dev(sn, gpu), n_rot=n_rot,
                        q_norm=dev(qn, gpu), eps=1e-6)
    torch.cuda.synchronize()
    assert qd.cpu().numpy().tobytes() == want.tobytes()


SHIFT_CASES = [
    # n_kv, hd, cap, n_rot, ring, keep, drop, n_pos
    (2, 128, 256, 128, False, 4, 50, 200),
    (1, 64, 64, 32, False, 0, 3, 64),
    (3, 256, 512, 256, True, 0, 100, 700),
    (2, 128, 256, 128, True, 10, 20, 200),
    (1, 96, 32, 0, False, 2, 5, 30),
]


@pytest.mark.parametrize("kv", [KV_I8, KV_I16])
@pytest.mark.parametrize("case", range(len(SHIFT_CASES)))
def test_cache_shift_bitwise(gpu, kv, case):
    n_kv, hd, cap, n_rot, ring, keep, drop, n_pos = SHIFT_CASES[case]
    rng = np.random.default_rng(200 + case)
    dt = np.int16 if kv == KV_I16 else np.int8
    top = 32767 if kv == KV_I16 else 127
    k = rng.integers(-top, top + 1, (n_kv, cap, hd)).astype(dt)
    v = rng.integers(-top, top + 1, (n_kv, cap, hd)).astype(dt)
    kz = rng.uniform(0.001, 0.02, (n_kv, cap)).astype(np.float32)
    vz = rng.uniform(0.001, 0.02, (n_kv, cap)).astype(np.float32)
    cs, sn = rope_tables([drop], max(n_rot, 2))
    cs, sn = cs[0][:n_rot // 2].copy(), sn[0][:n_rot // 2].copy()
    gk, gv, gkz, gvz = (dev(x, gpu) for x in (k, v, kz, vz))
    c = jm.attention.cache(gk, gv, gkz, gvz, kv_type=kv, ring=ring)
    print(f"shift case {case} kv {kv}", flush=True)
    jm.attention.cache_shift(c, keep=keep, drop=drop, n_pos=n_pos,
                             cs=dev(cs, gpu) if n_rot else None,
                             sn=dev(sn, gpu) if n_rot else None, n_rot=n_rot)
    torch.cuda.synchronize()
    orc.cache_shift(k, v, kz, vz, keep=keep, drop=drop, n_pos=n_pos, cs=cs,
                    sn=sn, n_rot=n_rot, ring=ring)
    assert np.array_equal(gk.cpu().numpy(), k)
    assert np.array_equal(gv.cpu().numpy(), v)
    assert gkz.cpu().numpy().tobytes() == kz.tobytes()
    assert gvz.cpu().numpy().tobytes() == vz.tobytes()


def copy_kv_reference(k, v, ks, vs, n_pos, rows, ring):
    """copy_kv's packing (model_state.c:175-218), written out in numpy."""
    cap = k.shape[1]
    pos = range(n_pos - rows, n_pos) if ring else range(rows)
    idx = [p % cap if ring else p for p in pos]
    return (np.ascontiguousarray(k[:, idx]), np.ascontiguousarray(v[:, idx]),
            np.ascontiguousarray(ks[:, idx]), np.ascontiguousarray(vs[:, idx]))


@pytest.mark.parametrize("ring,n_pos,rows", [(False, 100, 100), (False, 256, 256),
                                             (True, 300, 256), (True, 1000, 200),
                                             (True, 100, 100)])
def test_cache_copy_layout_and_round_trip(gpu, ring, n_pos, rows):
    n_kv, cap, hd = 3, 256, 64
    rng = np.random.default_rng(n_pos + rows)
    k = rng.integers(-127, 128, (n_kv, cap, hd)).astype(np.int8)
    v = rng.integers(-127, 128, (n_kv, cap, hd)).astype(np.int8)
    ks = rng.uniform(0.001, 0.02, (n_kv, cap)).astype(np.float32)
    vs = rng.uniform(0.001, 0.02, (n_kv, cap)).astype(np.float32)
    gk, gv, gks, gvs = (dev(x, gpu) for x in (k, v, ks, vs))
    c = jm.attention.cache(gk, gv, gks, gvs, kv_type=KV_I8, ring=ring)
    bk = np.zeros((n_kv, rows, hd), np.int8)
    bv = np.zeros_like(bk)
    bks = np.zeros((n_kv, rows), np.float32)
    bvs = np.zeros_like(bks)
    jm.attention.cache_copy(c, n_pos=n_pos, rows=rows, k=bk, v=bv, ks=bks,
                            vs=bvs, out=True)
    torch.cuda.synchronize()
    want = copy_kv_reference(k, v, ks, vs, n_pos, rows, ring)
    for got, w in zip((bk, bv, bks, bvs), want):
        assert got.tobytes() == w.tobytes()
    # back into a cleared cache: the same rows again, nothing else
    for t in (gk, gv, gks, gvs):
        t.zero_()
    jm.attention.cache_copy(c, n_pos=n_pos, rows=rows, k=bk, v=bv, ks=bks,
                            vs=bvs, out=False)
    torch.cuda.synchronize()
    idx = [p % cap if ring else p for p in
           (range(n_pos - rows, n_pos) if ring else range(rows))]
    assert np.array_equal(gk.cpu().numpy()[:, idx], k[:, idx])
    assert np.array_equal(gvs.cpu().numpy()[:, idx], vs[:, idx])
    rest = np.setdiff1d(np.arange(cap), idx)
    assert not gk.cpu().numpy()[:, rest].any()


@pytest.mark.parametrize("path", ["split", "prefill"])
@pytest.mark.parametrize("gate_mode", [jm.GATE_NONE, jm.GATE_ELEM])
def test_q8k_output_bitwise(gpu, path, gate_mode):
    h, kvh, hd, L = 32, 8, 128, 700
    n = 1 if path == "split" else 100
    rng = np.random.default_rng(11)
    k = rng.standard_normal((kvh, L, hd)).astype(np.float16)
    v = rng.standard_normal((kvh, L, hd)).astype(np.float16)
    q = rng.standard_normal((n, h, hd)).astype(np.float32)
    g = rng.standard_normal((n, h, hd)).astype(np.float32)
    out = torch.zeros((n, h, hd), dtype=torch.float32, device=gpu)
    blocks = torch.zeros((n, h * hd // 256, jm.attention.Q8K_BYTES),
                         dtype=torch.uint8, device=gpu)
    with jm.Attention(h, kvh, hd, L) as a:
        a.run_dev(KV_F16, [dict(k=dev(k, gpu), v=dev(v, gpu), q=dev(q, gpu),
                                out=out, gate=dev(g, gpu), cap=L, n=n,
                                pos0=L - n, out_q8k=blocks)],
                  gate_mode=gate_mode, path=path)
        torch.cuda.synchronize()
    o = out.cpu().numpy()
    want = orc.q8k_quantize(o.reshape(n, h * hd))
    assert blocks.cpu().numpy().tobytes() == want.tobytes()
    ref = orc.run(q, k, v, n_head=h, n_kv=kvh, hd=hd, pos0=L - n, kv=KV_F16,
                  threads=threads(), block=64)
    if gate_mode:
        orc.gate(ref, g)
    assert within(abs_err(o, ref), TOL_F16_ABS, "abs_err(o, ref)")


@pytest.mark.parametrize("geom", [(32, 8, 128, 1), (8, 2, 96, 3),
                                  (16, 2, 256, 1), (16, 4, 64, 5),
                                  (4, 1, 512, 2)])
@pytest.mark.parametrize("gate_mode", [jm.GATE_NONE, jm.GATE_HEAD])
def test_q8k_fused_merge(gpu, geom, gate_mode):
    """The split path's merge quantizes its own output, a Q8_K block a
    workgroup (blocks across heads for head sizes 64, 96 and 128, half a
    head at 512): the blocks equal the restatement of janas_q8k_quantize
    over the output bit for bit, and the output equals the same call's
    without Q8_K bit for bit (a second sequence of the launch asks for
    none)."""
    h, kvh, hd, n = geom
    L = 900
    rng = np.random.default_rng(hd + n)
    k = rng.standard_normal((kvh, L, hd)).astype(np.float16)
    v = rng.standard_normal((kvh, L, hd)).astype(np.float16)
    q = rng.standard_normal((n, h, hd)).astype(np.float32)
    g = rng.standard_normal((n, h)).astype(np.float32)
    kd, vd, qd, gd = dev(k, gpu), dev(v, gpu), dev(q, gpu), dev(g, gpu)
    nb = h * hd // 256
    outs = [torch.zeros((n, h, hd), dtype=torch.float32, device=gpu)
            for _ in range(3)]
    blocks = torch.zeros((n, nb, jm.attention.Q8K_BYTES), dtype=torch.uint8,
                         device=gpu)
    seq = dict(k=kd, v=vd, q=qd, gate=gd, cap=L, n=n, pos0=L - n)
    with jm.Attention(h, kvh, hd, L) as a:
        a.run_dev(KV_F16, [dict(seq, out=outs[0], out_q8k=blocks),
                           dict(seq, out=outs[1])],
                  gate_mode=gate_mode, path="split")
        a.run_dev(KV_F16, [dict(seq, out=outs[2])], gate_mode=gate_mode,
                  path="split")
        torch.cuda.synchronize()
    o = [x.cpu().numpy() for x in outs]
    assert np.array_equal(o[0].view(np.int32), o[2].view(np.int32))
    assert np.array_equal(o[1].view(np.int32), o[2].view(np.int32))
    want = orc.q8k_quantize(o[0].reshape(n, h * hd))
    assert blocks.cpu().numpy().tobytes() == want.tobytes()
    ref = orc.run(q, k, v, n_head=h, n_kv=kvh, hd=hd, pos0=L - n, kv=KV_F16,
                  threads=threads())
    if gate_mode:
        orc.gate(ref, g, per_head=True)
    assert within(abs_err(o[0], ref), TOL_F16_ABS, "vs oracle")


def test_q8k_output_needs_whole_blocks(gpu):
    h, kvh, hd, L = 3, 1, 64, 256   # 192 numbers a token: no whole block
    k = torch.zeros((kvh, L, hd), dtype=torch.float16, device=gpu)
    q = torch.zeros((1, h, hd), dtype=torch.float32, device=gpu)
    blocks = torch.zeros((1, 1, jm.attention.Q8K_BYTES), dtype=torch.uint8,
                         device=gpu)
    with jm.Attention(h, kvh, hd, L) as a:
        with pytest.raises(jm.AttnError) as e:
            a.run_dev(KV_F16, [dict(k=k, v=k, q=q, out=torch.empty_like(q),
                                    cap=L, n=1, pos0=L - 1, out_q8k=blocks)])
        assert e.value.code == -1


@pytest.mark.parametrize("kv", [KV_I8, KV_I16])
def test_written_cache_attends_like_the_reference(gpu, kv):
    """Tokens 0 .. 299 written on the device, then the last 4 attend it; the
    restatement writes and attends the same tokens on the CPU."""
    h, kvh, hd, n_rot, cap, npos = 16, 2, 128, 128, 512, 300
    rng = np.random.default_rng(77)
    k = rng.standard_normal((npos, kvh, hd)).astype(np.float32)
    v = rng.standard_normal((npos, kvh, hd)).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    q = rng.standard_normal((4, h, hd)).astype(np.float32)
    cs, sn = rope_tables(range(npos), n_rot)
    dt = np.int16 if kv == KV_I16 else np.int8
    kc = np.zeros((kvh, cap, hd), dt)
    vc, kz, vz = np.zeros_like(kc), np.zeros((kvh, cap), np.float32), \
        np.zeros((kvh, cap), np.float32)
    orc.cache_write(k.copy(), v.copy(), cs=cs, sn=sn, n_rot=n_rot, pos0=0,
                    kc=kc, vc=vc, kz=kz, vz=vz, k_norm=kn, eps=1e-6)
    c, (gk, gv, gks, gvs) = device_cache(gpu, kvh, cap, hd, kv)
    for s in range(0, npos, 64):   # in blocks, as the engine writes them
        e = min(npos, s + 64)
        jm.attention.cache_write(c, dev(k[s:e], gpu), dev(v[s:e], gpu),
                                 cs=dev(cs[s:e], gpu), sn=dev(sn[s:e], gpu),
                                 n_rot=n_rot, pos0=s, k_norm=dev(kn, gpu),
                                 eps=1e-6)
    out = torch.zeros((4, h, hd), dtype=torch.float32, device=gpu)
    with jm.Attention(h, kvh, hd, cap) as a:
        a.run_dev(kv, [dict(k=gk, v=gv, ks=gks, vs=gvs, q=dev(q, gpu), out=out,
                            cap=cap, n=4, pos0=npos - 4)])
        torch.cuda.synchronize()
    ref = orc.run(q, kc, vc, kz, vz, n_head=h, n_kv=kvh, hd=hd,
                  pos0=npos - 4, kv=kv, threads=threads())
    assert within(abs_err(out.cpu().numpy(), ref), TOL_FLOAT_ABS, "abs_err(out.cpu().numpy(), ref)")


@pytest.mark.parametrize("geom", [
    (32, 8, 128, 2048, 0, KV_F16),     # DMA kernel, one segment: write_out
    (32, 8, 128, 1024, 0, KV_F16),     # two-halves kernel
    (32, 8, 128, 300, 600, KV_F16),    # key segments: the segment merge
    (16, 2, 256, 700, 100, KV_F16),    # a block is one row
    (16, 4, 64, 900, 0, KV_F16),       # a block is four rows
    (32, 8, 128, 800, 0, KV_I8),       # the exact kernel
    (16, 2, 256, 600, 0, KV_I16),      # the exact kernel, two planes
    (8, 2, 96, 300, 0, KV_F16),        # no whole rows a block: a pass
    (8, 8, 128, 400, 0, KV_F16),       # a block's heads in two KV heads
    (4, 1, 512, 200, 0, KV_F16),       # the register-staged kernel
])
@pytest.mark.parametrize("gate_mode", [jm.GATE_NONE, jm.GATE_ELEM])
def test_prefill_q8k(gpu, geom, gate_mode):
    """A prompt that asks for Q8_K output on the prefill path: the kernel
    writes the blocks with its output (head sizes 64, 128, 256, a block's
    heads in one KV head's group), the segment merge with its, or a pass
    over the output does (other shapes). Every way: the blocks equal the
    restatement of janas_q8k_quantize over the output bit for bit, and the
    output equals the same sequence's without Q8_K bit for bit, both in one
    launch and alone."""
    h, kvh, hd, n, pos0, kv = geom
    L = pos0 + n
    rng = np.random.default_rng(hd + n + kv)
    if kv == KV_F16:
        k = rng.standard_normal((kvh, L, hd)).astype(np.float16)
        v = rng.standard_normal((kvh, L, hd)).astype(np.float16)
        ks = vs = None
    else:
        top = 127 if kv == KV_I8 else 32767
        dt = np.int8 if kv == KV_I8 else np.int16
        kf = rng.standard_normal((kvh, L, hd)).astype(np.float32)
        vf = rng.standard_normal((kvh, L, hd)).astype(np.float32)
        ks = (np.abs(kf).max(axis=2) / top).astype(np.float32)
        vs = (np.abs(vf).max(axis=2) / top).astype(np.float32)
        k = np.rint(kf / ks[..., None]).astype(dt)
        v = np.rint(vf / vs[..., None]).astype(dt)
    q = rng.standard_normal((n, h, hd)).astype(np.float32)
    g = rng.standard_normal((n, h, hd)).astype(np.float32)
    seq = dict(k=dev(k, gpu), v=dev(v, gpu), q=dev(q, gpu), gate=dev(g, gpu),
               cap=L, n=n, pos0=pos0)
    if ks is not None:
        seq.update(ks=dev(ks, gpu), vs=dev(vs, gpu))
    outs = [torch.full((n, h, hd), float("nan"), device=gpu) for _ in range(3)]
    blocks = torch.zeros((n, h * hd // 256, jm.attention.Q8K_BYTES),
                         dtype=torch.uint8, device=gpu)
    with jm.Attention(h, kvh, hd, L, 1, jm.FLOAT) as a:
        a.run_dev(kv, [dict(seq, out=outs[0], out_q8k=blocks),
                       dict(seq, out=outs[1])], gate_mode=gate_mode,
                  path="prefill")
        a.run_dev(kv, [dict(seq, out=outs[2])], gate_mode=gate_mode,
                  path="prefill")
        torch.cuda.synchronize()
        assert a.status() == 0
    o = [x.cpu().numpy() for x in outs]
    assert np.array_equal(o[0].view(np.int32), o[2].view(np.int32))
    assert np.array_equal(o[1].view(np.int32), o[2].view(np.int32))
    want = orc.q8k_quantize(o[0].reshape(n, h * hd))
    assert blocks.cpu().numpy().tobytes() == want.tobytes()
