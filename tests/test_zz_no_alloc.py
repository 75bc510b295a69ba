"""janas_attn_run_dev_noalloc: the same results as janas_attn_run_dev,
bit for bit, with its partials in the device's fixed array - two calls in
a row (a long decode, then a smaller block and a prompt chunk whose key
segments need partials), and a call needing more than the array is refused
with JANAS_ATTN_ERANGE."""
import numpy as np
import pytest
import torch

import janas_amd
from cases import normal
from janas_amd import Attention

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 64 << 20


def dev(x, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def both(a, kv, seqs, gate_mode, noalloc_outs):
    """run_dev into the seqs' outs, then run_dev_noalloc into noalloc_outs
    (same inputs)."""
    a.run_dev(kv, seqs, gate_mode=gate_mode)
    seqs2 = [dict(s, out=o) for s, o in zip(seqs, noalloc_outs)]
    a.run_dev(kv, seqs2, gate_mode=gate_mode, path="noalloc")
    torch.cuda.synchronize()


def test_noalloc_equals_run_dev_twice(gpu):
    # call 1: config 4's decode (16 / 2 / 256, 32k positions, gated)
    h, kvh, hd, L = 16, 2, 256, 32768
    k = dev(normal(101, kvh * L * hd).reshape(kvh, L, hd).astype(np.float16), gpu)
    v = dev(normal(103, kvh * L * hd).reshape(kvh, L, hd).astype(np.float16), gpu)
    q = dev(normal(107, h * hd).reshape(1, h, hd), gpu)
    g = dev(normal(109, h * hd).reshape(1, h, hd), gpu)
    out, out2 = torch.empty_like(q), torch.full_like(q, float("nan"))
    with Attention(h, kvh, hd, L) as a:
        a.set_scale(1.0 / 16.0)
        both(a, janas_amd.KV_F16, [dict(k=k, v=v, q=q, out=out, gate=g, cap=L,
                                        n=1, pos0=L - 1)],
             janas_amd.GATE_ELEM, [out2])
    assert torch.equal(out, out2)
    # call 2, smaller: a 16-token block (split path) and a 512-token chunk
    # of a prompt at 4096 (prefill path, split into key segments) over an
    # int8 cache, 32 / 8 / 128
    h, kvh, hd, L = 32, 8, 128, 4608
    k8 = np.clip(np.rint(normal(111, kvh * L * hd) * 30), -127, 127).astype(np.int8)
    v8 = np.clip(np.rint(normal(113, kvh * L * hd) * 30), -127, 127).astype(np.int8)
    ks = (0.01 + 0.01 * np.abs(normal(117, kvh * L))).astype(np.float32)
    vs = (0.01 + 0.01 * np.abs(normal(119, kvh * L))).astype(np.float32)
    kd, vd = dev(k8.reshape(kvh, L, hd), gpu), dev(v8.reshape(kvh, L, hd), gpu)
    ksd, vsd = dev(ks.reshape(kvh, L), gpu), dev(vs.reshape(kvh, L), gpu)
    qa = dev(normal(121, 16 * h * hd).reshape(16, h, hd), gpu)
    qb = dev(normal(123, 512 * h * hd).reshape(512, h, hd), gpu)
    oa, ob = torch.empty_like(qa), torch.empty_like(qb)
    oa2, ob2 = torch.full_like(qa, float("nan")), torch.full_like(qb, float("nan"))
    with Attention(h, kvh, hd, L) as a:
        both(a, janas_amd.KV_I8,
             [dict(k=kd, v=vd, ks=ksd, vs=vsd, q=qa, out=oa, cap=L, n=16, pos0=3000),
              dict(k=kd, v=vd, ks=ksd, vs=vsd, q=qb, out=ob, cap=L, n=512, pos0=4096)],
             janas_amd.GATE_NONE, [oa2, ob2])
    assert torch.equal(oa, oa2)
    assert torch.equal(ob, ob2)


@pytest.mark.parametrize("L,fits", [(16128, True), (16384, False), (65536, False)])
def test_noalloc_refuses_more_than_the_array(gpu, L, fits):
    """The array's capacity for the split path's partials: a row of m, l and
    hd values takes (hd + 2) x 4 bytes, a launch n_kv x chunks x n x group
    rows (the m, l pairs padded to 256 bytes). A 64-token block over 8 KV
    heads of 128 (32 query heads) at positions L - 64 .. L - 1 takes 2048
    rows a chunk: 63 chunks (L = 16128: 67,092,480 bytes) fit in the
    67,108,864, 64 chunks (L = 16384: 68,157,440) do not and are refused
    with ERANGE, as is 64k. The block that fits equals janas_attn_run_dev's
    result bit for bit."""
    h, kvh, hd = 32, 8, 128
    k = torch.zeros((kvh, L, hd), dtype=torch.float16, device=gpu)
    q = dev(normal(161, 64 * h * hd).reshape(64, h, hd), gpu)
    out = torch.full_like(q, float("nan"))
    chunks = (L + 255) // 256
    rows = kvh * chunks * 64 * (h // kvh)
    need = (rows * 2 * 4 + 255) // 256 * 256 + rows * hd * 4
    assert (need <= NOALLOC_BYTES) == fits
    seq = dict(k=k, v=k, q=q, out=out, cap=L, n=64, pos0=L - 64)
    with Attention(h, kvh, hd, L) as a:
        if not fits:
            with pytest.raises(janas_amd.AttnError) as e:
                a.run_dev(janas_amd.KV_F16, [seq], path="noalloc")
            assert e.value.code == janas_amd.ERANGE
            return
        a.run_dev(janas_amd.KV_F16, [seq], path="noalloc")
        want = torch.full_like(q, float("nan"))
        a.run_dev(janas_amd.KV_F16, [dict(seq, out=want)])
        torch.cuda.synchronize()
    assert torch.equal(out, want)


def test_noalloc_under_graph_capture(gpu):
    """The entry point's reason: code under HIP graph capture. A decode
    step (f16, gated) and a 16-token block over an int8 cache, captured
    into one graph through janas_attn_run_dev_noalloc and replayed three
    times - with eager work in between that overwrites the device's
    partials array - each replay equal bit for bit to the eager result."""
    h, kvh, hd, L = 16, 2, 256, 4096
    k = dev(normal(131, kvh * L * hd).reshape(kvh, L, hd).astype(np.float16), gpu)
    v = dev(normal(133, kvh * L * hd).reshape(kvh, L, hd).astype(np.float16), gpu)
    q = dev(normal(137, h * hd).reshape(1, h, hd), gpu)
    g = dev(normal(139, h * hd).reshape(1, h, hd), gpu)
    k8 = np.clip(np.rint(normal(141, kvh * L * hd) * 30), -127, 127).astype(np.int8)
    v8 = np.clip(np.rint(normal(143, kvh * L * hd) * 30), -127, 127).astype(np.int8)
    ks = dev((0.01 + 0.01 * np.abs(normal(147, kvh * L))).astype(np.float32).reshape(kvh, L), gpu)
    vs = dev((0.01 + 0.01 * np.abs(normal(149, kvh * L))).astype(np.float32).reshape(kvh, L), gpu)
    kd, vd = dev(k8.reshape(kvh, L, hd), gpu), dev(v8.reshape(kvh, L, hd), gpu)
    qb = dev(normal(151, 16 * h * hd).reshape(16, h, hd), gpu)
    qo = dev(normal(153, 16 * h * hd).reshape(16, h, hd), gpu)
    want_a, want_b = torch.empty_like(q), torch.empty_like(qb)
    out_a, out_b = torch.empty_like(q), torch.empty_like(qb)
    scratch_out = torch.empty_like(qb)
    s = torch.cuda.Stream()
    with Attention(h, kvh, hd, L) as a:
        def calls(oa, ob, path):
            return [a.prepare(janas_amd.KV_F16, [dict(k=k, v=v, q=q, out=oa, gate=g, cap=L,
                                                      n=1, pos0=L - 1)],
                              gate_mode=janas_amd.GATE_ELEM, stream=s.cuda_stream,
                              path=path),
                    a.prepare(janas_amd.KV_I8, [dict(k=kd, v=vd, ks=ks, vs=vs, q=qb, out=ob,
                                                     cap=L, n=16, pos0=L - 16)],
                              stream=s.cuda_stream, path=path)]
        with torch.cuda.stream(s):
            for f in calls(want_a, want_b, "auto"):
                f()
            captured = calls(out_a, out_b, "noalloc")
            for f in captured:   # once outside the capture
                f()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            for f in captured:
                f()
        torch.cuda.synchronize()
        other = a.prepare(janas_amd.KV_I8, [dict(k=kd, v=vd, ks=ks, vs=vs, q=qo,
                                                 out=scratch_out, cap=L, n=16, pos0=1000)],
                          stream=s.cuda_stream, path="noalloc")
        for _ in range(3):
            out_a.zero_()
            out_b.zero_()
            with torch.cuda.stream(s):
                other()          # eager: overwrites the partials array
                graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_a, want_a)
            assert torch.equal(out_b, want_b)
        assert a.status() == 0
