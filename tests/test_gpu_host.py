"""Host-side behaviour of the library on the GPU: the drop-in's staging
buffers follow the cache's element size, calls on different streams share
an instance's partials safely, and a failing janas_attn_run can return
instead of aborting (janas_attn_set_abort), leaving NaN in a host output
and its failure kept in janas_attn_status."""
import numpy as np
import pytest
import torch

import janas_amd
from attn_helpers import TOL_FLOAT_ABS, abs_err, threads, within
from cases import normal
from janas_amd import Attention
from oracle import orc

pytestmark = pytest.mark.gpu


def int_cache(seed, n_kv, n_ctx, hd, dtype):
    """int8 / int16 keys or values and their per-row scales, seeded: rows
    of N(0, 1) numbers quantized as the engine does it (the largest
    magnitude of a row becomes 127 or 32767, model_attn.c:126-145)."""
    top = 127 if dtype == np.int8 else 32767
    x = normal(seed, n_kv * n_ctx * hd).reshape(n_kv, n_ctx, hd)
    mx = np.abs(x).max(axis=2, keepdims=True)
    q = np.rint(x * (top / mx)).astype(dtype)
    return q, (mx[..., 0] / top).astype(np.float32)


def reference(q, k, ks, v, vs, kv, pos0, h, n_kv, hd):
    return orc.run(q, k, v, ks, vs, n_head=h, n_kv=n_kv, hd=hd, pos0=pos0,
                   kv=kv, threads=threads())


def test_staging_follows_kv16_toggle(gpu):
    """An int8 host-pointer call, then set_kv16(1) and an int16 one on the
    same instance: the staging buffers grow to the 16-bit cache (before,
    they kept the int8 size and the copy overran them)."""
    h, n_kv, hd, n_ctx, pos0 = 8, 2, 128, 1024, 1000
    q = normal(5, 3 * h * hd).reshape(3, h, hd)
    k8, ks8 = int_cache(11, n_kv, n_ctx, hd, np.int8)
    v8, vs8 = int_cache(13, n_kv, n_ctx, hd, np.int8)
    k16, ks16 = int_cache(17, n_kv, n_ctx, hd, np.int16)
    v16, vs16 = int_cache(19, n_kv, n_ctx, hd, np.int16)
    with Attention(h, n_kv, hd, n_ctx, 1, janas_amd.FLOAT) as a:
        out8 = np.zeros_like(q)
        a.run(q, k8, ks8, v8, vs8, 3, pos0, out8)
        a.set_kv16(True)
        out16 = np.zeros_like(q)
        a.run(q, k16, ks16, v16, vs16, 3, pos0, out16)
        a.set_kv16(False)
        out8b = np.zeros_like(q)
        a.run(q, k8, ks8, v8, vs8, 3, pos0, out8b)
        assert a.status() == 0
    ref8 = reference(q, k8, ks8, v8, vs8, orc.KV_I8, pos0, h, n_kv, hd)
    ref16 = reference(q, k16, ks16, v16, vs16, orc.KV_I16, pos0, h, n_kv, hd)
    assert within(abs_err(out8, ref8), TOL_FLOAT_ABS, "abs_err(out8, ref8)")
    assert within(abs_err(out16, ref16), TOL_FLOAT_ABS, "abs_err(out16, ref16)")
    assert np.array_equal(out8, out8b)


def test_two_streams_share_partials(gpu):
    """Calls alternating between two streams on one instance, the second
    stream's call growing the partials while the first's may still run:
    every output equals the same call made alone."""
    h, n_kv, hd = 16, 2, 128
    n_ctx = 8192
    dev = gpu
    k = torch.from_numpy(normal(31, n_kv * n_ctx * hd).reshape(n_kv, n_ctx, hd)
                         .astype(np.float16)).to(dev)
    v = torch.from_numpy(normal(37, n_kv * n_ctx * hd).reshape(n_kv, n_ctx, hd)
                         .astype(np.float16)).to(dev)
    q1 = torch.from_numpy(normal(41, h * hd).reshape(1, h, hd)).to(dev)
    q2 = torch.from_numpy(normal(43, 48 * h * hd).reshape(48, h, hd)).to(dev)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def call(a, q, n, pos0, out, stream):
        a.run_dev(janas_amd.KV_F16, [dict(k=k, v=v, q=q, out=out, cap=n_ctx,
                                          n=n, pos0=pos0)],
                  stream=stream.cuda_stream if stream is not None else None,
                  path="split")

    # alone, on the default stream of a fresh instance each
    want1 = torch.empty_like(q1)
    want2 = torch.empty_like(q2)
    with Attention(h, n_kv, hd, 256) as a:
        call(a, q1, 1, n_ctx - 1, want1, None)
        torch.cuda.synchronize()
    with Attention(h, n_kv, hd, 256) as a:
        call(a, q2, 48, n_ctx - 48, want2, None)
        torch.cuda.synchronize()
    # interleaved on two streams; the instance starts with small partials
    outs1 = [torch.full_like(q1, float("nan")) for _ in range(3)]
    outs2 = [torch.full_like(q2, float("nan")) for _ in range(3)]
    with Attention(h, n_kv, hd, 256) as a:
        for i in range(3):
            call(a, q1, 1, n_ctx - 1, outs1[i], s1)
            call(a, q2, 48, n_ctx - 48, outs2[i], s2)
        torch.cuda.synchronize()
        assert a.status() == 0
    for o in outs1:
        assert torch.equal(o, want1)
    for o in outs2:
        assert torch.equal(o, want2)


def test_run_returns_instead_of_abort(gpu):
    """With janas_attn_set_abort(0) a call janas_attn_run refuses (more
    tokens than a block, positions past the cache) returns, the host
    output NaN; argument errors are not kept as the device status."""
    h, n_kv, hd, n_ctx = 4, 1, 64, 512
    k, ks = int_cache(3, n_kv, n_ctx, hd, np.int8)
    v, vs = int_cache(7, n_kv, n_ctx, hd, np.int8)
    with Attention(h, n_kv, hd, n_ctx) as a:
        a.set_abort(False)
        q = normal(9, 65 * h * hd).reshape(65, h, hd)
        out = np.zeros_like(q)
        a.run(q, k, ks, v, vs, 65, 0, out)
        assert np.isnan(out).all()
        q = normal(9, 2 * h * hd).reshape(2, h, hd)
        out = np.zeros_like(q)
        a.run(q, k, ks, v, vs, 2, n_ctx - 1, out)
        assert np.isnan(out).all()
        assert a.status() == 0
        # and the instance still works
        out = np.zeros_like(q)
        a.run(q, k, ks, v, vs, 2, 100, out)
        ref = reference(q, k, ks, v, vs, orc.KV_I8, 100, h, n_kv, hd)
        assert within(abs_err(out, ref), TOL_FLOAT_ABS, "abs_err(out, ref)")
        a.clear_status()
        assert a.status() == 0
