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


def imported_case(kv_dtype, n_kv=2, h=8, hd=128, n_ctx=1024, seed=61):
    k, ks = int_cache(seed, n_kv, n_ctx, hd, kv_dtype)
    v, vs = int_cache(seed + 2, n_kv, n_ctx, hd, kv_dtype)
    return k, ks, v, vs


def staged(h, n_kv, hd, n_ctx, kv16, ring, q, k, ks, v, vs, n, pos0):
    """The same call through the staging path (nothing imported)."""
    out = np.zeros_like(q)
    with Attention(h, n_kv, hd, n_ctx, 1, janas_amd.FLOAT) as a:
        a.set_kv16(kv16)
        a.set_ring(ring)
        a.run(q, k, ks, v, vs, n, pos0, out)
        assert a.status() == 0
    return out


@pytest.mark.parametrize("kv16", [False, True])
def test_imported_cache_equals_staging(kv16, gpu):
    """janas_attn_run over an imported host cache (janas_attn_import) reads
    the device copy: a decode and a 64-token block equal the staging path
    bit for bit and the oracle within the FLOAT bar; the rows of a call's
    positions are taken from the host at the call (the engine writes them
    just before), a change anywhere else is not seen until janas_attn_sync,
    and after janas_attn_forget the call stages the host cache again."""
    h, n_kv, hd, n_ctx = 8, 2, 128, 1024
    dt = np.int16 if kv16 else np.int8
    kvt = orc.KV_I16 if kv16 else orc.KV_I8
    k, ks, v, vs = imported_case(dt)
    q1 = normal(71, h * hd).reshape(1, h, hd)
    q64 = normal(73, 64 * h * hd).reshape(64, h, hd)
    with Attention(h, n_kv, hd, n_ctx, 1, janas_amd.FLOAT) as a:
        a.set_kv16(kv16)
        for arr in (k, ks, v, vs):
            assert a.import_host(arr) == 0
        assert a.import_host(k[1]) == 0          # inside an import: nothing new
        # a decode at 700 and a block at 900..963
        for q, n, pos0 in ((q1, 1, 700), (q64, 64, 900)):
            out = np.zeros_like(q)
            a.run(q, k, ks, v, vs, n, pos0, out)
            assert a.status() == 0
            ref_st = staged(h, n_kv, hd, n_ctx, kv16, False, q, k, ks, v, vs, n, pos0)
            assert np.array_equal(out.view(np.int32), ref_st.view(np.int32))
            ref = reference(q, k, ks, v, vs, kvt, pos0, h, n_kv, hd)
            assert within(abs_err(out, ref), TOL_FLOAT_ABS, f"imported n={n} vs oracle")
        # the engine writes the next block's rows 964..1003, then calls
        rng = np.random.default_rng(5)
        k[:, 964:1004] = rng.integers(-100, 100, (n_kv, 40, hd)).astype(dt)
        vs[:, 964:1004] *= np.float32(1.5)
        q40 = normal(79, 40 * h * hd).reshape(40, h, hd)
        out = np.zeros_like(q40)
        a.run(q40, k, ks, v, vs, 40, 964, out)
        ref_st = staged(h, n_kv, hd, n_ctx, kv16, False, q40, k, ks, v, vs, 40, 964)
        assert np.array_equal(out.view(np.int32), ref_st.view(np.int32))
        # a change before pos0 is the caller's to sync
        old = staged(h, n_kv, hd, n_ctx, kv16, False, q1, k, ks, v, vs, 1, 1003)
        k[:, 100:110] = -k[:, 100:110]
        new = staged(h, n_kv, hd, n_ctx, kv16, False, q1, k, ks, v, vs, 1, 1003)
        assert not np.array_equal(old, new)
        out = np.zeros_like(q1)
        a.run(q1, k, ks, v, vs, 1, 1003, out)
        assert np.array_equal(out.view(np.int32), old.view(np.int32))
        assert a.sync(k) == 0
        a.run(q1, k, ks, v, vs, 1, 1003, out)
        assert np.array_equal(out.view(np.int32), new.view(np.int32))
        # the device copy back to the host
        k_dev_view = k.copy()
        k[:] = 0
        assert a.sync(k, to_device=False) == 0
        assert np.array_equal(k, k_dev_view)
        # forgotten: staged again, so a host change is seen at once
        a.forget(k)
        k[:, 200:210] = -k[:, 200:210]
        after = staged(h, n_kv, hd, n_ctx, kv16, False, q1, k, ks, v, vs, 1, 1003)
        a.run(q1, k, ks, v, vs, 1, 1003, out)
        assert np.array_equal(out.view(np.int32), after.view(np.int32))
        assert a.status() == 0


def test_imported_ring_cache_takes_wrapped_rows(gpu):
    """A ring (position p in row p mod n_ctx, window 200): a block at
    positions 480..543 writes rows 480..511 and 0..31, and the call over the
    imported cache takes both runs from the host."""
    h, n_kv, hd, n_ctx, window = 8, 2, 128, 512, 200
    k, ks, v, vs = imported_case(np.int8, n_ctx=n_ctx, seed=91)
    q = normal(93, 64 * h * hd).reshape(64, h, hd)
    with Attention(h, n_kv, hd, n_ctx, 1, janas_amd.FLOAT) as a:
        a.set_ring(True)
        a.set_window(window)
        for arr in (k, ks, v, vs):
            assert a.import_host(arr) == 0
        rng = np.random.default_rng(9)
        for rows in (slice(480, 512), slice(0, 32)):
            k[:, rows] = rng.integers(-120, 120, (n_kv, 32, hd)).astype(np.int8)
            v[:, rows] = rng.integers(-120, 120, (n_kv, 32, hd)).astype(np.int8)
            ks[:, rows] *= np.float32(0.5)
        out = np.zeros_like(q)
        a.run(q, k, ks, v, vs, 64, 480, out)
        assert a.status() == 0
    ref = np.zeros_like(q)
    with Attention(h, n_kv, hd, n_ctx, 1, janas_amd.FLOAT) as b:
        b.set_ring(True)
        b.set_window(window)
        b.run(q, k, ks, v, vs, 64, 480, ref)
    assert np.array_equal(out.view(np.int32), ref.view(np.int32))


def test_import_refuses_partial_overlap(gpu):
    """An import that overlaps another in part is refused, one inside it is
    a no-op, a sync outside every import is refused."""
    h, n_kv, hd, n_ctx = 8, 2, 64, 256
    buf = np.zeros(4096, np.int8)
    with Attention(h, n_kv, hd, n_ctx, 1, janas_amd.FLOAT) as a:
        assert a.import_host(buf[1024:3072]) == 0
        assert a.import_host(buf[2048:4096]) == janas_amd.EINVAL
        assert a.import_host(buf[1024:2048]) == 0
        assert a.sync(buf[0:512]) == janas_amd.EINVAL
        assert a.sync(buf[1500:1600]) == 0
        a.forget(buf[1024:3072])
        assert a.sync(buf[1500:1600]) == janas_amd.EINVAL
        assert a.import_host(buf[2048:4096]) == 0
