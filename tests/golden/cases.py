"""Golden cases: the geometries, the inputs' generator and the calls.

The reference keeps no golden vectors for its attention (its unit test,
tests/test_attention.c, draws random data and compares against an in-test
double-precision softmax). These cases cover what that test covers -
chunk boundaries, GQA groups of 8, 4 and 3, a block against token-by-token
calls, sixteen-bit keys and values with a window and a score scale, spans
that see past their own position (set_last) - plus a ring cache and
decode-shaped calls, at sizes small enough to commit their outputs.

Inputs come from a counter-based generator (splitmix64 of seed and index), so
they are the same on every machine and cheap to rebuild; each fixture stores
a digest of them next to the reference's outputs.
"""
import hashlib

import numpy as np

KV_I8, KV_I16, KV_F16, KV_F32 = 0, 1, 2, 3

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix(seed, count):
    """count 64-bit words: splitmix64 of seed + i * golden gamma."""
    with np.errstate(over="ignore"):
        z = (np.uint64(seed) +
             np.arange(1, count + 1, dtype=np.uint64) *
             np.uint64(0x9E3779B97F4A7C15))
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed, count, lo, hi):
    """floats in [lo, hi) from 24 random bits, as test_attention.c:59-65."""
    u = (splitmix(seed, count) >> np.uint64(40)).astype(np.float32)
    u *= np.float32(1.0 / (1 << 24))
    return (np.float32(lo) + np.float32(hi - lo) * u).astype(np.float32)


def normal(seed, count):
    """N(0, 1) by Box-Muller over two uniform streams (float32)."""
    u1 = (splitmix(seed, count) >> np.uint64(11)).astype(np.float64)
    u2 = (splitmix(seed ^ 0x5DEECE66D, count) >> np.uint64(11)).astype(
        np.float64)
    u1 = (u1 + 0.5) * (1.0 / (1 << 53))
    u2 = u2 * (1.0 / (1 << 53))
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(
        np.float32)


# name: (n_head, n_kv, hd, n_ctx, pos0, n, kv, extra)
CASES = {
    # decode, one token, the first position
    "i8_16x2x128_p0_n1": dict(n_head=16, n_kv=2, hd=128, n_ctx=1, pos0=0,
                              n=1, kv=KV_I8),
    # a block from the start (test_attention.c:348), smaller heads
    "i8_4x2x64_p0_n64": dict(n_head=4, n_kv=2, hd=64, n_ctx=64, pos0=0, n=64,
                             kv=KV_I8),
    # across a chunk boundary, GQA 8 (test_attention.c:349)
    "i8_8x1x128_p250_n17": dict(n_head=8, n_kv=1, hd=128, n_ctx=267,
                                pos0=250, n=17, kv=KV_I8),
    # qwen3moe heads 32/4/128 at a decode step past two chunks
    "i8_32x4x128_p600_n1": dict(n_head=32, n_kv=4, hd=128, n_ctx=601,
                                pos0=600, n=1, kv=KV_I8),
    # three heads a group (test_attention.c:352)
    "i8_6x2x64_p511_n3": dict(n_head=6, n_kv=2, hd=64, n_ctx=514, pos0=511,
                              n=3, kv=KV_I8),
    # a window, no ring
    "i8_4x1x64_p600_n8_w300": dict(n_head=4, n_kv=1, hd=64, n_ctx=608,
                                   pos0=600, n=8, kv=KV_I8, window=300),
    # sixteen bits, window and ring, score scale 0.02 (test_attention.c:355)
    "i16_4x1x64_p1030_n5_w64_ring": dict(n_head=4, n_kv=1, hd=64, n_ctx=512,
                                         pos0=1030, n=5, kv=KV_I16, window=64,
                                         ring=True, scale=0.02),
    # Gemma 4's full layers: 16 bits, hd 512 (test_attention.c:356)
    "i16_2x1x512_p100_n3": dict(n_head=2, n_kv=1, hd=512, n_ctx=103,
                                pos0=100, n=3, kv=KV_I16, scale=0.02),
    # a span that sees past itself, across calls of 64 (test_attention.c:358)
    "i8_4x2x64_p200_n100_both": dict(n_head=4, n_kv=2, hd=64, n_ctx=300,
                                     pos0=200, n=100, kv=KV_I8,
                                     picture=(230, 290)),
    # the reference test's own geometry, 16/2/256, across a chunk boundary
    # (test_attention.c:347-350)
    "i8_16x2x256_p254_n5": dict(n_head=16, n_kv=2, hd=256, n_ctx=259,
                                pos0=254, n=5, kv=KV_I8),
    # head size 512 over an eight-bit cache
    "i8_2x1x512_p300_n3": dict(n_head=2, n_kv=1, hd=512, n_ctx=303,
                               pos0=300, n=3, kv=KV_I8),
    # unit scales and integer keys: the float element types' pin
    "i8unit_8x2x128_p300_n4": dict(n_head=8, n_kv=2, hd=128, n_ctx=304,
                                   pos0=300, n=4, kv=KV_I8, unit=True),
}


def make_inputs(name, seed=0x9E3779B97F4A7C15):
    """The case's q, k, ks, v, vs (and last) as the reference's test draws
    them: int8 keys and values from U(-127, 127) truncated, int16 from
    U(-32767, 32767), scales U(0.001, 0.02) (/258 for 16 bits), q U(-3, 3)
    (test_attention.c:108-117, :270-279)."""
    c = CASES[name]
    h, kvh, hd, cap, n = c["n_head"], c["n_kv"], c["hd"], c["n_ctx"], c["n"]
    base = int.from_bytes(hashlib.sha256(name.encode()).digest()[:8],
                          "little") ^ seed
    cells, rows = kvh * cap * hd, kvh * cap
    if c["kv"] == KV_I16:
        k = uniform(base + 1, cells, -32767, 32767).astype(np.int32).astype(
            np.int16)
        v = uniform(base + 2, cells, -32767, 32767).astype(np.int32).astype(
            np.int16)
        ks = uniform(base + 3, rows, 0.001, 0.02) / np.float32(258.0)
        vs = uniform(base + 4, rows, 0.001, 0.02) / np.float32(258.0)
    else:
        k = uniform(base + 1, cells, -127, 127).astype(np.int32).astype(
            np.int8)
        v = uniform(base + 2, cells, -127, 127).astype(np.int32).astype(
            np.int8)
        ks = uniform(base + 3, rows, 0.001, 0.02)
        vs = uniform(base + 4, rows, 0.001, 0.02)
    if c.get("unit"):
        ks = np.ones(rows, np.float32)
        vs = np.ones(rows, np.float32)
    q = uniform(base + 5, n * h * hd, -3, 3)
    if c.get("unit"):
        q = q * np.float32(0.02)  # scores of order one over 128 products
    last = None
    if "picture" in c:
        pic, pic_end = c["picture"]
        p = c["pos0"] + np.arange(n)
        last = np.where((p >= pic) & (p < pic_end), pic_end - 1, p).astype(
            np.uint32)
    return dict(q=q.reshape(n, h, hd).astype(np.float32),
                k=k.reshape(kvh, cap, hd), v=v.reshape(kvh, cap, hd),
                ks=ks.reshape(kvh, cap).astype(np.float32),
                vs=vs.reshape(kvh, cap).astype(np.float32), last=last)


def digest(inputs):
    h = hashlib.sha256()
    for key in ("q", "k", "ks", "v", "vs", "last"):
        a = inputs[key]
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def int16_case(name):
    """The reference's INT16 scores apply: an int8 cache, head size a
    multiple of 16 (attention.c:975-977, :1061-1066)."""
    c = CASES[name]
    return c["kv"] == KV_I8 and c["hd"] % 16 == 0


def call_kwargs(name):
    c = CASES[name]
    return dict(n_head=c["n_head"], n_kv=c["n_kv"], hd=c["hd"],
                pos0=c["pos0"], kv=c["kv"], scale=c.get("scale"),
                window=c.get("window", 0), ring=c.get("ring", False))
