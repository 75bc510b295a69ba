"""The CPU restatement of the cache-side rules (oracle/cache_oracle.c),
pinned before the GPU is compared with it:

* Q8_K (quant.c:150-200): bit for bit against the reference's own
  janas_q8k_quantize, compiled from its sources (oracle/_ref), and against
  the closed form of the block's fields;
* the cache write (model_attn.c:75-146): the quantization rule in closed
  form where no rotation or norm is applied, the NeoX rotation against
  float64 rotation matrices, the rms norm against float64, ring rows;
* the shift (model.c:263-377): rows move by `drop`, values and their scales
  unchanged, keys turned back by the float64 inverse rotation.

Each check is shown to fail on a planted mistake (a flipped rotation sign,
pairs (i, i+1) instead of (i, i+half), a dropped norm weight, a truncating
quantizer), planted in a copy of the oracle's output on the CPU.
"""
import numpy as np
import pytest

from oracle import orc

RNG = np.random.default_rng(20261201)


def rope_tables(positions, n_rot, base=10000.0):
    half = n_rot // 2
    inv = base ** (-2.0 * np.arange(half) / n_rot)
    ang = np.outer(np.asarray(positions, np.float64), inv)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


# ---- Q8_K -------------------------------------------------------------

def q8k_inputs():
    x = np.random.default_rng(7).standard_normal((6, 512)).astype(np.float32)
    x[1, :256] = 0.0                                  # an all-zero block
    x[2] *= 1e4                                       # large numbers
    x[3, 256:] = np.float32(127.0) * np.linspace(-1, 1, 256, dtype=np.float32)
    x[4, :256] = 0.5                                  # ties at x * id
    x[5, 7] = 1e-30                                   # a tiny one
    return x


def test_q8k_bitwise_equals_compiled_reference():
    try:
        ref = orc.ref_q8k_quantize(q8k_inputs())
    except FileNotFoundError:
        pytest.skip("reference not built in this container")
    assert orc.q8k_quantize(q8k_inputs()).tobytes() == ref.tobytes()


def q8k_closed_form_ok(x, y):
    """The block's fields from their definitions (quant.h:283-300)."""
    xb = x.reshape(-1, 256)
    yb = y.reshape(-1)
    for b in range(xb.shape[0]):
        amax = np.abs(xb[b]).max()
        d = np.float32(amax / np.float32(127.0))
        if yb[b]["d"] != d:
            return False
        if d > 0:
            q = np.rint(xb[b] * (np.float32(1.0) / d)).clip(-127, 127)
            if not np.array_equal(yb[b]["qs"], q.astype(np.int8)):
                return False
        if not np.array_equal(yb[b]["bsums"],
                              yb[b]["qs"].astype(np.int32).reshape(16, 16).sum(1)):
            return False
        if not np.array_equal(yb[b]["bsums2"],
                              yb[b]["bsums"].astype(np.int32).reshape(8, 2).sum(1)):
            return False
        for k in range(8):
            xs = xb[b, 32 * k:32 * k + 32]
            d32 = np.float32(np.abs(xs).max() / np.float32(127.0))
            if yb[b]["d32"][k] != d32:
                return False
    return True


def test_q8k_closed_form_and_planted_truncation():
    x = q8k_inputs()
    y = orc.q8k_quantize(x)
    assert q8k_closed_form_ok(x, y)
    bad = y.copy()
    xb = x.reshape(-1, 256)
    for b in range(bad.size):
        d = bad.reshape(-1)[b]["d"]
        if d > 0:   # truncation instead of rounding
            bad.reshape(-1)[b]["qs"] = np.trunc(xb[b] / d).clip(-127, 127)
    assert not q8k_closed_form_ok(x, bad)


# ---- the cache write -------------------------------------------------

def write(k, v, *, wide=False, cap=64, pos0=0, n_rot=None, k_norm=None,
          v_norm=False, ring=False, cs=None, sn=None):
    n, n_kv, hd = k.shape
    n_rot = hd if n_rot is None else n_rot
    if cs is None:
        cs, sn = rope_tables(range(pos0, pos0 + n), n_rot)
    dt = np.int16 if wide else np.int8
    kc = np.zeros((n_kv, cap, hd), dt)
    vc = np.zeros_like(kc)
    kz = np.zeros((n_kv, cap), np.float32)
    vz = np.zeros_like(kz)
    kk, vv = k.copy(), v.copy()
    orc.cache_write(kk, vv, cs=cs, sn=sn, n_rot=n_rot, pos0=pos0, kc=kc,
                    vc=vc, kz=kz, vz=vz, k_norm=k_norm, v_norm=v_norm,
                    ring=ring)
    return kc, vc, kz, vz


def test_quantization_closed_form_without_rotation():
    """cs = 1, sn = 0 and no norm: the row is only quantized, and the
    stored numbers are rint(x * 127 / max|x|) with scale max|x| / 127."""
    n, n_kv, hd = 3, 2, 64
    k = RNG.standard_normal((n, n_kv, hd)).astype(np.float32)
    v = RNG.standard_normal((n, n_kv, hd)).astype(np.float32)
    cs = np.ones((n, hd // 2), np.float32)
    sn = np.zeros((n, hd // 2), np.float32)
    for wide, top in ((False, 127.0), (True, 32767.0)):
        kc, vc, kz, vz = write(k, v, wide=wide, cs=cs, sn=sn, pos0=5)
        for j in range(n):
            for h in range(n_kv):
                for x, c, z in ((k, kc, kz), (v, vc, vz)):
                    row = x[j, h]
                    m = np.abs(row).max()
                    assert z[h, 5 + j] == np.float32(m / np.float32(top))
                    want = np.rint(row * np.float32(np.float32(top) / m))
                    assert np.array_equal(c[h, 5 + j], want.astype(c.dtype))


def rotation_ok(k, kc, kz, positions, n_rot, quanta=1.0):
    """Dequantized keys against the float64 NeoX rotation of k."""
    cs, sn = rope_tables(positions, n_rot)
    half = n_rot // 2
    for j in range(k.shape[0]):
        for h in range(k.shape[1]):
            x = k[j, h].astype(np.float64)
            want = x.copy()
            a, b = x[:half], x[half:n_rot]
            want[:half] = a * cs[j] - b * sn[j]
            want[half:n_rot] = a * sn[j] + b * cs[j]
            got = kc[h, positions[j]].astype(np.float64) * kz[h, positions[j]]
            if np.abs(got - want).max() > quanta * kz[h, positions[j]]:
                return False
    return True


def test_rotation_against_float64_and_planted_mistakes():
    n, n_kv, hd, n_rot = 4, 2, 128, 96
    k = RNG.standard_normal((n, n_kv, hd)).astype(np.float32)
    v = RNG.standard_normal((n, n_kv, hd)).astype(np.float32)
    pos = list(range(10, 10 + n))
    kc, vc, kz, vz = write(k, v, wide=True, pos0=10, n_rot=n_rot, cap=32)
    assert rotation_ok(k, kc, kz, pos, n_rot)
    # planted: the rotation turned the other way
    cs, sn = rope_tables(pos, n_rot)
    bad = write(k, v, wide=True, pos0=10, n_rot=n_rot, cap=32, cs=cs, sn=-sn)
    assert not rotation_ok(k, bad[0], bad[2], pos, n_rot)
    # planted: pairs (2i, 2i + 1) instead of (i, i + half)
    perm = np.arange(hd)
    perm[:n_rot] = np.concatenate([np.arange(0, n_rot, 2),
                                   np.arange(1, n_rot, 2)])
    kp = np.ascontiguousarray(k[:, :, perm])
    bad = write(kp, v, wide=True, pos0=10, n_rot=n_rot, cap=32)
    unperm = np.empty_like(bad[0])
    unperm[:, :, perm] = bad[0]
    assert not rotation_ok(k, unperm, bad[2], pos, n_rot)


def test_norm_against_float64_and_planted_dropped_weight():
    n, n_kv, hd = 2, 3, 64
    k = (3.0 * RNG.standard_normal((n, n_kv, hd))).astype(np.float32)
    v = (5.0 * RNG.standard_normal((n, n_kv, hd))).astype(np.float32)
    w = RNG.uniform(0.5, 1.5, hd).astype(np.float32)
    eps = 1e-6
    cs = np.ones((n, hd // 2), np.float32)
    sn = np.zeros((n, hd // 2), np.float32)

    def norm_ok(kc, kz, vc, vz, weight):
        for j in range(n):
            for h in range(n_kv):
                x = k[j, h].astype(np.float64)
                want = x / np.sqrt((x * x).mean() + eps) * weight
                got = kc[h, j] * np.float64(kz[h, j])
                if np.abs(got - want).max() > 1.0 * kz[h, j]:
                    return False
                y = v[j, h].astype(np.float64)
                wv = y / np.sqrt((y * y).mean() + eps)
                if np.abs(vc[h, j] * np.float64(vz[h, j]) - wv).max() > vz[h, j]:
                    return False
        return True

    got = write(k, v, wide=True, cs=cs, sn=sn, k_norm=w, v_norm=True)
    assert norm_ok(got[0], got[2], got[1], got[3], w)
    bad = write(k, v, wide=True, cs=cs, sn=sn, k_norm=np.ones(hd, np.float32),
                v_norm=True)
    assert not norm_ok(bad[0], bad[2], bad[1], bad[3], w)


def test_ring_rows():
    n, n_kv, hd, cap = 5, 1, 32, 256
    k = RNG.standard_normal((n, n_kv, hd)).astype(np.float32)
    v = RNG.standard_normal((n, n_kv, hd)).astype(np.float32)
    cs, sn = rope_tables(range(254, 259), hd)
    a = write(k, v, cap=cap, pos0=254, ring=True, cs=cs, sn=sn)
    rows = [(254 + j) % cap for j in range(n)]
    assert set(np.nonzero(a[2][0])[0]) == set(rows)


# ---- the shift -------------------------------------------------------

def filled_cache(n_kv, cap, hd, n_pos, wide, n_rot):
    k = RNG.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
    v = RNG.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
    kc, vc, kz, vz = write(k, v, wide=wide, cap=cap, n_rot=n_rot)
    return kc, vc, kz, vz


@pytest.mark.parametrize("wide", [False, True])
def test_shift_moves_rows_and_turns_keys_back(wide):
    n_kv, cap, hd, n_rot = 2, 64, 64, 64
    keep, drop, n_pos = 4, 7, 40
    kc, vc, kz, vz = filled_cache(n_kv, cap, hd, n_pos, wide, n_rot)
    k0, v0, kz0, vz0 = kc.copy(), vc.copy(), kz.copy(), vz.copy()
    cs, sn = rope_tables([drop], n_rot)
    orc.cache_shift(kc, vc, kz, vz, keep=keep, drop=drop, n_pos=n_pos,
                    cs=cs[0], sn=sn[0], n_rot=n_rot)
    move = n_pos - keep - drop
    # kept rows untouched, values and their scales moved as they are
    assert np.array_equal(kc[:, :keep], k0[:, :keep])
    assert np.array_equal(vc[:, keep:keep + move], v0[:, keep + drop:n_pos])
    assert np.array_equal(vz[:, keep:keep + move], vz0[:, keep + drop:n_pos])
    # keys: the old key rotated back by drop positions, in float64
    half = n_rot // 2
    c, s = cs[0].astype(np.float64), sn[0].astype(np.float64)
    for h in range(n_kv):
        for i in range(move):
            x = k0[h, keep + drop + i] * np.float64(kz0[h, keep + drop + i])
            want = x.copy()
            want[:half] = x[:half] * c + x[half:] * s
            want[half:] = x[half:] * c - x[:half] * s
            got = kc[h, keep + i] * np.float64(kz[h, keep + i])
            assert np.abs(got - want).max() <= kz[h, keep + i]


def test_shift_ring_keeps_the_last_positions():
    n_kv, cap, hd = 1, 256, 32
    n_pos, keep, drop = 300, 0, 20
    k = RNG.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
    v = RNG.standard_normal((n_pos, n_kv, hd)).astype(np.float32)
    kc, vc, kz, vz = write(k, v, cap=cap, ring=True, n_rot=0,
                           cs=np.zeros((n_pos, 0), np.float32),
                           sn=np.zeros((n_pos, 0), np.float32))
    v0 = vc.copy()
    orc.cache_shift(kc, vc, kz, vz, keep=keep, drop=drop, n_pos=n_pos,
                    cs=np.zeros(0, np.float32), sn=np.zeros(0, np.float32),
                    n_rot=0, ring=True)
    lo = max(keep + drop, n_pos - cap)
    for p in range(lo, n_pos):
        assert np.array_equal(vc[0, (p - drop) % cap], v0[0, p % cap])


def test_rotate_then_unrotate_is_identity_within_quanta():
    hd, n_rot = 128, 128
    row_f = RNG.standard_normal(hd).astype(np.float32)
    m = np.abs(row_f).max()
    row = np.rint(row_f * np.float32(32767 / m)).astype(np.int16)
    z = np.float32(m / 32767)
    cs, sn = rope_tables([9], n_rot)
    # turning "back" by -angle turns forward; then back again
    fwd = row.copy()
    z1 = orc.unrotate_row(fwd, z, cs[0], -sn[0])
    z2 = orc.unrotate_row(fwd, z1, cs[0], sn[0])
    assert np.abs(fwd * np.float64(z2) - row * np.float64(z)).max() <= 2 * z2


def q_prep_ok(q, got, w, cs, sn, n_rot, eps, tol=2e-6):
    """orc_q_prep against its closed form in float64: each (token, head)
    row rms-normalized with weights w (model_attn.c:93-94), then rotated in
    pairs (i, i + n_rot / 2) by the token's angles (model_attn.c:95-96,
    model_impl.h:635-644); within tol of the largest magnitude."""
    n, n_head, hd = q.shape
    half = n_rot // 2
    for j in range(n):
        for h in range(n_head):
            x = q[j, h].astype(np.float64)
            if w is not None:
                x = x / np.sqrt((x * x).mean() + eps) * w
            a, b = x[:half].copy(), x[half:n_rot].copy()
            x[:half] = a * cs[j] - b * sn[j]
            x[half:n_rot] = a * sn[j] + b * cs[j]
            if np.abs(got[j, h] - x).max() > tol * max(1.0, np.abs(x).max()):
                return False
    return True


def test_q_prep_against_float64_and_planted_mistakes():
    """The query side of qkv_item: norm, then rotation; the bound is a few
    float roundings. Planted mistakes - the rotation turned the other way,
    the norm's weights dropped, pairs (2i, 2i + 1) - are caught."""
    n, n_head, hd, n_rot, eps = 3, 4, 128, 96, 1e-6
    q = (2.0 * RNG.standard_normal((n, n_head, hd))).astype(np.float32)
    w = RNG.uniform(0.5, 1.5, hd).astype(np.float32)
    cs, sn = rope_tables(range(40, 40 + n), n_rot)

    def prep(x, **kw):
        x = np.ascontiguousarray(x.copy())
        orc.q_prep(x, **kw)
        return x

    got = prep(q, cs=cs, sn=sn, n_rot=n_rot, q_norm=w, eps=eps)
    assert q_prep_ok(q, got, w, cs, sn, n_rot, eps)
    # no norm: the rotation alone, and columns past n_rot untouched
    got = prep(q, cs=cs, sn=sn, n_rot=n_rot)
    assert q_prep_ok(q, got, None, cs, sn, n_rot, eps)
    assert np.array_equal(got[:, :, n_rot:], q[:, :, n_rot:])
    # planted mistakes
    bad = prep(q, cs=cs, sn=-sn, n_rot=n_rot, q_norm=w, eps=eps)
    assert not q_prep_ok(q, bad, w, cs, sn, n_rot, eps)
    bad = prep(q, cs=cs, sn=sn, n_rot=n_rot, q_norm=np.ones(hd, np.float32),
               eps=eps)
    assert not q_prep_ok(q, bad, w, cs, sn, n_rot, eps)
    perm = np.arange(hd)
    perm[:n_rot] = np.concatenate([np.arange(0, n_rot, 2),
                                   np.arange(1, n_rot, 2)])
    bad = prep(q[:, :, perm], cs=cs, sn=sn, n_rot=n_rot)
    unperm = np.empty_like(bad)
    unperm[:, :, perm] = bad
    assert not q_prep_ok(q, unperm, None, cs, sn, n_rot, eps)
