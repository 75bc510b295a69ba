"""ctypes bindings of the CPU checker - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module. It wraps two shared libraries built by oracle/Makefile:

* ``liborc_attn.so``: this repo's C restatement of the reference attention
  (oracle/attn_oracle.c), generic over the cache's element type, and of the
  cache-side rules - cache write, shift, Q8_K (oracle/cache_oracle.c);
* ``_ref/libjanas_ref_attn.so``: the reference's own attention compiled from
  /root/reference/src/llm/attention.c and its few dependencies, driven through
  its public header (src/llm/attention.h:58-112). It is used to write the
  golden fixtures and to pin the restatement.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORC_LIB = os.path.join(HERE, "liborc_attn.so")
REF_LIB = os.path.join(HERE, "_ref", "libjanas_ref_attn.so")

KV_I8, KV_I16, KV_F16, KV_F32 = 0, 1, 2, 3
KV_DTYPE = {KV_I8: np.int8, KV_I16: np.int16, KV_F16: np.float16,
            KV_F32: np.float32}
CHUNK = 256

_u32 = ctypes.c_uint32
_vp = ctypes.c_void_p


class _Geom(ctypes.Structure):
    _fields_ = [("n_head", _u32), ("n_kv", _u32), ("hd", _u32),
                ("n_ctx", _u32), ("scale", ctypes.c_float),
                ("window", _u32), ("ring", ctypes.c_int), ("kv", ctypes.c_int),
                ("int16", ctypes.c_int)]


_orc = None


def orc():
    """The restatement's library; built on demand in this container."""
    global _orc
    if _orc is None:
        if not os.path.exists(ORC_LIB):
            raise FileNotFoundError(
                f"{ORC_LIB} missing: run `make -C oracle` (or build())")
        lib = ctypes.CDLL(ORC_LIB)
        lib.orc_attn_run.argtypes = [ctypes.POINTER(_Geom), _vp, _vp, _vp, _vp,
                                     _vp, _u32, _u32, _vp, _vp, ctypes.c_int]
        lib.orc_attn_run.restype = ctypes.c_int
        lib.orc_attn_exact.argtypes = [ctypes.POINTER(_Geom), _vp, _vp, _vp,
                                       _vp, _vp, _u32, _u32, _vp, _vp]
        lib.orc_attn_exact.restype = ctypes.c_int
        lib.orc_gate.argtypes = [_vp, ctypes.c_int, _u32, _u32, _u32, _vp]
        lib.orc_gate.restype = None
        lib.orc_exp_det.argtypes = [ctypes.c_float]
        lib.orc_exp_det.restype = ctypes.c_float
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f16_to_f32.restype = ctypes.c_float
        lib.orc_ring_positions.argtypes = [_u32, _u32]
        lib.orc_ring_positions.restype = _u32
        lib.orc_q8k_quantize.argtypes = [_vp, _vp, ctypes.c_size_t]
        lib.orc_q8k_quantize.restype = None
        lib.orc_cache_write.argtypes = [_vp, _vp, _vp, ctypes.c_float, _vp,
                                        _vp, _u32, ctypes.c_int, _u32, _u32,
                                        _u32, _u32, _u32, ctypes.c_int,
                                        ctypes.c_int, _vp, _vp, _vp, _vp]
        lib.orc_cache_write.restype = None
        lib.orc_q_prep.argtypes = [_vp, _vp, ctypes.c_float, _vp, _vp, _u32,
                                   _u32, _u32, _u32]
        lib.orc_q_prep.restype = None
        lib.orc_unrotate_row.argtypes = [_vp, _vp, _u32, _u32, _vp, _vp,
                                         ctypes.c_int]
        lib.orc_unrotate_row.restype = None
        lib.orc_cache_shift.argtypes = [_vp, _vp, _vp, _vp, _u32, _u32, _u32,
                                        ctypes.c_int, ctypes.c_int, _u32, _u32,
                                        _u32, _vp, _vp, _u32]
        lib.orc_cache_shift.restype = ctypes.c_int
        _orc = lib
    return _orc


def _ptr(a):
    return None if a is None else a.ctypes.data


def _geom(n_head, n_kv, hd, n_ctx, kv, scale=None, window=0, ring=False,
          int16=False):
    return _Geom(n_head, n_kv, hd, n_ctx,
                 1.0 / np.sqrt(np.float32(hd)) if scale is None else scale,
                 window, 1 if ring else 0, kv, 1 if int16 else 0)


def _check_inputs(q, k, v, ks, vs, kv):
    assert q.dtype == np.float32 and q.flags.c_contiguous
    assert k.dtype == KV_DTYPE[kv] and v.dtype == KV_DTYPE[kv]
    assert k.flags.c_contiguous and v.flags.c_contiguous
    if kv in (KV_I8, KV_I16):
        assert ks.dtype == np.float32 and vs.dtype == np.float32


def run(q, k, v, ks=None, vs=None, *, n_head, n_kv, hd, pos0, kv,
        scale=None, window=0, ring=False, last=None, threads=8, block=None,
        int16=False):
    """The restatement over n = q.shape[0] tokens from pos0. k, v are
    n_kv x n_ctx x hd. block: cut the call into pieces of that many tokens,
    as the engine does (model_attn.c:343-353); None runs it whole. int16:
    the reference's INT16 scores (int8 caches, hd a multiple of 16)."""
    _check_inputs(q, k, v, ks, vs, kv)
    n = q.shape[0]
    n_ctx = k.shape[1]
    g = _geom(n_head, n_kv, hd, n_ctx, kv, scale, window, ring, int16)
    out = np.zeros((n, n_head, hd), np.float32)
    last = None if last is None else np.ascontiguousarray(last, np.uint32)
    step = n if block is None else block
    for s in range(0, n, step):
        m = min(step, n - s)
        qs = np.ascontiguousarray(q[s:s + m])
        os_ = np.zeros((m, n_head, hd), np.float32)
        ls = None if last is None else np.ascontiguousarray(last[s:s + m])
        rc = orc().orc_attn_run(ctypes.byref(g), _ptr(qs), _ptr(k), _ptr(ks),
                                _ptr(v), _ptr(vs), m, pos0 + s, _ptr(ls),
                                _ptr(os_), threads)
        if rc != 0:
            raise ValueError("orc_attn_run rejected the call")
        out[s:s + m] = os_
    return out


def exact(q, k, v, ks=None, vs=None, *, n_head, n_kv, hd, pos0, kv,
          scale=None, window=0, ring=False, last=None):
    """The closed form in double precision."""
    _check_inputs(q, k, v, ks, vs, kv)
    n = q.shape[0]
    g = _geom(n_head, n_kv, hd, k.shape[1], kv, scale, window, ring)
    out = np.zeros((n, n_head, hd), np.float64)
    last = None if last is None else np.ascontiguousarray(last, np.uint32)
    rc = orc().orc_attn_exact(ctypes.byref(g), _ptr(q), _ptr(k), _ptr(ks),
                              _ptr(v), _ptr(vs), n, pos0, _ptr(last),
                              _ptr(out))
    if rc != 0:
        raise ValueError("orc_attn_exact rejected the call")
    return out


def gate(out, g, per_head=False):
    """out *= sigmoid(g), in place; returns out."""
    n, n_head, hd = out.shape
    g = np.ascontiguousarray(g, np.float32)
    orc().orc_gate(_ptr(g), 1 if per_head else 0, n, n_head, hd, _ptr(out))
    return out


def exp_det(x):
    return orc().orc_exp_det(float(x))


def ring_positions(window, n):
    return orc().orc_ring_positions(window, n)


# struct janas_block_q8k (src/llm/quant.h:283-300), 628 bytes
Q8K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16),
                ("d32", "<f4", 8), ("qs32", "i1", 256),
                ("bsums32", "<i2", 16), ("bsums2", "<i2", 8)])
assert Q8K.itemsize == 628


def q8k_quantize(x):
    """x (..., 256 m) float32 -> (..., m) Q8K blocks, the restatement of
    janas_q8k_quantize (quant.c:174-200)."""
    x = np.ascontiguousarray(x, np.float32)
    assert x.shape[-1] % 256 == 0
    y = np.zeros(x.shape[:-1] + (x.shape[-1] // 256,), Q8K)
    orc().orc_q8k_quantize(_ptr(x), _ptr(y), x.size)
    return y


def ref_q8k_quantize(x):
    """The reference's own janas_q8k_quantize (compiled quant.c)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(x.shape[:-1] + (x.shape[-1] // 256,), Q8K)
    lib = RefAttention.lib()
    lib.janas_q8k_quantize.argtypes = [_vp, _vp, ctypes.c_size_t]
    lib.janas_q8k_quantize.restype = None
    lib.janas_q8k_quantize(_ptr(x), _ptr(y), x.size)
    return y


def cache_write(k, v, *, cs, sn, n_rot, pos0, kc, vc, kz, vz, k_norm=None,
                eps=1e-6, v_norm=False, ring=False):
    """qkv_item's K/V part (model_attn.c:75-146): k, v (n, n_kv, hd) float32
    are normalized / turned in place and written at eight (kc int8) or
    sixteen (kc int16) bits into kc, vc (n_kv, cap, hd) and kz, vz
    (n_kv, cap)."""
    n, n_kv, hd = k.shape
    cap = kc.shape[1]
    wide = kc.dtype == np.int16
    assert k.dtype == np.float32 and v.dtype == np.float32
    assert k.flags.c_contiguous and v.flags.c_contiguous
    cs = np.ascontiguousarray(cs, np.float32)
    sn = np.ascontiguousarray(sn, np.float32)
    kn = None if k_norm is None else np.ascontiguousarray(k_norm, np.float32)
    orc().orc_cache_write(_ptr(k), _ptr(v), _ptr(kn), eps, _ptr(cs), _ptr(sn),
                          n_rot, 1 if v_norm else 0, n, n_kv, hd, pos0, cap,
                          1 if ring else 0, 1 if wide else 0, _ptr(kc),
                          _ptr(vc), _ptr(kz), _ptr(vz))


def q_prep(q, *, cs, sn, n_rot, q_norm=None, eps=1e-6):
    """The query side of qkv_item, in place on q (n, n_head, hd)."""
    n, n_head, hd = q.shape
    cs = np.ascontiguousarray(cs, np.float32)
    sn = np.ascontiguousarray(sn, np.float32)
    qn = None if q_norm is None else np.ascontiguousarray(q_norm, np.float32)
    orc().orc_q_prep(_ptr(q), _ptr(qn), eps, _ptr(cs), _ptr(sn), n_rot, n,
                     n_head, hd)


def unrotate_row(row, scale, cs, sn):
    """unrotate_row (model.c:263-290) on one int8 / int16 row in place;
    returns the new scale."""
    sc = np.array([scale], np.float32)
    cs = np.ascontiguousarray(cs, np.float32)
    sn = np.ascontiguousarray(sn, np.float32)
    orc().orc_unrotate_row(_ptr(row), _ptr(sc), row.shape[0], cs.shape[0],
                           _ptr(cs), _ptr(sn), 1 if row.dtype == np.int16 else 0)
    return float(sc[0])


def cache_shift(k, v, kz, vz, *, keep, drop, n_pos, cs, sn, n_rot,
                ring=False):
    """One slot of janas_llm_model_shift (model.c:304-377), in place."""
    n_kv, cap, hd = k.shape
    cs = np.ascontiguousarray(cs, np.float32)
    sn = np.ascontiguousarray(sn, np.float32)
    rc = orc().orc_cache_shift(_ptr(k), _ptr(v), _ptr(kz), _ptr(vz), n_kv,
                               hd, cap, 1 if ring else 0,
                               1 if k.dtype == np.int16 else 0, keep, drop,
                               n_pos, _ptr(cs), _ptr(sn), n_rot)
    if rc != 0:
        raise ValueError("orc_cache_shift rejected the call")


class RefAttention:
    """The reference's compiled attention through its own API:
    janas_attn_create / set_* / run (attention.h). scores: FLOAT (1, the
    exact path) or INT16 (2) - never AUTO, whose calibration times the host
    and writes under the home directory. The JANAS_ATTN environment variable
    overrides it in the reference (attention.c:965-974): callers clear it."""

    _lib = None

    @classmethod
    def lib(cls):
        if cls._lib is None:
            if not os.path.exists(REF_LIB):
                raise FileNotFoundError(f"{REF_LIB} missing")
            lib = ctypes.CDLL(REF_LIB)
            lib.janas_pool_create.argtypes = [ctypes.c_int, _vp]
            lib.janas_pool_create.restype = _vp
            lib.janas_pool_destroy.argtypes = [_vp]
            lib.janas_attn_create.argtypes = [_u32, _u32, _u32, _u32,
                                              ctypes.c_int, ctypes.c_int]
            lib.janas_attn_create.restype = _vp
            lib.janas_attn_destroy.argtypes = [_vp]
            lib.janas_attn_set_scale.argtypes = [_vp, ctypes.c_float]
            lib.janas_attn_set_window.argtypes = [_vp, _u32]
            lib.janas_attn_set_kv16.argtypes = [_vp, ctypes.c_int]
            lib.janas_attn_set_ring.argtypes = [_vp, ctypes.c_int]
            lib.janas_attn_set_last.argtypes = [_vp, _vp]
            lib.janas_attn_scores_mode.argtypes = [_vp]
            lib.janas_attn_scores_mode.restype = ctypes.c_int
            lib.janas_attn_part_bytes.argtypes = [_u32, _u32, _u32, _u32]
            lib.janas_attn_part_bytes.restype = ctypes.c_size_t
            lib.janas_attn_ring_positions.argtypes = [_u32, _u32]
            lib.janas_attn_ring_positions.restype = _u32
            lib.janas_attn_run.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                           _u32, _u32, _vp]
            lib.janas_attn_run.restype = None
            cls._lib = lib
        return cls._lib

    def __init__(self, n_head, n_kv, hd, n_ctx, threads=4, scores=1):
        if scores not in (1, 2):
            raise ValueError("FLOAT (1) or INT16 (2) only")
        lib = self.lib()
        self.pool = lib.janas_pool_create(threads, None)
        self.a = lib.janas_attn_create(n_head, n_kv, hd, n_ctx, threads,
                                       scores)
        if not self.pool or not self.a:
            raise RuntimeError("janas_attn_create failed")
        self.n_head, self.hd = n_head, hd

    def close(self):
        lib = self.lib()
        if self.a:
            lib.janas_attn_destroy(self.a)
        if self.pool:
            lib.janas_pool_destroy(self.pool)
        self.a = self.pool = None

    def run(self, q, k, ks, v, vs, pos0, last=None):
        n = q.shape[0]
        out = np.zeros((n, self.n_head, self.hd), np.float32)
        self._last = None
        if last is not None:
            self._last = np.ascontiguousarray(last, np.uint32)
            self.lib().janas_attn_set_last(self.a, _ptr(self._last))
        self.lib().janas_attn_run(self.a, self.pool, _ptr(q), _ptr(k),
                                  _ptr(ks), _ptr(v), _ptr(vs), n, pos0,
                                  _ptr(out))
        return out
