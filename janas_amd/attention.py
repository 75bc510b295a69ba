"""Python mirror of the engine's attention interface, over libjanas_attn.so.

``Attention`` follows the reference's C API (src/llm/attention.h:58-112)
name for name - create / set_scale / set_window / set_kv16 / set_ring /
set_last / scores_mode / scores_auto / run / destroy - and adds the device
extension of include/janas_attn.h (``run_dev``: f16 / f32 / int8 / int16
caches, several sequences, the fused gate, a stream).

Arrays may be numpy arrays (host memory: janas_attn_run stages them through
the device, as the C entry point does) or anything with ``data_ptr()``
(torch tensors on the GPU: used in place). There is no CPU path: without the
built library this module raises on import of the library.
"""
import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libjanas_attn.so")
HEADER = os.path.join(ROOT, "include", "janas_attn.h")

MAX_BLOCK = 64
AUTO, FLOAT, INT16 = 0, 1, 2
KV_I8, KV_I16, KV_F16, KV_F32 = 0, 1, 2, 3
GATE_NONE, GATE_ELEM, GATE_HEAD = 0, 1, 2
ERRORS = {0: "ok", -1: "EINVAL", -2: "ERANGE", -3: "ENOMEM", -4: "EDEVICE",
          -5: "ENOTSUP"}
OK, EINVAL, ERANGE, ENOMEM, EDEVICE, ENOTSUP = 0, -1, -2, -3, -4, -5

_u32 = ctypes.c_uint32
_vp = ctypes.c_void_p


class Seq(ctypes.Structure):
    """struct janas_attn_seq (include/janas_attn.h)."""
    _fields_ = [("k", _vp), ("v", _vp), ("ks", _vp), ("vs", _vp),
                ("q", _vp), ("out", _vp), ("gate", _vp), ("last", _vp),
                ("cap", _u32), ("n", _u32), ("pos0", _u32),
                ("last_max", _u32), ("out_q8k", _vp)]


class Cache(ctypes.Structure):
    """struct janas_attn_cache (include/janas_attn.h Part 3)."""
    _fields_ = [("k", _vp), ("v", _vp), ("ks", _vp), ("vs", _vp),
                ("n_kv", _u32), ("head_dim", _u32), ("cap", _u32),
                ("kv_type", ctypes.c_int), ("ring", ctypes.c_int)]


Q8K_BYTES = 628  # struct janas_attn_q8k


class AttnError(RuntimeError):
    def __init__(self, code, what):
        super().__init__(f"{what}: {ERRORS.get(code, code)}")
        self.code = code


_lib = None


def lib():
    """The C-ABI library, loaded once; raises if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with "
                          "`python -m janas_amd.build` (there is no CPU "
                          "fallback)")
    L = ctypes.CDLL(LIB_PATH)
    L.janas_attn_part_bytes.argtypes = [_u32, _u32, _u32, _u32]
    L.janas_attn_part_bytes.restype = ctypes.c_size_t
    L.janas_attn_create.argtypes = [_u32, _u32, _u32, _u32, ctypes.c_int,
                                    ctypes.c_int]
    L.janas_attn_create.restype = _vp
    L.janas_attn_destroy.argtypes = [_vp]
    L.janas_attn_destroy.restype = None
    L.janas_attn_set_scale.argtypes = [_vp, ctypes.c_float]
    L.janas_attn_set_window.argtypes = [_vp, _u32]
    L.janas_attn_set_kv16.argtypes = [_vp, ctypes.c_int]
    L.janas_attn_set_ring.argtypes = [_vp, ctypes.c_int]
    L.janas_attn_ring_positions.argtypes = [_u32, _u32]
    L.janas_attn_ring_positions.restype = _u32
    L.janas_attn_set_last.argtypes = [_vp, _vp]
    L.janas_attn_scores_mode.argtypes = [_vp]
    L.janas_attn_scores_mode.restype = ctypes.c_int
    L.janas_attn_scores_auto.argtypes = [_vp]
    L.janas_attn_scores_auto.restype = ctypes.c_int
    L.janas_attn_run.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32,
                                 _u32, _vp]
    L.janas_attn_run.restype = None
    for name in ("janas_attn_run_dev", "janas_attn_run_dev_split",
                 "janas_attn_run_dev_prefill", "janas_attn_run_dev_noalloc"):
        f = getattr(L, name)
        f.argtypes = [_vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(Seq),
                      _u32, _vp]
        f.restype = ctypes.c_int
    L.janas_attn_run_dev_kernels.argtypes = [_vp, ctypes.c_int, ctypes.c_int,
                                             ctypes.POINTER(Seq), _u32, _vp,
                                             ctypes.c_int]
    L.janas_attn_run_dev_kernels.restype = ctypes.c_int
    L.janas_attn_status.argtypes = [_vp]
    L.janas_attn_status.restype = ctypes.c_int
    L.janas_attn_clear_status.argtypes = [_vp]
    L.janas_attn_clear_status.restype = None
    L.janas_attn_set_abort.argtypes = [_vp, ctypes.c_int]
    L.janas_attn_set_abort.restype = None
    L.janas_attn_import.argtypes = [_vp, _vp, ctypes.c_size_t]
    L.janas_attn_import.restype = ctypes.c_int
    L.janas_attn_sync.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.c_int]
    L.janas_attn_sync.restype = ctypes.c_int
    L.janas_attn_forget.argtypes = [_vp, _vp]
    L.janas_attn_forget.restype = None
    L.janas_attn_strerror.argtypes = [ctypes.c_int]
    L.janas_attn_strerror.restype = ctypes.c_char_p
    L.janas_attn_cache_write.argtypes = [ctypes.POINTER(Cache), _vp, _vp,
                                         _vp, ctypes.c_float, _vp, _vp, _u32,
                                         ctypes.c_int, _u32, _u32, _vp]
    L.janas_attn_cache_write.restype = ctypes.c_int
    L.janas_attn_q_prep.argtypes = [_vp, _vp, ctypes.c_float, _vp, _vp, _u32,
                                    _u32, _u32, _u32, _vp]
    L.janas_attn_q_prep.restype = ctypes.c_int
    L.janas_attn_cache_shift.argtypes = [ctypes.POINTER(Cache), _u32, _u32,
                                         _u32, _vp, _vp, _u32, _vp]
    L.janas_attn_cache_shift.restype = ctypes.c_int
    L.janas_attn_cache_copy.argtypes = [ctypes.POINTER(Cache), _u32, _u32,
                                        _vp, _vp, _vp, _vp, ctypes.c_int, _vp]
    L.janas_attn_cache_copy.restype = ctypes.c_int
    L.janas_attn_prof_enable.argtypes = [_vp, ctypes.c_int]
    L.janas_attn_prof_read.argtypes = [_vp, ctypes.POINTER(_u32),
                                       ctypes.POINTER(ctypes.c_double)]
    L.janas_attn_prof_read.restype = ctypes.c_int
    _lib = L
    return L


def header_functions():
    """The function names include/janas_attn.h declares."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(janas_attn_\w+)\s*\(", text)))


def ptr(x):
    """Address of a numpy array, a torch tensor or an int; None for None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    return x.ctypes.data


def part_bytes(n_head, n_kv, head_dim, n_ctx):
    return lib().janas_attn_part_bytes(n_head, n_kv, head_dim, n_ctx)


def ring_positions(window, n):
    return lib().janas_attn_ring_positions(window, n)


def strerror(code):
    return lib().janas_attn_strerror(code).decode()


class Attention:
    """One attention instance: janas_attn_create(n_head, n_head_kv,
    head_dim, n_ctx, n_threads, scores)."""

    def __init__(self, n_head, n_kv, head_dim, n_ctx, threads=1,
                 scores=AUTO):
        self._a = lib().janas_attn_create(n_head, n_kv, head_dim, n_ctx,
                                          threads, scores)
        if not self._a:
            raise ValueError("janas_attn_create refused "
                             f"{n_head}/{n_kv}/{head_dim}/{n_ctx}")
        self.n_head, self.n_kv, self.hd, self.n_ctx = (n_head, n_kv,
                                                       head_dim, n_ctx)
        self._last = None

    def close(self):
        if self._a:
            lib().janas_attn_destroy(self._a)
            self._a = None

    destroy = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_scale(self, scale):
        lib().janas_attn_set_scale(self._a, scale)

    def set_window(self, window):
        lib().janas_attn_set_window(self._a, window)

    def set_kv16(self, on):
        lib().janas_attn_set_kv16(self._a, 1 if on else 0)

    def set_ring(self, on):
        lib().janas_attn_set_ring(self._a, 1 if on else 0)

    def set_last(self, last):
        """last: a host uint32 array kept alive until the next run."""
        self._last = last
        lib().janas_attn_set_last(self._a, ptr(last))

    def scores_mode(self):
        return lib().janas_attn_scores_mode(self._a)

    def scores_auto(self):
        return lib().janas_attn_scores_auto(self._a)

    def run(self, q, k, ks, v, vs, n, pos0, out):
        """janas_attn_run: synchronous; numpy (host) or device arrays."""
        lib().janas_attn_run(self._a, None, ptr(q), ptr(k), ptr(ks), ptr(v),
                             ptr(vs), n, pos0, ptr(out))
        self._last = None

    def status(self):
        """janas_attn_status: the first device failure kept, or 0."""
        return lib().janas_attn_status(self._a)

    def clear_status(self):
        lib().janas_attn_clear_status(self._a)

    def set_abort(self, on):
        """janas_attn_set_abort: whether janas_attn_run aborts on a
        failure (the default) or returns with a NaN output."""
        lib().janas_attn_set_abort(self._a, 1 if on else 0)

    def import_host(self, arr):
        """janas_attn_import of a host numpy array's bytes (the array
        must stay alive while imported): 0 or a JANAS_ATTN_E* code."""
        return lib().janas_attn_import(self._a, ptr(arr), arr.nbytes)

    def sync(self, arr, to_device=True):
        """janas_attn_sync of a host array (or a view into an imported
        one)."""
        return lib().janas_attn_sync(self._a, ptr(arr), arr.nbytes,
                                     1 if to_device else 0)

    def forget(self, arr):
        """janas_attn_forget of the import holding arr's first byte."""
        lib().janas_attn_forget(self._a, ptr(arr))

    def prepare(self, kv_type, seqs, gate_mode=GATE_NONE, stream=None,
                path="auto"):
        """The call janas_attn_run_dev would make, with its arguments built
        once: returns a function of no arguments that makes it (the arrays
        must stay alive). seqs: dicts with k, v, ks, vs, q, out, gate, last
        (device arrays or addresses), cap, n, pos0, last_max."""
        arr = (Seq * len(seqs))()
        for i, s in enumerate(seqs):
            arr[i] = Seq(ptr(s["k"]), ptr(s["v"]), ptr(s.get("ks")),
                         ptr(s.get("vs")), ptr(s["q"]), ptr(s["out"]),
                         ptr(s.get("gate")), ptr(s.get("last")), s["cap"],
                         s["n"], s["pos0"], s.get("last_max", 0),
                         ptr(s.get("out_q8k")))
        a, n, st = self._a, len(seqs), ptr(stream)
        if path in ("split-kernel", "merge-kernel"):
            # one kernel of the split path alone (measurement)
            kern = 1 if path == "split-kernel" else 2
            f = lib().janas_attn_run_dev_kernels

            def fn(a_, kv_, g_, arr_, n_, st_):
                return f(a_, kv_, g_, arr_, n_, st_, kern)
        else:
            fn = {"auto": lib().janas_attn_run_dev,
                  "split": lib().janas_attn_run_dev_split,
                  "prefill": lib().janas_attn_run_dev_prefill,
                  "noalloc": lib().janas_attn_run_dev_noalloc}[path]

        def call():
            rc = fn(a, kv_type, gate_mode, arr, n, st)
            if rc != 0:
                raise AttnError(rc, f"janas_attn_run_dev ({path})")
        call.keep = (arr, seqs)
        return call

    def run_dev(self, kv_type, seqs, gate_mode=GATE_NONE, stream=None,
                path="auto"):
        """janas_attn_run_dev over a list of sequences (see prepare)."""
        self.prepare(kv_type, seqs, gate_mode, stream, path)()

    def prof_enable(self, on=True):
        lib().janas_attn_prof_enable(self._a, 1 if on else 0)

    def prof_read(self):
        """{kernel: (launches, ms)} for split, merge and prefill."""
        counts = (_u32 * 3)()
        ms = (ctypes.c_double * 3)()
        rc = lib().janas_attn_prof_read(self._a, counts, ms)
        if rc != 0:
            raise AttnError(rc, "janas_attn_prof_read")
        return {name: (counts[i], ms[i])
                for i, name in enumerate(("split", "merge", "prefill"))}


# ---- Part 3: the cache around the attention --------------------------------

def _check(rc, what):
    if rc != 0:
        raise AttnError(rc, what)


def cache(k, v, ks=None, vs=None, *, kv_type, ring=False):
    """struct janas_attn_cache over device tensors k, v (n_kv, cap, hd) and
    ks, vs (n_kv, cap)."""
    n_kv, cap, hd = k.shape
    return Cache(ptr(k), ptr(v), ptr(ks), ptr(vs), n_kv, hd, cap, kv_type,
                 1 if ring else 0)


def cache_write(c, k, v, *, cs, sn, n_rot, pos0, k_norm=None, eps=1e-6,
                v_norm=False, stream=None):
    """janas_attn_cache_write: k, v (n, n_kv, hd) device floats."""
    _check(lib().janas_attn_cache_write(ctypes.byref(c), ptr(k), ptr(v),
                                        ptr(k_norm), eps, ptr(cs), ptr(sn),
                                        n_rot, 1 if v_norm else 0, pos0,
                                        k.shape[0], ptr(stream)),
           "janas_attn_cache_write")


def q_prep(q, *, cs, sn, n_rot, q_norm=None, eps=1e-6, stream=None):
    """janas_attn_q_prep on q (n, n_head, hd), in place."""
    n, n_head, hd = q.shape
    _check(lib().janas_attn_q_prep(ptr(q), ptr(q_norm), eps, ptr(cs), ptr(sn),
                                   n_rot, n, n_head, hd, ptr(stream)),
           "janas_attn_q_prep")


def cache_shift(c, *, keep, drop, n_pos, cs, sn, n_rot, stream=None):
    """janas_attn_cache_shift."""
    _check(lib().janas_attn_cache_shift(ctypes.byref(c), keep, drop, n_pos,
                                        ptr(cs), ptr(sn), n_rot, ptr(stream)),
           "janas_attn_cache_shift")


def cache_copy(c, *, n_pos, rows, k, v, ks=None, vs=None, out=True,
               stream=None):
    """janas_attn_cache_copy: out=True cache -> buffers, else back."""
    _check(lib().janas_attn_cache_copy(ctypes.byref(c), n_pos, rows, ptr(k),
                                       ptr(v), ptr(ks), ptr(vs),
                                       1 if out else 0, ptr(stream)),
           "janas_attn_cache_copy")
