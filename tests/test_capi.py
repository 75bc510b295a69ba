"""The C-ABI library on the CPU: it loads, exports every function its
header declares, and its host-only entry points keep the reference's
meaning (attention.c:984-992, :1048-1054). No GPU call is made."""
import ctypes
import os
import subprocess

import pytest

import janas_amd
from janas_amd.attention import header_functions, lib
from oracle import orc


def test_library_exports_every_declared_function():
    names = header_functions()
    assert len(names) >= 12
    L = lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_reference_entry_points_all_declared():
    """The twelve entry points of src/llm/attention.h:58-112."""
    ref = {"janas_attn_part_bytes", "janas_attn_create", "janas_attn_destroy",
           "janas_attn_set_scale", "janas_attn_set_window",
           "janas_attn_set_kv16", "janas_attn_set_ring",
           "janas_attn_ring_positions", "janas_attn_set_last",
           "janas_attn_scores_mode", "janas_attn_scores_auto",
           "janas_attn_run"}
    assert ref <= set(header_functions())


@pytest.mark.parametrize("geom", [(32, 8, 128, 1024), (16, 2, 256, 32768),
                                  (12, 4, 64, 600), (16, 1, 512, 4096),
                                  (8, 0, 64, 100)])
def test_part_bytes_matches_reference_formula(geom):
    h, kv, d, n_ctx = geom
    if kv == 0:
        assert janas_amd.part_bytes(h, kv, d, n_ctx) == 0
        return
    chunks = (n_ctx + 255) // 256
    want = kv * chunks * 64 * (h // kv) * (d + 2) * 4
    assert janas_amd.part_bytes(h, kv, d, n_ctx) == want


def test_part_bytes_matches_compiled_reference():
    try:
        R = orc.RefAttention.lib()
    except FileNotFoundError:
        pytest.skip("reference not built here")
    for g in [(32, 8, 128, 1024), (16, 2, 256, 32768), (12, 4, 64, 600)]:
        assert janas_amd.part_bytes(*g) == R.janas_attn_part_bytes(*g)


@pytest.mark.parametrize("w,n", [(0, 1), (64, 5), (256, 64), (1000, 17),
                                 (4096, 1)])
def test_ring_positions(w, n):
    assert janas_amd.ring_positions(w, n) == orc.ring_positions(w, n)


def test_create_rejects_reference_bad_geometry_without_device_calls():
    """attention.c:998-1000: these are refused before any device call."""
    L = lib()
    for args in [(8, 0, 64, 100, 1, 0), (9, 2, 64, 100, 1, 0),
                 (8, 2, 60, 100, 1, 0), (8, 2, 520, 100, 1, 0),
                 (8, 2, 64, 100, 0, 0)]:
        assert not L.janas_attn_create(*args)


def test_strerror_covers_codes():
    for code in (0, -1, -2, -3, -4, -5):
        assert janas_amd.strerror(code)
    assert "unknown" in janas_amd.strerror(-99)


def test_scores_mode_is_float_without_instance():
    L = lib()
    assert L.janas_attn_scores_mode(None) == janas_amd.FLOAT
    assert L.janas_attn_scores_auto(None) == 0


def test_no_cpu_fallback_when_library_missing(monkeypatch, tmp_path):
    """The product path raises when the HIP library is absent."""
    import janas_amd.attention as at
    monkeypatch.setattr(at, "_lib", None)
    monkeypatch.setattr(at, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(ImportError):
        at.lib()


def test_status_of_no_instance_is_einval():
    """janas_attn_status(NULL) reports an argument error; clear and
    set_abort accept NULL (no device call)."""
    L = lib()
    assert L.janas_attn_status(None) == janas_amd.EINVAL
    L.janas_attn_clear_status(None)
    L.janas_attn_set_abort(None, 0)



REF_SRC = "/root/reference/src"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "llm", "attention.h")),
                    reason="the reference's sources are not here (only in the "
                           "build container)")
def test_reference_header_caller_links_unchanged(tmp_path):
    """A C caller written against the reference's own header
    (src/llm/attention.h, as model_attn.c includes it) compiles and links
    against libjanas_attn.so with no change, every one of the twelve entry
    points bound; run, it calls the two that need no device and checks
    them against the reference's formulas (attention.c:984-992,
    :1048-1054)."""
    src = tmp_path / "caller.c"
    src.write_text(r'''
#include <stdio.h>
#include "llm/attention.h"

/* every entry point model_attn.c and model_assist.c call, bound */
static void *bound[] = {
    (void *)janas_attn_part_bytes, (void *)janas_attn_create,
    (void *)janas_attn_destroy, (void *)janas_attn_set_scale,
    (void *)janas_attn_set_window, (void *)janas_attn_set_kv16,
    (void *)janas_attn_set_ring, (void *)janas_attn_ring_positions,
    (void *)janas_attn_set_last, (void *)janas_attn_scores_mode,
    (void *)janas_attn_scores_auto, (void *)janas_attn_run,
};

int main(void)
{
    for (unsigned i = 0; i < sizeof bound / sizeof bound[0]; i++)
        if (!bound[i])
            return 2;
    size_t pb = janas_attn_part_bytes(32, 8, 128, 1024);
    uint32_t rp = janas_attn_ring_positions(4096, 64);
    printf("%zu %u\n", pb, rp);
    return 0;
}
''')
    exe = tmp_path / "caller"
    libdir = os.path.dirname(janas_amd.attention.LIB_PATH)
    cmd = ["gcc", "-std=gnu11", "-O1", "-I", REF_SRC, "-I",
           os.path.join(os.path.dirname(REF_SRC), "include"), str(src),
           "-o", str(exe), "-L", libdir, "-ljanas_attn",
           f"-Wl,-rpath,{libdir}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    pb, rp = (int(x) for x in r.stdout.split())
    assert pb == 8 * 4 * janas_amd.MAX_BLOCK * 4 * 130 * 4
    assert rp == (4096 + 64 + 256 + 255) // 256 * 256


def test_import_entry_points_reject_null_without_a_device():
    """janas_attn_import / _sync refuse a null instance, pointer or size
    before any device call; janas_attn_forget of nothing is a no-op."""
    L = lib()
    buf = ctypes.create_string_buffer(64)
    addr = ctypes.addressof(buf)
    assert L.janas_attn_import(None, addr, 64) == janas_amd.EINVAL
    assert L.janas_attn_sync(None, addr, 64, 1) == janas_amd.EINVAL
    L.janas_attn_forget(None, addr)
