"""The C-ABI library on the CPU: it loads, exports every function its
header declares, and its host-only entry points keep the reference's
meaning (attention.c:984-992, :1048-1054). No GPU call is made."""
import ctypes

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

