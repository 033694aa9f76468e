"""C-ABI checks that need no GPU: the library loads, exports every function the
public headers declare, and rejects invalid arguments with the documented
codes before touching the device."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent

WHA_ERR_INVALID, WHA_ERR_UNSUPPORTED, WHA_ERR_WORKSPACE = -1, -2, -4

# Several checks below pass made-up device addresses (1 << 20, 0x100000) that
# validation must reject before any launch.  On a machine with a visible GPU a
# validation regression would launch a kernel on an unmapped address, so those
# checks run only where no GPU device node exists.
no_device = pytest.mark.skipif(Path("/dev/kfd").exists(),
                               reason="passes made-up device pointers; runs only where no GPU is visible")


def declared_functions():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(wha_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_expected_entry_points(pkg):
    names = declared_functions()
    assert set(pkg.EXPORTED_SYMBOLS) == names


def test_library_exports_every_declared_symbol(pkg):
    L = pkg.lib()
    for name in declared_functions():
        assert hasattr(L, name), name


def test_version(pkg):
    assert "gfx950" in pkg.version()


def _layout(pkg, B=1, H=2, T=16, D=64):
    return pkg.layout_bhtd(B, H, T, D)


def _call_fwd(pkg, layout, scale=0.125, ptr=1 << 20):
    p = ctypes.c_void_p(ptr)
    return pkg.lib().wha_attn_fwd(p, p, p, p, None, ctypes.byref(layout) if layout is not None else None,
                                  scale, None)


@no_device
def test_invalid_layouts_are_rejected(pkg):
    L = pkg.lib()
    assert _call_fwd(pkg, None) == WHA_ERR_INVALID
    assert b"layout is NULL" in L.wha_last_error()
    for bad in (dict(B=0), dict(H=-1), dict(T=0), dict(D=0)):
        assert _call_fwd(pkg, _layout(pkg, **bad)) == WHA_ERR_INVALID
        assert b"must be positive" in L.wha_last_error()
    assert _call_fwd(pkg, _layout(pkg, D=129)) == WHA_ERR_UNSUPPORTED
    assert b"128" in L.wha_last_error()
    lay = _layout(pkg)
    lay.stride_t = 32  # < D
    assert _call_fwd(pkg, lay) == WHA_ERR_INVALID
    assert b"strides" in L.wha_last_error()


@no_device
def test_invalid_scale_and_null_pointers_are_rejected(pkg):
    L = pkg.lib()
    lay = _layout(pkg)
    for s in (0.0, -1.0, float("inf"), float("nan")):
        assert _call_fwd(pkg, lay, scale=s) == WHA_ERR_INVALID
        assert b"scale" in L.wha_last_error()
    assert _call_fwd(pkg, lay, ptr=0) == WHA_ERR_INVALID
    assert b"non-NULL" in L.wha_last_error()
    null = ctypes.c_void_p(0)
    rc = L.wha_attn_bwd(*([null] * 9), None, 0, ctypes.byref(lay), 0.125, None)
    assert rc == WHA_ERR_INVALID
    rc = L.wha_attn_bwd_from_probs(*([null] * 8), None, 0, ctypes.byref(lay), 0.125, None)
    assert rc == WHA_ERR_INVALID
    rc = L.wha_decode_fwd(*([null] * 5), None, 0, ctypes.byref(lay), 0.125, None)
    assert rc == WHA_ERR_INVALID


def test_workspace_sizes(pkg):
    L = pkg.lib()
    lay = pkg.layout_bhtd(8, 12, 1024, 64)
    n = L.wha_attn_bwd_workspace_size(ctypes.byref(lay))
    assert n >= 8 * 12 * 1024 * 4 and n % 256 == 0
    assert L.wha_attn_bwd_from_probs_workspace_size(ctypes.byref(lay)) >= 8 * 12 * 1024 * 4
    dec = pkg.layout_bhtd(64, 12, 8192, 64)
    assert L.wha_decode_workspace_size(ctypes.byref(dec)) > 0
    bad = pkg.layout_bhtd(0, 1, 1, 1)
    assert L.wha_attn_bwd_workspace_size(ctypes.byref(bad)) == 0


def test_host_entry_points_validate_before_device_use(pkg):
    L = pkg.lib()
    f = np.zeros(64, dtype=np.float32)
    fp = f.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    assert L.wha_host_attention_core_fwd(fp, fp, fp, 4, 10, 3, fp) == WHA_ERR_INVALID   # 10 % 3 != 0
    assert b"divisible" in L.wha_last_error()
    assert L.wha_host_attention_core_fwd(fp, fp, fp, 0, 8, 2, fp) == WHA_ERR_INVALID
    assert L.wha_host_attention_backward(fp, fp, fp, fp, fp, 4, 8, 0, fp, fp, fp) == WHA_ERR_INVALID


def test_backend_mirror_checks_shapes(pkg):
    be = pkg.HipBackend()
    q = np.zeros((4, 8), np.float32)
    with pytest.raises(ValueError):
        be.attention_backward(q, q, q, q, np.zeros((3, 4, 4), np.float32), 2)  # att heads != n_head
    with pytest.raises(ValueError):
        be.attention_core(q[0], q, q, 2)
    with pytest.raises(RuntimeError):
        be.attention_core(q, q, q, 3)  # 8 % 3 != 0, rejected by the C ABI as a panic would


def test_padded_dims_cover_the_configs():
    # head_dim of the BASELINE configs: 42, 48, 64, 128 (all <= 128)
    src = (ROOT / "wave-engine_amd" / "csrc" / "wha_launch.hpp").read_text()
    assert "D <= 128" in src


@no_device
def test_probs_rows_validates_rows(pkg):
    L = pkg.lib()
    lay = pkg.layout_bhtd(1, 2, 16, 64)
    p = ctypes.c_void_p(1 << 20)
    rows = (ctypes.c_int32 * 2)(3, 16)  # 16 is outside [0, 16)
    assert L.wha_attn_probs_rows(p, p, p, rows, 2, p, ctypes.byref(lay), 0.125, None) == WHA_ERR_INVALID
    assert b"outside" in L.wha_last_error()
    assert L.wha_attn_probs_rows(p, p, p, rows, 0, p, ctypes.byref(lay), 0.125, None) == WHA_ERR_INVALID
    assert L.wha_attn_probs_rows(p, p, p, rows, 257, p, ctypes.byref(lay), 0.125, None) == WHA_ERR_INVALID


def test_head_stats_follow_the_monitor_definitions(pkg):
    """analyze_attention (src/monitors/attn_monitor.rs:26-80) on hand-made rows."""
    rows = np.array([[0.25, 0.25, 0.5, 0.0], [0.0, 0.0, 0.0, 1.0], [0.4, 0.2, 0.4, 0.0]], np.float32)
    st = pkg.attention_head_stats(rows)
    ent0 = -(0.25 * np.log(0.25) * 2 + 0.5 * np.log(0.5))
    np.testing.assert_allclose(st["entropy"], [ent0, 0.0, -(2 * 0.4 * np.log(0.4) + 0.2 * np.log(0.2))], rtol=1e-6)
    np.testing.assert_array_equal(st["top_position"], [2, 3, 0])   # first maximum wins ties
    np.testing.assert_allclose(st["max_weight"], [0.5, 1.0, 0.4])
    np.testing.assert_allclose(st["self_attn_frac"], [0.0, 1.0, 0.0])


def _wave_structs(pkg, B=1, T=8, E=64, H=2, C=16):
    p = 1 << 20
    w = pkg._WaveWeightsC(*([p] * 7))
    cache = pkg._WaveCacheC(*([p] * 7))
    return pkg.WaveShape(B, T, E, H, C), w, cache


@no_device
def test_wave_entry_points_validate_before_device_use(pkg):
    L = pkg.lib()
    p = ctypes.c_void_p(1 << 20)
    sh, w, cache = _wave_structs(pkg)
    for bad, msg in ((dict(E=63), b"divisible"), (dict(C=31), b"content_dim"), (dict(E=258, H=1), b"128"),
                     (dict(E=258, H=129), b"n_head"), (dict(T=0), b"positive")):
        s2, _, _ = _wave_structs(pkg, **bad)
        rc = L.wha_wave_fwd(p, ctypes.byref(w), ctypes.byref(s2), p, ctypes.byref(cache), None, 0, None)
        assert rc in (WHA_ERR_INVALID, WHA_ERR_UNSUPPORTED) and msg in L.wha_last_error(), L.wha_last_error()
    nw = pkg._WaveWeightsC(*([1 << 20] * 6 + [None]))
    assert L.wha_wave_fwd(p, ctypes.byref(nw), ctypes.byref(sh), p, ctypes.byref(cache), None, 0,
                          None) == WHA_ERR_INVALID
    nc = pkg._WaveCacheC(*([1 << 20] * 6 + [None]))
    assert L.wha_wave_fwd(p, ctypes.byref(w), ctypes.byref(sh), p, ctypes.byref(nc), None, 0,
                          None) == WHA_ERR_INVALID
    # the bucket-sparse family (default from T = 1024) needs its workspace; a
    # short one is refused before anything is enqueued
    big, _, _ = _wave_structs(pkg, B=2, T=1024, E=768, H=12)
    need = L.wha_wave_fwd_workspace_size(ctypes.byref(big))
    assert need > 0
    rc = L.wha_wave_fwd(p, ctypes.byref(w), ctypes.byref(big), p, ctypes.byref(cache), p, need - 16, None)
    assert rc == WHA_ERR_WORKSPACE and b"workspace" in L.wha_last_error(), L.wha_last_error()
    # shapes that only take the all-pairs family need none
    assert L.wha_wave_fwd_workspace_size(ctypes.byref(sh)) >= 0
    some = pkg._WaveGradsC(1 << 20, 1 << 20, None, None, None, None, None, None)  # neither all nor none
    rc = L.wha_wave_bwd(p, p, ctypes.byref(w), ctypes.byref(sh), ctypes.byref(cache), ctypes.byref(some), None, 0,
                        None)
    assert rc == WHA_ERR_INVALID and b"all non-NULL or all NULL" in L.wha_last_error()
    rows = (ctypes.c_int32 * 1)(8)
    assert L.wha_wave_probs_rows(ctypes.byref(cache), ctypes.byref(sh), rows, 1, p, None) == WHA_ERR_INVALID


def test_wave_kernel_family_switch(pkg):
    """wha_wave_set_bucket_sparse: modes 0..2 (default 2, automatic), anything
    else rejected with -1 and the mode unchanged; the backward workspace covers
    the sparse family's score-gradient blocks (one [T16][64] block per 64
    sorted keys) and sorted operands whatever the mode."""
    L = pkg.lib()
    prev = L.wha_wave_set_bucket_sparse(2)
    try:
        assert prev in (0, 1, 2)
        assert L.wha_wave_set_bucket_sparse(7) == -1 and L.wha_wave_set_bucket_sparse(-1) == -1
        assert L.wha_wave_set_bucket_sparse(0) == 2
        assert L.wha_wave_set_bucket_sparse(1) == 0
        assert L.wha_wave_set_bucket_sparse(2) == 1
        assert pkg.wave_set_bucket_sparse("auto") == 2 and pkg.wave_set_bucket_sparse(False) == 2
        with pytest.raises(ValueError):
            pkg.wave_set_bucket_sparse(5)
    finally:
        L.wha_wave_set_bucket_sparse(prev)
    B, T, E, H, C = 8, 1024, 768, 12, 16
    sh = pkg.WaveShape(B, T, E, H, C)
    n = L.wha_wave_bwd_workspace_size(ctypes.byref(sh))
    sparse_ds = B * H * (T // 64) * T * 64 * 4
    assert n > sparse_ds + B * T * E * 4 * 2


@no_device
def test_wave_kv_entry_points_validate(pkg):
    L = pkg.lib()
    p = ctypes.c_void_p(1 << 20)
    sh, w, _ = _wave_structs(pkg, B=2, T=1)
    kv = pkg._WaveKvC(1 << 20, 1 << 20, 1 << 20, 1 << 20, 16)
    lens = (ctypes.c_int32 * 2)(3, 16)  # 16 leaves no room to append
    assert L.wha_wave_kv_decode(p, ctypes.byref(w), ctypes.byref(sh), ctypes.byref(kv), lens, p, None, 0,
                                None) == WHA_ERR_INVALID
    assert b"lengths[1]" in L.wha_last_error()
    sh2, _, _ = _wave_structs(pkg, B=2, T=4)
    lens = (ctypes.c_int32 * 2)(3, 4)
    assert L.wha_wave_kv_decode(p, ctypes.byref(w), ctypes.byref(sh2), ctypes.byref(kv), lens, p, None, 0,
                                None) == WHA_ERR_INVALID
    assert b"T must be 1" in L.wha_last_error()
    big, _, _ = _wave_structs(pkg, B=300, T=1)
    lens = (ctypes.c_int32 * 300)()
    assert L.wha_wave_kv_decode(p, ctypes.byref(w), ctypes.byref(big), ctypes.byref(kv), lens, p, None, 0,
                                None) == WHA_ERR_UNSUPPORTED
    long_prompt, _, _ = _wave_structs(pkg, B=1, T=17)
    assert L.wha_wave_kv_prefill(p, ctypes.byref(w), ctypes.byref(long_prompt), ctypes.byref(kv), p, None, 0,
                                 None) == WHA_ERR_INVALID
    assert b"capacity" in L.wha_last_error()
    assert L.wha_wave_kv_decode_workspace_size(ctypes.byref(sh), 0) == 0


@no_device
def test_scores_size_and_kept_pair_validation(pkg):
    """wha_attn_scores_size: the causal half in 64-key column blocks (rows
    64kt..Tp-1 of block kt) for the covered layouts, 0 elsewhere; the kept pair
    rejects a missing or misaligned scores buffer before touching the device."""
    L = pkg.lib()
    B, H, T = 8, 12, 1024
    rows = sum(T - 64 * kt for kt in range(T // 64))
    assert L.wha_attn_scores_size(ctypes.byref(pkg.layout_bhtd(B, H, T, 64))) == B * H * rows * 64 * 4
    assert L.wha_attn_scores_size(ctypes.byref(pkg.layout_seq(B, T, 12, 768))) == B * H * rows * 64 * 4
    for D in (100, 128, 52, 48, 44, 36):
        assert L.wha_attn_scores_size(ctypes.byref(pkg.layout_bhtd(8, 16, 100, D))) > 0
        # small problems (fewer than 256 tiles of 64 rows, T <= 1024) run the split-sweep kernels: nothing kept
        assert L.wha_attn_scores_size(ctypes.byref(pkg.layout_bhtd(2, 2, 100, D))) == 0
    assert L.wha_attn_scores_size(ctypes.byref(pkg.layout_bhtd(1, 2, 2048, 64))) > 0
    for D in (32, 42, 16, 50):
        assert L.wha_attn_scores_size(ctypes.byref(pkg.layout_bhtd(8, 16, 100, D))) == 0
    odd = pkg.layout_bhtd(8, 16, 100, 64)
    odd.stride_t = 66
    assert L.wha_attn_scores_size(ctypes.byref(odd)) == 0
    assert L.wha_attn_scores_size(ctypes.byref(pkg.layout_bhtd(0, 1, 1, 64))) == 0

    lay = pkg.layout_bhtd(8, 16, 128, 64)   # 256 tiles of 64 rows: not a small problem, scores are kept
    p = ctypes.c_void_p(0x100000)
    rc = L.wha_attn_fwd_keep(p, p, p, p, p, None, ctypes.byref(lay), 0.125, None)
    assert rc == WHA_ERR_INVALID and b"scores" in L.wha_last_error()
    rc = L.wha_attn_fwd_keep(p, p, p, p, p, ctypes.c_void_p(0x100004), ctypes.byref(lay), 0.125, None)
    assert rc == WHA_ERR_INVALID and b"aligned" in L.wha_last_error()
    rc = L.wha_attn_bwd_kept(*([p] * 6), ctypes.c_void_p(0x100004), p, p, p, None, 0, ctypes.byref(lay), 0.125,
                             None)
    assert rc == WHA_ERR_INVALID and b"aligned" in L.wha_last_error()
    rc = L.wha_attn_bwd_kept(*([p] * 6), None, p, p, p, None, 0, ctypes.byref(lay), 0.125, None)
    assert rc == WHA_ERR_INVALID and b"scores" in L.wha_last_error()
    null = ctypes.c_void_p(0)
    rc = L.wha_attn_bwd_kept(*([null] * 10), None, 0, ctypes.byref(lay), 0.125, None)
    assert rc == WHA_ERR_INVALID and b"non-NULL" in L.wha_last_error()


@no_device
def test_overlapping_strides_are_rejected(pkg):
    """One layout describes the outputs too, so rows of distinct (b,h,t) must
    not overlap: zero or too-small head/batch strides are rejected, the
    [B,H,T,D], [B][T][H*D] and fused [B][T][3E] column-slice layouts pass."""
    L = pkg.lib()
    B, H, T, D = 2, 3, 16, 64
    E = H * D
    for sb, sh, st in ((H * T * D, 0, D), (0, T * D, D), (H * T * D, D, D), (T * D, T * D, D),
                       (H * T * D, T * D - 1, D), (T * 3 * E, D // 2, 3 * E)):
        lay = pkg.layout_bhtd(B, H, T, D)
        lay.stride_b, lay.stride_h, lay.stride_t = sb, sh, st
        assert _call_fwd(pkg, lay) == WHA_ERR_INVALID, (sb, sh, st)
        assert b"overlap" in L.wha_last_error()
    # the accepted layouts fail later, at the NULL pointer check, not at the strides
    for sb, sh, st in ((H * T * D, T * D, D), (T * E, D, E), (T * 3 * E, D, 3 * E)):
        lay = pkg.layout_bhtd(B, H, T, D)
        lay.stride_b, lay.stride_h, lay.stride_t = sb, sh, st
        assert _call_fwd(pkg, lay, ptr=0) == WHA_ERR_INVALID
        assert b"non-NULL" in L.wha_last_error(), L.wha_last_error()
    # extent-1 dimensions may have any stride (a single head or sequence)
    lay = pkg.layout_bhtd(1, 1, T, D)
    lay.stride_b, lay.stride_h = 0, 0
    assert _call_fwd(pkg, lay, ptr=0) == WHA_ERR_INVALID and b"non-NULL" in L.wha_last_error()


def test_plan_keeps_scores_only_for_aligned_tensors():
    """AttnPlan chooses the kept-scores pair only when every tensor is 16-byte
    aligned; the C ABI runs the recompute pair for unaligned ones, so both
    sides agree (source check: the plan tests data_ptr() % 16)."""
    src = (ROOT / "wave-engine_amd" / "__init__.py").read_text()
    assert "data_ptr() % 16 == 0" in src
    api = (ROOT / "wave-engine_amd" / "csrc" / "wha_api.hip").read_text()
    assert api.count("wha_attn_scores_size(layout) > 0 && vec") == 2


def test_noalloc_decode_rejects_layouts_beyond_its_scratch(pkg):
    """wha_decode_fwd_noalloc checks the split-K scratch size (16 MiB static
    array) before the pointers, so NULL pointers with a too-large layout get
    WHA_ERR_WORKSPACE and nothing reaches the device."""
    L = pkg.lib()
    WHA_ERR_WORKSPACE = -4
    null = ctypes.c_void_p(0)
    big = pkg.layout_bhtd(64, 12, 1 << 17, 64)             # 768 (b,h) x 128 splits x 66 floats
    assert L.wha_decode_workspace_size(ctypes.byref(big)) > 16 << 20
    rc = L.wha_decode_fwd_noalloc(null, null, null, null, None, ctypes.byref(big), 0.125, None)
    assert rc == WHA_ERR_WORKSPACE and b"static" in L.wha_last_error(), L.wha_last_error()
    fits = pkg.layout_bhtd(64, 12, 8192, 64)               # the decode config: 1.6 MB of partials
    assert L.wha_decode_workspace_size(ctypes.byref(fits)) <= 16 << 20
    rc = L.wha_decode_fwd_noalloc(null, null, null, null, None, ctypes.byref(fits), 0.125, None)
    assert rc == WHA_ERR_INVALID and b"non-NULL" in L.wha_last_error()
