"""wave-engine_amd: MI355X (gfx950) causal attention tier for wave-engine.

Python host side of the C ABI declared in ``include/wave_hip_attn.h`` and
implemented by ``libwave_hip_attn.so`` (built in-tree by ``Makefile``).  It binds
the library with ctypes and hands it device pointers and the current HIP stream
of torch tensors -- torch is only the allocator and stream provider here; every
FLOP runs in the hand-written HIP kernels under ``csrc/``.  There is no CPU or
torch fallback: if the library is missing or the device is not a GPU, calls
raise.

Two levels mirror the reference interface:

* ``HipBackend`` -- the two attention methods of wave-engine's
  ``ComputeBackend`` trait (``src/common/compute.rs:42-43``, ``:163-173``), projections
  included, with the
  reference's per-sequence ``[T][n_embd]`` layout and host arrays, raising
  ``RuntimeError`` where the reference panics.
* ``attn_fwd`` / ``attn_bwd`` / ``attn_bwd_from_probs`` / ``decode_fwd`` -- batched
  device entry points on torch tensors in any strided ``[B,H,T,D]`` view.

The directory name contains a hyphen, so it is loaded by path (see
``__graft_entry__.load_package``) under the module name ``wave_engine_amd``.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libwave_hip_attn.so"

# C-ABI symbols declared in include/wave_hip_attn.h
EXPORTED_SYMBOLS = (
    "wha_last_error", "wha_version",
    "wha_attn_fwd", "wha_attn_bwd_workspace_size", "wha_attn_bwd",
    "wha_attn_bwd_from_probs_workspace_size", "wha_attn_bwd_from_probs",
    "wha_attn_scores_size", "wha_attn_fwd_keep", "wha_attn_bwd_kept",
    "wha_decode_workspace_size", "wha_decode_fwd", "wha_decode_fwd_noalloc", "wha_attn_probs_rows",
    "wha_wave_fwd_workspace_size", "wha_wave_fwd", "wha_wave_bwd_workspace_size", "wha_wave_bwd", "wha_wave_probs_rows",
    "wha_wave_set_bucket_sparse",
    "wha_wave_kv_prefill_workspace_size", "wha_wave_kv_prefill", "wha_wave_kv_decode_workspace_size",
    "wha_wave_kv_decode", "wha_host_wave_attention_forward", "wha_host_wave_attention_backward",
    "wha_linear_fwd", "wha_linear_bwd_dx", "wha_linear_bwd_dw_workspace_size", "wha_linear_bwd_dw",
    "wha_host_attention_core_fwd", "wha_host_attention_backward", "wha_host_attention",
    "wha_synth_normal",
    "wha_timing_enable", "wha_timing_reset", "wha_timing_read",
)

WHA_OK = 0


class WaveLayout(ctypes.Structure):
    """wha_layout: element (b,h,t,d) at b*stride_b + h*stride_h + t*stride_t + d."""
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("T", ctypes.c_int32),
                ("D", ctypes.c_int32), ("stride_b", ctypes.c_int64),
                ("stride_h", ctypes.c_int64), ("stride_t", ctypes.c_int64)]

    def __repr__(self):
        return (f"WaveLayout(B={self.B}, H={self.H}, T={self.T}, D={self.D}, "
                f"strides=({self.stride_b}, {self.stride_h}, {self.stride_t}))")


class WaveShape(ctypes.Structure):
    """wha_wave_shape."""
    _fields_ = [("B", ctypes.c_int32), ("T", ctypes.c_int32), ("n_embd", ctypes.c_int32),
                ("n_head", ctypes.c_int32), ("content_dim", ctypes.c_int32)]


class _WaveWeightsC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("harmonic_raw", "proj_w", "proj_b", "v_w", "v_b", "out_w", "out_b")]


class _WaveCacheC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("proj", "values", "feat", "phase", "bucket", "merged", "lse")]


class _WaveGradsC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("d_x", "d_harmonic_raw", "d_proj_w", "d_proj_b", "d_v_w", "d_v_b",
                                                "d_out_w", "d_out_b")]


class _WaveKvC(ctypes.Structure):
    _fields_ = [("cs", ctypes.c_void_p), ("bucket", ctypes.c_void_p), ("phase", ctypes.c_void_p),
                ("values", ctypes.c_void_p), ("capacity", ctypes.c_int32)]


def layout_bhtd(B, H, T, D) -> WaveLayout:
    """Contiguous [B,H,T,D]."""
    return WaveLayout(B, H, T, D, H * T * D, T * D, D)


def layout_seq(B, T, n_head, n_embd) -> WaveLayout:
    """Reference per-sequence layout [T][n_embd] batched as [B][T][n_embd]."""
    D = n_embd // n_head
    return WaveLayout(B, n_head, T, D, T * n_embd, D, n_embd)


def build() -> None:
    """Compile libwave_hip_attn.so for gfx950 with the package Makefile."""
    subprocess.run(["make", "-s", "-C", str(PKG_DIR), "-j8"], check=True)


_lib = None


def lib():
    """The loaded C library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               f"or `make -C {PKG_DIR}`; there is no fallback path")
        # torch bundles its own HIP runtime under the same soname
        # (libamdhip64.so.7).  Load it first so that this library binds to the
        # runtime torch allocates with; loading /opt/rocm's copy first leaves
        # torch unable to see the device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(str(LIB_PATH))
        vp, f32p, lp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(WaveLayout)
        sz, i32 = ctypes.c_size_t, ctypes.c_int32
        L.wha_last_error.restype = ctypes.c_char_p
        L.wha_version.restype = ctypes.c_char_p
        L.wha_attn_fwd.argtypes = [vp, vp, vp, vp, vp, lp, ctypes.c_float, vp]
        L.wha_attn_bwd_workspace_size.argtypes = [lp]
        L.wha_attn_bwd_workspace_size.restype = sz
        L.wha_attn_bwd.argtypes = [vp] * 9 + [vp, sz, lp, ctypes.c_float, vp]
        L.wha_attn_bwd_from_probs_workspace_size.argtypes = [lp]
        L.wha_attn_bwd_from_probs_workspace_size.restype = sz
        L.wha_attn_bwd_from_probs.argtypes = [vp] * 8 + [vp, sz, lp, ctypes.c_float, vp]
        L.wha_attn_scores_size.argtypes = [lp]
        L.wha_attn_scores_size.restype = sz
        L.wha_attn_fwd_keep.argtypes = [vp] * 6 + [lp, ctypes.c_float, vp]
        L.wha_attn_bwd_kept.argtypes = [vp] * 10 + [vp, sz, lp, ctypes.c_float, vp]
        L.wha_decode_workspace_size.argtypes = [lp]
        L.wha_decode_workspace_size.restype = sz
        L.wha_decode_fwd.argtypes = [vp] * 5 + [vp, sz, lp, ctypes.c_float, vp]
        L.wha_decode_fwd_noalloc.argtypes = [vp] * 5 + [lp, ctypes.c_float, vp]
        i64 = ctypes.c_int64
        L.wha_linear_fwd.argtypes = [vp, i64, vp, vp, vp, i64, i64, i32, i32, vp]
        L.wha_linear_bwd_dx.argtypes = [vp, i64, vp, vp, i64, i64, i32, i32, vp]
        L.wha_linear_bwd_dw_workspace_size.argtypes = [i64, i32, i32]
        L.wha_linear_bwd_dw_workspace_size.restype = sz
        L.wha_linear_bwd_dw.argtypes = [vp, i64, vp, i64, vp, vp, i64, i32, i32, vp, sz, vp]
        L.wha_host_attention.argtypes = [f32p] * 5 + [i32, i32, i32, f32p]
        L.wha_host_attention_core_fwd.argtypes = [f32p, f32p, f32p, i32, i32, i32, f32p]
        L.wha_host_attention_backward.argtypes = [f32p] * 5 + [i32, i32, i32] + [f32p] * 3
        L.wha_attn_probs_rows.argtypes = [vp, vp, vp, ctypes.POINTER(ctypes.c_int32), i32, vp, lp, ctypes.c_float, vp]
        wsp, wwp = ctypes.POINTER(WaveShape), ctypes.POINTER(_WaveWeightsC)
        wcp, wgp = ctypes.POINTER(_WaveCacheC), ctypes.POINTER(_WaveGradsC)
        L.wha_wave_fwd_workspace_size.argtypes = [wsp]
        L.wha_wave_fwd_workspace_size.restype = sz
        L.wha_wave_fwd.argtypes = [vp, wwp, wsp, vp, wcp, vp, sz, vp]
        L.wha_wave_bwd_workspace_size.argtypes = [wsp]
        L.wha_wave_bwd_workspace_size.restype = sz
        L.wha_wave_bwd.argtypes = [vp, vp, wwp, wsp, wcp, wgp, vp, sz, vp]
        L.wha_wave_probs_rows.argtypes = [wcp, wsp, ctypes.POINTER(ctypes.c_int32), i32, vp, vp]
        L.wha_wave_set_bucket_sparse.argtypes = [ctypes.c_int]
        L.wha_host_wave_attention_forward.argtypes = [f32p, wwp, i32, i32, i32, i32, f32p, vp]
        L.wha_host_wave_attention_backward.argtypes = [f32p, f32p, wwp, i32, i32, i32, i32, wgp]
        kvp = ctypes.POINTER(_WaveKvC)
        L.wha_wave_kv_prefill_workspace_size.argtypes = [wsp]
        L.wha_wave_kv_prefill_workspace_size.restype = sz
        L.wha_wave_kv_prefill.argtypes = [vp, wwp, wsp, kvp, vp, vp, sz, vp]
        L.wha_wave_kv_decode_workspace_size.argtypes = [wsp, i32]
        L.wha_wave_kv_decode_workspace_size.restype = sz
        L.wha_wave_kv_decode.argtypes = [vp, wwp, wsp, kvp, ctypes.POINTER(ctypes.c_int32), vp, vp, sz, vp]
        L.wha_synth_normal.argtypes = [ctypes.POINTER(ctypes.c_uint64), f32p, sz, ctypes.c_double, ctypes.c_int]
        L.wha_synth_normal.restype = ctypes.c_int
        L.wha_timing_enable.argtypes = [ctypes.c_int]
        L.wha_timing_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_int64)]
        for name in EXPORTED_SYMBOLS:
            if name not in ("wha_last_error", "wha_version") and not name.endswith("_size"):
                getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


class WaveHipError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed with code {code}: {msg}")
        self.code = code


def _check(fn, rc):
    if rc != WHA_OK:
        raise WaveHipError(fn, rc, lib().wha_last_error().decode())


def version() -> str:
    return lib().wha_version().decode()


# ------------------------------------------------------------------ torch plumbing

def _torch():
    import torch
    return torch


def _stream_ptr(t):
    torch = _torch()
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def layout_of(t) -> WaveLayout:
    """Layout of a 4-D [B,H,T,D] float32 cuda tensor view (unit stride on D)."""
    torch = _torch()
    if t.dim() != 4:
        raise ValueError(f"expected a 4-D [B,H,T,D] tensor, got shape {tuple(t.shape)}")
    if t.dtype != torch.float32:
        raise TypeError(f"expected float32, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError("expected a device (cuda/hip) tensor")
    if t.stride(3) != 1 and t.shape[3] > 1:
        raise ValueError("the head dimension must have unit stride")
    B, H, T, D = t.shape
    return WaveLayout(B, H, T, D, t.stride(0), t.stride(1), t.stride(2))


def _same_layout(L, *ts):
    for t in ts:
        l2 = layout_of(t)
        if (l2.B, l2.H, l2.T, l2.D, l2.stride_b, l2.stride_h, l2.stride_t) != \
                (L.B, L.H, L.T, L.D, L.stride_b, L.stride_h, L.stride_t):
            raise ValueError(f"all tensors must share one layout: {L} vs {l2}")


def default_scale(D: int) -> float:
    """1/sqrt(head_dim) rounded to f32, as src/common/compute.rs:362 computes it."""
    return float(np.float32(1.0) / np.sqrt(np.float32(D)))


def attn_scores_bytes(L: WaveLayout) -> int:
    """Bytes of the scores buffer a training forward keeps for its backward
    (wha_attn_scores_size; 0 where the layout's kernels cannot keep them)."""
    return int(lib().wha_attn_scores_size(ctypes.byref(L)))


def attn_scores_buffer(L: WaveLayout, device):
    """A scores buffer for attn_fwd(..., scores=) / attn_bwd(..., scores=), or
    None where attn_scores_bytes(L) is 0 (nothing to keep)."""
    n = attn_scores_bytes(L)
    return _torch().empty(n // 4, dtype=_torch().float32, device=device) if n else None


def attn_fwd(q, k, v, scale=None, want_lse=True, out=None, lse=None, scores=None):
    """Fused causal forward on [B,H,T,D] views.  Returns (o, lse) with lse
    [B,H,T] (natural-log row log-sum-exp), or o alone when want_lse=False.
    scores (attn_scores_buffer): also keep the raw scores for attn_bwd(...,
    scores=) (wha_attn_fwd_keep)."""
    torch = _torch()
    L = layout_of(q)
    _same_layout(L, k, v)
    if out is None:
        out = torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=q.device)
    _same_layout(L, out)
    if want_lse and lse is None:
        lse = torch.empty((L.B, L.H, L.T), dtype=torch.float32, device=q.device)
    s = default_scale(L.D) if scale is None else float(scale)
    if scores is not None:
        _check("wha_attn_fwd_keep", lib().wha_attn_fwd_keep(_ptr(q), _ptr(k), _ptr(v), _ptr(out),
                                                            _ptr(lse) if want_lse else None, _ptr(scores),
                                                            ctypes.byref(L), s, _stream_ptr(q)))
    else:
        _check("wha_attn_fwd", lib().wha_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(out),
                                                  _ptr(lse) if want_lse else None,
                                                  ctypes.byref(L), s, _stream_ptr(q)))
    return (out, lse) if want_lse else out


def attn_bwd(q, k, v, o, do, lse, scale=None, workspace=None, dq=None, dk=None, dv=None, scores=None):
    """Fused causal backward (P recomputed from lse; with scores, from the
    scores attn_fwd kept: wha_attn_bwd_kept).  Returns (dq, dk, dv)."""
    torch = _torch()
    L = layout_of(q)
    _same_layout(L, k, v, o, do)
    dq = torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=q.device) if dq is None else dq
    dk = torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=q.device) if dk is None else dk
    dv = torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=q.device) if dv is None else dv
    _same_layout(L, dq, dk, dv)
    s = default_scale(L.D) if scale is None else float(scale)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    if scores is not None:
        _check("wha_attn_bwd_kept", lib().wha_attn_bwd_kept(
            _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(do), _ptr(lse.contiguous()), _ptr(scores), _ptr(dq),
            _ptr(dk), _ptr(dv), _ptr(workspace), ws_bytes, ctypes.byref(L), s, _stream_ptr(q)))
    else:
        _check("wha_attn_bwd", lib().wha_attn_bwd(
            _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(do), _ptr(lse.contiguous()), _ptr(dq), _ptr(dk), _ptr(dv),
            _ptr(workspace), ws_bytes, ctypes.byref(L), s, _stream_ptr(q)))
    return dq, dk, dv


def attn_probs_rows(q, k, lse, rows, scale=None):
    """Rows of P recomputed from q, k and the forward's lse: returns [B,H,len(rows),T]
    with out[b,h,r,j] = softmax row rows[r] (zeros past the causal limit)."""
    torch = _torch()
    L = layout_of(q)
    _same_layout(L, k)
    rows = [int(r) for r in rows]
    arr = (ctypes.c_int32 * len(rows))(*rows)
    out = torch.empty((L.B, L.H, len(rows), L.T), dtype=torch.float32, device=q.device)
    s = default_scale(L.D) if scale is None else float(scale)
    _check("wha_attn_probs_rows", lib().wha_attn_probs_rows(_ptr(q), _ptr(k), _ptr(lse.contiguous()), arr, len(rows),
                                                            _ptr(out), ctypes.byref(L), s, _stream_ptr(q)))
    return out


def attention_head_stats(last_rows):
    """Per-head statistics of attention rows, as analyze_attention computes them
    for the last position (src/monitors/attn_monitor.rs:26-80): for each row
    (..., T) holding position t = T-1's weights, entropy = sum(-p ln p) over p > 0,
    the first maximum weight and its position, and the self-attention weight p[t].
    Returns a dict of numpy arrays shaped like last_rows without the last axis."""
    p = np.asarray(last_rows, dtype=np.float32)
    pos = p.shape[-1] - 1
    with np.errstate(divide="ignore", invalid="ignore"):
        ent = np.where(p > 0, -p * np.log(p), 0.0).astype(np.float32).sum(-1)
    top = p.argmax(-1)
    mx = np.take_along_axis(p, top[..., None], -1)[..., 0]
    mx = np.maximum(mx, 0.0)
    return {"entropy": ent, "max_weight": mx, "top_position": top, "self_attn_frac": p[..., pos]}


def attn_bwd_workspace_bytes(L: WaveLayout) -> int:
    return int(lib().wha_attn_bwd_workspace_size(ctypes.byref(L)))


def attn_bwd_from_probs(do, q, k, v, att, scale=None, workspace=None):
    """Backward with att [B,H,T,T] used as given (the reference contract)."""
    torch = _torch()
    L = layout_of(q)
    _same_layout(L, k, v, do)
    if tuple(att.shape) != (L.B, L.H, L.T, L.T) or not att.is_contiguous():
        raise ValueError(f"att must be a contiguous [B,H,T,T] tensor, got {tuple(att.shape)}")
    dq, dk, dv = (torch.empty_strided(q.shape, q.stride(), dtype=q.dtype, device=q.device) for _ in range(3))
    s = default_scale(L.D) if scale is None else float(scale)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("wha_attn_bwd_from_probs", lib().wha_attn_bwd_from_probs(
        _ptr(do), _ptr(q), _ptr(k), _ptr(v), _ptr(att), _ptr(dq), _ptr(dk), _ptr(dv),
        _ptr(workspace), ws_bytes, ctypes.byref(L), s, _stream_ptr(q)))
    return dq, dk, dv


def decode_fwd(q, k_cache, v_cache, scale=None, want_lse=False, workspace=None):
    """Single-token decode: q [B,H,D] against a [B,H,Tk,D] cache view."""
    torch = _torch()
    L = layout_of(k_cache)
    _same_layout(L, v_cache)
    if tuple(q.shape) != (L.B, L.H, L.D) or not q.is_contiguous():
        raise ValueError(f"q must be a contiguous [B,H,D] tensor, got {tuple(q.shape)}")
    o = torch.empty_like(q)
    lse = torch.empty((L.B, L.H), dtype=torch.float32, device=q.device) if want_lse else None
    s = default_scale(L.D) if scale is None else float(scale)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("wha_decode_fwd", lib().wha_decode_fwd(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(o), _ptr(lse) if want_lse else None,
        _ptr(workspace), ws_bytes, ctypes.byref(L), s, _stream_ptr(q)))
    return (o, lse) if want_lse else o


def decode_fwd_noalloc(q, k_cache, v_cache, scale=None, want_lse=False, out=None, lse=None):
    """decode_fwd through wha_decode_fwd_noalloc: the split-K partials live in
    the library's static device scratch (no allocation inside the call; calls
    that overlap on one GPU race).  out / lse may be preallocated."""
    torch = _torch()
    L = layout_of(k_cache)
    _same_layout(L, v_cache)
    if tuple(q.shape) != (L.B, L.H, L.D) or not q.is_contiguous():
        raise ValueError(f"q must be a contiguous [B,H,D] tensor, got {tuple(q.shape)}")
    o = torch.empty_like(q) if out is None else out
    if want_lse and lse is None:
        lse = torch.empty((L.B, L.H), dtype=torch.float32, device=q.device)
    s = default_scale(L.D) if scale is None else float(scale)
    _check("wha_decode_fwd_noalloc", lib().wha_decode_fwd_noalloc(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(o), _ptr(lse) if want_lse else None,
        ctypes.byref(L), s, _stream_ptr(q)))
    return (o, lse) if want_lse else o


def _rows_of(t, name):
    """(rows, row stride) of a 2-D float32 device tensor with unit column stride."""
    torch = _torch()
    if t.dim() != 2 or t.dtype != torch.float32 or not t.is_cuda:
        raise ValueError(f"{name}: expected a 2-D float32 device tensor, got {tuple(t.shape)} {t.dtype}")
    if t.stride(1) != 1 and t.shape[1] > 1:
        raise ValueError(f"{name}: columns must be contiguous")
    return t.shape[0], t.stride(0)


def linear_fwd(x, w, b=None, out=None):
    """y[m] = b + W x[m] for the rows of x [M][K] (w [N][K] contiguous, b [N] or None)."""
    torch = _torch()
    M, ldx = _rows_of(x, "x")
    N, K = w.shape
    if not w.is_contiguous() or x.shape[1] != K:
        raise ValueError("w must be a contiguous [N][K] tensor matching x's columns")
    y = torch.empty((M, N), dtype=torch.float32, device=x.device) if out is None else out
    _, ldy = _rows_of(y, "out")
    _check("wha_linear_fwd", lib().wha_linear_fwd(_ptr(x), ldx, _ptr(w), _ptr(b) if b is not None else None,
                                                  _ptr(y), ldy, M, N, K, _stream_ptr(x)))
    return y


def linear_bwd_dx(dy, w, out=None):
    """dx[m] = W^T dy[m] (linear_backward_dx_batch)."""
    torch = _torch()
    M, lddy = _rows_of(dy, "dy")
    N, K = w.shape
    dx = torch.empty((M, K), dtype=torch.float32, device=dy.device) if out is None else out
    _, lddx = _rows_of(dx, "out")
    _check("wha_linear_bwd_dx", lib().wha_linear_bwd_dx(_ptr(dy), lddy, _ptr(w), _ptr(dx), lddx, M, N, K,
                                                        _stream_ptr(dy)))
    return dx


def linear_bwd_dw(dy, x, compute_bias=True, workspace=None):
    """(d_w [N][K], d_b [N] or None) = outer_product_accum(dy, x, compute_bias)."""
    torch = _torch()
    M, lddy = _rows_of(dy, "dy")
    M2, ldx = _rows_of(x, "x")
    if M2 != M:
        raise ValueError("dy and x must have the same number of rows")
    N, K = dy.shape[1], x.shape[1]
    dw = torch.empty((N, K), dtype=torch.float32, device=dy.device)
    db = torch.empty(N, dtype=torch.float32, device=dy.device) if compute_bias else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check("wha_linear_bwd_dw", lib().wha_linear_bwd_dw(
        _ptr(dy), lddy, _ptr(x), ldx, _ptr(dw), _ptr(db) if db is not None else None, M, N, K,
        _ptr(workspace), ws_bytes, _stream_ptr(dy)))
    return dw, db


class AttnPlan:
    """Launches bound once to a fixed set of [B,H,T,D] tensors: layouts, pointers,
    scale, workspace and stream are validated and marshalled at construction, so
    fwd() and bwd() are one C call each (for training loops and benchmarks where
    per-call Python checks would cost as much as the kernels).  A plan with
    backward tensors keeps the forward's scores for its backward
    (wha_attn_fwd_keep / wha_attn_bwd_kept) unless keep_scores=False."""

    def __init__(self, q, k, v, o, lse, do=None, dq=None, dk=None, dv=None, workspace=None, scale=None,
                 keep_scores=True):
        torch = _torch()
        L = layout_of(q)
        _same_layout(L, k, v, o)
        if tuple(lse.shape) != (L.B, L.H, L.T) or not lse.is_contiguous():
            raise ValueError("lse must be a contiguous [B,H,T] tensor")
        self.layout = L
        self._keep = [q, k, v, o, lse, do, dq, dk, dv, workspace]
        s = ctypes.c_float(default_scale(L.D) if scale is None else float(scale))
        st = _stream_ptr(q)
        self._fwd_args = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), ctypes.byref(L), s, st)
        self._bwd_args = None
        self._f = lib().wha_attn_fwd
        self._b = lib().wha_attn_bwd
        self._fname, self._bname = "wha_attn_fwd", "wha_attn_bwd"
        # the kept pair needs 16-byte-aligned tensors (the C ABI otherwise runs the recompute pair)
        aligned = do is not None and all(t.data_ptr() % 16 == 0 for t in (q, k, v, o, do, dq, dk, dv))
        scores = attn_scores_buffer(L, q.device) if (aligned and keep_scores) else None
        if do is not None:
            _same_layout(L, do, dq, dk, dv)
            need = attn_bwd_workspace_bytes(L)
            if workspace is None:
                workspace = torch.empty(need // 4, dtype=torch.float32, device=q.device)
                self._keep.append(workspace)
            ws_bytes = workspace.numel() * workspace.element_size()
            self._bwd_args = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(do), _ptr(lse), _ptr(dq), _ptr(dk),
                              _ptr(dv), _ptr(workspace), ctypes.c_size_t(ws_bytes), ctypes.byref(L), s, st)
        if scores is not None:
            self._keep.append(scores)
            a = self._fwd_args
            self._fwd_args = a[:5] + (_ptr(scores),) + a[5:]
            a = self._bwd_args
            self._bwd_args = a[:6] + (_ptr(scores),) + a[6:]
            self._f, self._b = lib().wha_attn_fwd_keep, lib().wha_attn_bwd_kept
            self._fname, self._bname = "wha_attn_fwd_keep", "wha_attn_bwd_kept"
        self.keeps_scores = scores is not None

    def fwd(self):
        rc = self._f(*self._fwd_args)
        if rc:
            _check(self._fname, rc)

    def bwd(self):
        if self._bwd_args is None:
            raise ValueError("this plan was built without backward tensors")
        rc = self._b(*self._bwd_args)
        if rc:
            _check(self._bname, rc)


def wave_set_bucket_sparse(mode) -> int:
    """Selects the wave attention's kernel family (process-wide): True / 1 =
    bucket-sparse (scores only in the 16 x 16 blocks of bucket-sorted
    positions the mask can admit), False / 0 = every causal pair, "auto" / 2
    (the default) = bucket-sparse from T = 1024.  Returns the previous mode."""
    m = 2 if mode == "auto" else int(mode)
    prev = lib().wha_wave_set_bucket_sparse(m)
    if prev < 0:
        raise ValueError(f"wave kernel family must be 0, 1 or 2 (got {mode!r})")
    return prev


# ------------------------------------------------------------------ timing

def timing_enable(on: bool = True):
    _check("wha_timing_enable", lib().wha_timing_enable(1 if on else 0))


def timing_reset():
    _check("wha_timing_reset", lib().wha_timing_reset())


def timing_read(kernel: str):
    """(total_ms, launches) of a kernel since the last reset."""
    ms, n = ctypes.c_double(0.0), ctypes.c_int64(0)
    _check("wha_timing_read", lib().wha_timing_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


# ------------------------------------------------------------------ reference-interface mirror

def _as_2d_f32(x, name):
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    if a.ndim != 2:
        raise ValueError(f"{name}: expected [T][n_embd], got shape {a.shape}")
    return a


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class LinearWeights:
    """LinearWeights (src/common/model.rs:175-180): w [out_dim][in_dim], b [out_dim]."""

    def __init__(self, w, b):
        self.w = np.ascontiguousarray(np.asarray(w, dtype=np.float32))
        self.b = np.ascontiguousarray(np.asarray(b, dtype=np.float32))


class AttentionWeights:
    """AttentionWeights (src/common/model.rs:189-195): c_attn [3E][E], c_proj [E][E], n_head."""

    def __init__(self, c_attn: LinearWeights, c_proj: LinearWeights, n_head: int):
        self.c_attn, self.c_proj, self.n_head = c_attn, c_proj, int(n_head)


class HipBackend:
    """The attention half of wave-engine's ``ComputeBackend`` on the HIP tier.

    Mirrors ``fn attention_backward(&self, d_pre_proj, q_all, k_all, v_all,
    att_weights, n_head) -> (d_q, d_k, d_v)`` (``src/common/compute.rs:163-173``)
    with ``CpuBackend``'s semantics (``:286-314``: att used as given), and the core
    of ``fn attention`` (``attention_cpu``, ``:377-409``).  Inputs are
    ``[T][n_embd]`` host arrays (lists of rows or 2-D arrays); outputs are
    ``[T][n_embd]`` float32 numpy arrays.  Failures raise ``RuntimeError`` where
    the reference panics."""

    def attention(self, weights: "AttentionWeights", x):
        """fn attention(&self, weights, x) (src/common/compute.rs:42-43): c_attn,
        causal attention core and c_proj on one sequence x [T][n_embd]."""
        xs = _as_2d_f32(x, "x")
        T, E = xs.shape
        wa, wp = weights.c_attn, weights.c_proj
        if wa.w.shape != (3 * E, E) or wa.b.shape != (3 * E,) or wp.w.shape != (E, E) or wp.b.shape != (E,):
            raise ValueError("weights: c_attn must be [3E][E] + [3E], c_proj [E][E] + [E]")
        out = np.empty((T, E), dtype=np.float32)
        _check("wha_host_attention", lib().wha_host_attention(_fp(xs), _fp(wa.w), _fp(wa.b), _fp(wp.w), _fp(wp.b),
                                                              T, E, weights.n_head, _fp(out)))
        return out

    def attention_core(self, q_all, k_all, v_all, n_head: int):
        q, k, v = (_as_2d_f32(a, n) for a, n in ((q_all, "q_all"), (k_all, "k_all"), (v_all, "v_all")))
        T, E = q.shape
        out = np.empty((T, E), dtype=np.float32)
        _check("wha_host_attention_core_fwd",
               lib().wha_host_attention_core_fwd(_fp(q), _fp(k), _fp(v), T, E, int(n_head), _fp(out)))
        return out

    def attention_backward(self, d_pre_proj, q_all, k_all, v_all, att_weights, n_head: int):
        d, q, k, v = (_as_2d_f32(a, n) for a, n in ((d_pre_proj, "d_pre_proj"), (q_all, "q_all"),
                                                    (k_all, "k_all"), (v_all, "v_all")))
        T, E = q.shape
        att = np.ascontiguousarray(np.asarray(att_weights, dtype=np.float32))
        if att.shape != (int(n_head), T, T):
            raise ValueError(f"att_weights: expected [n_head][T][T] = {(n_head, T, T)}, got {att.shape}")
        dq, dk, dv = (np.empty((T, E), dtype=np.float32) for _ in range(3))
        _check("wha_host_attention_backward",
               lib().wha_host_attention_backward(_fp(d), _fp(q), _fp(k), _fp(v), _fp(att), T, E,
                                                 int(n_head), _fp(dq), _fp(dk), _fp(dv)))
        return dq, dk, dv

    # ---- wave attention on host arrays (src/common/attn.rs:90-511)

    @staticmethod
    def _wave_host_weights(w):
        arrs = {k: np.ascontiguousarray(np.asarray(w[k], dtype=np.float32))
                for k in ("hraw", "proj_w", "proj_b", "v_w", "v_b", "out_w", "out_b")}
        H, P, E = arrs["proj_w"].shape
        c = _WaveWeightsC(*(a.ctypes.data for a in arrs.values()))
        return arrs, c, H, P - 2, E

    def wave_attention_forward(self, weights, x, n_bands=None, want_phases=False):
        """wave_attention_forward (attn.rs:90-305) on one sequence x [T][n_embd];
        weights: mapping of packed host arrays (hraw, proj_w [H][2+C][E], proj_b,
        v_w, v_b, out_w, out_b).  Returns out (and phases [H][T])."""
        arrs, c, H, C, E = self._wave_host_weights(weights)
        xs = _as_2d_f32(x, "x")
        T = xs.shape[0]
        if xs.shape[1] != E or (n_bands is not None and 2 * n_bands != E):
            raise ValueError("x must be [T][n_embd] with n_embd = 2 * n_bands")
        out = np.empty((T, E), dtype=np.float32)
        ph = np.empty((H, T), dtype=np.float32)
        _check("wha_host_wave_attention_forward", lib().wha_host_wave_attention_forward(
            _fp(xs), ctypes.byref(c), T, E, H, C, _fp(out), ctypes.c_void_p(ph.ctypes.data)))
        return (out, ph) if want_phases else out

    def wave_attention_backward(self, weights, x, d_attn_out, full=True):
        """wave_attention_backward_full (attn.rs:346-430), or _pathway (:432-511)
        when full is False (d_normed only).  The forward is recomputed from x."""
        arrs, c, H, C, E = self._wave_host_weights(weights)
        xs, d = _as_2d_f32(x, "x"), _as_2d_f32(d_attn_out, "d_attn_out")
        T = xs.shape[0]
        hd = E // H
        g = dict(d_x=np.empty((T, E), np.float32))
        if full:
            g.update(d_hraw=np.empty(H, np.float32), d_proj_w=np.empty((H, 2 + C, E), np.float32),
                     d_proj_b=np.empty((H, 2 + C), np.float32), d_v_w=np.empty((H, hd, hd), np.float32),
                     d_v_b=np.empty((H, hd), np.float32), d_out_w=np.empty((E, E), np.float32),
                     d_out_b=np.empty(E, np.float32))
        keys = ("d_x", "d_hraw", "d_proj_w", "d_proj_b", "d_v_w", "d_v_b", "d_out_w", "d_out_b")
        gc = _WaveGradsC(*((g[k].ctypes.data if k in g else None) for k in keys))
        _check("wha_host_wave_attention_backward", lib().wha_host_wave_attention_backward(
            _fp(xs), _fp(d), ctypes.byref(c), T, E, H, C, ctypes.byref(gc)))
        return g if full else g["d_x"]


# ------------------------------------------------------------------ synthetic inputs

# ------------------------------------------------------------------ wave attention
# Mirror of the harmonic coherence attention interface (src/common/attn.rs:17-511):
# the same names, weights and results, on device tensors, batched over B
# sequences.  Weight layout: include/wave_hip_attn.h (wha_wave_weights).

class WaveAttnWeights:
    """WaveAttnWeights (src/common/attn.rs:39-46) for all heads, as device
    float32 tensors: harmonic_raw [H], proj_w [H][2+C][E] (phase rows r, s then
    content rows), proj_b [H][2+C], v_w [H][hd][hd], v_b [H][hd], out_w [E][E],
    out_b [E]."""

    _NAMES = ("harmonic_raw", "proj_w", "proj_b", "v_w", "v_b", "out_w", "out_b")

    def __init__(self, harmonic_raw, proj_w, proj_b, v_w, v_b, out_w, out_b):
        torch = _torch()
        vals = (harmonic_raw, proj_w, proj_b, v_w, v_b, out_w, out_b)
        for name, t in zip(self._NAMES, vals):
            if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
                raise ValueError(f"{name} must be a contiguous float32 device tensor")
            setattr(self, name, t)
        H, P, E = proj_w.shape
        hd = E // H if H else 0
        want = {"harmonic_raw": (H,), "proj_b": (H, P), "v_w": (H, hd, hd), "v_b": (H, hd), "out_w": (E, E),
                "out_b": (E,)}
        for name, shp in want.items():
            if tuple(getattr(self, name).shape) != shp:
                raise ValueError(f"{name}: expected shape {shp}, got {tuple(getattr(self, name).shape)}")
        if H == 0 or E % H:
            raise ValueError(f"n_embd {E} is not divisible by n_head {H}")
        self.n_head, self.content_dim, self.n_embd = H, P - 2, E

    @classmethod
    def from_heads(cls, heads, out_proj_w, out_proj_b, device="cuda"):
        """From the reference's per-head fields (WaveAttnHeadWeights,
        attn.rs:17-37): each head a mapping with harmonic_raw, phase_proj_w [2][E],
        phase_proj_b [2], v_proj_w [hd][hd], v_proj_b [hd], content_proj_w [C][E]
        (empty: no content projection) and content_proj_b [C]."""
        torch = _torch()
        f = lambda a: np.asarray(a, dtype=np.float32)
        cdims = {len(h.get("content_proj_w", [])) for h in heads}
        if len(cdims) != 1:
            raise ValueError("every head must have the same content_dim")
        rows_w, rows_b = [], []
        for h in heads:
            cw = f(h.get("content_proj_w", [])).reshape(-1, f(h["phase_proj_w"]).shape[1])
            rows_w.append(np.concatenate([f(h["phase_proj_w"]), cw], axis=0))
            rows_b.append(np.concatenate([f(h["phase_proj_b"]), f(h.get("content_proj_b", []))]))
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)
        return cls(t([h["harmonic_raw"] for h in heads]), t(np.stack(rows_w)), t(np.stack(rows_b)),
                   t(np.stack([f(h["v_proj_w"]) for h in heads])), t(np.stack([f(h["v_proj_b"]) for h in heads])),
                   t(out_proj_w), t(out_proj_b))

    def _c(self):
        return _WaveWeightsC(*(t.data_ptr() for t in (getattr(self, n) for n in self._NAMES)))


class WaveAttnCache:
    """Forward intermediates (the role of WaveAttnCache, attn.rs:48-70) on the
    device; ``normed`` is the input the forward read, as in the reference."""

    def __init__(self, shape: WaveShape, device):
        torch = _torch()
        B, T, E, H, C = shape.B, shape.T, shape.n_embd, shape.n_head, shape.content_dim
        e = lambda *s, dt=torch.float32: torch.empty(*s, dtype=dt, device=device)
        self.shape = shape
        self.proj = e(B, T, H, 2 + C)
        self.values = e(B, T, E)
        self.feat = e(B, H, T, 32)
        self.phase = e(B, H, T)
        self.bucket = e(B, H, T, dt=torch.int32)
        self.merged = e(B, T, E)
        self.lse = e(B, H, T)
        self.normed = None

    def _c(self):
        return _WaveCacheC(*(t.data_ptr() for t in (self.proj, self.values, self.feat, self.phase, self.bucket,
                                                     self.merged, self.lse)))


class WaveAttnGrads:
    """WaveAttnGrads (attn.rs:328-336): per-head weight gradients in the packed
    layout of WaveAttnWeights (summed over the batch), out_proj gradients and
    d_normed."""

    def __init__(self, d_normed, d_harmonic_raw, d_proj_w, d_proj_b, d_v_w, d_v_b, out_proj_w, out_proj_b):
        self.d_normed, self.d_harmonic_raw = d_normed, d_harmonic_raw
        self.d_proj_w, self.d_proj_b, self.d_v_w, self.d_v_b = d_proj_w, d_proj_b, d_v_w, d_v_b
        self.out_proj_w, self.out_proj_b = out_proj_w, out_proj_b


class WaveAttnRows:
    """Lazy view of att_weights_all: rows are recomputed on the device from the
    cache (the forward never materialises [H][T][T])."""

    def __init__(self, cache: WaveAttnCache):
        self.cache = cache

    def rows(self, rows):
        return wave_probs_rows(self.cache, rows)

    def last_rows(self):
        """[B][H][T]: the row attn_monitor reads (src/monitors/attn_monitor.rs:26-80)."""
        return self.rows([self.cache.shape.T - 1])[:, :, 0, :]


def _wave_x(x, weights: WaveAttnWeights):
    torch = _torch()
    if x.dim() == 2:
        x = x.unsqueeze(0)
    if x.dim() != 3 or x.shape[2] != weights.n_embd:
        raise ValueError(f"x must be [B][T][{weights.n_embd}] (or [T][{weights.n_embd}]), got {tuple(x.shape)}")
    if not (x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()):
        raise ValueError("x must be a contiguous float32 device tensor")
    return x


def wave_fwd_workspace_bytes(shape: WaveShape) -> int:
    return int(lib().wha_wave_fwd_workspace_size(ctypes.byref(shape)))


def wave_attention_forward(weights: WaveAttnWeights, x, n_bands=None, return_pathway_cache=True, out=None,
                           workspace=None):
    """wave_attention_forward (src/common/attn.rs:90-305) on x [B][T][n_embd]
    (or one sequence [T][n_embd]).  Returns (out, att_weights, cache): att_weights
    is a WaveAttnRows view; cache is None unless return_pathway_cache.
    workspace: a float32 device tensor of at least wave_fwd_workspace_bytes
    (allocated here when None)."""
    torch = _torch()
    x = _wave_x(x, weights)
    if n_bands is not None and 2 * n_bands != weights.n_embd:
        raise ValueError(f"n_bands {n_bands} does not match n_embd {weights.n_embd}")
    B, T, E = x.shape
    shape = WaveShape(B, T, E, weights.n_head, weights.content_dim)
    cache = WaveAttnCache(shape, x.device)
    cache.normed = x
    if out is None:
        out = torch.empty_like(x)
    ws = workspace
    if ws is None:
        ws = torch.empty(wave_fwd_workspace_bytes(shape) // 4 + 64, dtype=torch.float32, device=x.device)
    _check("wha_wave_fwd", lib().wha_wave_fwd(_ptr(x), ctypes.byref(weights._c()), ctypes.byref(shape), _ptr(out),
                                               ctypes.byref(cache._c()), _ptr(ws), ws.numel() * 4,
                                               _stream_ptr(x)))
    return out, WaveAttnRows(cache), (cache if return_pathway_cache else None)


def wave_bwd_workspace_bytes(shape: WaveShape) -> int:
    return int(lib().wha_wave_bwd_workspace_size(ctypes.byref(shape)))


def _wave_bwd(weights, cache, d_attn_out, full, workspace=None):
    torch = _torch()
    if cache is None or cache.normed is None:
        raise ValueError("the backward needs the forward's pathway cache")
    x = cache.normed
    d = d_attn_out.unsqueeze(0) if d_attn_out.dim() == 2 else d_attn_out
    if tuple(d.shape) != tuple(x.shape) or not d.is_contiguous() or d.dtype != torch.float32:
        raise ValueError(f"d_attn_out must be a contiguous float32 tensor of shape {tuple(x.shape)}")
    H, C, E = weights.n_head, weights.content_dim, weights.n_embd
    hd = E // H
    dev = x.device
    z = lambda *s: torch.empty(*s, dtype=torch.float32, device=dev)
    d_x = torch.empty_like(x)
    g = dict(d_harmonic_raw=z(H), d_proj_w=z(H, 2 + C, E), d_proj_b=z(H, 2 + C), d_v_w=z(H, hd, hd),
             d_v_b=z(H, hd), d_out_w=z(E, E), d_out_b=z(E)) if full else {}
    gc = _WaveGradsC(d_x.data_ptr(), *((g[k].data_ptr() if full else None) for k in
                                      ("d_harmonic_raw", "d_proj_w", "d_proj_b", "d_v_w", "d_v_b", "d_out_w",
                                       "d_out_b")))
    shape = cache.shape
    ws = workspace
    if ws is None:
        ws = torch.empty(wave_bwd_workspace_bytes(shape) // 4 + 64, dtype=torch.float32, device=dev)
    _check("wha_wave_bwd", lib().wha_wave_bwd(_ptr(x), _ptr(d), ctypes.byref(weights._c()), ctypes.byref(shape),
                                               ctypes.byref(cache._c()), ctypes.byref(gc), _ptr(ws),
                                               ws.numel() * 4, _stream_ptr(x)))
    if not full:
        return d_x
    return WaveAttnGrads(d_x, g["d_harmonic_raw"], g["d_proj_w"], g["d_proj_b"], g["d_v_w"], g["d_v_b"],
                         g["d_out_w"], g["d_out_b"])


def wave_attention_backward_full(weights: WaveAttnWeights, cache: WaveAttnCache, d_attn_out, workspace=None):
    """wave_attention_backward_full (attn.rs:346-430): WaveAttnGrads."""
    return _wave_bwd(weights, cache, d_attn_out, True, workspace)


def wave_attention_backward_pathway(weights: WaveAttnWeights, cache: WaveAttnCache, d_attn_out, workspace=None):
    """wave_attention_backward_pathway (attn.rs:432-511): d_normed only."""
    return _wave_bwd(weights, cache, d_attn_out, False, workspace)


def wave_probs_rows(cache: WaveAttnCache, rows):
    """Rows of att_weights_all from the cache: [B][H][len(rows)][T] (0 where
    the bucket mask excludes a key, -inf after the diagonal)."""
    torch = _torch()
    rows = [int(r) for r in rows]
    arr = (ctypes.c_int32 * len(rows))(*rows)
    sh = cache.shape
    out = torch.empty(sh.B, sh.n_head, len(rows), sh.T, dtype=torch.float32, device=cache.lse.device)
    _check("wha_wave_probs_rows", lib().wha_wave_probs_rows(ctypes.byref(cache._c()), ctypes.byref(sh), arr,
                                                             len(rows), _ptr(out), _stream_ptr(out)))
    return out


# ------------------------------------------------------------------ wave KV cache (serving)

class WaveKvCache:
    """One layer's KV cache for B concurrent sequences (the per-layer part of
    KvCache, src/common/kv_cache.rs:35-89): per (sequence, head) cos/sin of
    n*phase, bucket, phase and value rows for up to `capacity` positions, plus
    the host-side count of cached positions per sequence (n_cached)."""

    def __init__(self, B: int, n_head: int, head_dim: int, capacity: int, device="cuda"):
        torch = _torch()
        self.B, self.n_head, self.head_dim, self.capacity = B, n_head, head_dim, capacity
        z = lambda *sh, dt=torch.float32: torch.zeros(*sh, dtype=dt, device=device)
        self.cs = z(B, n_head, capacity, 2)
        self.bucket = z(B, n_head, capacity, dt=torch.int32)
        self.phase = z(B, n_head, capacity)
        self.values = z(B, n_head, capacity, head_dim)
        self.lengths = [0] * B

    def _c(self, b0=0):
        """C view of sequences b0.. (pointer offsets into the batch)."""
        return _WaveKvC(self.cs[b0:].data_ptr(), self.bucket[b0:].data_ptr(), self.phase[b0:].data_ptr(),
                        self.values[b0:].data_ptr(), self.capacity)


def prefill_attention(weights: WaveAttnWeights, x, cache: WaveKvCache, first_seq: int = 0, workspace=None):
    """prefill's attention (kv_cache.rs:121-193) for prompts x [b][T][n_embd] of
    sequences first_seq .. first_seq+b-1 of the cache: returns out (after
    out_proj) and sets those sequences' cached positions to T."""
    torch = _torch()
    x = _wave_x(x, weights)
    nb, T, E = x.shape
    if first_seq < 0 or first_seq + nb > cache.B:
        raise ValueError("sequence range outside the cache")
    shape = WaveShape(nb, T, E, weights.n_head, weights.content_dim)
    ws = workspace
    if ws is None:
        ws = torch.empty(int(lib().wha_wave_kv_prefill_workspace_size(ctypes.byref(shape))) // 4 + 64,
                         dtype=torch.float32, device=x.device)
    out = torch.empty_like(x)
    _check("wha_wave_kv_prefill", lib().wha_wave_kv_prefill(
        _ptr(x), ctypes.byref(weights._c()), ctypes.byref(shape), ctypes.byref(cache._c(first_seq)), _ptr(out),
        _ptr(ws), ws.numel() * 4, _stream_ptr(x)))
    for b in range(first_seq, first_seq + nb):
        cache.lengths[b] = T
    return out


def wave_kv_decode_workspace_bytes(shape: WaveShape, capacity: int) -> int:
    return int(lib().wha_wave_kv_decode_workspace_size(ctypes.byref(shape), capacity))


def forward_one_attention(weights: WaveAttnWeights, x, cache: WaveKvCache, workspace=None):
    """forward_one's attention (kv_cache.rs:263-335) for one new token of every
    sequence: x [B][n_embd] -> out [B][n_embd]; appends the tokens and advances
    the cached counts (kv_cache.rs:358)."""
    torch = _torch()
    if x.dim() != 2 or x.shape[0] != cache.B or x.shape[1] != weights.n_embd:
        raise ValueError(f"x must be [{cache.B}][{weights.n_embd}]")
    if not (x.is_cuda and x.dtype == torch.float32 and x.is_contiguous()):
        raise ValueError("x must be a contiguous float32 device tensor")
    shape = WaveShape(cache.B, 1, weights.n_embd, weights.n_head, weights.content_dim)
    ws = workspace
    if ws is None:
        ws = torch.empty(wave_kv_decode_workspace_bytes(shape, cache.capacity) // 4 + 64, dtype=torch.float32,
                         device=x.device)
    lens = (ctypes.c_int32 * cache.B)(*cache.lengths)
    out = torch.empty_like(x)
    _check("wha_wave_kv_decode", lib().wha_wave_kv_decode(
        _ptr(x), ctypes.byref(weights._c()), ctypes.byref(shape), ctypes.byref(cache._c()), lens, _ptr(out),
        _ptr(ws), ws.numel() * 4, _stream_ptr(x)))
    cache.lengths = [n + 1 for n in cache.lengths]
    return out


class SynthStream:
    """Seeded normal draws from the library's generator: xorshift64 exactly as
    the reference's Rng (src/common/rng.rs:24-34) with Box-Muller pairs
    (u1 = 1 - next_f32, u2 = next_f32) evaluated in double."""

    def __init__(self, seed: int = 42):
        if seed == 0:
            raise ValueError("xorshift64 seed must be non-zero")
        self.state = ctypes.c_uint64(seed)

    def normal(self, n: int, stddev: float = 1.0, nthreads: int = 0) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        rc = lib().wha_synth_normal(ctypes.byref(self.state), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                    n, float(stddev), int(nthreads))
        if rc != 0:
            raise ValueError("wha_synth_normal: invalid state")
        return out


def synth_inputs(B: int, H: int, T: int, D: int, seed: int = 42, with_do: bool = True):
    """BASELINE inputs: Q, K, V ~ N(0,1)/sqrt(D), then dO ~ N(0,1), drawn in that
    order from one stream, each in [B][H][T][D] row-major order (numpy float32)."""
    g = SynthStream(seed)
    n = B * H * T * D
    sd = 1.0 / math.sqrt(float(D))
    out = [g.normal(n, sd).reshape(B, H, T, D) for _ in range(3)]
    if with_do:
        out.append(g.normal(n, 1.0).reshape(B, H, T, D))
    return tuple(out)
