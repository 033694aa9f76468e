"""CPU oracle for wave-engine's dot-product causal attention.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or the timed CPU baseline) -- never as the thing measured or shipped.
The product library in ``wave-engine_amd/`` does not depend on it.

The arithmetic lives in ``wave_attn_oracle.c`` (built by ``oracle/Makefile``
into ``liboracle.so``): a reference-order f32 restatement of

* ``attention_cpu`` core, ``src/common/compute.rs:377-409``
* ``CpuBackend::attention_backward``, ``src/common/compute.rs:286-314``
* ``attention_backward_single``, ``src/cpu/backward.rs:313-363``
* ``Rng::next_u64`` / ``next_f32``, ``src/common/rng.rs:24-34``
* the projections: ``linear_batch_cpu`` (``src/common/compute.rs:441-468``),
  ``linear_backward_dx_only`` (``src/common/math/backward.rs:36-46``),
  ``outer_product_accum`` (``src/common/compute.rs:263-282``) and ``attention_cpu``
  end to end (``:357-414``)

plus an f64 twin of the same loops (ground truth).  This module only moves
numpy arrays in and out of it, converting between the device layout
``[B, H, T, D]`` and the reference's per-sequence ``[T][H*D]`` layout.

Pins (each in ``tests/``): the reference's softmax-backward,
value-aggregation and out-projection-backward known-answer tests
(``src/common/math/attn_backward.rs:336-379``),
closed forms (T=1, Q=0, constant V, equal K rows), invariants (row sums,
sum of dK over keys, causality, linearity in V), an independent matrix-form
numpy restatement in f64, and a central finite-difference check of the
backward in f64.  The generator's xorshift step is pinned by its full-period
property over GF(2); its Box-Muller layer is this build's own definition and is
pinned by committed check values only.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


def build() -> None:
    """Compile liboracle.so with its Makefile."""
    subprocess.run(["make", "-s", "-C", str(_HERE), "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        u64p = ctypes.POINTER(ctypes.c_uint64)
        L.wao_xorshift64_next.argtypes = [u64p]
        L.wao_xorshift64_next.restype = ctypes.c_uint64
        L.wao_next_f32.argtypes = [u64p]
        L.wao_next_f32.restype = ctypes.c_float
        L.wao_fill_normal.argtypes = [u64p, _f32p, ctypes.c_size_t, ctypes.c_double]
        L.wao_fill_normal.restype = None
        for sfx, p, real in (("f32", _f32p, ctypes.c_float), ("f64", _f64p, ctypes.c_double)):
            vp = ctypes.c_void_p
            f = getattr(L, f"wao_attention_core_fwd_{sfx}")
            f.argtypes = [p, p, p, ctypes.c_int, ctypes.c_int, ctypes.c_int, p, vp, vp]
            f.restype = None
            f = getattr(L, f"wao_attention_backward_{sfx}")
            f.argtypes = [p, p, p, p, p, ctypes.c_int, ctypes.c_int, ctypes.c_int, p, p, p]
            f.restype = None
            f = getattr(L, f"wao_softmax_backward_row_{sfx}")
            f.argtypes = [p, p, ctypes.c_int, p]
            f.restype = None
            f = getattr(L, f"wao_value_backward_row_{sfx}")
            f.argtypes = [p, p, p, ctypes.c_long, p, ctypes.c_int, ctypes.c_int, p]
            f.restype = None
            f = getattr(L, f"wao_linear_{sfx}")
            f.argtypes = [p, p, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, p]
            f.restype = None
            f = getattr(L, f"wao_linear_backward_dx_{sfx}")
            f.argtypes = [p, p, ctypes.c_int, ctypes.c_int, ctypes.c_int, p]
            f.restype = None
            f = getattr(L, f"wao_outer_product_accum_{sfx}")
            f.argtypes = [p, p, ctypes.c_int, ctypes.c_int, ctypes.c_int, p, vp]
            f.restype = None
            f = getattr(L, f"wao_attention_full_{sfx}")
            f.argtypes = [p, p, p, p, p, ctypes.c_int, ctypes.c_int, ctypes.c_int, p]
            f.restype = None
            f = getattr(L, f"wao_decode_{sfx}")
            f.argtypes = [p, p, p, ctypes.c_int, ctypes.c_int, ctypes.c_int, p, vp]
            f.restype = None
        L.wao_batch_fwd_bwd_f32.argtypes = [ctypes.c_int] * 4 + [_f32p] * 3 + [ctypes.c_void_p] + \
            [_f32p] + [ctypes.c_void_p] * 3 + [ctypes.c_int]
        L.wao_batch_fwd_bwd_f32.restype = ctypes.c_int
        _lib = L
    return _lib


def _dt(precision: str):
    if precision == "f32":
        return np.float32
    if precision == "f64":
        return np.float64
    raise ValueError(precision)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- generator

class Xorshift64:
    """Rng (src/common/rng.rs:5-45) state, advanced by the C restatement."""

    def __init__(self, seed: int = 42):
        if seed == 0:
            raise ValueError("xorshift64 seed must be non-zero")
        self.state = ctypes.c_uint64(seed)

    def next_u64(self) -> int:
        return int(lib().wao_xorshift64_next(ctypes.byref(self.state)))

    def next_f32(self) -> float:
        return float(lib().wao_next_f32(ctypes.byref(self.state)))

    def normal(self, n: int, stddev: float = 1.0) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().wao_fill_normal(ctypes.byref(self.state), out, n, float(stddev))
        return out


def synth_inputs(B: int, H: int, T: int, D: int, seed: int = 42, with_do: bool = True):
    """BASELINE inputs: Q, K, V ~ N(0,1)/sqrt(D), then dO ~ N(0,1), drawn in that
    order from one xorshift64 stream, each in [B][H][T][D] row-major order."""
    rng = Xorshift64(seed)
    n = B * H * T * D
    sd = 1.0 / np.sqrt(float(D))
    q = rng.normal(n, sd).reshape(B, H, T, D)
    k = rng.normal(n, sd).reshape(B, H, T, D)
    v = rng.normal(n, sd).reshape(B, H, T, D)
    if not with_do:
        return q, k, v
    do = rng.normal(n, 1.0).reshape(B, H, T, D)
    return q, k, v, do


# ---------------------------------------------------------------- layouts

def bhtd_to_seq(x: np.ndarray) -> np.ndarray:
    """[B,H,T,D] -> [B,T,H*D] (reference per-sequence layout)."""
    B, H, T, D = x.shape
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3).reshape(B, T, H * D))


def seq_to_bhtd(x: np.ndarray, H: int) -> np.ndarray:
    B, T, E = x.shape
    return np.ascontiguousarray(x.reshape(B, T, H, E // H).transpose(0, 2, 1, 3))


# ---------------------------------------------------------------- per sequence

def core_fwd(q, k, v, n_head: int, precision: str = "f32", want_att=False, want_lse=False):
    """attention_cpu core on one sequence. q,k,v: [T][E]. Returns out (and att
    [H][T][T], lse [H][T] when asked)."""
    dt = _dt(precision)
    q, k, v = _c(q, dt), _c(k, dt), _c(v, dt)
    T, E = q.shape
    out = np.empty((T, E), dtype=dt)
    att = np.empty((n_head, T, T), dtype=dt) if want_att else None
    lse = np.empty((n_head, T), dtype=dt) if want_lse else None
    getattr(lib(), f"wao_attention_core_fwd_{precision}")(
        q, k, v, T, E, n_head, out,
        att.ctypes.data if att is not None else None,
        lse.ctypes.data if lse is not None else None)
    res = [out]
    if want_att:
        res.append(att)
    if want_lse:
        res.append(lse)
    return res[0] if len(res) == 1 else tuple(res)


def attention_backward(d_pre_proj, q, k, v, att, n_head: int, precision: str = "f32"):
    """CpuBackend::attention_backward on one sequence. att: [H][T][T]."""
    dt = _dt(precision)
    d_pre_proj, q, k, v, att = (_c(a, dt) for a in (d_pre_proj, q, k, v, att))
    T, E = q.shape
    dq, dk, dv = (np.empty((T, E), dtype=dt) for _ in range(3))
    getattr(lib(), f"wao_attention_backward_{precision}")(d_pre_proj, q, k, v, att, T, E, n_head, dq, dk, dv)
    return dq, dk, dv


def softmax_backward_row(att, d_att, precision: str = "f32"):
    dt = _dt(precision)
    att, d_att = _c(att, dt), _c(d_att, dt)
    out = np.empty_like(att)
    getattr(lib(), f"wao_softmax_backward_row_{precision}")(att, d_att, att.shape[0], out)
    return out


def value_backward_row(d_out, v, dv, att, precision: str = "f32"):
    """Value-aggregation step for one head and position: returns d_att (length
    n = len(att)) and accumulates att[ki]*d_out into dv[ki] in place."""
    dt = _dt(precision)
    d_out, v, att = _c(d_out, dt), _c(v, dt), _c(att, dt)
    if dv.dtype != dt or not dv.flags.c_contiguous:
        raise ValueError("dv must be a C-contiguous array of the working precision")
    n, D = len(att), d_out.shape[0]
    d_att = np.empty(n, dtype=dt)
    getattr(lib(), f"wao_value_backward_row_{precision}")(d_out, v, dv, v.shape[1], att, n, D, d_att)
    return d_att


def decode_one(q, k, v, n_head: int, precision: str = "f32", want_lse=False):
    """One query [E] against a cache [Tk][E], every key visible."""
    dt = _dt(precision)
    q, k, v = _c(q, dt), _c(k, dt), _c(v, dt)
    Tk, E = k.shape
    out = np.empty(E, dtype=dt)
    lse = np.empty(n_head, dtype=dt) if want_lse else None
    getattr(lib(), f"wao_decode_{precision}")(q, k, v, Tk, E, n_head, out,
                                              lse.ctypes.data if lse is not None else None)
    return (out, lse) if want_lse else out


# ---------------------------------------------------------------- projections

def linear(x, w, b=None, precision: str = "f32"):
    """linear_batch_cpu: y[m] = b + W x[m] for the rows of x [M][K]; w [N][K]."""
    dt = _dt(precision)
    x, w = _c(x, dt), _c(w, dt)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=dt)
    bb = _c(b, dt) if b is not None else None
    getattr(lib(), f"wao_linear_{precision}")(x, w, bb.ctypes.data if bb is not None else None, M, N, K, y)
    return y


def linear_backward_dx(dy, w, precision: str = "f32"):
    """linear_backward_dx_only per row: dx[m] = W^T dy[m]."""
    dt = _dt(precision)
    dy, w = _c(dy, dt), _c(w, dt)
    M, N = dy.shape
    K = w.shape[1]
    dx = np.empty((M, K), dtype=dt)
    getattr(lib(), f"wao_linear_backward_dx_{precision}")(dy, w, M, N, K, dx)
    return dx


def outer_product_accum(dy, x, compute_bias: bool, precision: str = "f32"):
    """CpuBackend::outer_product_accum: (d_w [N][K], d_b [N])."""
    dt = _dt(precision)
    dy, x = _c(dy, dt), _c(x, dt)
    M, N = dy.shape
    K = x.shape[1]
    dw = np.empty((N, K), dtype=dt)
    db = np.zeros(N, dtype=dt)
    getattr(lib(), f"wao_outer_product_accum_{precision}")(dy, x, M, N, K, dw,
                                                          db.ctypes.data if compute_bias else None)
    return dw, db


def attention_full(x, wa, ba, wp, bp, n_head: int, precision: str = "f32"):
    """attention_cpu end to end (c_attn, core, c_proj) on one sequence x [T][E]."""
    dt = _dt(precision)
    x, wa, ba, wp, bp = (_c(a, dt) for a in (x, wa, ba, wp, bp))
    T, E = x.shape
    out = np.empty((T, E), dtype=dt)
    getattr(lib(), f"wao_attention_full_{precision}")(x, wa, ba, wp, bp, T, E, n_head, out)
    return out


# ---------------------------------------------------------------- batched [B,H,T,D]

def fwd_bhtd(q, k, v, precision: str = "f32", want_lse=False):
    """Forward over a [B,H,T,D] batch, one reference call per sequence.
    Returns O [B,H,T,D] (and LSE [B,H,T])."""
    B, H, T, D = q.shape
    qs, ks, vs = bhtd_to_seq(q), bhtd_to_seq(k), bhtd_to_seq(v)
    outs, lses = [], []
    for b in range(B):
        r = core_fwd(qs[b], ks[b], vs[b], H, precision, want_lse=want_lse)
        if want_lse:
            outs.append(r[0])
            lses.append(r[1])
        else:
            outs.append(r)
    o = seq_to_bhtd(np.stack(outs), H)
    return (o, np.stack(lses)) if want_lse else o


def fwd_bwd_bhtd(q, k, v, do, precision: str = "f32", nthreads: int = 1):
    """Forward then backward (att from the oracle's own forward) over a
    [B,H,T,D] batch, one sequence per task (nthreads > 1: a thread pool; the C
    calls release the GIL).  Returns O, dQ, dK, dV in [B,H,T,D] and LSE [B,H,T]."""
    B, H, T, D = q.shape
    qs, ks, vs, dos = (bhtd_to_seq(a) for a in (q, k, v, do))

    def one(b):
        o, att, lse = core_fwd(qs[b], ks[b], vs[b], H, precision, want_att=True, want_lse=True)
        dq, dk, dv = attention_backward(dos[b], qs[b], ks[b], vs[b], att, H, precision)
        return o, dq, dk, dv, lse

    if nthreads > 1:
        from concurrent.futures import ThreadPoolExecutor
        with ThreadPoolExecutor(min(nthreads, B)) as ex:
            res = list(ex.map(one, range(B)))
    else:
        res = [one(b) for b in range(B)]
    cv = lambda i: seq_to_bhtd(np.stack([r[i] for r in res]), H)
    return cv(0), cv(1), cv(2), cv(3), np.stack([r[4] for r in res])


def batch_fwd_bwd_f32_threaded(q_seq, k_seq, v_seq, do_seq, n_head: int, nthreads: int):
    """Threaded reference-order f32 forward+backward over [B][T][E] sequences
    (one thread per sequence).  Returns out, dq, dk, dv [B][T][E]."""
    q_seq, k_seq, v_seq = (_c(a, np.float32) for a in (q_seq, k_seq, v_seq))
    B, T, E = q_seq.shape
    out = np.empty_like(q_seq)
    if do_seq is None:
        lib().wao_batch_fwd_bwd_f32(B, T, E, n_head, q_seq, k_seq, v_seq, None, out,
                                    None, None, None, nthreads)
        return out
    do_seq = _c(do_seq, np.float32)
    dq, dk, dv = (np.empty_like(q_seq) for _ in range(3))
    lib().wao_batch_fwd_bwd_f32(B, T, E, n_head, q_seq, k_seq, v_seq, do_seq.ctypes.data, out,
                                dq.ctypes.data, dk.ctypes.data, dv.ctypes.data, nthreads)
    return out, dq, dk, dv


# ---------------------------------------------------------------- wave attention
# Restatement of src/common/attn.rs:72-430 and src/common/math/attn_backward.rs
# (C body in wave_core.inc).  Weights are a dict of arrays in the flattened layout
#   hraw [H], proj_w [H][2+C][E] (rows r, s, then content), proj_b [H][2+C],
#   v_w [H][hd][hd], v_b [H][hd], out_w [E][E], out_b [E].

_WAVE_KEYS = ("hraw", "proj_w", "proj_b", "v_w", "v_b", "out_w", "out_b")


def _ptr(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _wave_fn(name, precision, restype=None):
    f = getattr(lib(), f"{name}_{precision}")
    f.restype = restype
    return f


def wave_dims(w):
    H, P, E = w["proj_w"].shape
    return H, P - 2, E


def phase_bucket(phase: float, precision: str = "f32") -> int:
    """phase_to_bucket (src/common/kv_cache.rs:66-70)."""
    real = ctypes.c_float if precision == "f32" else ctypes.c_double
    f = _wave_fn("wao_phase_bucket", precision, ctypes.c_int)
    f.argtypes = [real]
    return int(f(phase))


def phases(r, s, precision: str = "f32"):
    """atan2(s, r) and its bucket for arrays of (r, s), with the reference's
    f32 (atan2f) or f64 operations (src/common/attn.rs:121-128, :169-174)."""
    dt = _dt(precision)
    r, s = _c(np.asarray(r).ravel(), dt), _c(np.asarray(s).ravel(), dt)
    ph = np.empty_like(r)
    bk = np.empty(r.shape, dtype=np.int32)
    f = _wave_fn("wao_phases", precision)
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long, ctypes.c_void_p, ctypes.c_void_p]
    f(r.ctypes.data, s.ctypes.data, r.size, ph.ctypes.data, bk.ctypes.data)
    return ph, bk


def wave_fwd(x, w, precision: str = "f32", phase_in=None):
    """wave_attention_forward on one sequence x [T][E].  phase_in [H][T]
    (optional) replays given phases.  Returns a dict with out, merged, att
    ([H][T][T], -inf after the diagonal as in the reference), phase [H][T],
    rs [H][T][2], content [H][T][C], values [H][T][hd], lse [H][T]."""
    dt = _dt(precision)
    x = _c(x, dt)
    ww = {k: _c(w[k], dt) for k in _WAVE_KEYS}
    H, C, E = wave_dims(ww)
    T = x.shape[0]
    hd = E // H
    ph_in = _c(phase_in, dt) if phase_in is not None else None
    r = dict(out=np.empty((T, E), dt), merged=np.empty((T, E), dt), att=np.empty((H, T, T), dt),
             phase=np.empty((H, T), dt), rs=np.empty((H, T, 2), dt), content=np.empty((H, T, max(C, 0)), dt),
             values=np.empty((H, T, hd), dt), lse=np.empty((H, T), dt))
    _wave_fn("wao_wave_fwd", precision)(
        _ptr(x), T, E, H, C, *(_ptr(ww[k]) for k in _WAVE_KEYS), _ptr(ph_in), _ptr(r["out"]), _ptr(r["merged"]),
        _ptr(r["att"]), _ptr(r["phase"]), _ptr(r["rs"]), _ptr(r["content"]) if C > 0 else None,
        _ptr(r["values"]), _ptr(r["lse"]))
    return r


def wave_bwd(x, w, d_out, precision: str = "f32", phase_in=None):
    """wave_attention_backward_full on one sequence.  Returns a dict with d_x,
    d_hraw, d_proj_w, d_proj_b, d_v_w, d_v_b, d_out_w, d_out_b."""
    dt = _dt(precision)
    x, d_out = _c(x, dt), _c(d_out, dt)
    ww = {k: _c(w[k], dt) for k in _WAVE_KEYS}
    H, C, E = wave_dims(ww)
    T = x.shape[0]
    hd = E // H
    ph_in = _c(phase_in, dt) if phase_in is not None else None
    g = dict(d_x=np.empty((T, E), dt), d_hraw=np.empty(H, dt), d_proj_w=np.empty((H, 2 + C, E), dt),
             d_proj_b=np.empty((H, 2 + C), dt), d_v_w=np.empty((H, hd, hd), dt), d_v_b=np.empty((H, hd), dt),
             d_out_w=np.empty((E, E), dt), d_out_b=np.empty(E, dt))
    _wave_fn("wao_wave_bwd", precision)(
        _ptr(x), T, E, H, C, *(_ptr(ww[k]) for k in _WAVE_KEYS), _ptr(ph_in), _ptr(d_out),
        *(_ptr(g[k]) for k in ("d_x", "d_hraw", "d_proj_w", "d_proj_b", "d_v_w", "d_v_b", "d_out_w", "d_out_b")))
    return g


def out_proj_backward(d_attn_out, merged, W, precision: str = "f32"):
    """out_proj_backward (attn_backward.rs:17-50): (d_out, d_w, d_b)."""
    dt = _dt(precision)
    d_attn_out, merged, W = (_c(a, dt) for a in (d_attn_out, merged, W))
    T, E = d_attn_out.shape
    d_out, d_w, d_b = np.empty((T, E), dt), np.empty((E, E), dt), np.empty(E, dt)
    _wave_fn("wao_out_proj_backward", precision)(_ptr(d_attn_out), _ptr(merged), _ptr(W), T, E, _ptr(d_out),
                                                 _ptr(d_w), _ptr(d_b))
    return d_out, d_w, d_b


def value_aggregation_backward(d_head, att, v, precision: str = "f32"):
    """value_aggregation_backward (attn_backward.rs:72-103): (d_att, d_v)."""
    dt = _dt(precision)
    d_head, att, v = (_c(a, dt) for a in (d_head, att, v))
    T, hd = d_head.shape
    d_att, d_v = np.empty((T, T), dt), np.empty((T, hd), dt)
    _wave_fn("wao_value_aggregation_backward", precision)(_ptr(d_head), _ptr(att), _ptr(v), T, hd, _ptr(d_att),
                                                          _ptr(d_v))
    return d_att, d_v


def wave_softmax_backward(d_att, att, precision: str = "f32"):
    """softmax_backward (attn_backward.rs:109-122) on [T][T]."""
    dt = _dt(precision)
    d_att, att = _c(d_att, dt), _c(att, dt)
    T = att.shape[0]
    out = np.empty((T, T), dt)
    _wave_fn("wao_wave_softmax_backward", precision)(_ptr(d_att), _ptr(att), T, _ptr(out))
    return out


def score_backward(d_scores, phases, n, att, cv=None, cs=0.0, precision: str = "f32"):
    """score_backward (attn_backward.rs:128-163): (d_delta, d_content or None, d_n)."""
    dt = _dt(precision)
    real = ctypes.c_float if precision == "f32" else ctypes.c_double
    d_scores, phases, att = (_c(a, dt) for a in (d_scores, phases, att))
    T = phases.shape[0]
    cvv = _c(cv, dt) if cv is not None else None
    C = cvv.shape[1] if cvv is not None else 0
    d_delta = np.empty((T, T), dt)
    d_c = np.empty((T, max(C, 1)), dt)
    f = _wave_fn("wao_score_backward", precision, real)
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, real, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, real,
                  ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    d_n = f(_ptr(d_scores), _ptr(phases), n, _ptr(att), _ptr(cvv), C, cs, T, _ptr(d_delta), _ptr(d_c))
    return d_delta, (d_c[:, :C] if cvv is not None else None), float(d_n)


def phase_subtraction_backward(d_delta, att, precision: str = "f32"):
    dt = _dt(precision)
    d_delta, att = _c(d_delta, dt), _c(att, dt)
    T = att.shape[0]
    out = np.empty(T, dt)
    _wave_fn("wao_phase_subtraction_backward", precision)(_ptr(d_delta), _ptr(att), T, _ptr(out))
    return out


def phase_projection_backward(d_phases, x, pw, pb, precision: str = "f32"):
    """phase_projection_backward (attn_backward.rs:190-231): (d_x, d_w, d_b)."""
    dt = _dt(precision)
    d_phases, x, pw, pb = (_c(a, dt) for a in (d_phases, x, pw, pb))
    T, E = x.shape
    d_x, d_w, d_b = np.empty((T, E), dt), np.empty((2, E), dt), np.empty(2, dt)
    _wave_fn("wao_phase_projection_backward", precision)(_ptr(d_phases), _ptr(x), _ptr(pw), _ptr(pb), T, E,
                                                         _ptr(d_x), _ptr(d_w), _ptr(d_b))
    return d_x, d_w, d_b


def value_projection_backward(d_v, x, offset, vw, precision: str = "f32"):
    """value_projection_backward (attn_backward.rs:237-263): (d_x, d_w, d_b)."""
    dt = _dt(precision)
    d_v, x, vw = (_c(a, dt) for a in (d_v, x, vw))
    T, E = x.shape
    hd = d_v.shape[1]
    d_x, d_w, d_b = np.empty((T, E), dt), np.empty((hd, hd), dt), np.empty(hd, dt)
    _wave_fn("wao_value_projection_backward", precision)(_ptr(d_v), _ptr(x), offset, hd, E, _ptr(vw), T,
                                                         _ptr(d_x), _ptr(d_w), _ptr(d_b))
    return d_x, d_w, d_b


def content_projection_backward(d_cv, x, cw, precision: str = "f32"):
    """content_projection_backward (attn_backward.rs:269-294): (d_x, d_w, d_b)."""
    dt = _dt(precision)
    d_cv, x, cw = (_c(a, dt) for a in (d_cv, x, cw))
    T, E = x.shape
    C = cw.shape[0]
    d_x, d_w, d_b = np.empty((T, E), dt), np.empty((C, E), dt), np.empty(C, dt)
    _wave_fn("wao_content_projection_backward", precision)(_ptr(d_cv), _ptr(x), _ptr(cw), T, E, C, _ptr(d_x),
                                                           _ptr(d_w), _ptr(d_b))
    return d_x, d_w, d_b


def combine_d_normed(d_phase, d_v, d_content=None, precision: str = "f32"):
    """combine_d_normed (attn_backward.rs:299-323): inputs [H][T][E]."""
    dt = _dt(precision)
    d_phase, d_v = _c(d_phase, dt), _c(d_v, dt)
    H, T, E = d_phase.shape
    dc = _c(d_content, dt) if d_content is not None and len(d_content) else None
    out = np.empty((T, E), dt)
    _wave_fn("wao_combine_d_normed", precision)(_ptr(d_phase), _ptr(d_v), _ptr(dc), H, T, E, _ptr(out))
    return out


def wave_kv_prefill(x, w, precision: str = "f32", phase_in=None):
    """kv_cache::prefill's attention (src/common/kv_cache.rs:121-193) on one
    prompt x [T][E]: no content bias.  Returns out, phase [H][T], values
    [H][T][hd], merged."""
    dt = _dt(precision)
    x = _c(x, dt)
    ww = {k: _c(w[k], dt) for k in _WAVE_KEYS}
    H, C, E = wave_dims(ww)
    T = x.shape[0]
    hd = E // H
    ph_in = _c(phase_in, dt) if phase_in is not None else None
    r = dict(out=np.empty((T, E), dt), phase=np.empty((H, T), dt), values=np.empty((H, T, hd), dt),
             merged=np.empty((T, E), dt))
    _wave_fn("wao_wave_kv_prefill", precision)(
        _ptr(x), T, E, H, C, *(_ptr(ww[k]) for k in _WAVE_KEYS), _ptr(ph_in), _ptr(r["out"]), _ptr(r["phase"]),
        _ptr(r["values"]), _ptr(r["merged"]))
    return r


def wave_kv_step(x, w, phases, values, n_cached: int, precision: str = "f32", phase_new_in=None):
    """kv_cache::forward_one's attention (src/common/kv_cache.rs:263-335) for one
    sequence: x [E] against cached phases [H][cap] and values [H][cap][hd]
    (entries 0..n_cached-1).  Returns out [E], phase_new [H], v_new [H][hd], merged [E]."""
    dt = _dt(precision)
    x = _c(x, dt)
    ww = {k: _c(w[k], dt) for k in _WAVE_KEYS}
    H, C, E = wave_dims(ww)
    hd = E // H
    phases, values = _c(phases, dt), _c(values, dt)
    cap = phases.shape[1]
    ph_in = _c(phase_new_in, dt) if phase_new_in is not None else None
    r = dict(out=np.empty(E, dt), phase_new=np.empty(H, dt), v_new=np.empty((H, hd), dt), merged=np.empty(E, dt))
    _wave_fn("wao_wave_kv_step", precision)(
        _ptr(x), E, H, C, *(_ptr(ww[k]) for k in _WAVE_KEYS), _ptr(phases), _ptr(values), cap, int(n_cached),
        _ptr(ph_in), _ptr(r["out"]), _ptr(r["phase_new"]), _ptr(r["v_new"]), _ptr(r["merged"]))
    return r
