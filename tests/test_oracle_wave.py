"""Pins of the wave (harmonic coherence) attention oracle, src/common/attn.rs:72-430
and src/common/math/attn_backward.rs:13-323, before it is trusted as the checker:
the reference's own known-answer tests, the bucket formula at hand-computed
points, an independent matrix-form numpy restatement in f64 with a brute-force
mask, closed forms, and central finite differences of the full backward in f64."""
import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from conftest import make_wave_weights

GOLDEN = Path(__file__).resolve().parent / "golden"


make_weights = make_wave_weights


# ------------------------------------------------------------ reference KATs

def test_reference_kats_on_wave_primitives():
    a = json.loads((GOLDEN / "attn_kat.json").read_text())
    k = a["softmax_backward"]
    ds = oracle.wave_softmax_backward(np.array(k["d_att"]), np.array(k["att"]))
    for e in k["expected"]:
        assert abs(ds[e["row"], e["col"]] - e["value"]) < e["tol"]
    k = a["value_aggregation_backward"]
    d_att, d_v = oracle.value_aggregation_backward(np.array(k["d_out"]), np.array(k["att"]), np.array(k["v"]))
    assert abs(d_att[0, 0] - k["expected_d_att_0_0"]) < k["tol"]
    np.testing.assert_allclose(d_v[0], k["expected_d_v_0"], atol=k["tol"])
    k = a["out_proj_backward"]
    d_out, d_w, d_b = oracle.out_proj_backward(np.array(k["d_attn"]), np.array(k["merged"]), np.array(k["w"]))
    ex = k["expected"]
    assert abs(d_out[0, 0] - ex["d_out_0_0"]) < k["tol"] and abs(d_out[0, 1] - ex["d_out_0_1"]) < k["tol"]
    assert abs(d_w[0, 0] - ex["d_w_0_0"]) < k["tol"] and abs(d_b[0] - ex["d_b_0"]) < k["tol"]

    w = json.loads((GOLDEN / "wave_kat.json").read_text())
    k = w["phase_projection_backward"]
    d_x, _, _ = oracle.phase_projection_backward(np.array(k["d_phases"]), np.array(k["x"]), np.array(k["w"]),
                                                 np.array(k["b"]))
    np.testing.assert_allclose(d_x[0], k["expected_d_x_0"], atol=k["tol"])
    k = w["value_projection_backward"]
    d_x, d_w, d_b = oracle.value_projection_backward(np.array(k["d_v"]), np.array(k["x"]), k["head_offset"],
                                                     np.array(k["w"]))
    ex = k["expected"]
    assert abs(d_x[0, 0] - ex["d_x_0_0"]) < k["tol"] and abs(d_x[0, 1] - ex["d_x_0_1"]) < k["tol"]
    assert abs(d_w[0, 0] - ex["d_w_0_0"]) < k["tol"] and abs(d_b[0] - ex["d_b_0"]) < k["tol"]
    k = w["combine_d_normed"]
    out = oracle.combine_d_normed(np.array(k["d_phase"]), np.array(k["d_v"]), None)
    np.testing.assert_allclose(out[0], k["expected_0"], atol=k["tol"])


# ------------------------------------------------------------ bucket formula

@pytest.mark.parametrize("precision", ["f32", "f64"])
def test_phase_bucket_at_hand_computed_points(precision):
    q = math.pi / 4
    cases = [(0.0, 0), (q * 0.999, 0), (q * 1.001, 1), (math.pi * 0.999, 3), (math.pi * 1.001, 4),
             (-math.pi * 1.001, 3), (-1e-3, 7), (-q * 1.001, 6), (2 * math.pi + 0.1, 0), (-2 * math.pi - 0.1, 7),
             (7 * q * 1.001, 7), (100.0, int((100.0 % (2 * math.pi)) / q)), (float("nan"), 0)]
    for phase, want in cases:
        assert oracle.phase_bucket(phase, precision) == want, (phase, want)


def test_phase_bucket_f32_rounding_at_boundaries():
    """The f32 formula step by step in numpy float32 (fmod exact, + and / rounded
    once each, truncation, clamp to 7), at the float neighbours of every bucket
    boundary in [-4 pi, 4 pi] and at random phases: pins the operation order,
    which decides the bucket of boundary phases."""
    tau = np.float32(2 * np.pi)
    width = np.float32(tau / np.float32(8))
    pts = []
    for k in range(-32, 33):
        b = np.float32(k * np.pi / 4)
        lo = b
        for _ in range(3):
            lo = np.nextafter(lo, np.float32(-np.inf))
        hi = b
        for _ in range(3):
            hi = np.nextafter(hi, np.float32(np.inf))
        x = lo
        while x <= hi:
            pts.append(x)
            x = np.nextafter(x, np.float32(np.inf))
    pts += list(np.random.default_rng(0).uniform(-20, 20, size=500).astype(np.float32))
    for p in pts:
        p = np.float32(p)
        nrm = np.fmod(np.fmod(p, tau) + tau, tau)
        want = min(int(nrm / width), 7)
        assert oracle.phase_bucket(float(p), "f32") == want, float(p)


# ------------------------------------------------------------ independent restatement

def numpy_wave_fwd(x, w, phase=None):
    """Matrix-form f64 restatement: the mask is built from its definition (causal,
    and key bucket within one of the query's bucket mod 8, or the previous
    position), not from bucket lists."""
    x = x.astype(np.float64)
    H, P, E = w["proj_w"].shape
    C = P - 2
    T = x.shape[0]
    hd = E // H
    merged = np.zeros((T, E))
    att_all = np.zeros((H, T, T))
    for h in range(H):
        raw = float(w["hraw"][h])
        n = raw if raw > 20 else math.log1p(math.exp(raw))
        proj = x @ w["proj_w"][h].astype(np.float64).T + w["proj_b"][h]
        ph = np.arctan2(proj[:, 1], proj[:, 0]) if phase is None else phase[h].astype(np.float64)
        bk = np.array([oracle.phase_bucket(p, "f64") for p in ph])
        mask = np.zeros((T, T), bool)
        for qi in range(T):
            for ki in range(qi + 1):
                rel = (bk[ki] - bk[qi]) % 8 in (0, 1, 7)
                mask[qi, ki] = rel or ki == qi - 1 or ki == qi
        s = np.cos(n * (ph[:, None] - ph[None, :]))
        if C > 0:
            c = proj[:, 2:]
            s = s + (c @ c.T) / math.sqrt(C)
        s = np.where(mask, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        v = x[:, h * hd:(h + 1) * hd] @ w["v_w"][h].astype(np.float64).T + w["v_b"][h]
        merged[:, h * hd:(h + 1) * hd] = p @ v
        att_all[h] = p
    out = merged @ w["out_w"].astype(np.float64).T + w["out_b"]
    return out, merged, att_all


@pytest.mark.parametrize("C", [0, 3, 16])
def test_oracle_matches_matrix_form(C):
    T, E, H = 40, 24, 3
    w = make_weights(H, C, E, seed=11 + C)
    x = np.random.default_rng(5).normal(size=(T, E)).astype(np.float32)
    want_out, want_merged, want_att = numpy_wave_fwd(x, w)
    r64 = oracle.wave_fwd(x, w, "f64")
    np.testing.assert_allclose(r64["merged"], want_merged, rtol=0, atol=1e-12)
    np.testing.assert_allclose(r64["out"], want_out, rtol=0, atol=1e-12)
    att = np.where(np.isneginf(r64["att"]), 0.0, r64["att"])
    np.testing.assert_allclose(att, want_att, rtol=0, atol=1e-14)
    # the f32 reference-order run agrees with the ground truth to f32 rounding
    r32 = oracle.wave_fwd(x, w, "f32", phase_in=r64["phase"].astype(np.float32))
    np.testing.assert_allclose(r32["out"], want_out, rtol=0, atol=2e-5)


def test_att_rows_follow_the_reference_contract():
    T, E, H, C = 33, 16, 2, 4
    w = make_weights(H, C, E, seed=3)
    x = np.random.default_rng(9).normal(size=(T, E)).astype(np.float32)
    r = oracle.wave_fwd(x, w, "f64")
    for h in range(H):
        for qi in range(T):
            row = r["att"][h, qi]
            assert np.all(np.isneginf(row[qi + 1:]))          # untouched past the diagonal (attn.rs:187, :240)
            assert abs(row[:qi + 1].sum() - 1.0) < 1e-12
            assert row[qi] > 0 and (qi == 0 or row[qi - 1] > 0)  # self and previous always attended
        # the sparsity pattern is the bucket relation
        bk = [oracle.phase_bucket(p, "f64") for p in r["phase"][h]]
        for qi in range(T):
            for ki in range(qi - 1):
                assert (r["att"][h, qi, ki] > 0) == ((bk[ki] - bk[qi]) % 8 in (0, 1, 7))
    np.testing.assert_allclose(np.exp(r["lse"]).shape, (H, T))


def test_closed_form_single_bucket_no_content():
    """Phase projection 0 with bias (r, s) = (1, 0): every phase is 0, one bucket,
    every score cos(0) = 1, so each row averages the causal prefix of the values
    and the harmonic gradient vanishes."""
    T, E, H = 17, 8, 2
    w = make_weights(H, 0, E, seed=1)
    w["proj_w"][:] = 0
    w["proj_b"][:, 0], w["proj_b"][:, 1] = 1.0, 0.0
    x = np.random.default_rng(2).normal(size=(T, E)).astype(np.float64)
    r = oracle.wave_fwd(x, w, "f64")
    hd = E // H
    for h in range(H):
        v = r["values"][h]
        want = np.cumsum(v, axis=0) / np.arange(1, T + 1)[:, None]
        np.testing.assert_allclose(r["merged"][:, h * hd:(h + 1) * hd], want, atol=1e-13)
    g = oracle.wave_bwd(x, w, np.random.default_rng(3).normal(size=(T, E)), "f64")
    np.testing.assert_allclose(g["d_hraw"], 0.0, atol=1e-14)
    np.testing.assert_allclose(g["d_proj_w"], 0.0, atol=1e-14)  # dS sums to zero per row, phases all equal


# ------------------------------------------------------------ finite differences

def _loss(x, w, dy, phase_ref):
    r = oracle.wave_fwd(x, w, "f64")
    same = all(oracle.phase_bucket(a, "f64") == oracle.phase_bucket(b, "f64")
               for a, b in zip(r["phase"].ravel(), phase_ref.ravel()))
    return float((r["out"] * dy).sum()), same


@pytest.mark.parametrize("C", [0, 4])
def test_backward_matches_finite_differences(C):
    T, E, H = 14, 12, 2
    w = {k: v.astype(np.float64) for k, v in make_weights(H, C, E, seed=21 + C).items()}
    rng = np.random.default_rng(8)
    x = rng.normal(size=(T, E))
    dy = rng.normal(size=(T, E))
    base = oracle.wave_fwd(x, w, "f64")
    g = oracle.wave_bwd(x, w, dy, "f64")
    eps = 1e-6
    checked = 0
    targets = [("x", None), ("hraw", "d_hraw"), ("proj_w", "d_proj_w"), ("proj_b", "d_proj_b"),
               ("v_w", "d_v_w"), ("v_b", "d_v_b"), ("out_w", "d_out_w"), ("out_b", "d_out_b")]
    for name, gname in targets:
        arr = x if name == "x" else w[name]
        grad = g["d_x"] if name == "x" else g[gname]
        for idx in [tuple(rng.integers(0, s) for s in arr.shape) for _ in range(6)]:
            old = arr[idx]
            arr[idx] = old + eps
            lp, okp = _loss(x, w, dy, base["phase"])
            arr[idx] = old - eps
            lm, okm = _loss(x, w, dy, base["phase"])
            arr[idx] = old
            if not (okp and okm):
                continue  # a bucket boundary lies inside the step: the loss is not differentiable there
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - grad[idx]) <= 1e-6 * max(1.0, abs(fd)), (name, idx, fd, grad[idx])
            checked += 1
    assert checked >= 40


# ------------------------------------------------------------ KV-cache serving

@pytest.mark.parametrize("precision", ["f32", "f64"])
def test_kv_prefill_is_the_forward_without_content(precision):
    """kv_cache::prefill scores phases only (kv_cache.rs:150-162): the forward
    with the content rows removed gives the same result."""
    T, E, H, C = 30, 24, 3, 4
    w = make_weights(H, C, E, seed=4)
    x = np.random.default_rng(1).normal(size=(T, E)).astype(np.float32)
    p = oracle.wave_kv_prefill(x, w, precision)
    w0 = dict(w, proj_w=w["proj_w"][:, :2].copy(), proj_b=w["proj_b"][:, :2].copy())
    f = oracle.wave_fwd(x, w0, precision)
    np.testing.assert_array_equal(p["out"], f["out"])
    np.testing.assert_array_equal(p["phase"], f["phase"])
    np.testing.assert_array_equal(p["values"], f["values"])


@pytest.mark.parametrize("precision", ["f32", "f64"])
def test_kv_step_equals_the_last_prefill_row(precision):
    """forward_one after prefilling t positions reproduces row t of a prefill
    over t+1 positions bit for bit (self score 1 = cos 0, the same mask and the
    same summation order), for every t."""
    T, E, H, C = 21, 16, 2, 3
    w = make_weights(H, C, E, seed=6)
    x = np.random.default_rng(2).normal(size=(T, E)).astype(np.float32)
    full = oracle.wave_kv_prefill(x, w, precision)
    cap = T + 3
    hd = E // H
    dt = np.float32 if precision == "f32" else np.float64
    phases = np.zeros((H, cap), dt)
    values = np.zeros((H, cap, hd), dt)
    for t in range(T):
        st = oracle.wave_kv_step(x[t], w, phases, values, t, precision)
        np.testing.assert_array_equal(st["out"], full["out"][t])
        np.testing.assert_array_equal(st["phase_new"], full["phase"][:, t])
        phases[:, t] = st["phase_new"]
        values[:, t] = st["v_new"]


def test_phases_follow_atan2_and_the_bucket_formula():
    """oracle.phases: f32 atan2 of (s, r) then phase_to_bucket, element by element
    equal to the scalar bucket function; f64 phases equal numpy's arctan2
    (closed forms at the axes and diagonals included)."""
    r = np.array([1.0, 0.0, -1.0, 0.0, 1.0, -1.0, 0.3, -2.5], np.float32)
    s = np.array([0.0, 1.0, 0.0, -1.0, 1.0, -1.0, 0.7, 0.1], np.float32)
    ph, bk = oracle.phases(r, s, "f32")
    np.testing.assert_allclose(ph[:6], [0.0, np.pi / 2, np.pi, -np.pi / 2, np.pi / 4, -3 * np.pi / 4], rtol=1e-7)
    assert bk.tolist() == [oracle.phase_bucket(float(p), "f32") for p in ph]
    assert bk[0] == 0 and bk[4] in (0, 1)           # pi/4 sits on the 0|1 bucket boundary
    ph64, _ = oracle.phases(r.astype(np.float64), s.astype(np.float64), "f64")
    np.testing.assert_array_equal(ph64, np.arctan2(s.astype(np.float64), r.astype(np.float64)))
    rng = np.random.default_rng(0)
    rr, ss = rng.normal(size=1000).astype(np.float32), rng.normal(size=1000).astype(np.float32)
    p2, b2 = oracle.phases(rr, ss, "f32")
    np.testing.assert_allclose(p2, np.arctan2(ss.astype(np.float64), rr.astype(np.float64)), atol=4e-7)
    assert b2.tolist() == [oracle.phase_bucket(float(p), "f32") for p in p2]
