"""Pins for the CPU oracle (runs on the CPU).

The oracle restates attention_cpu (src/common/compute.rs:377-409) and
attention_backward_single (src/cpu/backward.rs:313-363).  Nothing here retypes
its formulas: the checks are the reference's own known-answer tests, an
independent matrix-form restatement in f64, closed forms, invariants and a
finite-difference check of the backward against the forward.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from conftest import errors

GOLDEN = Path(__file__).resolve().parent / "golden"


def rand_seq(T, H, D, seed, scale_qk=None):
    rng = np.random.default_rng(seed)
    E = H * D
    sd = 1.0 / np.sqrt(D) if scale_qk is None else scale_qk
    q = (rng.standard_normal((T, E)) * sd).astype(np.float32)
    k = (rng.standard_normal((T, E)) * sd).astype(np.float32)
    v = (rng.standard_normal((T, E)) * sd).astype(np.float32)
    do = rng.standard_normal((T, E)).astype(np.float32)
    return q, k, v, do


def matrix_form(q, k, v, do, H):
    """Independent restatement: whole-matrix causal attention and its gradient in f64,
    per head, from the textbook formulas (no loops over positions)."""
    T, E = q.shape
    D = E // H
    sc = 1.0 / np.sqrt(np.float64(np.float32(D)))
    out = np.zeros((T, E)); dq = np.zeros((T, E)); dk = np.zeros((T, E)); dv = np.zeros((T, E))
    lse = np.zeros((H, T)); P_all = np.zeros((H, T, T))
    mask = np.tril(np.ones((T, T), dtype=bool))
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        Q, K, V, dO = (a[:, sl].astype(np.float64) for a in (q, k, v, do))
        S = np.where(mask, Q @ K.T * sc, -np.inf)
        m = S.max(axis=1, keepdims=True)
        Pu = np.exp(S - m)
        l = Pu.sum(axis=1, keepdims=True)
        P = Pu / l
        out[:, sl] = P @ V
        dP = dO @ V.T
        dS = P * (dP - (P * dP).sum(axis=1, keepdims=True))
        dq[:, sl] = dS @ K * sc
        dk[:, sl] = dS.T @ Q * sc
        dv[:, sl] = P.T @ dO
        lse[h] = (m + np.log(l))[:, 0]
        P_all[h] = P
    return out, dq, dk, dv, lse, P_all


def oracle_fwd_bwd(q, k, v, do, H, precision):
    o, att, lse = oracle.core_fwd(q, k, v, H, precision, want_att=True, want_lse=True)
    dq, dk, dv = oracle.attention_backward(do, q, k, v, att, H, precision)
    return o, dq, dk, dv, lse, att


# ------------------------------------------------------------ reference KATs

def test_softmax_backward_kat():
    """src/common/math/attn_backward.rs:352-365, through the oracle's softmax-Jacobian step."""
    kat = json.loads((GOLDEN / "attn_kat.json").read_text())["softmax_backward"]
    att, d_att = np.array(kat["att"]), np.array(kat["d_att"])
    for prec in ("f32", "f64"):
        rows = [oracle.softmax_backward_row(att[qi, :qi + 1], d_att[qi, :qi + 1], prec) for qi in range(2)]
        for e in kat["expected"]:
            assert abs(rows[e["row"]][e["col"]] - e["value"]) <= e["tol"], (prec, e)


def test_value_aggregation_backward_kat():
    """src/common/math/attn_backward.rs:367-379, through the oracle's value step,
    accumulating over query positions as the reference's driver does."""
    kat = json.loads((GOLDEN / "attn_kat.json").read_text())["value_aggregation_backward"]
    att, v, d_out = (np.array(kat[x]) for x in ("att", "v", "d_out"))
    for prec in ("f32", "f64"):
        dt = np.float32 if prec == "f32" else np.float64
        dv = np.zeros((2, 2), dtype=dt)
        d_att = [oracle.value_backward_row(d_out[qi], v, dv, att[qi, :qi + 1], prec) for qi in range(2)]
        assert abs(d_att[0][0] - kat["expected_d_att_0_0"]) <= kat["tol"]
        np.testing.assert_allclose(dv[0], kat["expected_d_v_0"], atol=kat["tol"])


def test_kats_through_full_backward():
    """Both KATs embedded in one call of the full backward (T=2, one head, D=2):
    V = I makes d_att[pos] = d_out[pos], so the softmax KAT's d_att = [[1,0],[2,4]]
    is produced by d_out = [[1,0],[2,4]]; Q = K = I then gives
    dQ[1] = scale*(dS[1][0]*K[0] + dS[1][1]*K[1]) = scale*[-0.42, 0.42]."""
    kat = json.loads((GOLDEN / "attn_kat.json").read_text())
    att = np.array(kat["softmax_backward"]["att"])[None]
    eye = np.eye(2)
    d_out = np.array(kat["softmax_backward"]["d_att"])
    dq, dk, dv = oracle.attention_backward(d_out, eye, eye, eye, att, 1, "f64")
    sc = 1.0 / np.sqrt(2.0)
    np.testing.assert_allclose(dq[1], sc * np.array([-0.42, 0.42]), atol=1e-12)
    np.testing.assert_allclose(dq[0], [0.0, 0.0], atol=1e-12)
    # dV[0] = att[0][0]*d_out[0] + att[1][0]*d_out[1]
    np.testing.assert_allclose(dv[0], [1.0 + 0.3 * 2.0, 0.0 + 0.3 * 4.0], atol=1e-12)
    va = kat["value_aggregation_backward"]
    dq, dk, dv = oracle.attention_backward(np.array(va["d_out"]), eye, eye, np.array(va["v"]),
                                           np.array(va["att"])[None], 1, "f64")
    np.testing.assert_allclose(dv[0], va["expected_d_v_0"], atol=1e-12)


# ------------------------------------------------------------ independent restatement

@pytest.mark.parametrize("T,H,D,seed", [(1, 1, 4, 0), (5, 2, 3, 1), (17, 3, 8, 2), (33, 4, 42, 3),
                                        (40, 2, 48, 4), (64, 1, 64, 5), (70, 2, 128, 6)])
def test_oracle_f64_matches_matrix_form(T, H, D, seed):
    q, k, v, do = rand_seq(T, H, D, seed)
    ref = matrix_form(q, k, v, do, H)
    got = oracle_fwd_bwd(q, k, v, do, H, "f64")
    for name, g, w in zip(("O", "dQ", "dK", "dV", "LSE", "att"), got, ref[:4] + (ref[4], ref[5])):
        ma, rl = errors(g, w)
        assert ma < 1e-12, (name, ma)


@pytest.mark.parametrize("T,H,D,seed", [(33, 4, 42, 3), (128, 2, 64, 7)])
def test_oracle_f32_close_to_f64(T, H, D, seed):
    q, k, v, do = rand_seq(T, H, D, seed)
    g32 = oracle_fwd_bwd(q, k, v, do, H, "f32")
    g64 = oracle_fwd_bwd(q, k, v, do, H, "f64")
    for name, a, b in zip(("O", "dQ", "dK", "dV"), g32, g64):
        ma, rl = errors(a, b)
        assert ma < 1e-5 and rl < 1e-5, (name, ma, rl)


# ------------------------------------------------------------ finite differences

def test_backward_matches_finite_differences():
    """Central differences of L = <dO, O(Q,K,V)> in f64 (the method of
    src/monitors/junctions/grad_check.rs:117; eps 1e-4 default there, smaller here
    because everything is f64)."""
    T, H, D = 9, 2, 5
    q, k, v, do = (a.astype(np.float64) for a in rand_seq(T, H, D, 11))
    _, dq, dk, dv, _, _ = oracle_fwd_bwd(q, k, v, do, H, "f64")

    def loss(q_, k_, v_):
        return float((oracle.core_fwd(q_, k_, v_, H, "f64") * do).sum())

    eps = 1e-6
    rng = np.random.default_rng(0)
    for which, grad in (("q", dq), ("k", dk), ("v", dv)):
        for _ in range(12):
            i, j = int(rng.integers(T)), int(rng.integers(H * D))
            args = {"q": q.copy(), "k": k.copy(), "v": v.copy()}
            args[which][i, j] += eps
            lp = loss(args["q"], args["k"], args["v"])
            args[which][i, j] -= 2 * eps
            lm = loss(args["q"], args["k"], args["v"])
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - grad[i, j]) <= 1e-7 + 1e-6 * abs(fd), (which, i, j, fd, grad[i, j])


# ------------------------------------------------------------ closed forms

def test_single_position():
    """T=1: O = V, dV = dO, dQ = dK = 0, LSE = score."""
    q, k, v, do = rand_seq(1, 3, 7, 21)
    o, dq, dk, dv, lse, _ = oracle_fwd_bwd(q, k, v, do, 3, "f64")
    np.testing.assert_allclose(o, v, atol=1e-15)
    np.testing.assert_allclose(dv, do, atol=1e-15)
    np.testing.assert_allclose(dq, 0, atol=1e-15)
    np.testing.assert_allclose(dk, 0, atol=1e-15)


def test_zero_queries_give_uniform_rows():
    """Q = 0: every score is 0, P is uniform over the causal prefix, so
    O[i] = mean(V[0..=i]), LSE_i = ln(i+1) and dK = 0."""
    T, H, D = 12, 2, 6
    _, k, v, do = rand_seq(T, H, D, 3)
    q = np.zeros_like(k)
    o, dq, dk, dv, lse, _ = oracle_fwd_bwd(q, k, v, do, H, "f64")
    cum = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, T + 1)[:, None]
    np.testing.assert_allclose(o, cum, atol=1e-14)
    np.testing.assert_allclose(lse, np.log(np.arange(1, T + 1))[None].repeat(H, 0), atol=1e-14)
    np.testing.assert_allclose(dk, 0, atol=1e-15)


def test_constant_values_and_equal_keys():
    """V rows all equal c -> O = c.  All K rows equal -> P uniform and dQ = 0."""
    T, H, D = 10, 2, 4
    q, k, v, do = rand_seq(T, H, D, 5)
    c = np.arange(H * D, dtype=np.float32) * 0.25 - 1.0
    v_const = np.tile(c, (T, 1))
    o = oracle.core_fwd(q, k, v_const, H, "f64")
    np.testing.assert_allclose(o, np.tile(c, (T, 1)), atol=1e-14)
    k_eq = np.tile(k[3], (T, 1))
    _, dq, _, _, _, att = oracle_fwd_bwd(q, k_eq, v, do, H, "f64")
    np.testing.assert_allclose(dq, 0, atol=1e-14)
    for h in range(H):
        for i in range(T):
            np.testing.assert_allclose(att[h, i, :i + 1], 1.0 / (i + 1), atol=1e-15)


# ------------------------------------------------------------ invariants

def test_invariants():
    T, H, D = 24, 3, 8
    q, k, v, do = rand_seq(T, H, D, 9)
    o, dq, dk, dv, lse, att = oracle_fwd_bwd(q, k, v, do, H, "f64")
    # softmax rows sum to 1 and are causal (the value_range.rs:117-119 contract)
    np.testing.assert_allclose(att.sum(-1), 1.0, atol=1e-14)
    assert np.all(np.triu(att, 1) == 0)
    # sum_j dS[i,j] = 0  =>  sum over keys of dK = 0 per head
    for h in range(H):
        np.testing.assert_allclose(dk[:, h * D:(h + 1) * D].sum(0), 0, atol=1e-13)
    # causality: changing K, V at position j leaves O[<j] unchanged
    j = 15
    k2, v2 = k.copy(), v.copy()
    k2[j] += 1.0
    v2[j] -= 2.0
    o2 = oracle.core_fwd(q, k2, v2, H, "f64")
    np.testing.assert_array_equal(o2[:j], o[:j])
    assert np.abs(o2[j:] - o[j:]).max() > 1e-3
    # linear in V
    v_b = rand_seq(T, H, D, 10)[2].astype(np.float64)
    a, b = 0.75, -1.5
    o_lin = oracle.core_fwd(q, k, a * v.astype(np.float64) + b * v_b, H, "f64")
    np.testing.assert_allclose(o_lin, a * o + b * oracle.core_fwd(q, k, v_b, H, "f64"), atol=1e-13)


def test_decode_is_last_causal_row():
    T, H, D = 31, 2, 16
    q, k, v, _ = rand_seq(T, H, D, 13)
    o, lse = oracle.core_fwd(q, k, v, H, "f64", want_lse=True)
    od, lsed = oracle.decode_one(q[-1], k, v, H, "f64", want_lse=True)
    np.testing.assert_array_equal(od, o[-1])
    np.testing.assert_array_equal(lsed, lse[:, -1])
    o32 = oracle.core_fwd(q, k, v, H, "f32")
    np.testing.assert_array_equal(oracle.decode_one(q[-1], k, v, H, "f32"), o32[-1])


def test_batched_threaded_driver_matches_per_sequence():
    B, H, T, D = 3, 2, 20, 8
    q, k, v, do = oracle.synth_inputs(B, H, T, D, seed=5)
    qs, ks, vs, dos = (oracle.bhtd_to_seq(a) for a in (q, k, v, do))
    out, dq, dk, dv = oracle.batch_fwd_bwd_f32_threaded(qs, ks, vs, dos, H, nthreads=3)
    O, dQ, dK, dV, _ = oracle.fwd_bwd_bhtd(q, k, v, do, "f32")
    for a, b in ((out, O), (dq, dQ), (dk, dK), (dv, dV)):
        np.testing.assert_array_equal(oracle.seq_to_bhtd(a, H), b)
