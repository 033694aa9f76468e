"""Pins for the oracle's projection restatements (CPU): linear_batch_cpu
(src/common/compute.rs:441-468), linear_backward_dx_only
(src/common/math/backward.rs:36-46), outer_product_accum
(src/common/compute.rs:263-282) and attention_cpu end to end (:357-414)."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_out_proj_backward_kat():
    """src/common/math/attn_backward.rs:336-349: identity W, two positions."""
    k = json.loads((GOLDEN / "attn_kat.json").read_text())["out_proj_backward"]
    d_attn, merged, w = (np.array(k[x]) for x in ("d_attn", "merged", "w"))
    for prec in ("f32", "f64"):
        d_out = oracle.linear_backward_dx(d_attn, w, prec)
        d_w, d_b = oracle.outer_product_accum(d_attn, merged, True, prec)
        e = k["expected"]
        assert abs(d_out[0][0] - e["d_out_0_0"]) < k["tol"]
        assert abs(d_out[0][1] - e["d_out_0_1"]) < k["tol"]
        assert abs(d_w[0][0] - e["d_w_0_0"]) < k["tol"]
        assert abs(d_b[0] - e["d_b_0"]) < k["tol"]


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 3, 7), (33, 17, 65), (64, 96, 32)])
def test_linear_family_matches_matrix_form(M, N, K):
    r = np.random.default_rng(M * 100 + N)
    x = r.standard_normal((M, K))
    w = r.standard_normal((N, K))
    b = r.standard_normal(N)
    dy = r.standard_normal((M, N))
    np.testing.assert_allclose(oracle.linear(x, w, b, "f64"), x @ w.T + b, atol=1e-12)
    np.testing.assert_allclose(oracle.linear(x, w, None, "f64"), x @ w.T, atol=1e-12)
    np.testing.assert_allclose(oracle.linear_backward_dx(dy, w, "f64"), dy @ w, atol=1e-12)
    dw, db = oracle.outer_product_accum(dy, x, True, "f64")
    np.testing.assert_allclose(dw, dy.T @ x, atol=1e-12)
    np.testing.assert_allclose(db, dy.sum(0), atol=1e-12)
    dw2, db2 = oracle.outer_product_accum(dy, x, False, "f64")
    np.testing.assert_allclose(dw2, dw, atol=0)
    assert np.all(db2 == 0)


def test_linear_closed_forms():
    r = np.random.default_rng(1)
    x = r.standard_normal((6, 4)).astype(np.float32)
    b = r.standard_normal(4).astype(np.float32)
    # identity weights: y = x + b exactly (each sum has one non-zero term)
    np.testing.assert_array_equal(oracle.linear(x, np.eye(4, dtype=np.float32), b, "f32"), x + b)
    # zero weights: y = b
    np.testing.assert_array_equal(oracle.linear(x, np.zeros((4, 4), np.float32), b, "f32"), np.tile(b, (6, 1)))


def test_attention_full_composes_projections_and_core():
    """attention_cpu = c_proj(core(split(c_attn(x)))) -- checked against the
    independent matrix form, and the identity-projection case reduces to the core."""
    T, H, D = 19, 3, 8
    E = H * D
    r = np.random.default_rng(7)
    x = r.standard_normal((T, E))
    wa, ba = r.standard_normal((3 * E, E)) / np.sqrt(E), r.standard_normal(3 * E)
    wp, bp = r.standard_normal((E, E)) / np.sqrt(E), r.standard_normal(E)
    got = oracle.attention_full(x, wa, ba, wp, bp, H, "f64")
    qkv = x @ wa.T + ba
    q, k, v = qkv[:, :E], qkv[:, E:2 * E], qkv[:, 2 * E:]
    mask = np.tril(np.ones((T, T), bool))
    o = np.zeros((T, E))
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        s = np.where(mask, q[:, sl] @ k[:, sl].T / np.sqrt(D), -np.inf)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        o[:, sl] = p @ v[:, sl]
    np.testing.assert_allclose(got, o @ wp.T + bp, atol=1e-12)
    # identity c_attn blocks and c_proj, zero biases: attention(x) = core(x, x, x)
    eye = np.eye(E)
    got_id = oracle.attention_full(x, np.vstack([eye, eye, eye]), np.zeros(3 * E), eye, np.zeros(E), H, "f64")
    np.testing.assert_allclose(got_id, oracle.core_fwd(x, x, x, H, "f64"), atol=1e-12)
