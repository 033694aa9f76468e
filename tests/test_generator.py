"""Seeded input generator: the oracle's restatement of the reference's Rng
(src/common/rng.rs:24-34) and the product library's multi-threaded copy.

The xorshift step is pinned by a property the triple (13, 7, 17) is chosen for:
the step is a linear map M over GF(2)^64 and, for the full-period triples of
Marsaglia's xorshift family, M has multiplicative order exactly 2^64 - 1.  A
wrong shift amount or direction almost surely breaks that.  The Box-Muller layer
is this build's own definition: pinned by committed check values and moments.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
ORDER = (1 << 64) - 1
PRIME_FACTORS = (3, 5, 17, 257, 641, 65537, 6700417)  # 2^64 - 1 = 3*5*17*257*641*65537*6700417


def _step_columns():
    cols = []
    for j in range(64):
        r = oracle.Xorshift64(1 << j)
        cols.append(r.next_u64())
    return cols


def _apply(cols, v):
    r = 0
    j = 0
    while v:
        if v & 1:
            r ^= cols[j]
        v >>= 1
        j += 1
    return r


def _matmul(a, b):
    return [_apply(a, c) for c in b]


def _matpow(cols, n):
    result = [1 << j for j in range(64)]
    p = cols
    while n:
        if n & 1:
            result = _matmul(p, result)
        p = _matmul(p, p)
        n >>= 1
    return result


def test_prime_factorisation_of_period():
    prod = 1
    for p in PRIME_FACTORS:
        prod *= p
    assert prod == ORDER


def test_xorshift_step_has_full_period():
    cols = _step_columns()
    ident = [1 << j for j in range(64)]
    assert _matpow(cols, ORDER) == ident
    for p in PRIME_FACTORS:
        assert _matpow(cols, ORDER // p) != ident, p


def test_next_f32_is_top_24_bits():
    r1, r2 = oracle.Xorshift64(42), oracle.Xorshift64(42)
    for _ in range(100):
        u = r1.next_u64()
        f = r2.next_f32()
        assert f == (u >> 40) / float(1 << 24)
        assert 0.0 <= f < 1.0


def test_committed_check_values():
    data = json.loads((GOLDEN / "gen_check.json").read_text())
    for case in data["cases"]:
        r = oracle.Xorshift64(case["seed"])
        assert [str(r.next_u64()) for _ in range(8)] == case["next_u64"]
        r = oracle.Xorshift64(case["seed"])
        assert [r.next_f32() for _ in range(8)] == case["next_f32"]
        r = oracle.Xorshift64(case["seed"])
        assert [float(x) for x in r.normal(9, 1.0)] == case["normal_stddev1"]
        assert str(r.state.value) == case["state_after_9_normals"]


def test_normal_moments():
    x = oracle.Xorshift64(7).normal(1_000_000, 1.0).astype(np.float64)
    assert abs(x.mean()) < 5e-3
    assert abs(x.var() - 1.0) < 5e-3
    assert abs((x ** 3).mean()) < 1e-2          # symmetric
    assert abs((x ** 4).mean() - 3.0) < 3e-2    # normal kurtosis


@pytest.mark.parametrize("n,threads", [(1, 1), (7, 1), (1000, 4), (3_000_001, 0), (2_500_000, 5)])
def test_library_generator_matches_oracle(pkg, n, threads):
    """The product's jump-ahead threaded generator reproduces the sequential stream."""
    a = oracle.Xorshift64(42)
    want = a.normal(n, 0.125)
    g = pkg.SynthStream(42)
    got = g.normal(n, 0.125, nthreads=threads)
    np.testing.assert_array_equal(got, want)
    assert g.state.value == a.state.value
    # and the stream continues identically
    np.testing.assert_array_equal(g.normal(5, 1.0), a.normal(5, 1.0))


def test_synth_inputs_draw_order(pkg):
    B, H, T, D = 2, 3, 5, 4
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=42)
    oq, ok, ov, odo = oracle.synth_inputs(B, H, T, D, seed=42)
    for a, b in ((q, oq), (k, ok), (v, ov), (do, odo)):
        np.testing.assert_array_equal(a, b)
    r = oracle.Xorshift64(42)
    np.testing.assert_array_equal(q.reshape(-1), r.normal(B * H * T * D, 0.5))
