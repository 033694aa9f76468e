"""The reference-interface mirrors on the GPU: the C++ HipBackend test program
(tests/cpp/test_hip_backend.cpp) and the Python HipBackend, both against the
CPU oracle with the reference's per-sequence [T][n_embd] layout and its
att-as-given backward contract (src/common/compute.rs:163-173, :286-314)."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from conftest import assert_parity

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


def test_cpp_host_mirror_program():
    exe = ROOT / "tests" / "cpp" / "test_hip_backend"
    assert exe.exists(), "build it with __graft_entry__.build()"
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=180)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout[-2000:]
    assert "test result: ok" in r.stdout


@pytest.mark.parametrize("T,E,H", [(64, 168, 4), (200, 384, 8), (300, 768, 12), (1, 64, 1)])
def test_python_host_mirror(pkg, T, E, H):
    g = oracle.Xorshift64(T + E)
    D = E // H
    q, k, v = (g.normal(T * E, 1.0 / np.sqrt(D)).reshape(T, E) for _ in range(3))
    d = g.normal(T * E, 1.0).reshape(T, E)
    o_ref, att = oracle.core_fwd(q, k, v, H, "f32", want_att=True)
    be = pkg.HipBackend()
    assert_parity("attention_core", be.attention_core(q, k, v, H), o_ref)
    dq, dk, dv = be.attention_backward(d, q.tolist(), k, v, att, H)  # rows as Vec<Vec<f32>> too
    rq, rk, rv = oracle.attention_backward(d, q, k, v, att, H, "f32")
    assert_parity("d_q", dq, rq)
    assert_parity("d_k", dk, rk)
    assert_parity("d_v", dv, rv)


@pytest.mark.parametrize("T,E,H", [(200, 384, 8), (300, 768, 12), (257, 1024, 8), (64, 224, 4)])
def test_host_backward_takes_the_direct_to_lds_kernels(pkg, T, E, H):
    """wha_host_attention_backward at head dims 48, 64, 128 and 56 (padded):
    the staged [T][E] operands are 16-byte aligned, so the exact-contract
    backward runs the direct-to-LDS kernels (Delta pass on the forward's tiles,
    key-stationary dK/dV/dS, dQ from dS), not the register-staged ones (timed
    as attn_bwd_probs_*_rs); results against the oracle."""
    g = oracle.Xorshift64(3 * T + E)
    D = E // H
    q, k, v = (g.normal(T * E, 1.0 / np.sqrt(D)).reshape(T, E) for _ in range(3))
    d = g.normal(T * E, 1.0).reshape(T, E)
    _, att = oracle.core_fwd(q, k, v, H, "f32", want_att=True)
    be = pkg.HipBackend()
    pkg.timing_enable(True)
    pkg.timing_reset()
    try:
        dq, dk, dv = be.attention_backward(d, q, k, v, att, H)
        fast = [pkg.timing_read(f"attn_bwd_probs_{n}")[1] for n in ("delta", "dkv", "dq")]
        slow = [pkg.timing_read(f"attn_bwd_probs_{n}_rs")[1] for n in ("delta", "dkv", "dq")]
    finally:
        pkg.timing_enable(False)
    assert fast == [1, 1, 1] and slow == [0, 0, 0], (fast, slow)
    rq, rk, rv = oracle.attention_backward(d, q, k, v, att, H, "f32")
    assert_parity("d_q", dq, rq)
    assert_parity("d_k", dk, rk)
    assert_parity("d_v", dv, rv)


@pytest.mark.parametrize("T,E,H,C", [(90, 64, 4, 16), (33, 168, 4, 0)])
def test_python_host_wave_mirror(pkg, T, E, H, C):
    """HipBackend's host-array wave attention (attn.rs:90-511) against the oracle
    replaying the device phases."""
    from conftest import make_wave_weights
    w = make_wave_weights(H, C, E, seed=T)
    rng = np.random.default_rng(T + 1)
    x = rng.normal(size=(T, E)).astype(np.float32)
    dy = (rng.normal(size=(T, E)) / np.sqrt(T)).astype(np.float32)
    be = pkg.HipBackend()
    out, ph = be.wave_attention_forward(w, x, n_bands=E // 2, want_phases=True)
    ref = oracle.wave_fwd(x, w, "f32", phase_in=ph)
    assert_parity("wave out", out, ref["out"])
    g = be.wave_attention_backward(w, x, dy)
    rg = oracle.wave_bwd(x, w, dy, "f32", phase_in=ph)
    for k in ("d_x", "d_hraw", "d_proj_w", "d_proj_b", "d_v_w", "d_v_b", "d_out_w", "d_out_b"):
        assert_parity(k, g[k], rg[k])
    np.testing.assert_array_equal(be.wave_attention_backward(w, x, dy, full=False), g["d_x"])
