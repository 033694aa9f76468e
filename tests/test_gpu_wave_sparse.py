"""The bucket-sparse wave attention kernels under bucket layouts that stress
their schedule, against the oracle (src/common/attn.rs:167-224: the mask
admits k <= q with bucket(k) within one of bucket(q) mod 8, or k = q - 1).

The phase projection is set so that the buckets take a chosen pattern:
every position in one bucket (every window is the whole sequence), two
opposite buckets 2 and 6 in random order (windows with gaps; most k = q - 1
pairs are admitted only by the previous-position rule, which lies outside
every window), and buckets 7 and 0 (windows that wrap around the bucket
order).  Each runs with both kernel families; forward (merged, LSE, out) and
backward (d_x and every weight gradient) meet the parity bar against the
oracle with the device's phases replayed.

d_harmonic_raw is a sum over positions of phi * dphi / n; with every phase
near zero (the wrap pattern) its terms cancel, and the f32 oracle itself is
1.1e-5 from the f64 oracle in relative L2 at T = 1024.  That gradient is
therefore checked against the f64 oracle, within the bar or twice the f32
oracle's own distance from f64, whichever is larger."""
import math

import numpy as np
import pytest

import oracle
from conftest import REL_L2, assert_parity, errors, make_wave_weights

pytestmark = pytest.mark.gpu

TAU = 2 * math.pi


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available()
    return torch, torch.device("cuda:0")


def _weights(H, C, E, pattern, seed):
    w = make_wave_weights(H, C, E, seed)
    pw, pb = w["proj_w"], w["proj_b"]
    pw[:, :2, :] = 0.0
    pb[:, :2] = 0.0
    if pattern == "one":
        th = 3.5 * TAU / 8  # the middle of bucket 3
        pb[:, 0], pb[:, 1] = math.cos(th), math.sin(th)
    elif pattern == "far":
        th = 2.5 * TAU / 8  # (r, s) = x0 (cos th, sin th): bucket 2 for x0 > 0, 6 for x0 < 0
        pw[:, 0, 0], pw[:, 1, 0] = math.cos(th), math.sin(th)
    elif pattern == "wrap":
        pb[:, 0] = 1.0      # (r, s) = (1, 0.3 x0): bucket 0 for x0 >= 0, 7 for x0 < 0 (|x0| < 3.3)
        pw[:, 1, 0] = 0.3
    return w


def _expected_buckets(pattern):
    return {"one": {3}, "far": {2, 6}, "wrap": {0, 7}}[pattern]


@pytest.mark.parametrize("pattern", ["one", "far", "wrap"])
@pytest.mark.parametrize("sparse", [True, False])
@pytest.mark.parametrize("B,T,E,H,C", [(2, 300, 128, 2, 16), (1, 1024, 256, 4, 5)])
def test_bucket_patterns_match_oracle(pkg, torch_dev, pattern, sparse, B, T, E, H, C):
    torch, dev = torch_dev
    print(f"wave pattern {pattern} sparse={sparse} B{B} T{T} E{E} H{H} C{C}", flush=True)
    prev = pkg.wave_set_bucket_sparse(sparse)
    try:
        w = _weights(H, C, E, pattern, seed=5 + T)
        rng = np.random.default_rng(T)
        x = rng.normal(size=(B, T, E)).astype(np.float32)
        x[..., 0] = np.clip(x[..., 0], -3.0, 3.0)
        dy = (rng.normal(size=(B, T, E)) / math.sqrt(B * T)).astype(np.float32)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        W = pkg.WaveAttnWeights(t(w["hraw"]), t(w["proj_w"]), t(w["proj_b"]), t(w["v_w"]), t(w["v_b"]),
                                t(w["out_w"]), t(w["out_b"]))
        out, _, cache = pkg.wave_attention_forward(W, t(x))
        grads = pkg.wave_attention_backward_full(W, cache, t(dy))
        torch.cuda.synchronize()
        bk = cache.bucket.cpu().numpy()
        assert set(np.unique(bk)) == _expected_buckets(pattern)
        phase = cache.phase.cpu().numpy()
        merged, lse = cache.merged.cpu().numpy(), cache.lse.cpu().numpy()
        refs = []
        for b in range(B):
            ref = oracle.wave_fwd(x[b], w, "f32", phase_in=phase[b])
            assert_parity(f"merged b{b}", merged[b], ref["merged"])
            assert_parity(f"lse b{b}", lse[b], ref["lse"])
            assert_parity(f"out b{b}", out[b].cpu().numpy(), ref["out"])
            refs.append(oracle.wave_bwd(x[b], w, dy[b], "f32", phase_in=phase[b]))
            refs[-1]["d_hraw64"] = oracle.wave_bwd(x[b], w, dy[b], "f64", phase_in=phase[b])["d_hraw"]
        got_dx = grads.d_normed.cpu().numpy()
        for b in range(B):
            assert_parity(f"d_x b{b}", got_dx[b], refs[b]["d_x"])
        s = lambda k: np.sum([r[k] for r in refs], axis=0, dtype=np.float64)
        h32, h64 = s("d_hraw"), s("d_hraw64")
        _, cond = errors(h32, h64)
        assert_parity("d_harmonic_raw vs f64", grads.d_harmonic_raw.cpu().numpy(), h64, rel_l2=max(REL_L2, 2 * cond))
        assert_parity("d_proj_w", grads.d_proj_w.cpu().numpy(), s("d_proj_w"))
        assert_parity("d_proj_b", grads.d_proj_b.cpu().numpy(), s("d_proj_b"))
        assert_parity("d_v_w", grads.d_v_w.cpu().numpy(), s("d_v_w"))
        assert_parity("d_v_b", grads.d_v_b.cpu().numpy(), s("d_v_b"))
        assert_parity("d_out_w", grads.out_proj_w.cpu().numpy(), s("d_out_w"))
        assert_parity("d_out_b", grads.out_proj_b.cpu().numpy(), s("d_out_b"))
    finally:
        pkg.wave_set_bucket_sparse(prev)


def test_families_agree_at_model_shape(pkg, torch_dev):
    """The 768-dim model shape (B=8, T=1024, 12 heads, content 16): the two
    kernel families on the same input agree within the parity bar (they sum
    in different orders), and the sparse family is deterministic."""
    torch, dev = torch_dev
    B, T, E, H, C = 8, 1024, 768, 12, 16
    print("wave families at the model shape", flush=True)
    w = make_wave_weights(H, C, E, seed=2024)
    x = np.random.default_rng(2025).normal(size=(B, T, E)).astype(np.float32)
    dy = (np.random.default_rng(2026).normal(size=(B, T, E)) / math.sqrt(B * T)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    W = pkg.WaveAttnWeights(t(w["hraw"]), t(w["proj_w"]), t(w["proj_b"]), t(w["v_w"]), t(w["v_b"]), t(w["out_w"]),
                            t(w["out_b"]))
    res = {}
    prev = pkg.wave_set_bucket_sparse(True)
    try:
        for sparse in (True, False, True):
            pkg.wave_set_bucket_sparse(sparse)
            out, _, cache = pkg.wave_attention_forward(W, t(x))
            g = pkg.wave_attention_backward_full(W, cache, t(dy))
            torch.cuda.synchronize()
            r = {"out": out.cpu().numpy(), "lse": cache.lse.cpu().numpy(), "d_x": g.d_normed.cpu().numpy(),
                 "d_proj_w": g.d_proj_w.cpu().numpy(), "d_v_w": g.d_v_w.cpu().numpy()}
            if sparse and sparse in res:
                for k in r:
                    np.testing.assert_array_equal(r[k], res[sparse][k], err_msg=k)
            res[sparse] = r
    finally:
        pkg.wave_set_bucket_sparse(prev)
    for k in res[True]:
        assert_parity(f"sparse vs dense {k}", res[True][k], res[False][k])
