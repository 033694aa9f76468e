"""The bucket-sparse wave attention kernels under bucket layouts that stress
their schedule, against the oracle (src/common/attn.rs:167-224: the mask
admits k <= q with bucket(k) within one of bucket(q) mod 8, or k = q - 1).

The phase projection is set so that the buckets take a chosen pattern:
every position in one bucket (every window is the whole sequence), two
opposite buckets 2 and 6 in random order (windows with gaps; most k = q - 1
pairs are admitted only by the previous-position rule, which lies outside
every window), buckets 7 and 0 (windows that wrap around the bucket
order), and every bucket with the content projections four times larger
("loud": each row's scores span tens of log2 units, so the bucket-sparse
forward's running maximum moves by more than its lazy threshold again and
again).  Each runs with both kernel families; forward (merged, LSE, out) and
backward (d_x and every weight gradient) meet the parity bar against the
oracle with the device's phases replayed.

d_harmonic_raw is a sum over positions of phi * dphi / n; with every phase
near zero (the wrap pattern) its terms cancel, and the f32 oracle itself is
1.1e-5 from the f64 oracle in relative L2 at T = 1024.  That gradient is
therefore checked against the f64 oracle, within the bar or twice the f32
oracle's own distance from f64, whichever is larger (as is every other
weight gradient, a sum over all positions; the max_abs bar applies per unit
of the largest entry, since the loud pattern's gradients reach ~5).  At T = 2500 the f32
oracle's distance (its sum runs over ~3.1M admitted pairs in order) measured
3.0e-5 (wrap), 2.1e-5 (natural) and 1.0e-6 (far): which pattern it happens to
sum well says nothing of the kernels, so above 2048 positions the bar is at
least 4e-5 for it and for d_proj_b.  The far pattern is the hard case for the
kernels: its phases take exactly two values, so every pair within a bucket has
sin(n delta) = 0, and the oracle's pair terms -sin(n delta) delta dS vanish
there, while the kernels form a position's share u_t = cos(n phi_t) G1 -
sin(n phi_t) G0 from feature sums G over the keys (the MFMA form of the
score), a difference of equal fp32 sums that leaves only rounding; d_r, d_s
and the harmonic partial phi_t u_t carry it.  Measured at T = 2500 (far,
bucket-sparse): d_harmonic_raw 2.4e-5 and d_proj_b 1.4e-5 from f64, every
other gradient and pattern within 6.4e-6."""
import math

import numpy as np
import pytest

import oracle
from conftest import MAX_ABS, REL_L2, assert_parity, errors, make_wave_weights

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
    elif pattern == "natural":
        return make_wave_weights(H, C, E, seed)
    elif pattern == "loud":
        # every bucket, content projections x4: content scores 16x larger, so
        # each row's scores span tens of log2 units and its running maximum
        # passes the lazy-rescale threshold (8 log2 units) repeatedly
        w = make_wave_weights(H, C, E, seed)
        w["proj_w"][:, 2:, :] *= 4.0
        w["proj_b"][:, 2:] *= 4.0
        return w
    return w


def _expected_buckets(pattern):
    return {"one": {3}, "far": {2, 6}, "wrap": {0, 7}, "natural": None, "loud": None}[pattern]


CASES = [(p, s, sh) for sh in ((2, 300, 128, 2, 16), (1, 1024, 256, 4, 5)) for s in (True, False)
         for p in ("one", "far", "wrap")]
# A ragged sequence above 1024 positions: the stable bucket sort then takes
# several passes of its 1024 threads, adding each pass's counts to the bucket
# bases, and the bucket windows are longer; the phases of the default weights
# give every bucket ("natural"), the adversarial patterns gaps and wrap-around.
CASES += [(p, True, (1, 2500, 256, 4, 16)) for p in ("natural", "far", "wrap")]
CASES += [("natural", False, (1, 2500, 256, 4, 16))]
# content scores spanning tens of log2 units (the sparse forward's lazy running max)
CASES += [("loud", s, sh) for sh in ((2, 300, 128, 2, 16), (1, 1024, 256, 4, 16)) for s in (True, False)]
# 263 chunks of 16 positions: bucket windows of about 100 chunks, so the one-wave
# kernels build their live-chunk lists over several groups of 64 window offsets
CASES += [("natural", True, (1, 4200, 128, 2, 16))]


@pytest.mark.parametrize("pattern,sparse,shape", CASES)
def test_bucket_patterns_match_oracle(pkg, torch_dev, pattern, sparse, shape):
    B, T, E, H, C = shape
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
        want = _expected_buckets(pattern)
        assert set(np.unique(bk)) == (want if want is not None else set(range(8)))
        phase = cache.phase.cpu().numpy()
        merged, lse = cache.merged.cpu().numpy(), cache.lse.cpu().numpy()
        refs = []
        for b in range(B):
            ref = oracle.wave_fwd(x[b], w, "f32", phase_in=phase[b])
            assert_parity(f"merged b{b}", merged[b], ref["merged"])
            assert_parity(f"lse b{b}", lse[b], ref["lse"])
            assert_parity(f"out b{b}", out[b].cpu().numpy(), ref["out"])
            refs.append((oracle.wave_bwd(x[b], w, dy[b], "f32", phase_in=phase[b]),
                         oracle.wave_bwd(x[b], w, dy[b], "f64", phase_in=phase[b])))
        got_dx = grads.d_normed.cpu().numpy()
        for b in range(B):
            assert_parity(f"d_x b{b}", got_dx[b], refs[b][0]["d_x"])
        # weight gradients: sums over every position of the batch, against the
        # f64 oracle within the bar or twice the f32 oracle's own distance
        for k, g in (("d_hraw", grads.d_harmonic_raw), ("d_proj_w", grads.d_proj_w), ("d_proj_b", grads.d_proj_b),
                     ("d_v_w", grads.d_v_w), ("d_v_b", grads.d_v_b), ("d_out_w", grads.out_proj_w),
                     ("d_out_b", grads.out_proj_b)):
            r32 = np.sum([r[0][k] for r in refs], axis=0, dtype=np.float64)
            r64 = np.sum([r[1][k] for r in refs], axis=0)
            ma32, cond = errors(r32, r64)
            floor = 4e-5 if (k in ("d_hraw", "d_proj_b") and T > 2048) else REL_L2
            got = g.cpu().numpy()
            print(f"{k} vs f64: rel_l2 {errors(got, r64)[1]:.2e} max_abs {errors(got, r64)[0]:.2e} (f32 oracle "
                  f"{cond:.2e}, {ma32:.2e}); vs f32 oracle {errors(got, r32)[1]:.2e}", flush=True)
            # max_abs: the bar per unit of the largest entry, or twice the f32
            # oracle's own error
            bar_abs = max(MAX_ABS * max(1.0, float(np.abs(r64).max())), 2 * ma32)
            assert_parity(f"{k} vs f64", got, r64, max_abs=bar_abs, rel_l2=max(floor, 2 * cond))
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


def test_forward_workspace_forms_agree(pkg, torch_dev):
    """wha_wave_fwd with a caller workspace (exactly wha_wave_fwd_workspace_size
    bytes) and with workspace NULL (the library-cached buffer) give the same
    bits on the bucket-sparse family at a ragged T above 1024."""
    import ctypes
    torch, dev = torch_dev
    B, T, E, H, C = 2, 1100, 256, 4, 16
    print("wave forward workspace forms", flush=True)
    w = make_wave_weights(H, C, E, seed=31)
    x = np.random.default_rng(32).normal(size=(B, T, E)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    W = pkg.WaveAttnWeights(t(w["hraw"]), t(w["proj_w"]), t(w["proj_b"]), t(w["v_w"]), t(w["v_b"]), t(w["out_w"]),
                            t(w["out_b"]))
    tx = t(x)
    shape = pkg.WaveShape(B, T, E, H, C)
    need = pkg.wave_fwd_workspace_bytes(shape)
    assert need > 0 and need % 4 == 0
    prev = pkg.wave_set_bucket_sparse(True)
    try:
        res = []
        for ws in (torch.empty(need // 4, dtype=torch.float32, device=dev), None):
            cache = pkg.WaveAttnCache(shape, dev)
            out = torch.empty_like(tx)
            rc = pkg.lib().wha_wave_fwd(ctypes.c_void_p(tx.data_ptr()), ctypes.byref(W._c()), ctypes.byref(shape),
                                        ctypes.c_void_p(out.data_ptr()), ctypes.byref(cache._c()),
                                        None if ws is None else ctypes.c_void_p(ws.data_ptr()),
                                        0 if ws is None else need, None)
            assert rc == 0, pkg.lib().wha_last_error()
            torch.cuda.synchronize()
            res.append((out.cpu().numpy(), cache.merged.cpu().numpy(), cache.lse.cpu().numpy()))
    finally:
        pkg.wave_set_bucket_sparse(prev)
    for a, b in zip(*res):
        np.testing.assert_array_equal(a, b)
