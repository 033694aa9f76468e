"""Wave (harmonic coherence) attention on the GPU against the oracle
(src/common/attn.rs:72-430): forward, cache, rows of att_weights_all, full and
pathway backward, with both kernel families (bucket-sparse and all pairs).
The oracle replays the device's phases (phase_in) so both sides form the same
bucket mask; the phases themselves, the projections and the buckets are
checked separately (the bucket bit for bit)."""
import math

import numpy as np
import pytest

import oracle
from conftest import assert_parity, make_wave_weights

pytestmark = pytest.mark.gpu

# (B, T, n_embd, n_head, content_dim): head_dim 12 (padded 48), 42, 64, 128, and the
# 768-dim model shape; 3 x 37 rows put a partial 16-row tile in the 64-wide per-head projections;
# head_dim 56 runs the 64-wide kernels with pad quads
CONFIGS = [(2, 100, 48, 4, 16), (1, 77, 168, 4, 0), (2, 200, 128, 2, 16), (2, 130, 256, 2, 5),
           (2, 1024, 768, 12, 16), (3, 1, 64, 2, 30), (1, 64, 64, 1, 3), (3, 37, 128, 2, 8),
           (2, 150, 112, 2, 16)]


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available()
    return torch, torch.device("cuda:0")


@pytest.fixture(params=["sparse", "dense"])
def family(request, pkg):
    """Both kernel families of wha_wave_fwd / wha_wave_bwd: bucket-sparse (the
    default) and all causal pairs."""
    prev = pkg.wave_set_bucket_sparse(request.param == "sparse")
    yield request.param
    pkg.wave_set_bucket_sparse(prev)


def _setup(pkg, torch, dev, B, T, E, H, C, seed):
    w = make_wave_weights(H, C, E, seed)
    x = np.random.default_rng(seed + 1).normal(size=(B, T, E)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    W = pkg.WaveAttnWeights(t(w["hraw"]), t(w["proj_w"]), t(w["proj_b"]), t(w["v_w"]), t(w["v_b"]),
                            t(w["out_w"]), t(w["out_b"]))
    return w, x, W, t(x)


@pytest.mark.parametrize("B,T,E,H,C", CONFIGS)
def test_wave_forward_matches_oracle(pkg, torch_dev, family, B, T, E, H, C):
    torch, dev = torch_dev
    print(f"wave fwd {family} B{B} T{T} E{E} H{H} C{C}", flush=True)
    w, x, W, tx = _setup(pkg, torch, dev, B, T, E, H, C, seed=7 + T)
    out, att_rows, cache = pkg.wave_attention_forward(W, tx)
    torch.cuda.synchronize()
    g = {k: getattr(cache, k).cpu().numpy() for k in ("proj", "values", "phase", "bucket", "merged", "lse")}
    hd = E // H
    for b in range(B):
        ref_own = oracle.wave_fwd(x[b], w, "f32")
        # projections: r, s, content and the per-head values
        assert_parity(f"rs b{b}", g["proj"][b][:, :, :2].transpose(1, 0, 2), ref_own["rs"])
        if C:
            assert_parity(f"content b{b}", g["proj"][b][:, :, 2:].transpose(1, 0, 2), ref_own["content"])
        assert_parity(f"values b{b}", g["values"][b].reshape(T, H, hd).transpose(1, 0, 2), ref_own["values"])
        # device atan2 within a few ulp of the f64 value of its own (r, s)
        rs = g["proj"][b][:, :, :2].astype(np.float64)
        ph64 = np.arctan2(rs[..., 1], rs[..., 0]).T
        assert np.abs(g["phase"][b] - ph64).max() <= 1e-6
        # buckets: bit for bit the reference's f32 formula on the device phases
        want_bk = np.array([[oracle.phase_bucket(float(p), "f32") for p in row] for row in g["phase"][b]])
        np.testing.assert_array_equal(g["bucket"][b], want_bk)
        # core and output with the device phases replayed
        ref = oracle.wave_fwd(x[b], w, "f32", phase_in=g["phase"][b])
        assert_parity(f"merged b{b}", g["merged"][b], ref["merged"])
        assert_parity(f"lse b{b}", g["lse"][b], ref["lse"])
        assert_parity(f"out b{b}", out[b].cpu().numpy(), ref["out"])
        # rows of att_weights_all on demand
        rows = sorted({r for r in (0, 1, T // 2, T - 1) if r < T})
        got_rows = att_rows.rows(rows)[b].cpu().numpy()
        want_rows = ref["att"][:, rows, :]
        assert np.array_equal(np.isneginf(got_rows), np.isneginf(want_rows))
        fin = ~np.isneginf(want_rows)
        assert_parity(f"att rows b{b}", got_rows[fin], want_rows[fin])
        assert np.array_equal(got_rows[fin] == 0, want_rows[fin] == 0)  # same sparsity pattern


@pytest.mark.parametrize("B,T,E,H,C", CONFIGS)
def test_wave_backward_matches_oracle(pkg, torch_dev, family, B, T, E, H, C):
    torch, dev = torch_dev
    print(f"wave bwd {family} B{B} T{T} E{E} H{H} C{C}", flush=True)
    w, x, W, tx = _setup(pkg, torch, dev, B, T, E, H, C, seed=11 + T)
    # d_out scaled by 1/sqrt(B*T) so that batch-summed weight gradients stay O(1)
    dy = (np.random.default_rng(T).normal(size=(B, T, E)) / math.sqrt(B * T)).astype(np.float32)
    tdy = torch.from_numpy(dy).to(dev)
    _, _, cache = pkg.wave_attention_forward(W, tx)
    grads = pkg.wave_attention_backward_full(W, cache, tdy)
    d_path = pkg.wave_attention_backward_pathway(W, cache, tdy)
    torch.cuda.synchronize()
    phase = cache.phase.cpu().numpy()
    refs = [oracle.wave_bwd(x[b], w, dy[b], "f32", phase_in=phase[b]) for b in range(B)]
    got_dx = grads.d_normed.cpu().numpy()
    for b in range(B):
        assert_parity(f"d_x b{b}", got_dx[b], refs[b]["d_x"])
    np.testing.assert_array_equal(d_path.cpu().numpy(), got_dx)  # pathway = full backward's d_normed
    s = lambda k: np.sum([r[k] for r in refs], axis=0, dtype=np.float64)
    # with T = 1 every softmax row has one entry, so the score gradient is exactly
    # zero in the reference (d_att - sum att*d_att = 0) and the phase/content
    # gradients vanish; the device's dP - Delta carries rounding noise instead, so
    # only the absolute bound applies (relative L2 is undefined for a zero reference)
    score_kw = dict(rel_l2=np.inf) if T == 1 else {}
    assert_parity("d_harmonic_raw", grads.d_harmonic_raw.cpu().numpy(), s("d_hraw"), **score_kw)
    assert_parity("d_proj_w", grads.d_proj_w.cpu().numpy(), s("d_proj_w"), **score_kw)
    assert_parity("d_proj_b", grads.d_proj_b.cpu().numpy(), s("d_proj_b"), **score_kw)
    assert_parity("d_v_w", grads.d_v_w.cpu().numpy(), s("d_v_w"))
    assert_parity("d_v_b", grads.d_v_b.cpu().numpy(), s("d_v_b"))
    assert_parity("d_out_w", grads.out_proj_w.cpu().numpy(), s("d_out_w"))
    assert_parity("d_out_b", grads.out_proj_b.cpu().numpy(), s("d_out_b"))


def test_wave_backward_is_deterministic(pkg, torch_dev, family):
    torch, dev = torch_dev
    B, T, E, H, C = 2, 300, 256, 4, 16
    w, x, W, tx = _setup(pkg, torch, dev, B, T, E, H, C, seed=3)
    tdy = torch.randn(B, T, E, device=dev) / math.sqrt(B * T)
    _, _, cache = pkg.wave_attention_forward(W, tx)
    g1 = pkg.wave_attention_backward_full(W, cache, tdy)
    g2 = pkg.wave_attention_backward_full(W, cache, tdy)
    for k in ("d_normed", "d_harmonic_raw", "d_proj_w", "d_v_w", "out_proj_w"):
        assert torch.equal(getattr(g1, k), getattr(g2, k)), k
