"""Wave-attention KV cache on the GPU (src/common/kv_cache.rs:93-356): ragged
prefills, batched decode steps over sequences of different lengths, and the
cache entries, against the oracle's prefill and forward_one restatements.  The
oracle replays the device phases so both sides form the same bucket masks."""
import numpy as np
import pytest

import oracle
from conftest import assert_parity, make_wave_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available()
    return torch, torch.device("cuda:0")


def _weights(pkg, torch, dev, H, C, E, seed):
    w = make_wave_weights(H, C, E, seed)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return w, pkg.WaveAttnWeights(t(w["hraw"]), t(w["proj_w"]), t(w["proj_b"]), t(w["v_w"]), t(w["v_b"]),
                                  t(w["out_w"]), t(w["out_b"]))


def _check_entries(cache, b, n, want_phase, want_values, n_head, w):
    ph = cache.phase[b, :, :n].cpu().numpy()
    np.testing.assert_array_equal(ph, want_phase) if want_phase is not None else None
    assert_parity(f"values seq{b}", cache.values[b, :, :n].cpu().numpy(), want_values)
    bk = cache.bucket[b, :, :n].cpu().numpy()
    np.testing.assert_array_equal(bk, [[oracle.phase_bucket(float(p), "f32") for p in row] for row in ph])
    cs = cache.cs[b, :, :n].cpu().numpy().astype(np.float64)
    hraw = w["hraw"].astype(np.float64)
    nh = np.where(hraw > 20, hraw, np.log1p(np.exp(hraw)))[:, None]
    np.testing.assert_allclose(cs[..., 0], np.cos(nh * ph), atol=2e-6)
    np.testing.assert_allclose(cs[..., 1], np.sin(nh * ph), atol=2e-6)


@pytest.mark.parametrize("E,H,C,prompts,steps,cap", [
    (64, 4, 16, (50, 130, 1), 5, 160),
    (168, 4, 0, (7, 33), 3, 48),
    (768, 12, 16, (300, 1000, 64, 513), 3, 1100),
    (256, 2, 16, (3000, 2500), 2, 3100),
])
def test_prefill_then_batched_decode(pkg, torch_dev, E, H, C, prompts, steps, cap):
    torch, dev = torch_dev
    print(f"kv E{E} H{H} C{C} prompts{prompts} steps{steps}", flush=True)
    w, W = _weights(pkg, torch, dev, H, C, E, seed=E + len(prompts))
    hd = E // H
    B = len(prompts)
    rng = np.random.default_rng(17)
    cache = pkg.WaveKvCache(B, H, hd, cap, dev)
    xs = [rng.normal(size=(T, E)).astype(np.float32) for T in prompts]
    # ragged prompts: one prefill per sequence into its slice of the batch cache
    for b, x in enumerate(xs):
        out = pkg.prefill_attention(W, torch.from_numpy(x).to(dev), cache, first_seq=b)
        torch.cuda.synchronize()
        T = prompts[b]
        ph = cache.phase[b, :, :T].cpu().numpy()
        ref = oracle.wave_kv_prefill(x, w, "f32", phase_in=ph)
        assert_parity(f"prefill out seq{b}", out[0].cpu().numpy(), ref["out"])
        # device phases vs f64 ground truth: an f32 projection error eps moves
        # phi by about eps / |(r, s)|
        g64 = oracle.wave_fwd(x, w, "f64")
        mag = np.hypot(g64["rs"][..., 0], g64["rs"][..., 1])
        dphi = np.abs(np.angle(np.exp(1j * (ph - g64["phase"]))))
        assert np.all(dphi <= 1e-6 + 2e-5 / mag)
        _check_entries(cache, b, T, None, ref["values"], H, w)
    assert cache.lengths == list(prompts)
    # decode steps for all sequences at once (different cached lengths)
    for step in range(steps):
        xn = rng.normal(size=(B, E)).astype(np.float32)
        lens = list(cache.lengths)
        before_ph = cache.phase.cpu().numpy()
        before_v = cache.values.cpu().numpy()
        out = pkg.forward_one_attention(W, torch.from_numpy(xn).to(dev), cache)
        torch.cuda.synchronize()
        assert cache.lengths == [n + 1 for n in lens]
        got = out.cpu().numpy()
        for b in range(B):
            n = lens[b]
            new_ph = cache.phase[b, :, n].cpu().numpy()
            ref = oracle.wave_kv_step(xn[b], w, before_ph[b], before_v[b], n, "f32", phase_new_in=new_ph)
            assert_parity(f"decode out step{step} seq{b}", got[b], ref["out"])
            assert_parity(f"appended v step{step} seq{b}", cache.values[b, :, n].cpu().numpy(), ref["v_new"])
            np.testing.assert_array_equal(cache.bucket[b, :, n].cpu().numpy(),
                                          [oracle.phase_bucket(float(p), "f32") for p in new_ph])
            # entries before the append are untouched
            np.testing.assert_array_equal(cache.phase[b, :, :n].cpu().numpy(), before_ph[b][:, :n])


def test_decode_from_an_empty_cache_returns_the_new_value(pkg, torch_dev):
    """n_cached = 0: the only score is the self score, so the merged head output
    is the new value row (kv_cache.rs:294, :312-320)."""
    torch, dev = torch_dev
    E, H, C = 64, 2, 16
    w, W = _weights(pkg, torch, dev, H, C, E, seed=5)
    cache = pkg.WaveKvCache(3, H, E // H, 8, dev)
    xn = np.random.default_rng(1).normal(size=(3, E)).astype(np.float32)
    out = pkg.forward_one_attention(W, torch.from_numpy(xn).to(dev), cache).cpu().numpy()
    for b in range(3):
        ref = oracle.wave_kv_step(xn[b], w, np.zeros((H, 8), np.float32), np.zeros((H, 8, E // H), np.float32), 0,
                                  "f32")
        assert_parity(f"empty-cache decode seq{b}", out[b], ref["out"])


def test_decode_rejects_a_full_cache(pkg, torch_dev):
    torch, dev = torch_dev
    E, H = 64, 2
    _, W = _weights(pkg, torch, dev, H, 0, E, seed=2)
    cache = pkg.WaveKvCache(1, H, E // H, 4, dev)
    cache.lengths = [4]
    with pytest.raises(pkg.WaveHipError):
        pkg.forward_one_attention(W, torch.zeros(1, E, device=dev), cache)
