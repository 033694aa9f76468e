"""Hardening checks of the GPU paths beyond plain parity:

- guard bands: every output, the LSE, the kept scores and the workspaces sit
  inside sentinel-filled margins (and, on the fused [B][T][3E] c_attn layout,
  beside columns that belong to other tensors); no kernel may write outside
  its tensor, at ragged T and every kernel family's head dims;
- NaN semantics: a NaN in V (forward) or dO (backward) reaches every output
  the reference's NaN reaches (src/cpu/backward.rs:313-363,
  src/common/compute.rs:377-409, masked entries never touched), and beyond it
  only outputs of causally later rows of the same tile (a masked probability or
  dS of exactly 0 still multiplies the NaN inside the MFMA);
- the kept-scores pair at the full 4096 preset against oracle slices;
- f64 ground truth at the full 768-dim config;
- the wave attention's buckets at the 768-dim model shape against the
  reference's own f32 operations (atan2f, phase_to_bucket) on the device's
  projections;
- unaligned tensors: the kept pair falls back to the recompute kernels;
- a sequence whose dS passes 2 GiB per head takes the register-staged backward.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_parity, errors, make_wave_weights, widen_b

pytestmark = pytest.mark.gpu

SENT = 0x7FC0DEAD   # a quiet NaN with a payload no kernel produces
MARGIN = 1024       # floats of guard band on each side (4 KB, keeps 16-byte alignment)


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch, torch.device("cuda:0")


class Guarded:
    """n floats of device memory between two sentinel-filled margins."""

    def __init__(self, torch, dev, n):
        self.n = n
        self.raw = torch.full((n + 2 * MARGIN,), SENT, dtype=torch.int32, device=dev)
        self.t = self.raw[MARGIN:MARGIN + n].view(torch.float32)

    def intact(self):
        return bool((self.raw[:MARGIN] == SENT).all()) and bool((self.raw[MARGIN + self.n:] == SENT).all())


def guarded_like(torch, dev, shape, fill=None):
    g = Guarded(torch, dev, int(np.prod(shape)))
    if fill is not None:
        g.t.copy_(torch.from_numpy(np.ascontiguousarray(fill, dtype=np.float32)).reshape(-1))
    return g, g.t.view(*shape)


# the last two: enough (b,h) heads for the paired block-to-tile mapping at a ragged T (odd tile count)
RAGGED = [(2, 3, 100, 64), (1, 2, 129, 128), (2, 2, 1000, 64), (1, 2, 77, 48), (2, 2, 65, 42), (1, 1, 200, 56),
          (1, 2, 33, 100), (2, 2, 97, 44), (8, 12, 900, 64), (8, 12, 900, 48)]


@pytest.mark.parametrize("B,H,T,D", RAGGED)
@pytest.mark.parametrize("keep,wide", [(False, False), (False, True), (True, True)])
def test_guard_bands_bhtd(pkg, torch_dev, B, H, T, D, keep, wide):
    """wide: the batch widened past the small-problem threshold (the 64-row tile
    kernels; small problems keep no scores)."""
    torch, dev = torch_dev
    if wide:
        B = widen_b(B, H, T)
    print(f"case guard bands B={B} H={H} T={T} D={D} keep={keep}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=500 + T + D)
    shape = (B, H, T, D)
    (_, tq), (_, tk), (_, tv), (_, tdo) = (guarded_like(torch, dev, shape, a) for a in (q, k, v, do))
    go, o = guarded_like(torch, dev, shape)
    gl, lse = guarded_like(torch, dev, (B, H, T))
    gdq, dq = guarded_like(torch, dev, shape)
    gdk, dk = guarded_like(torch, dev, shape)
    gdv, dv = guarded_like(torch, dev, shape)
    L = pkg.layout_of(tq)
    gws = Guarded(torch, dev, (pkg.attn_bwd_workspace_bytes(L) + 3) // 4)
    nsc = pkg.attn_scores_bytes(L) // 4 if keep else 0
    gsc = Guarded(torch, dev, nsc) if nsc else None
    sc = gsc.t if gsc else None
    pkg.attn_fwd(tq, tk, tv, out=o, lse=lse, scores=sc)
    pkg.attn_bwd(tq, tk, tv, o, tdo, lse, workspace=gws.t, dq=dq, dk=dk, dv=dv, scores=sc)
    torch.cuda.synchronize()
    for name, g in (("O", go), ("LSE", gl), ("dQ", gdq), ("dK", gdk), ("dV", gdv), ("workspace", gws),
                    ("scores", gsc)):
        if g is not None:
            assert g.intact(), f"{name}: a kernel wrote into the guard band"
    sel = sorted({0, B - 1})
    ref = oracle.fwd_bwd_bhtd(q[sel], k[sel], v[sel], do[sel], "f32")
    for name, got, want in zip(("O", "dQ", "dK", "dV"), (o, dq, dk, dv), ref[:4]):
        assert_parity(name, got[sel].cpu().numpy(), want)


def _fused_views(buf, B, T, H, D):
    """q, k, v [B,H,T,D] views of a [B][T][3E] c_attn row (compute.rs:368-375)."""
    E = H * D
    return [buf.view(B, T, 3 * E)[:, :, c * E:(c + 1) * E].view(B, T, H, D).permute(0, 2, 1, 3) for c in range(3)]


@pytest.mark.parametrize("B,H,T,D", [(2, 3, 100, 64), (2, 2, 130, 48), (1, 4, 129, 128), (2, 2, 70, 42)])
@pytest.mark.parametrize("keep,wide", [(False, False), (False, True), (True, True)])
def test_guard_bands_fused_c_attn_layout(pkg, torch_dev, B, H, T, D, keep, wide):
    """q, k, v are column slices of one [B][T][3E] buffer; o is written into the
    q columns of another such buffer, whose k and v columns must stay untouched;
    dq, dk, dv fill the three slices of a [B][T][3E] gradient buffer."""
    torch, dev = torch_dev
    if wide:
        B = widen_b(B, H, T)
    print(f"case fused layout guard bands B={B} H={H} T={T} D={D} keep={keep}", flush=True)
    E = H * D
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=900 + T)
    seq = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(B, T, E)
    qkv = np.concatenate([seq(q), seq(k), seq(v)], axis=2)
    _, tqkv = guarded_like(torch, dev, (B, T, 3 * E), qkv)
    tq, tk, tv = _fused_views(tqkv, B, T, H, D)
    _, tdo_buf = guarded_like(torch, dev, (B, T, 3 * E), np.concatenate([seq(do)] * 3, axis=2))
    tdo = _fused_views(tdo_buf, B, T, H, D)[0]
    gob, obuf = guarded_like(torch, dev, (B, T, 3 * E))
    o = _fused_views(obuf, B, T, H, D)[0]
    gl, lse = guarded_like(torch, dev, (B, H, T))
    gd, dbuf = guarded_like(torch, dev, (B, T, 3 * E))
    dq, dk, dv = _fused_views(dbuf, B, T, H, D)
    L = pkg.layout_of(tq)
    gws = Guarded(torch, dev, (pkg.attn_bwd_workspace_bytes(L) + 3) // 4)
    nsc = pkg.attn_scores_bytes(L) // 4 if keep else 0
    gsc = Guarded(torch, dev, nsc) if nsc else None
    sc = gsc.t if gsc else None
    pkg.attn_fwd(tq, tk, tv, out=o, lse=lse, scores=sc)
    pkg.attn_bwd(tq, tk, tv, o, tdo, lse, workspace=gws.t, dq=dq, dk=dk, dv=dv, scores=sc)
    torch.cuda.synchronize()
    for name, g in (("obuf", gob), ("LSE", gl), ("d_qkv", gd), ("workspace", gws), ("scores", gsc)):
        if g is not None:
            assert g.intact(), f"{name}: a kernel wrote into the guard band"
    untouched = obuf.view(torch.int32)[:, :, E:]
    assert bool((untouched == SENT).all()), "o's writes reached the k/v columns of its [B][T][3E] buffer"
    sel = sorted({0, B - 1})
    ref = oracle.fwd_bwd_bhtd(q[sel], k[sel], v[sel], do[sel], "f32")
    for name, got, want in zip(("O", "dQ", "dK", "dV"), (o, dq, dk, dv), ref[:4]):
        assert_parity(name, got[sel].cpu().numpy(), want)


@pytest.mark.parametrize("B,H,T,D", [(2, 2, 100, 64), (1, 2, 77, 48), (2, 1, 130, 128)])
def test_guard_bands_from_probs(pkg, torch_dev, B, H, T, D):
    torch, dev = torch_dev
    import ctypes
    print(f"case from-probs guard bands B={B} H={H} T={T} D={D}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=77 + T)
    tq, tk, tv, tdo = (torch.from_numpy(a).to(dev) for a in (q, k, v, do))
    o, lse = pkg.attn_fwd(tq, tk, tv)
    att_d = torch.cat([pkg.attn_probs_rows(tq, tk, lse, range(r, min(T, r + 256))) for r in range(0, T, 256)],
                      dim=2).contiguous()
    L = pkg.layout_of(tq)
    gws = Guarded(torch, dev, (int(pkg.lib().wha_attn_bwd_from_probs_workspace_size(ctypes.byref(L))) + 3) // 4)
    shape = (B, H, T, D)
    gdq, dq = guarded_like(torch, dev, shape)
    gdk, dk = guarded_like(torch, dev, shape)
    gdv, dv = guarded_like(torch, dev, shape)
    s = pkg.default_scale(D)
    rc = pkg.lib().wha_attn_bwd_from_probs(pkg._ptr(tdo), pkg._ptr(tq), pkg._ptr(tk), pkg._ptr(tv), pkg._ptr(att_d),
                                           pkg._ptr(dq), pkg._ptr(dk), pkg._ptr(dv), pkg._ptr(gws.t),
                                           gws.n * 4, ctypes.byref(L), s, pkg._stream_ptr(tq))
    assert rc == 0, pkg.lib().wha_last_error()
    torch.cuda.synchronize()
    for name, g in (("dQ", gdq), ("dK", gdk), ("dV", gdv), ("workspace", gws)):
        assert g.intact(), f"{name}: a kernel wrote into the guard band"
    ref = oracle.fwd_bwd_bhtd(q, k, v, do, "f32")
    for name, got, want in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref[1:4]):
        assert_parity(name, got.cpu().numpy(), want)


@pytest.mark.parametrize("B,H,Tk,D", [(3, 4, 1000, 64), (2, 2, 333, 48), (1, 3, 2049, 128)])
def test_guard_bands_decode(pkg, torch_dev, B, H, Tk, D):
    torch, dev = torch_dev
    import ctypes
    print(f"case decode guard bands B={B} H={H} Tk={Tk} D={D}", flush=True)
    g = pkg.SynthStream(5 + Tk)
    sd = 1.0 / np.sqrt(D)
    q = g.normal(B * H * D, sd).reshape(B, H, D)
    kc = g.normal(B * H * Tk * D, sd).reshape(B, H, Tk, D)
    vc = g.normal(B * H * Tk * D, sd).reshape(B, H, Tk, D)
    tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, kc, vc))
    L = pkg.layout_of(tk)
    gws = Guarded(torch, dev, (int(pkg.lib().wha_decode_workspace_size(ctypes.byref(L))) + 3) // 4)
    go, o = guarded_like(torch, dev, (B, H, D))
    gl, lse = guarded_like(torch, dev, (B, H))
    rc = pkg.lib().wha_decode_fwd(pkg._ptr(tq), pkg._ptr(tk), pkg._ptr(tv), pkg._ptr(o), pkg._ptr(lse),
                                  pkg._ptr(gws.t), gws.n * 4, ctypes.byref(L), pkg.default_scale(D),
                                  pkg._stream_ptr(tq))
    assert rc == 0, pkg.lib().wha_last_error()
    torch.cuda.synchronize()
    for name, gg in (("O", go), ("LSE", gl), ("workspace", gws)):
        assert gg.intact(), f"{name}: a kernel wrote into the guard band"
    for b, h in ((0, 0), (B - 1, H - 1)):
        assert_parity(f"decode b{b}h{h}", o[b, h].cpu().numpy(), oracle.decode_one(q[b, h], kc[b, h], vc[b, h], 1))


# ------------------------------------------------------------------ NaN semantics

def _nan_map(a):
    return np.isnan(a)


@pytest.mark.parametrize("T,D,j", [(200, 64, 77), (200, 64, 128), (150, 48, 70), (300, 128, 131), (90, 42, 40),
                                   (100, 64, 99)])
@pytest.mark.parametrize("keep,wide", [(False, False), (False, True), (True, True)])
def test_nan_in_v_forward_superset(pkg, torch_dev, T, D, j, keep, wide):
    """NaN at V[b=0,h=1,j,d=5]: the reference's O[i][5] is NaN exactly for
    i >= j (P[i][j] > 0; masked entries are never touched).  The device must
    give NaN there, and may give it beyond only in column 5 of rows
    64*floor(j/64) <= i < j (queries whose tile also computes key j's block,
    where the masked P = 0 multiplies the NaN).  Other heads stay finite."""
    torch, dev = torch_dev
    print(f"case NaN in V T={T} D={D} j={j} keep={keep}", flush=True)
    B, H, dcol = 2, 2, 5
    B = widen_b(B, H, T) if wide else B   # wide: the 64-row tile kernels, else the small-problem ones
    q, k, v, _ = pkg.synth_inputs(B, H, T, D, seed=31 + j)
    v = v.copy()
    v[0, 1, j, dcol] = np.nan
    tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    L = pkg.layout_of(tq)
    sc = pkg.attn_scores_buffer(L, dev) if keep else None
    o, lse = pkg.attn_fwd(tq, tk, tv, scores=sc)
    torch.cuda.synchronize()
    got = _nan_map(o.cpu().numpy())
    ref = np.zeros_like(got)
    ref[0, 1, j:, dcol] = True
    assert (got & ref).sum() == ref.sum(), "a NaN the reference produces is missing"
    extra = got & ~ref
    allowed = np.zeros_like(got)
    allowed[0, 1, 64 * (j // 64):j, dcol] = True
    assert not (extra & ~allowed).any(), f"NaN outside the documented tile superset: {np.argwhere(extra & ~allowed)[:5]}"
    assert np.isfinite(lse.cpu().numpy()).all()
    print(f"  reference NaN {int(ref.sum())}, extra in-tile NaN {int(extra.sum())}", flush=True)


@pytest.mark.parametrize("T,D,i", [(200, 64, 77), (200, 64, 127), (150, 48, 70), (300, 128, 131), (90, 42, 40),
                                   (100, 64, 99)])
@pytest.mark.parametrize("keep,wide", [(False, False), (False, True), (True, True)])
def test_nan_in_do_backward_superset(pkg, torch_dev, T, D, i, keep, wide):
    """NaN at dO[b=0,h=1,i,d=3] with finite Q, K, V: in the reference
    (src/cpu/backward.rs:335-361) d_att[i][*] and att_d_att_sum of row i are NaN,
    so dQ[i][:] is NaN, dK[k][:] for every k <= i, and dV[k][3] for every
    k <= i; nothing else.  The device must give NaN there, and may give it
    beyond only in the same columns of key rows i < k < 64*floor(i/64) + 80
    (keys whose 16-key wave group also swept query i's tile)."""
    torch, dev = torch_dev
    print(f"case NaN in dO T={T} D={D} i={i} keep={keep}", flush=True)
    B, H, dcol = 2, 2, 3
    B = widen_b(B, H, T) if wide else B
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=41 + i)
    do = do.copy()
    do[0, 1, i, dcol] = np.nan
    tq, tk, tv, tdo = (torch.from_numpy(a).to(dev) for a in (q, k, v, do))
    L = pkg.layout_of(tq)
    sc = pkg.attn_scores_buffer(L, dev) if keep else None
    o, lse = pkg.attn_fwd(tq, tk, tv, scores=sc)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, scores=sc)
    torch.cuda.synchronize()
    hi = min(T, 64 * (i // 64) + 80)
    for name, t, ref_rows, cols in (("dQ", dq, slice(i, i + 1), slice(None)), ("dK", dk, slice(0, i + 1), slice(None)),
                                     ("dV", dv, slice(0, i + 1), slice(dcol, dcol + 1))):
        got = _nan_map(t.cpu().numpy())
        ref = np.zeros_like(got)
        ref[0, 1, ref_rows, cols] = True
        assert (got & ref).sum() == ref.sum(), f"{name}: a NaN the reference produces is missing"
        extra = got & ~ref
        allowed = np.zeros_like(got)
        if name != "dQ":
            allowed[0, 1, i + 1:hi, cols] = True
        assert not (extra & ~allowed).any(), \
            f"{name}: NaN outside the documented tile superset: {np.argwhere(extra & ~allowed)[:5]}"
        print(f"  {name}: reference NaN {int(ref.sum())}, extra in-tile NaN {int(extra.sum())}", flush=True)


# ------------------------------------------------------------------ full-size checks

def test_kept_pair_4096_preset_full(pkg, torch_dev):
    """The kept-scores pair at the full 4096 preset (B=4, H=32, T=2048, D=128;
    a 1.1 GB score buffer, the last slice's scores at its end): oracle on sampled
    (b,h) slices -- including the last one, whose scores sit at the end of the
    buffer -- and the whole-output identities."""
    torch, dev = torch_dev
    from test_gpu_parity import check_identities, threaded_ref, report
    B, H, T, D = 4, 32, 2048, 128
    print("case kept pair 4096 preset", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=42)
    tq, tk, tv, tdo = (torch.from_numpy(a).to(dev) for a in (q, k, v, do))
    sc = pkg.attn_scores_buffer(pkg.layout_of(tq), dev)
    assert sc is not None and sc.numel() * 4 > 1 << 30
    o, lse = pkg.attn_fwd(tq, tk, tv, scores=sc)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, scores=sc)
    torch.cuda.synchronize()
    o, dq, dk, dv = (x.cpu().numpy() for x in (o, dq, dk, dv))
    for b, h in ((0, 0), (3, 31), (2, 9)):
        sl = lambda a: a[b:b + 1, h:h + 1]
        ref = threaded_ref(sl(q), sl(k), sl(v), sl(do), nthreads=1)
        report(f"kept 4096 b{b}h{h}", (sl(o), sl(dq), sl(dk), sl(dv)), ref)
    check_identities(q, k, v, do, o, dq, dk, dv)


def test_long_sequence_takes_the_register_staged_backward(pkg, torch_dev):
    """T = 32768 on one head: its dS (2.15 GB) is past the 2 GiB a buffer
    descriptor of the direct-to-LDS backward spans, so the pair keeps no scores
    and the backward runs the register-staged kernels.  Causality pins the first
    256 rows exactly (their O, LSE and dQ depend on those rows only: the oracle
    on the prefix), the whole-output identities the rest."""
    torch, dev = torch_dev
    from test_gpu_parity import check_identities
    B, H, T, D = 1, 1, 32768, 64
    print("case long sequence T=32768", flush=True)
    assert pkg.attn_scores_bytes(pkg.layout_bhtd(B, H, T, D)) == 0
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=5)
    tq, tk, tv, tdo = (torch.from_numpy(a).to(dev) for a in (q, k, v, do))
    o, lse = pkg.attn_fwd(tq, tk, tv)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse)
    torch.cuda.synchronize()
    o, lse, dq, dk, dv = (x.cpu().numpy() for x in (o, lse, dq, dk, dv))
    P = 256
    prefix = [np.ascontiguousarray(a[:, :, :P]) for a in (q, k, v, do)]
    r32 = oracle.fwd_bwd_bhtd(*prefix, "f32")
    r64 = oracle.fwd_bwd_bhtd(*prefix, "f64")
    assert_parity("O prefix", o[:, :, :P], r32[0])
    assert_parity("dQ prefix", dq[:, :, :P], r32[1])
    assert np.abs(lse[:, :, :P] - r64[4]).max() < 2e-5
    check_identities(q, k, v, do, o, dq, dk, dv)


@pytest.mark.parametrize("keep", [False, True])
def test_f64_ground_truth_768(pkg, torch_dev, keep):
    """The full 768-dim config against the f64 oracle (ground truth) and the f32
    oracle (the parity bar); the device must be no further from f64 than the
    bar, and the errors are printed for the record."""
    torch, dev = torch_dev
    B, H, T, D = 8, 12, 1024, 64
    print(f"case f64 ground truth 768 keep={keep}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=42)
    tq, tk, tv, tdo = (torch.from_numpy(a).to(dev) for a in (q, k, v, do))
    sc = pkg.attn_scores_buffer(pkg.layout_of(tq), dev) if keep else None
    o, lse = pkg.attn_fwd(tq, tk, tv, scores=sc)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, scores=sc)
    torch.cuda.synchronize()
    got = [x.cpu().numpy() for x in (o, dq, dk, dv)]
    r64 = oracle.fwd_bwd_bhtd(q, k, v, do, "f64", nthreads=8)
    from test_gpu_parity import threaded_ref
    r32 = threaded_ref(q, k, v, do)
    for name, g, w64, w32 in zip(("O", "dQ", "dK", "dV"), got, r64[:4], r32):
        ma64, rl64 = errors(g, w64)
        mc, rc = errors(w32, w64)
        ma32, rl32 = assert_parity(name, g, w32)
        assert ma64 <= 1e-4 and rl64 <= 1e-5, f"{name}: vs f64 max_abs={ma64:.2e} rel_l2={rl64:.2e}"
        print(f"768 {'kept' if keep else 'recompute'} {name}: gpu vs f64 max_abs={ma64:.2e} rel_l2={rl64:.2e} | "
              f"cpu f32 vs f64 max_abs={mc:.2e} rel_l2={rc:.2e} | gpu vs cpu f32 max_abs={ma32:.2e} "
              f"rel_l2={rl32:.2e}", flush=True)


def test_wave_buckets_match_reference_f32_ops_768(pkg, torch_dev):
    """At the 768-dim wave shape (B=8, T=1024, 12 heads, content 16) the device's
    phase and bucket of every position against the reference's own f32
    operations (atan2f, then phase_to_bucket) applied to the device's (r, s):
    the bucket is index work, so every flip is counted and none is allowed."""
    torch, dev = torch_dev
    B, T, E, H, C = 8, 1024, 768, 12, 16
    print("case wave buckets 768", flush=True)
    w = make_wave_weights(H, C, E, seed=2024)
    x = np.random.default_rng(2025).normal(size=(B, T, E)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    W = pkg.WaveAttnWeights(t(w["hraw"]), t(w["proj_w"]), t(w["proj_b"]), t(w["v_w"]), t(w["v_b"]), t(w["out_w"]),
                            t(w["out_b"]))
    _, _, cache = pkg.wave_attention_forward(W, t(x))
    torch.cuda.synchronize()
    proj = cache.proj.cpu().numpy()                     # [B][T][H][2+C]
    r = proj[..., 0].transpose(0, 2, 1)                 # [B][H][T]
    s = proj[..., 1].transpose(0, 2, 1)
    ph_ref, bk_ref = oracle.phases(r, s, "f32")
    ph_dev = cache.phase.cpu().numpy().ravel()
    bk_dev = cache.bucket.cpu().numpy().ravel()
    flips = int((bk_dev != bk_ref).sum())
    ulp = np.abs(ph_dev.view(np.int32).astype(np.int64) - ph_ref.view(np.int32).astype(np.int64))
    print(f"wave 768: {ph_dev.size} positions, bucket flips {flips}, phases equal to atan2f {(ulp == 0).mean():.4f}, "
          f"max phase difference {int(ulp.max())} ulp", flush=True)
    assert flips == 0
    # the device phase is atan2 rounded once from double: at most 1 ulp from the host's atan2f
    # (glibc's is itself within 1 ulp of the correctly rounded value)
    assert int(ulp.max()) <= 1
    cr = np.arctan2(s.astype(np.float64), r.astype(np.float64)).astype(np.float32).ravel()
    assert (ph_dev == cr).mean() > 0.999


def test_kept_pair_falls_back_on_unaligned_tensors(pkg, torch_dev):
    """Views at an odd float offset are not 16-byte aligned: the kept pair then
    runs the recompute kernels (scores untouched) and still meets the bar, and
    AttnPlan does not choose the kept pair."""
    torch, dev = torch_dev
    B, H, T, D = widen_b(1, 2, 130), 2, 130, 64   # not a small problem: the layout keeps scores
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=3)
    n = B * H * T * D

    def unaligned(a):
        buf = torch.empty(n + 1, device=dev)
        buf[1:].copy_(torch.from_numpy(a).reshape(-1))
        return buf[1:].view(B, H, T, D)

    tq, tk, tv, tdo = (unaligned(a) for a in (q, k, v, do))
    assert tq.data_ptr() % 16 != 0
    sc = pkg.attn_scores_buffer(pkg.layout_of(tq), dev)
    sc.fill_(float("nan"))
    o, lse = pkg.attn_fwd(tq, tk, tv, scores=sc)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, scores=sc)
    torch.cuda.synchronize()
    assert bool(torch.isnan(sc).all()), "the unaligned forward wrote kept scores"
    sel = [0, B - 1]
    ref = oracle.fwd_bwd_bhtd(q[sel], k[sel], v[sel], do[sel], "f32")
    for name, got, want in zip(("O", "dQ", "dK", "dV"), (o, dq, dk, dv), ref[:4]):
        assert_parity(name, got[sel].cpu().numpy(), want)
    o2, lse2 = torch.empty_like(tq), torch.empty(B, H, T, device=dev)
    dq2, dk2, dv2 = (torch.empty_like(tq) for _ in range(3))
    plan = pkg.AttnPlan(tq, tk, tv, o2, lse2, tdo, dq2, dk2, dv2)
    assert not plan.keeps_scores


def test_small_problems_take_the_split_sweep_kernels(pkg, torch_dev):
    """Dispatch: below 256 tiles of 64 rows (and T <= 1024) the backward is the
    one-kernel small path (no statistics pass, no separate dQ pass, no kept
    scores); above it the 64-row tile kernels run with their statistics pass."""
    torch, dev = torch_dev
    for (B, H, T, D), small in (((4, 4, 256, 42), True), ((1, 2, 200, 64), True), ((16, 4, 256, 64), False),
                                ((1, 2, 1100, 64), False)):
        q, k, v, do = (torch.from_numpy(a).to(dev) for a in pkg.synth_inputs(B, H, T, D, seed=1))
        assert (pkg.attn_scores_bytes(pkg.layout_of(q)) == 0) == (small or D % 4 != 0)
        pkg.timing_reset()
        pkg.timing_enable(True)
        o, lse = pkg.attn_fwd(q, k, v)
        pkg.attn_bwd(q, k, v, o, do, lse)
        torch.cuda.synchronize()
        pkg.timing_enable(False)
        n_delta = pkg.timing_read("attn_bwd_delta")[1]
        n_dkv = pkg.timing_read("attn_bwd_dkv")[1]
        n_dq = pkg.timing_read("attn_bwd_dq")[1]
        pkg.timing_reset()
        assert n_dkv == 1 and n_delta == n_dq == (0 if small else 1), (B, H, T, D, n_delta, n_dkv, n_dq)
