"""GPU parity of the kept-scores training pair (wha_attn_fwd_keep, then
wha_attn_bwd_kept reading the forward's scores instead of recomputing Q K^T)
against the CPU oracle (src/common/compute.rs:377-409, src/cpu/backward.rs:313-363),
at the same bar as the fused pair: max-abs <= 1e-4 and relative L2 <= 1e-5 for
O, dQ, dK and dV against the f32 oracle.  Shapes the kept pair does not cover
(wha_attn_scores_size = 0) must behave exactly as wha_attn_fwd / wha_attn_bwd.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_parity, errors, widen_b

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch, torch.device("cuda:0")


def run_pair(pkg, torch, dev, q, k, v, do, keep):
    tq, tk, tv, tdo = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (q, k, v, do))
    L = pkg.layout_of(tq)
    sc = pkg.attn_scores_buffer(L, dev) if keep else None
    if keep and sc is not None:
        sc.fill_(float("nan"))  # entries the forward does not write must never be used unmasked
    o, lse = pkg.attn_fwd(tq, tk, tv, scores=sc)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, scores=sc)
    torch.cuda.synchronize()
    return [x.cpu().numpy() for x in (o, lse, dq, dk, dv)], sc is not None


SHAPES = [(1, 1, 1, 64), (1, 2, 17, 64), (2, 2, 100, 64), (3, 1, 48, 64), (2, 3, 130, 64),
          (1, 1, 257, 128), (1, 2, 129, 100), (2, 2, 97, 56), (1, 3, 40, 52), (1, 2, 65, 124),
          (2, 3, 63, 48), (1, 2, 65, 42), (1, 4, 200, 8), (2, 2, 97, 44), (1, 3, 70, 36)]


@pytest.mark.parametrize("B,H,T,D", SHAPES)
def test_kept_pair_small_shapes(pkg, torch_dev, B, H, T, D):
    """Ragged shapes with the batch widened past the small-problem threshold
    (small problems keep no scores); the oracle on the first and last sequence."""
    torch, dev = torch_dev
    B = widen_b(B, H, T)
    print(f"case kept B={B} H={H} T={T} D={D}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=2000 + T + D)
    got, kept = run_pair(pkg, torch, dev, q, k, v, do, keep=True)
    covered = pkg.attn_scores_bytes(pkg.layout_bhtd(B, H, T, D)) > 0
    assert kept == covered
    assert covered == (D % 4 == 0 and 32 < D <= 128)
    sel = sorted({0, B - 1})
    q, k, v, do = (a[sel] for a in (q, k, v, do))
    got = [a[sel] for a in got]
    r32 = oracle.fwd_bwd_bhtd(q, k, v, do, "f32")
    r64 = oracle.fwd_bwd_bhtd(q, k, v, do, "f64")
    for i, n in enumerate(("O", "dQ", "dK", "dV")):
        g = got[[0, 2, 3, 4][i]]
        ma, rl = assert_parity(f"kept B{B}H{H}T{T}D{D} {n}", g, r32[i])
        print(f"  {n}: vs f32 max_abs={ma:.2e} rel_l2={rl:.2e} | vs f64 {errors(g, r64[i])[1]:.2e}", flush=True)
    assert np.abs(got[1] - r64[4]).max() < 2e-5
    # the recompute pair on the same inputs: same softmax, scores rounded in another order
    qw, kw, vw, dow = pkg.synth_inputs(B, H, T, D, seed=2000 + T + D)
    ref, _ = run_pair(pkg, torch, dev, qw, kw, vw, dow, keep=False)
    ref = [a[sel] for a in ref]
    # the same forward kernel at every head dim (keeping the scores only adds their stores)
    assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1])
    for a, b in zip(got, ref):
        assert errors(a, b)[1] < 1e-6


def test_kept_pair_headline_config(pkg, torch_dev):
    """768-dim config at full size (seed 42) against the threaded f32 oracle,
    through AttnPlan (the bench's launch path), two steps in a row."""
    torch, dev = torch_dev
    B, H, T, D = 8, 12, 1024, 64
    print("case kept headline", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=42)
    tq, tk, tv, tdo = (torch.from_numpy(a).to(dev) for a in (q, k, v, do))
    o = torch.empty_like(tq)
    lse = torch.empty((B, H, T), dtype=torch.float32, device=dev)
    dq, dk, dv = (torch.empty_like(tq) for _ in range(3))
    plan = pkg.AttnPlan(tq, tk, tv, o, lse, tdo, dq, dk, dv)
    assert plan.keeps_scores
    for _ in range(2):
        plan.fwd()
        plan.bwd()
    torch.cuda.synchronize()
    out, rq, rk, rv = oracle.batch_fwd_bwd_f32_threaded(
        *(oracle.bhtd_to_seq(a) for a in (q, k, v, do)), H, nthreads=16)
    for n, g, r in (("O", o, out), ("dQ", dq, rq), ("dK", dk, rk), ("dV", dv, rv)):
        ma, rl = assert_parity(f"kept headline {n}", g.cpu().numpy(), oracle.seq_to_bhtd(r, H))
        print(f"  {n}: max_abs={ma:.2e} rel_l2={rl:.2e}", flush=True)


def test_kept_pair_384_config(pkg, torch_dev):
    """384-dim config (D = 48, kept pair on the exact 48-wide direct-to-LDS
    kernels) at full size, seed 42, against the threaded f32 oracle."""
    torch, dev = torch_dev
    B, H, T, D = 16, 8, 512, 48
    print("case kept 384-dim", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=42)
    got, kept = run_pair(pkg, torch, dev, q, k, v, do, keep=True)
    assert kept
    out, rq, rk, rv = oracle.batch_fwd_bwd_f32_threaded(
        *(oracle.bhtd_to_seq(a) for a in (q, k, v, do)), H, nthreads=16)
    for n, g, r in (("O", got[0], out), ("dQ", got[2], rq), ("dK", got[3], rk), ("dV", got[4], rv)):
        ma, rl = assert_parity(f"kept 384 {n}", g, oracle.seq_to_bhtd(r, H))
        print(f"  {n}: max_abs={ma:.2e} rel_l2={rl:.2e}", flush=True)


def test_kept_pair_4096_slice(pkg, torch_dev):
    """4096 preset (D = 128, T = 2048) on one (b,h) slice against the oracle."""
    torch, dev = torch_dev
    print("case kept 4096 slice", flush=True)
    q, k, v, do = pkg.synth_inputs(1, 2, 2048, 128, seed=42)
    got, kept = run_pair(pkg, torch, dev, q, k, v, do, keep=True)
    assert kept
    sl = lambda a: a[:, 1:2]
    out, rq, rk, rv = oracle.batch_fwd_bwd_f32_threaded(
        *(oracle.bhtd_to_seq(sl(a)) for a in (q, k, v, do)), 1, nthreads=1)
    for n, g, r in (("O", got[0], out), ("dQ", got[2], rq), ("dK", got[3], rk), ("dV", got[4], rv)):
        assert_parity(f"kept 4096 {n}", sl(g), oracle.seq_to_bhtd(r, 1))


def test_kept_pair_fused_qkv_layout_is_bit_identical(pkg, torch_dev):
    """The kept pair on q, k, v read in place from one fused c_attn output
    [B][T][3E] (the reference layout, stride_t = 3E; src/common/compute.rs:368-375)
    and dq, dk, dv written into one [B][T][3E] gradient buffer gives the same bits
    as on contiguous [B,H,T,D] tensors."""
    torch, dev = torch_dev
    for (B, H, T, D) in ((widen_b(2, 12, 300), 12, 300, 64), (widen_b(1, 4, 130), 4, 130, 48),
                         (widen_b(1, 2, 200), 2, 200, 128)):
        print(f"case kept fused-qkv B={B} H={H} T={T} D={D}", flush=True)
        E = H * D
        q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=6)
        base, kept = run_pair(pkg, torch, dev, q, k, v, do, keep=True)
        assert kept
        qkv = torch.from_numpy(np.concatenate([oracle.bhtd_to_seq(a) for a in (q, k, v)], axis=-1)).to(dev)
        heads = lambda buf, c, w: buf.view(B, T, w)[:, :, c * E:(c + 1) * E].view(B, T, H, D).permute(0, 2, 1, 3)
        tq, tk, tv = (heads(qkv, c, 3 * E) for c in range(3))
        # o and dO share q's layout (one wha_layout per call): 3E-wide buffers, first E columns
        dobuf = torch.zeros(B, T, 3 * E, device=dev)
        dobuf[:, :, :E] = torch.from_numpy(oracle.bhtd_to_seq(do)).to(dev)
        tdo = heads(dobuf, 0, 3 * E)
        o = heads(torch.empty(B, T, 3 * E, device=dev), 0, 3 * E)
        grads = torch.empty(B, T, 3 * E, device=dev)
        dq, dk, dv = (heads(grads, c, 3 * E) for c in range(3))
        sc = pkg.attn_scores_buffer(pkg.layout_of(tq), dev)
        _, lse = pkg.attn_fwd(tq, tk, tv, out=o, scores=sc)
        pkg.attn_bwd(tq, tk, tv, o, tdo, lse, dq=dq, dk=dk, dv=dv, scores=sc)
        torch.cuda.synchronize()
        got = [x.contiguous().cpu().numpy() for x in (o, lse, dq, dk, dv)]
        for a, b_ in zip(got, base):
            np.testing.assert_array_equal(a, b_)


def test_kept_backward_reads_only_scores_the_forward_wrote(pkg, torch_dev):
    """wha_attn_fwd_keep on tensors that are not 16-byte aligned falls back to
    the recompute forward and leaves the score buffer untouched.  A backward
    that then gets aligned copies of the same tensors must recompute the
    scores, not read the buffer: here it holds NaN (never written) in the
    first case, and scores of other inputs (a kept forward before the
    fallback) in the second.  Both backwards must meet the bar against the
    oracle."""
    torch, dev = torch_dev
    B, H, T, D = widen_b(1, 4, 200), 4, 200, 64
    L = pkg.layout_bhtd(B, H, T, D)
    assert pkg.attn_scores_bytes(L) > 0

    def unaligned(a):
        buf = torch.empty(a.size + 1, dtype=torch.float32, device=dev)
        t = buf[1:].view(a.shape)
        t.copy_(torch.from_numpy(np.ascontiguousarray(a)))
        assert t.data_ptr() % 16 != 0
        return t

    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=77)
    q2, k2, v2, _ = pkg.synth_inputs(B, H, T, D, seed=78)
    sel = [0, B - 1]
    ref = oracle.fwd_bwd_bhtd(*(a[sel] for a in (q, k, v, do)), "f32")
    for case in ("never written", "other inputs"):
        print(f"case kept fallback: {case}", flush=True)
        sc = pkg.attn_scores_buffer(L, dev)
        sc.fill_(float("nan"))
        if case == "other inputs":
            # a kept forward of other inputs fills the buffer with their scores
            t2 = [torch.from_numpy(a).to(dev) for a in (q2, k2, v2)]
            pkg.attn_fwd(*t2, scores=sc)
        uq, uk, uv = (unaligned(a) for a in (q, k, v))
        uo = unaligned(np.zeros_like(q))
        _, lse = pkg.attn_fwd(uq, uk, uv, out=uo, scores=sc)
        tq, tk, tv, tdo = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (q, k, v, do))
        o = uo.clone()  # fresh (aligned) storage
        assert o.data_ptr() % 16 == 0
        dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, scores=sc)
        torch.cuda.synchronize()
        for n, g, r in zip(("O", "dQ", "dK", "dV"), (o, dq, dk, dv), ref):
            assert_parity(f"kept fallback ({case}) {n}", g.cpu().numpy()[sel], r)
