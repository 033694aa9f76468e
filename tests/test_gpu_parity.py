"""GPU parity of the fused forward/backward against the CPU oracle
(reference-order f32 restatement of src/common/compute.rs:377-409 and
src/cpu/backward.rs:313-363), through the C ABI.

Bar (from the north star): max-abs <= 1e-4 and relative L2 <= 1e-5 for O, dQ, dK
and dV against the f32 oracle on identical seeded inputs; errors against the f64
oracle are printed as ground truth.  Full-size configs that the oracle cannot
finish in seconds are checked on a sample of (b, h) slices plus size-independent
identities over the whole output.
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


def to_dev(torch, dev, *arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in arrs]


def gpu_fwd_bwd(pkg, torch, dev, q, k, v, do):
    tq, tk, tv, tdo = to_dev(torch, dev, q, k, v, do)
    o, lse = pkg.attn_fwd(tq, tk, tv)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse)
    torch.cuda.synchronize()
    return [x.cpu().numpy() for x in (o, lse, dq, dk, dv)]


def report(tag, got, ref32, ref64=None):
    names = ("O", "dQ", "dK", "dV")
    for i, n in enumerate(names):
        ma, rl = assert_parity(f"{tag} {n}", got[i], ref32[i])
        msg = f"{tag} {n}: vs f32 max_abs={ma:.2e} rel_l2={rl:.2e}"
        if ref64 is not None:
            ma64, rl64 = errors(got[i], ref64[i])
            mc, rc = errors(ref32[i], ref64[i])
            msg += f" | vs f64 gpu={rl64:.2e} cpu_f32={rc:.2e}"
        print(msg, flush=True)


# as given these are small problems (the split-sweep kernels); widened (wide=True) they run the
# 64-row tile kernels, one tile per block; the last one has enough heads for paired tiles at ragged T
SMALL = [(1, 1, 1, 64), (1, 2, 17, 64), (2, 3, 63, 48), (1, 2, 65, 42), (2, 2, 100, 64),
         (1, 1, 257, 128), (2, 2, 130, 32), (1, 1, 64, 16), (1, 4, 200, 8), (1, 2, 129, 100),
         (3, 1, 48, 64), (2, 2, 97, 56), (1, 3, 40, 52), (2, 2, 97, 44), (1, 3, 70, 36), (8, 12, 900, 64),
         (8, 12, 900, 48)]


@pytest.mark.parametrize("wide", [False, True])
@pytest.mark.parametrize("B,H,T,D", SMALL)
def test_fused_small_shapes(pkg, torch_dev, B, H, T, D, wide):
    """Each shape as given (the small-problem kernels) and with the batch widened
    past the small-problem threshold (the 64-row tile kernels), the oracle run
    on the first and last sequence of the widened batch."""
    torch, dev = torch_dev
    if wide:
        B = widen_b(B, H, T)
    print(f"case fused B={B} H={H} T={T} D={D}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=1000 + T + D)
    o, lse, dq, dk, dv = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
    sel = sorted({0, B - 1})
    q, k, v, do, o, lse, dq, dk, dv = (a[sel] for a in (q, k, v, do, o, lse, dq, dk, dv))
    r32 = oracle.fwd_bwd_bhtd(q, k, v, do, "f32")
    r64 = oracle.fwd_bwd_bhtd(q, k, v, do, "f64")
    report(f"B{B}H{H}T{T}D{D}", (o, dq, dk, dv), r32, r64)
    # lse is not a reference output; check it against the f64 oracle's m + ln(sum)
    lse64 = r64[4]
    assert np.abs(lse - lse64).max() < 2e-5


def threaded_ref(q, k, v, do, nthreads=16):
    B, H, T, D = q.shape
    out, dq, dk, dv = oracle.batch_fwd_bwd_f32_threaded(
        *(oracle.bhtd_to_seq(a) for a in (q, k, v, do)), H, nthreads=nthreads)
    return [oracle.seq_to_bhtd(a, H) for a in (out, dq, dk, dv)]


@pytest.mark.parametrize("name,B,H,T,D", [("168-dim", 4, 4, 256, 42), ("384-dim", 16, 8, 512, 48),
                                          ("768-dim", 8, 12, 1024, 64)])
def test_baseline_configs_full(pkg, torch_dev, name, B, H, T, D):
    """BASELINE configs 1-3 at full size, seed 42, against the threaded f32 oracle."""
    torch, dev = torch_dev
    print(f"case config {name}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=42)
    o, lse, dq, dk, dv = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
    ref = threaded_ref(q, k, v, do)
    report(name, (o, dq, dk, dv), ref)


def test_4096_preset_sampled(pkg, torch_dev):
    """Config 4 (B=4, H=32, T=2048, D=128): oracle on sampled (b,h) slices, and
    size-independent identities over every slice."""
    torch, dev = torch_dev
    B, H, T, D = 4, 32, 2048, 128
    print("case config 4096 preset", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=42)
    o, lse, dq, dk, dv = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
    for b, h in ((0, 0), (3, 31), (1, 17)):
        sl = lambda a: a[b:b + 1, h:h + 1]
        ref = threaded_ref(sl(q), sl(k), sl(v), sl(do), nthreads=1)
        report(f"4096 b{b}h{h}", (sl(o), sl(dq), sl(dk), sl(dv)), ref)
    check_identities(q, k, v, do, o, dq, dk, dv)


def check_identities(q, k, v, do, o, dq, dk, dv):
    """Identities that hold for every (b,h) at any size:
    sum_j dV_j = sum_i dO_i (rows of P sum to 1); sum_j dK_j = 0 (rows of dS sum
    to 0); sum_i Q_i.dQ_i = sum_j K_j.dK_j (S is bilinear in Q and K)."""
    f = lambda a: a.astype(np.float64)
    lhs = f(dv).sum(2)
    rhs = f(do).sum(2)
    assert np.abs(lhs - rhs).max() <= 1e-3 * max(1.0, np.abs(rhs).max())
    sdk = f(dk).sum(2)
    assert np.abs(sdk).max() <= 1e-3
    a = (f(q) * f(dq)).sum((2, 3))
    b = (f(k) * f(dk)).sum((2, 3))
    assert np.abs(a - b).max() <= 1e-3 * max(1.0, np.abs(a).max())
    for x in (o, dq, dk, dv):
        assert np.isfinite(x).all()


def test_identities_headline(pkg, torch_dev):
    torch, dev = torch_dev
    q, k, v, do = pkg.synth_inputs(8, 12, 1024, 64, seed=7)
    o, lse, dq, dk, dv = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
    check_identities(q, k, v, do, o, dq, dk, dv)


def test_reference_layout_is_bit_identical(pkg, torch_dev):
    """The reference's per-sequence [T][H*D] layout (batched [B][T][E]) is read in
    place through strides and gives the same bits as [B,H,T,D]."""
    torch, dev = torch_dev
    # small problems and (widened batches) the 64-row tile kernels
    for (B, H, T, D) in ((2, 12, 300, 64), (2, 4, 256, 42), (widen_b(2, 12, 300), 12, 300, 64),
                         (widen_b(2, 4, 256), 4, 256, 42)):
        q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=5)
        base = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
        seq = [torch.from_numpy(oracle.bhtd_to_seq(a)).to(dev) for a in (q, k, v, do)]
        views = [x.view(B, T, H, D).permute(0, 2, 1, 3) for x in seq]  # strided [B,H,T,D] views
        o, lse = pkg.attn_fwd(*views[:3])
        dq, dk, dv = pkg.attn_bwd(views[0], views[1], views[2], o, views[3], lse)
        torch.cuda.synchronize()
        got = [x.contiguous().cpu().numpy() for x in (o, lse, dq, dk, dv)]
        for a, b_ in zip(got, base):
            np.testing.assert_array_equal(a, b_)


@pytest.mark.parametrize("wide", [False, True])
def test_deterministic(pkg, torch_dev, wide):
    torch, dev = torch_dev
    q, k, v, do = pkg.synth_inputs(widen_b(2, 4, 333) if wide else 2, 4, 333, 64, seed=3)
    a = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
    b = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("offset,D", [(1, 42), (2, 42), (2, 64), (0, 33), (4, 48)])
def test_small_chunk_unit_widths(pkg, torch_dev, offset, D):
    """The small-problem kernels read their chunks in units of 4, 2 or 1 floats,
    the widest that the strides, the head dim and every tensor's alignment allow:
    views at an odd float offset (1-float units), at an 8-byte offset (2-float
    units at an even head dim), an odd head dim (1-float units) and 16-byte
    aligned views (4-float units at head dim 48) all meet the bar."""
    torch, dev = torch_dev
    B, H, T = 2, 3, 77
    print(f"case small chunk units offset={offset} D={D}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=500 + D + offset)
    n = B * H * T * D

    def at_offset(a):
        buf = torch.empty(n + offset, device=dev)
        buf[offset:].copy_(torch.from_numpy(a).reshape(-1))
        return buf[offset:].view(B, H, T, D)

    tq, tk, tv, tdo = (at_offset(a) for a in (q, k, v, do))
    o, lse = pkg.attn_fwd(tq, tk, tv)
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse)
    torch.cuda.synchronize()
    ref = oracle.fwd_bwd_bhtd(q, k, v, do, "f32")
    for name, got, want in zip(("O", "dQ", "dK", "dV"), (o, dq, dk, dv), ref[:4]):
        assert_parity(f"units offset={offset} D={D} {name}", got.cpu().numpy(), want)


@pytest.mark.parametrize("stride_t", [64, 1 << 25])
def test_small_problem_row_stride_limit(pkg, torch_dev, stride_t):
    """The small-problem kernels address a chunk's 16 rows with 32-bit byte
    offsets, so a row stride whose 16 rows span 2 GiB (2^25 floats) sends even a
    tiny problem to the 64-row tile kernels; with T = 1 the views stay a few
    floats long.  Both routes meet the bar."""
    torch, dev = torch_dev
    B, H, T, D = 2, 3, 1, 64
    print(f"case small row stride {stride_t}", flush=True)
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=77)
    strides = (H * D, D, stride_t, 1)

    def view(a=None):
        t = torch.empty_strided((B, H, T, D), strides, dtype=torch.float32, device=dev)
        if a is not None:
            t.copy_(torch.from_numpy(a))
        return t

    tq, tk, tv, tdo = (view(a) for a in (q, k, v, do))
    o, lse = pkg.attn_fwd(tq, tk, tv, out=view())
    dq, dk, dv = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, dq=view(), dk=view(), dv=view())
    torch.cuda.synchronize()
    ref = oracle.fwd_bwd_bhtd(q, k, v, do, "f32")
    for name, got, want in zip(("O", "dQ", "dK", "dV"), (o, dq, dk, dv), ref[:4]):
        assert_parity(f"row stride {stride_t} {name}", got.cpu().numpy(), want)


@pytest.mark.parametrize("wide", [False, True])
def test_causality(pkg, torch_dev, wide):
    """Changing K and V at position j leaves O, LSE and dQ of rows < j unchanged."""
    torch, dev = torch_dev
    B, H, T, D = (widen_b(1, 2, 200) if wide else 1), 2, 200, 64
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=8)
    a = gpu_fwd_bwd(pkg, torch, dev, q, k, v, do)
    j = 150
    k2, v2 = k.copy(), v.copy()
    k2[:, :, j] += 0.5
    v2[:, :, j] -= 1.0
    b = gpu_fwd_bwd(pkg, torch, dev, q, k2, v2, do)
    for x, y in zip(a[:3], b[:3]):
        np.testing.assert_array_equal(x[:, :, :j], y[:, :, :j])


def test_nan_propagates(pkg, torch_dev):
    """A NaN in Q row t makes O row t NaN and leaves other rows finite; a NaN in K
    row j reaches every row that attends to j."""
    torch, dev = torch_dev
    B, H, T, D = 1, 1, 130, 64
    q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=9)
    q2 = q.copy()
    q2[0, 0, 77, 5] = np.nan
    o, lse, dq, dk, dv = gpu_fwd_bwd(pkg, torch, dev, q2, k, v, do)
    assert np.isnan(o[0, 0, 77]).all()
    assert np.isfinite(np.delete(o[0, 0], 77, axis=0)).all()
    assert np.isnan(dq[0, 0, 77]).any()
    k2 = k.copy()
    k2[0, 0, 90, 1] = np.nan
    o, lse, dq, dk, dv = gpu_fwd_bwd(pkg, torch, dev, q, k2, v, do)
    assert np.isnan(o[0, 0, 90:]).all(axis=1).all()
    assert np.isfinite(o[0, 0, :64]).all()  # query tiles before the key's tile never see it


def test_from_probs_matches_reference_contract(pkg, torch_dev):
    """wha_attn_bwd_from_probs uses att as given (compute.rs:286-314): softmax
    rows from the forward, and also arbitrary rows that are not a softmax of
    Q K^T; masked entries (j > t) hold garbage that must never be read."""
    torch, dev = torch_dev
    rng = np.random.default_rng(0)
    for (B, H, T, D) in ((2, 3, 100, 64), (1, 4, 96, 42), (1, 2, 257, 128), (1, 2, 130, 56), (1, 1, 70, 100),
                         (1, 2, 130, 48), (1, 1, 70, 44)):
        print(f"case from_probs B={B} H={H} T={T} D={D}", flush=True)
        q, k, v, do = pkg.synth_inputs(B, H, T, D, seed=11)
        qs, ks, vs, dos = (oracle.bhtd_to_seq(a) for a in (q, k, v, do))
        for kind in ("softmax", "arbitrary"):
            atts, refs = [], []
            for b in range(B):
                if kind == "softmax":
                    _, att = oracle.core_fwd(qs[b], ks[b], vs[b], H, "f32", want_att=True)
                else:
                    att = np.tril(rng.random((H, T, T)).astype(np.float32))
                refs.append(oracle.attention_backward(dos[b], qs[b], ks[b], vs[b], att, H, "f32"))
                att = att.copy()
                att[:, np.triu_indices(T, 1)[0], np.triu_indices(T, 1)[1]] = np.nan
                atts.append(att)
            att_all = np.stack(atts)
            tq, tk, tv, tdo, tatt = to_dev(torch, dev, q, k, v, do, att_all)
            dq, dk, dv = pkg.attn_bwd_from_probs(tdo, tq, tk, tv, tatt)
            torch.cuda.synchronize()
            for i, (name, got) in enumerate((("dQ", dq), ("dK", dk), ("dV", dv))):
                want = oracle.seq_to_bhtd(np.stack([r[i] for r in refs]), H)
                ma, rl = assert_parity(f"from_probs {kind} {name}", got.cpu().numpy(), want)
                print(f"from_probs {kind} B{B}H{H}T{T}D{D} {name}: max_abs={ma:.2e} rel_l2={rl:.2e}",
                      flush=True)


@pytest.mark.parametrize("B,H,Tk,D", [(4, 3, 1000, 64), (2, 2, 77, 42), (3, 2, 4097, 128),
                                      (2, 1, 1, 64), (1, 2, 300, 48)])
def test_decode_matches_last_causal_row(pkg, torch_dev, B, H, Tk, D):
    torch, dev = torch_dev
    print(f"case decode B={B} H={H} Tk={Tk} D={D}", flush=True)
    g = pkg.SynthStream(77 + Tk)
    sd = 1.0 / np.sqrt(D)
    q = g.normal(B * H * D, sd).reshape(B, H, D)
    kc = g.normal(B * H * Tk * D, sd).reshape(B, H, Tk, D)
    vc = g.normal(B * H * Tk * D, sd).reshape(B, H, Tk, D)
    tq, tk, tv = to_dev(torch, dev, q, kc, vc)
    o, lse = pkg.decode_fwd(tq, tk, tv, want_lse=True)
    torch.cuda.synchronize()
    o, lse = o.cpu().numpy(), lse.cpu().numpy()
    ref = np.empty_like(o)
    ref_lse = np.empty((B, H))
    for b in range(B):
        qseq = q[b].reshape(H * D)
        kseq = kc[b].transpose(1, 0, 2).reshape(Tk, H * D)
        vseq = vc[b].transpose(1, 0, 2).reshape(Tk, H * D)
        ref[b] = oracle.decode_one(qseq, kseq, vseq, H, "f32").reshape(H, D)
        ref_lse[b] = oracle.decode_one(qseq, kseq, vseq, H, "f64", want_lse=True)[1]
    assert_parity("decode O", o, ref)
    assert np.abs(lse - ref_lse).max() < 2e-5


def test_decode_full_config_sampled(pkg, torch_dev):
    """Config 5: 64 single-token queries x 12 heads against 8192 cached keys (D=64)."""
    torch, dev = torch_dev
    B, H, Tk, D = 64, 12, 8192, 64
    print("case decode config 5", flush=True)
    g = pkg.SynthStream(42)
    sd = 1.0 / np.sqrt(D)
    q = g.normal(B * H * D, sd).reshape(B, H, D)
    kc = torch.from_numpy(g.normal(B * H * Tk * D, sd).reshape(B, H, Tk, D)).to(dev)
    vc = torch.from_numpy(g.normal(B * H * Tk * D, sd).reshape(B, H, Tk, D)).to(dev)
    o = pkg.decode_fwd(torch.from_numpy(q).to(dev), kc, vc).cpu().numpy()
    for b, h in ((0, 0), (63, 11), (17, 5)):
        kseq = kc[b, h].cpu().numpy()
        vseq = vc[b, h].cpu().numpy()
        ref = oracle.decode_one(q[b, h], kseq, vseq, 1, "f32")
        assert_parity(f"decode b{b}h{h}", o[b, h], ref)
    assert np.isfinite(o).all()


def test_workspace_explicit_and_too_small(pkg, torch_dev):
    torch, dev = torch_dev
    q, k, v, do = pkg.synth_inputs(1, 2, 64, 64, seed=4)
    tq, tk, tv, tdo = to_dev(torch, dev, q, k, v, do)
    o, lse = pkg.attn_fwd(tq, tk, tv)
    need = pkg.attn_bwd_workspace_bytes(pkg.layout_of(tq))
    ws = torch.empty(need // 4, dtype=torch.float32, device=dev)
    a = pkg.attn_bwd(tq, tk, tv, o, tdo, lse, workspace=ws)
    b = pkg.attn_bwd(tq, tk, tv, o, tdo, lse)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    small = torch.empty(4, dtype=torch.float32, device=dev)
    with pytest.raises(pkg.WaveHipError) as e:
        pkg.attn_bwd(tq, tk, tv, o, tdo, lse, workspace=small)
    assert e.value.code == -4


def test_kernel_timing_hooks(pkg, torch_dev):
    """Per-kernel event timing on the 64-row tile kernels (a layout above the
    small-problem threshold, which runs no separate statistics pass)."""
    torch, dev = torch_dev
    q, k, v, do = pkg.synth_inputs(widen_b(1, 2, 128), 2, 128, 64, seed=4)
    tq, tk, tv, tdo = to_dev(torch, dev, q, k, v, do)
    pkg.timing_reset()
    pkg.timing_enable(True)
    try:
        for _ in range(3):
            o, lse = pkg.attn_fwd(tq, tk, tv)
            pkg.attn_bwd(tq, tk, tv, o, tdo, lse)
        torch.cuda.synchronize()
        for name in ("attn_fwd", "attn_bwd_delta", "attn_bwd_dq", "attn_bwd_dkv"):
            ms, n = pkg.timing_read(name)
            assert n == 3 and ms > 0, (name, ms, n)
    finally:
        pkg.timing_enable(False)
        pkg.timing_reset()
