"""GPU parity of the projection GEMMs and of ComputeBackend::attention with its
c_attn / c_proj projections (src/common/compute.rs:357-414), through the C ABI.
Small shapes against the reference-order f32 oracle; the headline-size GEMMs
against an f64 matrix product (the oracle's scalar loops would take minutes)."""
import numpy as np
import pytest

import oracle
from conftest import assert_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available()
    return torch, torch.device("cuda:0")


def rnd(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


# (333, 64, 64): the 64 x 64 projection kernel (head64_gemm_kernel) with a partial 16-row tile, forward with
# and without bias and the non-accumulating input gradient
SHAPES = [(1, 1, 1), (37, 45, 29), (300, 130, 70), (129, 257, 128), (1000, 768, 384), (64, 2304, 768),
          (333, 64, 64)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_linear_fwd_dx_dw(pkg, torch_dev, M, N, K):
    torch, dev = torch_dev
    print(f"case linear M={M} N={N} K={K}", flush=True)
    # unit-scale activations and 1/sqrt(rows)-scale upstream gradients keep every
    # output O(1), the regime the max-abs part of the parity bar is stated for
    x, w, b, dy = rnd((M, K), 1), rnd((N, K), 2, 1 / np.sqrt(K)), rnd(N, 3), rnd((M, N), 4, 1 / np.sqrt(M))
    tx, tw, tb, tdy = (torch.from_numpy(a).to(dev) for a in (x, w, b, dy))
    y = pkg.linear_fwd(tx, tw, tb)
    y_nb = pkg.linear_fwd(tx, tw)
    dx = pkg.linear_bwd_dx(tdy, tw)
    dw, db = pkg.linear_bwd_dw(tdy, tx, compute_bias=True)
    torch.cuda.synchronize()
    assert_parity("y", y.cpu().numpy(), oracle.linear(x, w, b, "f32"))
    assert_parity("y (no bias)", y_nb.cpu().numpy(), oracle.linear(x, w, None, "f32"))
    assert_parity("dx", dx.cpu().numpy(), oracle.linear_backward_dx(dy, w, "f32"))
    rw, rb = oracle.outer_product_accum(dy, x, True, "f32")
    assert_parity("dw", dw.cpu().numpy(), rw)
    assert_parity("db", db.cpu().numpy(), rb)


def test_linear_strided_rows(pkg, torch_dev):
    """Rows with a stride: q/k/v column blocks of a fused [T][3E] buffer."""
    torch, dev = torch_dev
    T, E = 200, 96
    qkv = rnd((T, 3 * E), 5)
    w, b = rnd((E, E), 6, 1 / np.sqrt(E)), rnd(E, 7)
    t = torch.from_numpy(qkv).to(dev)
    for c in range(3):
        view = t[:, c * E:(c + 1) * E]
        y = pkg.linear_fwd(view, torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev))
        assert_parity(f"block {c}", y.cpu().numpy(), oracle.linear(qkv[:, c * E:(c + 1) * E], w, b, "f32"))


def test_headline_projection_sizes_vs_f64(pkg, torch_dev):
    """c_attn and c_proj of the 768-dim config over the whole batch (M = 8*1024 rows)."""
    torch, dev = torch_dev
    M, E = 8192, 768
    x = rnd((M, E), 8)
    for N in (3 * E, E):
        w, b, dy = rnd((N, E), 9, 1 / np.sqrt(E)), rnd(N, 10), rnd((M, N), 11, 1 / np.sqrt(M))
        tx, tw, tb, tdy = (torch.from_numpy(a).to(dev) for a in (x, w, b, dy))
        y = pkg.linear_fwd(tx, tw, tb).cpu().numpy()
        dx = pkg.linear_bwd_dx(tdy, tw).cpu().numpy()
        dw, db = (a.cpu().numpy() for a in pkg.linear_bwd_dw(tdy, tx))
        x64, w64, dy64 = x.astype(np.float64), w.astype(np.float64), dy.astype(np.float64)
        assert_parity(f"y N={N}", y, x64 @ w64.T + b)
        assert_parity(f"dx N={N}", dx, dy64 @ w64)
        assert_parity(f"dw N={N}", dw, dy64.T @ x64)
        assert_parity(f"db N={N}", db, dy64.sum(0))


def test_dw_is_deterministic(pkg, torch_dev):
    torch, dev = torch_dev
    dy = torch.from_numpy(rnd((4096, 300), 12, 1 / 64)).to(dev)
    x = torch.from_numpy(rnd((4096, 200), 13)).to(dev)
    a = [t.cpu().numpy() for t in pkg.linear_bwd_dw(dy, x)]
    b = [t.cpu().numpy() for t in pkg.linear_bwd_dw(dy, x)]
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)


@pytest.mark.parametrize("T,E,H", [(64, 168, 4), (130, 384, 8), (256, 768, 12), (1, 64, 2)])
def test_backend_attention_with_projections(pkg, T, E, H):
    x = rnd((T, E), 20)
    wa, ba = rnd((3 * E, E), 21, 1 / np.sqrt(E)), rnd(3 * E, 22, 0.1)
    wp, bp = rnd((E, E), 23, 1 / np.sqrt(E)), rnd(E, 24, 0.1)
    weights = pkg.AttentionWeights(pkg.LinearWeights(wa, ba), pkg.LinearWeights(wp, bp), H)
    got = pkg.HipBackend().attention(weights, x)
    assert_parity("attention", got, oracle.attention_full(x, wa, ba, wp, bp, H, "f32"))
