"""P-row export for the monitors that read materialised attention rows
(src/monitors/attn_monitor.rs:26-80, softmax_rows contract at
src/monitors/junctions/value_range.rs:117-121), checked against the oracle's
materialised att rows."""
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


@pytest.mark.parametrize("B,H,T,D", [(2, 3, 100, 64), (1, 4, 77, 42), (1, 2, 300, 128), (2, 2, 1, 48)])
def test_probs_rows_match_oracle_att(pkg, torch_dev, B, H, T, D):
    torch, dev = torch_dev
    q, k, v = pkg.synth_inputs(B, H, T, D, seed=31 + T, with_do=False)
    tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    _, lse = pkg.attn_fwd(tq, tk, tv)
    rows = sorted({0, T // 2, T - 1})
    got = pkg.attn_probs_rows(tq, tk, lse, rows).cpu().numpy()
    qs, ks, vs = (oracle.bhtd_to_seq(a) for a in (q, k, v))
    for b in range(B):
        _, att = oracle.core_fwd(qs[b], ks[b], vs[b], H, "f32", want_att=True)
        assert_parity(f"P rows b{b}", got[b], att[:, rows, :])


def test_softmax_rows_contract_and_head_stats(pkg, torch_dev):
    """Rows in [0, 1 + 1e-5] summing to 1 within 1e-4 (the softmax_rows contract),
    and analyze_attention's statistics of the last row match the oracle's."""
    torch, dev = torch_dev
    B, H, T, D = 8, 12, 1024, 64
    q, k, v = pkg.synth_inputs(B, H, T, D, seed=42, with_do=False)
    tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    _, lse = pkg.attn_fwd(tq, tk, tv)
    rows = [0, 1, 511, T - 1]
    p = pkg.attn_probs_rows(tq, tk, lse, rows).cpu().numpy().astype(np.float64)
    assert p.min() >= 0.0 and p.max() <= 1.0 + 1e-5
    for r_i, t in enumerate(rows):
        np.testing.assert_allclose(p[:, :, r_i, :].sum(-1), 1.0, atol=1e-4)
        assert np.all(p[:, :, r_i, t + 1:] == 0.0)
    stats = pkg.attention_head_stats(p[:, :, -1, :].astype(np.float32))
    qs, ks, vs = (oracle.bhtd_to_seq(a) for a in (q, k, v))
    for b in (0, 7):
        _, att = oracle.core_fwd(qs[b], ks[b], vs[b], H, "f32", want_att=True)
        ref = pkg.attention_head_stats(att[:, -1, :])
        np.testing.assert_allclose(stats["entropy"][b], ref["entropy"], atol=1e-4)
        np.testing.assert_allclose(stats["max_weight"][b], ref["max_weight"], atol=1e-6)
        np.testing.assert_array_equal(stats["top_position"][b], ref["top_position"])
        np.testing.assert_allclose(stats["self_attn_frac"][b], ref["self_attn_frac"], atol=1e-6)
