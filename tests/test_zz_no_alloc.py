"""wha_decode_fwd_noalloc (split-K partials in the library's static device
scratch, no allocation inside the call) against wha_decode_fwd (workspace
path) through the C ABI: identical bits for O and LSE on two calls in a row,
the second with a smaller input, then the first shape again; plus the f32
oracle's decode row on the first call."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import assert_parity

pytestmark = pytest.mark.gpu


def _inputs(pkg, B, H, T, D, seed):
    g = pkg.SynthStream(seed)
    sd = 1.0 / np.sqrt(D)
    q = g.normal(B * H * D, sd).reshape(B, H, D)
    kc = g.normal(B * H * T * D, sd).reshape(B, H, T, D)
    vc = g.normal(B * H * T * D, sd).reshape(B, H, T, D)
    return q, kc, vc


@pytest.mark.parametrize("shapes", [[(8, 12, 5000, 64), (3, 4, 700, 48), (8, 12, 5000, 64)]])
def test_noalloc_decode_matches_workspace_decode(pkg, shapes):
    import oracle
    dev = torch.device("cuda:0")
    for i, (B, H, T, D) in enumerate(shapes):
        print(f"noalloc decode call {i}: B={B} H={H} T={T} D={D}", flush=True)
        q, kc, vc = _inputs(pkg, B, H, T, D, seed=100 + i)
        tq, tk, tv = (torch.from_numpy(a).to(dev) for a in (q, kc, vc))
        ws = torch.empty(int(pkg.lib().wha_decode_workspace_size(ctypes.byref(pkg.layout_of(tk)))) // 4 + 64,
                         device=dev)
        o_ref, lse_ref = pkg.decode_fwd(tq, tk, tv, want_lse=True, workspace=ws)
        o, lse = pkg.decode_fwd_noalloc(tq, tk, tv, want_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), f"call {i}: O differs from wha_decode_fwd"
        assert torch.equal(lse, lse_ref), f"call {i}: LSE differs from wha_decode_fwd"
        if i == 0:
            # the f32 oracle's decode row for two (b, h) of the first call
            for b, h in ((0, 0), (B - 1, H - 1)):
                want = oracle.decode_one(q[b, h], kc[b, h], vc[b, h], 1, "f32")
                assert_parity(f"O[{b},{h}]", o[b, h].cpu().numpy(), want)
