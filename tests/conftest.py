"""Shared fixtures.  Tests marked ``gpu`` need an MI355X (run with -m gpu on the
GPU box); everything else runs on the CPU."""
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

# parity bar from the north star: max-abs <= 1e-4 and relative L2 <= 1e-5
MAX_ABS = 1e-4
REL_L2 = 1e-5


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


def widen_b(B, H, T, blocks=256):
    """The smallest batch B' >= B at which a [B',H,T,D] layout leaves the
    small-problem kernels for the 64-row tile kernels (B'*H*ceil(T/64) >= 256;
    rows longer than 1024 never take the small path), so that a small test
    shape can exercise either kernel family."""
    return max(B, -(-blocks // (H * ((T + 63) // 64))))


def errors(got, want):
    """(max_abs, rel_l2) of got vs want, both promoted to float64."""
    g = np.asarray(got, dtype=np.float64)
    w = np.asarray(want, dtype=np.float64)
    max_abs = float(np.abs(g - w).max()) if g.size else 0.0
    den = float(np.linalg.norm(w))
    rel = float(np.linalg.norm(g - w) / den) if den > 0 else float(np.linalg.norm(g - w))
    return max_abs, rel


def assert_parity(name, got, want, max_abs=MAX_ABS, rel_l2=REL_L2):
    ma, rl = errors(got, want)
    assert np.isfinite(ma) and ma <= max_abs and rl <= rel_l2, \
        f"{name}: max_abs={ma:.3e} (<= {max_abs:g}) rel_l2={rl:.3e} (<= {rel_l2:g})"
    return ma, rl


def make_wave_weights(H, C, E, seed, dtype=np.float32):
    """Wave-attention weights in the packed layout (harmonic_raw, proj_w
    [H][2+C][E], proj_b, v_w [H][hd][hd], v_b, out_w [E][E], out_b), scaled so
    that projections of a unit-variance input are O(1)."""
    rng = np.random.default_rng(seed)
    hd = E // H
    w = dict(
        hraw=rng.normal(0.5, 1.0, size=H),
        proj_w=rng.normal(0, 1.0 / np.sqrt(E), size=(H, 2 + C, E)),
        proj_b=rng.normal(0, 0.1, size=(H, 2 + C)),
        v_w=rng.normal(0, 1.0 / np.sqrt(hd), size=(H, hd, hd)),
        v_b=rng.normal(0, 0.1, size=(H, hd)),
        out_w=rng.normal(0, 1.0 / np.sqrt(E), size=(E, E)),
        out_b=rng.normal(0, 0.1, size=E),
    )
    return {k: v.astype(dtype) for k, v in w.items()}
