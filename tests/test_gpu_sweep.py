"""Seeded random shapes through the main entry points, against the oracle.

The other GPU tests choose their shapes by hand (tile and chunk boundaries,
job rounds, segment counts, the benchmark configurations).  This sweep draws
shapes from fixed seeds over the ranges the kernels accept, so that
combinations nobody picked (a ragged last tile with an odd head width and a
job count just past a round, say) are exercised too.  Each case states its
shape in its test id.  Checks are the same as the hand-picked tests':
softmax MHA forward and backward (with and without lse) against
ref_mha_fwd / ref_mha_bwd (kernel_test.cpp:12-93); the two_stage linear
chain and the fused pair against the linear-attention oracle
(kernel_test.cpp:96-193).
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, normal_inputs
from test_gpu_linbwd import check_fused_kattn
from test_gpu_linear import check_kattn
from test_gpu_mha import _run_bwd, _run_fwd

pytestmark = pytest.mark.gpu

_DH = [1, 2, 3, 4, 5, 7, 8, 12, 16, 20, 31, 32, 33, 48, 63, 64, 65, 96, 100, 127, 128, 129,
       160, 200, 255, 256]


def _mha_shapes(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        Dh = int(rng.choice(_DH))
        B = int(rng.integers(1, 4))
        H = int(rng.integers(1, 5))
        # bound the oracle's work (B H S^2 Dh) to a few seconds
        smax = int(min(600, np.sqrt(4.0e8 / (B * H * Dh))))
        S = int(rng.integers(1, max(2, smax)))
        out.append((B, S, H, Dh))
    return out


def _lin_shapes(n, seed, wmax):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        # full-width rows (the 16-byte path) two times in five
        D = wmax if rng.random() < 0.4 else int(rng.integers(1, wmax + 1))
        E = wmax if rng.random() < 0.4 else int(rng.integers(1, wmax + 1))
        B = int(rng.integers(1, 7))
        # short sequences (one or two segments, the quadratic form) a third of the time
        S = int(rng.integers(1, 200 if rng.random() < 0.33 else (1200 if wmax <= 64 else 300)))
        out.append((B, S, D, E))
    return out


@pytest.mark.parametrize("B,S,H,Dh", _mha_shapes(40, 2026))
def test_mha_random_shapes(dev, B, S, H, Dh):
    """Forward (O, lse), then the backward with the forward's lse and without
    it (the reference's signature, which recomputes the statistics)."""
    Q, K, V, dO = normal_inputs((B * S, H * Dh), (B * S, H * Dh), 31 * S + 7 * H + Dh)
    O, lse = _run_fwd(dev, Q, K, V, B, S, H, Dh, want_lse=True)
    assert_close(O, orc.mha_fwd(Q, K, V, B, S, H, Dh, nthreads=8), "O")
    assert np.all(np.isfinite(lse))
    ref = orc.mha_bwd(Q, K, V, O, dO, B, S, H, Dh, nthreads=8)
    for lse_arg, tag in ((lse, "lse"), (None, "no-lse")):
        got = _run_bwd(dev, Q, K, V, O, dO, B, S, H, Dh, lse=lse_arg)
        for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
            assert_close(g, r, f"{tag} {name}")


@pytest.mark.parametrize("B,S,D,E", _lin_shapes(24, 4096, 64))
def test_linear_chain_random_shapes(dev, B, S, D, E):
    """two_stage chain (fwd with z_cache and state, step 1, dQ, dK/dV) at
    narrow widths: the chunked scan, or the quadratic form at S <= 128."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 17 * S + 5 * D + E)
    check_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"B{B}S{S}D{D}E{E}")


@pytest.mark.parametrize("B,S,D,E", _lin_shapes(24, 8192, 64))
def test_linear_fused_random_shapes(dev, B, S, D, E):
    """The fused pair, with and without the forward's context."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 19 * S + 3 * D + E)
    for use_ctx in (False, True):
        check_fused_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"B{B}S{S}D{D}E{E}",
                          use_ctx=use_ctx)


@pytest.mark.parametrize("B,S,D,E", _lin_shapes(12, 512, 512))
def test_linear_wide_random_shapes(dev, B, S, D, E):
    """Widths up to 512 (the quadratic form above 64) through the chain."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 23 * S + D + 11 * E)
    check_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"B{B}S{S}D{D}E{E}")
