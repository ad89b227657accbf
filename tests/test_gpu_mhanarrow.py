"""GPU parity tests of the narrow-head MHA kernels (mhanarrow.hip): heads of at
most 16 columns on sequences whose rows fit in LDS (S rounded up to 16, times
8 columns for Dh <= 8 or 16 otherwise, at most 4096 floats) take one workgroup
per head through the same C ABI calls (cxg_mha_fwd / cxg_mha_bwd /
cxg_mha_bwd_noalloc).  TwoStageGPT's stage 1 is the reference's shape for
them: B = 32, S = 256, H = 64, Dh = 8 (two_stage_train.cpp:168-170).

Forward O and lse against the oracle, the backward with lse and without it
(the reference's signature, statistics recomputed in the kernel) against the
oracle fed the GPU's forward output, as the reference's own kernel test does
(src/TwoStage/kernel_test.cpp:246, :405).
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, normal_inputs

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _launches(name):
    import cxxgpt_attn as cx
    return cx.prof_query(name)[1]


def _run(dev, Q, K, V, dO, B, S, H, Dh):
    """Forward (O, lse), then the backward with and without lse; returns the
    outputs and the narrow kernels' launch counts."""
    import torch
    import cxxgpt_attn as cx
    tQ, tK, tV, tdO = (_t(a, dev) for a in (Q, K, V, dO))
    O = torch.full_like(tQ, float("nan"))
    lse = torch.full((B * H * S,), float("nan"), device=dev)
    torch.cuda.synchronize()
    cx.prof_reset()
    cx.prof_enable(True)
    cx.mha_fwd(tQ, tK, tV, O, B, S, H, Dh, lse=lse)
    grads = {}
    for use_lse in (True, False):
        outs = [torch.full_like(tQ, float("nan")) for _ in range(3)]
        cx.mha_bwd(tQ, tK, tV, O, tdO, *outs, B, S, H, Dh, lse=lse if use_lse else None)
        grads[use_lse] = outs
    torch.cuda.synchronize()
    counts = (_launches("mha_nar_fwd"), _launches("mha_nar_bwd"), _launches("mha_fwd"),
              _launches("mha_bwd"))
    cx.prof_enable(False)
    cx.prof_reset()
    return (O.cpu().numpy(), lse.cpu().numpy(),
            {k: [g.cpu().numpy() for g in v] for k, v in grads.items()}, counts)


@pytest.mark.parametrize("B,S,H,Dh", [
    (32, 256, 64, 8),    # TwoStageGPT stage 1 (BH a multiple of 8: heads grouped by XCD)
    (3, 100, 5, 7),      # ragged S, Dh not a multiple of 4 (scalar loads)
    (2, 33, 3, 4),
    (1, 512, 2, 8),      # the longest sequence at Dh <= 8
    (2, 256, 3, 16),     # the longest at 16 columns; no spare column for the row sums
    (2, 250, 4, 12),     # 16-column padding with a spare column
    (1, 1, 1, 8),        # one row
    (2, 17, 9, 1),       # one column, two row blocks
    (4, 64, 6, 2),
])
def test_narrow_heads(dev, B, S, H, Dh):
    Q, K, V, dO = normal_inputs((B * S, H * Dh), (B * S, H * Dh), 17 * S + 5 * H + Dh)
    O, lse, grads, counts = _run(dev, Q, K, V, dO, B, S, H, Dh)
    assert counts == (1, 2, 0, 0), f"launches (nar fwd, nar bwd, mha fwd, mha bwd): {counts}"
    rO, rlse = orc.mha_fwd(Q, K, V, B, S, H, Dh, nthreads=8, want_lse=True)
    tag = f"B{B}S{S}H{H}Dh{Dh}"
    assert_close(O, rO, f"{tag} O")
    assert_close(lse, rlse, f"{tag} lse")
    rdQ, rdK, rdV = orc.mha_bwd(Q, K, V, O, dO, B, S, H, Dh, nthreads=8)
    for use_lse, (dQ, dK, dV) in grads.items():
        assert_close(dQ, rdQ, f"{tag} dQ lse={use_lse}")
        assert_close(dK, rdK, f"{tag} dK lse={use_lse}")
        assert_close(dV, rdV, f"{tag} dV lse={use_lse}")


@pytest.mark.parametrize("std", [1.5, 2.0])
def test_narrow_heads_large_scores(dev, std):
    """Scores spread over many units of log2 (up to |s| = 30 at std 2): the
    forward's and the statistics' reference maximum moves several times along
    a row (the lazy rescale), and the probabilities of most keys underflow.
    Larger inputs are not a parity case: at std 3 the fp32 oracle's own dQ
    is off the float64 gradient by more than the bar (the rounding of O and
    Di, whose difference dP - Di cancels)."""
    B, S, H, Dh = 2, 300, 4, 8
    Q, K, V, dO = normal_inputs((B * S, H * Dh), (B * S, H * Dh), 99 + int(std))
    Q, K = Q * std, K * std
    O, lse, grads, counts = _run(dev, Q, K, V, dO, B, S, H, Dh)
    assert counts[:2] == (1, 2)
    rO, rlse = orc.mha_fwd(Q, K, V, B, S, H, Dh, nthreads=8, want_lse=True)
    assert_close(O, rO, f"std{std} O")
    assert_close(lse, rlse, f"std{std} lse")
    rdQ, rdK, rdV = orc.mha_bwd(Q, K, V, O, dO, B, S, H, Dh, nthreads=8)
    for use_lse, (dQ, dK, dV) in grads.items():
        assert_close(dQ, rdQ, f"std{std} dQ lse={use_lse}")
        assert_close(dK, rdK, f"std{std} dK lse={use_lse}")
        assert_close(dV, rdV, f"std{std} dV lse={use_lse}")


@pytest.mark.parametrize("B,S,H,Dh", [(1, 513, 2, 8), (1, 257, 2, 12), (2, 64, 2, 17)])
def test_beyond_narrow_limits(dev, B, S, H, Dh):
    """Just past the LDS limit or 16 columns: the 64-row tile kernels."""
    Q, K, V, dO = normal_inputs((B * S, H * Dh), (B * S, H * Dh), 3 * S + Dh)
    O, lse, grads, counts = _run(dev, Q, K, V, dO, B, S, H, Dh)
    assert counts[0] == 0 and counts[1] == 0 and counts[2] == 1, counts
    assert_close(O, orc.mha_fwd(Q, K, V, B, S, H, Dh, nthreads=8), "O")
    rdQ, rdK, rdV = orc.mha_bwd(Q, K, V, O, dO, B, S, H, Dh, nthreads=8)
    assert_close(grads[True][0], rdQ, "dQ")
    assert_close(grads[True][1], rdK, "dK")
    assert_close(grads[True][2], rdV, "dV")


def test_narrow_noalloc(dev):
    """The allocation-free backward takes the same narrow kernel (it needs no
    scratch); its results against the workspace path's."""
    import torch
    import cxxgpt_attn as cx
    B, S, H, Dh = 4, 200, 8, 8
    Q, K, V, dO = (_t(a, dev) for a in normal_inputs((B * S, H * Dh), (B * S, H * Dh), 5150))
    O = torch.empty_like(Q)
    cx.mha_fwd(Q, K, V, O, B, S, H, Dh)
    ref = [torch.full_like(Q, float("nan")) for _ in range(3)]
    cx.mha_bwd(Q, K, V, O, dO, *ref, B, S, H, Dh)
    got = [torch.full_like(Q, float("nan")) for _ in range(3)]
    cx.mha_bwd_noalloc(Q, K, V, O, dO, *got, B, S, H, Dh)
    torch.cuda.synchronize()
    for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
        assert_close(g.cpu().numpy(), r.cpu().numpy(), f"noalloc narrow {name}")
