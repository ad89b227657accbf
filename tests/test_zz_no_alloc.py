"""GPU test of the allocation-free MHA backward (cxg_mha_bwd_noalloc).

The entry point keeps its scratch (Di and the statistics pass's lse) in a
static device array instead of a workspace.  Its results must match
cxg_mha_bwd's on the same inputs (to the parity bar: dQ is summed with float
atomics, whose order varies between calls), over two calls in a row, the
second on a smaller problem (the array keeps the first call's contents), with
and without the forward's lse; a problem beyond the array's capacity is
refused before any launch.
"""
import numpy as np
import pytest

from helpers import assert_close, normal_inputs

pytestmark = pytest.mark.gpu


def _run_pair(dev, B, S, H, Dh, seed, use_lse):
    import torch
    import cxxgpt_attn as cx
    shape = (B * S, H * Dh)
    Q, K, V, dO = (torch.from_numpy(a).to(dev) for a in normal_inputs(shape, shape, seed))
    O = torch.empty_like(Q)
    lse = torch.empty(B * H * S, device=dev) if use_lse else None
    cx.mha_fwd(Q, K, V, O, B, S, H, Dh, lse=lse)
    ref = [torch.full_like(Q, float("nan")) for _ in range(3)]
    cx.mha_bwd(Q, K, V, O, dO, *ref, B, S, H, Dh, lse=lse)
    got = [torch.full_like(Q, float("nan")) for _ in range(3)]
    cx.mha_bwd_noalloc(Q, K, V, O, dO, *got, B, S, H, Dh, lse=lse)
    torch.cuda.synchronize()
    for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
        assert_close(g.cpu().numpy(), r.cpu().numpy(),
                     f"noalloc B{B}S{S}H{H}Dh{Dh} lse={use_lse} {name}")


@pytest.mark.parametrize("use_lse", [True, False])
def test_noalloc_matches_workspace_path(dev, use_lse):
    # C2's shape, then a smaller ragged one on the same (dirty) scratch array
    _run_pair(dev, 8, 256, 12, 64, 1000, use_lse)
    _run_pair(dev, 2, 77, 3, 32, 1001, use_lse)


def test_noalloc_rejects_oversize(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(16, device=dev)
    P = cx._ptr
    rows = cx.MHA_BWD_NOALLOC_MAX_ROWS
    st = cx.call_status("cxg_mha_bwd_noalloc", *[P(t)] * 9, 1, rows + 1, 1, 64,
                        cx._stream(None))
    assert st == cx.CXG_ERR_WORKSPACE
    # the capacity check precedes the pointer checks: NULL outputs give
    # CXG_ERR_WORKSPACE one row past the limit and CXG_ERR_NULL at it, so the
    # limit itself is accepted by the size check (no launch either way)
    st = cx.call_status("cxg_mha_bwd_noalloc", *[P(t)] * 6, None, None, None, 1, rows + 1, 1,
                        64, cx._stream(None))
    assert st == cx.CXG_ERR_WORKSPACE
    st = cx.call_status("cxg_mha_bwd_noalloc", *[P(t)] * 6, None, None, None, 1, rows, 1, 64,
                        cx._stream(None))
    assert st == cx.CXG_ERR_NULL
