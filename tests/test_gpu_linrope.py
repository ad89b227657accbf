"""GPU parity tests of TwoStageGPT's stage 2 with RoPE fused into the
linear-attention kernels (cxg_kattn_rope_fwd / cxg_kattn_rope_bwd).

The reference's stage 2 rotates q and k in place over the whole feature width
(rope_fwd(lqc, lkc, B, S, E, E), two_stage_gpt.hpp:113), runs kernel_attn_fwd
on the rotated tensors, and in the backward runs bwd_step1 / bwd_dQ /
bwd_dKdV on them and rotates dq, dk back (rope_bwd, :149-160).  Each case
here composes the oracle the same way: orc.rope(+1) on Q and K, the
kattn_fwd / step1 / dQ / dKdV restatements on the rotated inputs (the
backward on the GPU's own O and den, as kernel_test.cpp:276-292 does), then
orc.rope(-1) on dQ and dK.  The fused entry points must match that chain and
leave Q and K unchanged; the cases cover the quadratic form (stage 2's
training width D = E = 512 and short sequences), the chunked scan with and
without the forward's context (D = E = 64, several segments), widths that
are not multiples of 4, D != E, and widths above 512 (rotation outside the
kernels).
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, normal_inputs

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _nan(dev, *shape):
    import torch
    return torch.full(shape, float("nan"), device=dev)


def _np(t):
    return t.cpu().numpy()


def rope_pair(dev, Q, K, V, dO, B, S, D, E, use_ctx):
    import torch
    import cxxgpt_attn as cx
    N = B * S
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    n = cx.lin_ctx_size(B, S, D, E) if use_ctx else 0
    ctx = torch.full((n // 4,), float("nan"), device=dev) if n else None
    cx.kattn_rope_fwd(tQ, tK, tV, O, den, B, S, D, E, ctx=ctx)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.kattn_rope_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, D, E, ctx=ctx)
    torch.cuda.synchronize()
    assert np.array_equal(_np(tQ), Q) and np.array_equal(_np(tK), K), "Q, K modified"
    return dict(O=_np(O), den=_np(den), dQ=_np(dQ), dK=_np(dK), dV=_np(dV))


def check_rope_pair(dev, Q, K, V, dO, B, S, D, E, tag, use_ctx=False):
    g = rope_pair(dev, Q, K, V, dO, B, S, D, E, use_ctx)
    tag = f"{tag}{' ctx' if use_ctx else ''}"
    Qr, Kr = orc.rope(Q, B, S, D, D, 1.0), orc.rope(K, B, S, D, D, 1.0)
    rO, rden, rzc = orc.kattn_fwd(Qr, Kr, V, B, S, D, E, nthreads=8)
    assert_close(g["O"], rO, f"{tag} O")
    assert_close(g["den"], rden, f"{tag} den")
    dnum, dden = orc.kattn_bwd_step1(g["O"], dO, g["den"], B * S, E)
    rdQr = orc.kattn_bwd_dQ(Kr, V, dnum, dden, rzc, Qr, B, S, D, E, nthreads=8)
    rdKr, rdV = orc.kattn_bwd_dKdV(Qr, Kr, V, dnum, dden, B, S, D, E, nthreads=8)
    assert_close(g["dQ"], orc.rope(rdQr, B, S, D, D, -1.0), f"{tag} dQ")
    assert_close(g["dK"], orc.rope(rdKr, B, S, D, D, -1.0), f"{tag} dK")
    assert_close(g["dV"], rdV, f"{tag} dV")


@pytest.mark.parametrize("B,S,D,E", [
    (4, 256, 512, 512),   # stage 2 at the training width (two_stage_train.cpp:168-170)
    (3, 100, 64, 64),     # short sequences: the quadratic form at narrow width
    (2, 77, 96, 64),      # D != E
    (1, 33, 258, 130),    # widths not multiples of 4
    (50, 112, 512, 512),  # a large batch, an odd block count
])
@pytest.mark.parametrize("use_ctx", [False, True])
def test_rope_quadratic_form(dev, B, S, D, E, use_ctx):
    """With the context, the block-score path's forward leaves the RoPE
    features and score blocks there for the backward (widths multiples of 16
    above 64; other shapes have no context to write)."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 41 * S + D + E)
    check_rope_pair(dev, Q, K, V, dO, B, S, D, E, tag=f"rope quad B{B}S{S}D{D}E{E}",
                    use_ctx=use_ctx)


@pytest.mark.parametrize("use_ctx", [False, True])
@pytest.mark.parametrize("B,S,D,E", [
    (8, 1024, 64, 64),    # several segments per sequence
    (96, 4096, 64, 64),   # C3's shape
    (2, 300, 32, 48),     # narrow widths (column masks)
    (3, 200, 6, 8),       # D not a multiple of 4
])
def test_rope_chunked_scan(dev, B, S, D, E, use_ctx):
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 43 * S + D + E)
    check_rope_pair(dev, Q, K, V, dO, B, S, D, E, tag=f"rope scan B{B}S{S}D{D}E{E}",
                    use_ctx=use_ctx)


def test_rope_wider_than_512(dev):
    B, S, D, E = 2, 40, 768, 520
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 47)
    check_rope_pair(dev, Q, K, V, dO, B, S, D, E, tag="rope generic")


def test_rope_errors(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(64, device=dev)
    P = cx._ptr
    st = cx._stream(None)
    # odd width: RoPE pairs columns
    assert cx.call_status("cxg_kattn_rope_fwd", *[P(t)] * 5, None, 0, 1, 4, 7, 8, st) == \
        cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_kattn_rope_bwd", *[P(t)] * 6, None, *[P(t)] * 3, 1, 4, 7, 8,
                          st) == cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_kattn_rope_fwd", *[P(t)] * 5, None, 0, 1, 4, 1026, 8, st) == \
        cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_kattn_rope_fwd", None, *[P(t)] * 4, None, 0, 1, 4, 8, 8, st) == \
        cx.CXG_ERR_NULL


def test_rope_refuses_plain_context(dev):
    """A context written by the plain ELU+1 forward holds unrotated sums: the
    RoPE backward refuses it (and the plain backward a RoPE forward's)."""
    import torch
    import cxxgpt_attn as cx
    B, S, D, E = 4, 1024, 64, 64
    N = B * S
    Q, K, V, dO = (_t(a, dev) for a in normal_inputs((N, D), (N, E), 49))
    n = cx.lin_ctx_size(B, S, D, E)
    assert n > 0
    ctx = torch.zeros(n // 4, device=dev)
    O, den = torch.empty(N, E, device=dev), torch.empty(N, device=dev)
    out = [torch.empty(N, D, device=dev) for _ in range(3)]
    cx.kattn_fwd_ctx(Q, K, V, O, den, ctx, B, S, D, E)
    st = cx.call_status("cxg_kattn_rope_bwd", *[cx._ptr(x) for x in (Q, K, V, O, dO, den, ctx)],
                        *[cx._ptr(x) for x in out], B, S, D, E, cx._stream(None))
    assert st == cx.CXG_ERR_WORKSPACE
    cx.kattn_rope_fwd(Q, K, V, O, den, B, S, D, E, ctx=ctx)
    st = cx.call_status("cxg_kattn_bwd", *[cx._ptr(x) for x in (Q, K, V, O, dO, den, ctx)],
                        *[cx._ptr(x) for x in out], B, S, D, E, cx._stream(None))
    assert st == cx.CXG_ERR_WORKSPACE
    torch.cuda.synchronize()
