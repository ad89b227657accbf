"""GPU parity tests of the rotary position embedding (C ABI cxg_rope_fwd/bwd).

Mirrors the reference's RoPE block (src/TwoStage/kernel_test.cpp:443-499):
forward and backward rotations against ref_rope (the C oracle), and the
round trip with Q and K one tensor; plus the shapes two_stage_gpt.hpp feeds
it (stage-1 heads :102/:174, the stage-2 full-width head :113/:160), long
sequences (angles up to S-1 radians), ragged and unaligned shapes, one
tensor only, and the argument checks.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, kernel_test_inputs, normal_inputs

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _run(dev, fn, Q, K, B, S, D, hd):
    import cxxgpt_attn as cx
    tQ = None if Q is None else _t(Q, dev)
    tK = None if K is None else _t(K, dev)
    getattr(cx, fn)(tQ, tK, B, S, D, hd)
    import torch
    torch.cuda.synchronize()
    return (None if tQ is None else tQ.cpu().numpy(), None if tK is None else tK.cpu().numpy())


def test_kernel_test_block(dev):
    r = kernel_test_inputs()["rope"]
    B, S, D, hd = r["B"], r["S"], r["D"], r["hd"]
    gQ, gK = _run(dev, "rope_fwd", r["Q"], r["K"], B, S, D, hd)
    assert_close(gQ, orc.rope(r["Q"], B, S, D, hd, 1.0), "rope fwd Q")
    assert_close(gK, orc.rope(r["K"], B, S, D, hd, 1.0), "rope fwd K")
    gdQ, gdK = _run(dev, "rope_bwd", r["dQ"], r["dK"], B, S, D, hd)
    assert_close(gdQ, orc.rope(r["dQ"], B, S, D, hd, -1.0), "rope bwd dQ")
    assert_close(gdK, orc.rope(r["dK"], B, S, D, hd, -1.0), "rope bwd dK")


def test_alias_round_trip(dev):
    """kernel_test.cpp:494-497: rope_fwd(Q, Q) then rope_bwd(Q, Q) restores Q; a
    tensor passed as both Q and K is rotated twice, like the reference."""
    import torch
    import cxxgpt_attn as cx
    r = kernel_test_inputs()["rope"]
    B, S, D, hd = r["B"], r["S"], r["D"], r["hd"]
    t = _t(r["Q"], dev)
    cx.rope_fwd(t, t, B, S, D, hd)
    torch.cuda.synchronize()
    twice = orc.rope(orc.rope(r["Q"], B, S, D, hd, 1.0), B, S, D, hd, 1.0)
    assert_close(t.cpu().numpy(), twice, "rope fwd aliased")
    cx.rope_bwd(t, t, B, S, D, hd)
    torch.cuda.synchronize()
    assert_close(t.cpu().numpy(), r["Q"], "rope round trip")


@pytest.mark.parametrize("B,S,D,hd", [
    (8, 256, 768, 64),     # stage-1 heads at the C2 shape
    (8, 256, 768, 768),    # stage 2: one head over the whole feature width
    (2, 4096, 768, 64),    # C5 sequence length: angles up to 4095 rad
    (3, 7, 10, 2),         # ragged: rows not a multiple of 4, D/2 not of 64
    (1, 1, 8, 8),
    (5, 33, 96, 32),
])
def test_shapes(dev, B, S, D, hd):
    Q, K, dQ, dK = normal_inputs((B * S, D), (B * S, D), 17 * S + D + hd)
    gQ, gK = _run(dev, "rope_fwd", Q, K, B, S, D, hd)
    assert_close(gQ, orc.rope(Q, B, S, D, hd, 1.0), "fwd Q")
    assert_close(gK, orc.rope(K, B, S, D, hd, 1.0), "fwd K")
    gdQ, gdK = _run(dev, "rope_bwd", dQ, dK, B, S, D, hd)
    assert_close(gdQ, orc.rope(dQ, B, S, D, hd, -1.0), "bwd dQ")
    assert_close(gdK, orc.rope(dK, B, S, D, hd, -1.0), "bwd dK")


def test_single_tensor_and_unaligned(dev):
    import torch
    import cxxgpt_attn as cx
    B, S, D, hd = 2, 50, 64, 16
    Q, K, _, _ = normal_inputs((B * S, D), (B * S, D), 77)
    gQ, gK = _run(dev, "rope_fwd", Q, None, B, S, D, hd)
    assert gK is None
    assert_close(gQ, orc.rope(Q, B, S, D, hd, 1.0), "Q only")
    _, gK = _run(dev, "rope_bwd", None, K, B, S, D, hd)
    assert_close(gK, orc.rope(K, B, S, D, hd, -1.0), "K only")
    # rows starting 4 bytes past an 8-byte boundary take the scalar path
    buf = torch.zeros(B * S * D + 1, device=dev)
    buf[1:] = _t(Q, dev).reshape(-1)
    view = buf[1:]
    cx.rope_fwd(view, None, B, S, D, hd)
    torch.cuda.synchronize()
    assert_close(view.cpu().numpy().reshape(B * S, D), orc.rope(Q, B, S, D, hd, 1.0), "unaligned")


def test_error_paths(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(64, device=dev)
    P = cx._ptr
    st = cx._stream(None)
    for args, want in (((P(t), P(t), 1, 2, 32, 3), cx.CXG_ERR_DIMS),     # odd head_dim
                       ((P(t), P(t), 1, 2, 30, 8), cx.CXG_ERR_DIMS),     # D % head_dim
                       ((P(t), P(t), 1, 2, 32, 0), cx.CXG_ERR_DIMS),
                       ((P(t), P(t), 1, 2, 2048, 2048), cx.CXG_ERR_DIMS),  # head_dim > 1024
                       ((None, None, 1, 2, 32, 8), cx.CXG_ERR_NULL),
                       ((None, None, 0, 2, 32, 8), cx.CXG_OK)):          # empty: nothing to do
        assert cx.call_status("cxg_rope_fwd", *args, st) == want, args


# ---------------------------------------------------------------- RoPE fused into MHA
def _fused_refs(Q, K, V, B, S, H, Dh):
    D = H * Dh
    Qr = orc.rope(Q, B, S, D, Dh, 1.0)
    Kr = orc.rope(K, B, S, D, Dh, 1.0)
    O, lse = orc.mha_fwd(Qr, Kr, V, B, S, H, Dh, nthreads=8, want_lse=True)
    return Qr, Kr, O, lse


@pytest.mark.parametrize("B,S,H,Dh", [
    (8, 256, 12, 64),    # the C2 shape (stage-1 heads of two_stage_gpt.hpp)
    (1, 1000, 2, 64),    # positions up to 999
    (2, 65, 2, 16), (1, 100, 3, 32), (1, 130, 2, 128), (1, 70, 1, 256), (3, 7, 2, 8),
    # narrow heads (one workgroup per head): TwoStageGPT's stage 1, the
    # longest sequence at Dh <= 8, Dh not a multiple of 4, 16-column padding
    (32, 256, 64, 8), (1, 512, 2, 8), (2, 100, 3, 6), (2, 250, 2, 12),
])
def test_fused_mha_rope(dev, B, S, H, Dh):
    """cxg_mha_rope_fwd/bwd == rope_fwd; fused_mha_fwd; fused_mha_bwd; rope_bwd
    (two_stage_gpt.hpp:102-106, :171-174), on the C oracle."""
    import torch
    import cxxgpt_attn as cx
    D = H * Dh
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, D), 31 * S + Dh)
    Qr, Kr, rO, rlse = _fused_refs(Q, K, V, B, S, H, Dh)
    tQ, tK, tV, tdO = (_t(a, dev) for a in (Q, K, V, dO))
    tO = torch.full_like(tQ, float("nan"))
    tl = torch.full((B * H * S,), float("nan"), device=dev)
    cx.mha_rope_fwd(tQ, tK, tV, tO, B, S, H, Dh, lse=tl)
    torch.cuda.synchronize()
    O = tO.cpu().numpy()
    assert_close(O, rO, "fused fwd O")
    assert_close(tl.cpu().numpy(), rlse, "fused fwd lse")
    np.testing.assert_array_equal(tQ.cpu().numpy(), Q)   # inputs are left unrotated
    np.testing.assert_array_equal(tK.cpu().numpy(), K)
    gQ, gK, gV = orc.mha_bwd(Qr, Kr, V, O, dO, B, S, H, Dh, nthreads=8)
    rdQ = orc.rope(gQ, B, S, D, Dh, -1.0)
    rdK = orc.rope(gK, B, S, D, Dh, -1.0)
    for use_lse in (True, False):
        outs = [torch.full_like(tQ, float("nan")) for _ in range(3)]
        cx.mha_rope_bwd(tQ, tK, tV, tO, tdO, *outs, B, S, H, Dh, lse=tl if use_lse else None)
        torch.cuda.synchronize()
        dQ, dK, dV = (o.cpu().numpy() for o in outs)
        assert_close(dQ, rdQ, f"fused dQ lse={use_lse}")
        assert_close(dK, rdK, f"fused dK lse={use_lse}")
        assert_close(dV, gV, f"fused dV lse={use_lse}")


def test_fused_mha_rope_rejects_odd_head_dim(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(64, device=dev)
    P = cx._ptr
    st = cx.call_status("cxg_mha_rope_fwd", P(t), P(t), P(t), P(t), None, 1, 2, 1, 7,
                        cx._stream(None))
    assert st == cx.CXG_ERR_DIMS
