"""GPU parity tests of the fused linear-attention backward (cxg_kattn_bwd, cxg_lin_bwd).

The fused entry does what the reference's callers do with three calls
(two_stage_gpt.hpp:149-157: kernel_attn_bwd_step1 -> _bwd_dQ -> _bwd_dKdV;
linear_gpt.hpp:154-167: the linear_cuda counterparts).  Each test runs the
GPU forward (z_cache not written, as a caller of the fused backward would),
then the fused backward on the GPU's own O and den, and checks dQ, dK, dV
against the oracle chain step1 -> dQ -> dKdV on the same O and den
(kernel_test.cpp:276-292 feeds its backward oracle the kernel's O the same
way), and against the reference's literal backward oracle
(kernel_test.cpp:128-193) where the shape is small.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, kernel_test_inputs, normal_inputs

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _nan(dev, *shape):
    import torch
    return torch.full(shape, float("nan"), device=dev)


def _np(t):
    return t.cpu().numpy()


def _ctx(dev, B, S, D, E):
    """Context buffer for the fused pair (None when the shape does not use one)."""
    import torch
    import cxxgpt_attn as cx
    n = cx.lin_ctx_size(B, S, D, E)
    return torch.full((n // 4,), float("nan"), device=dev) if n else None


def fused_kattn(dev, Q, K, V, dO, B, S, D, E, use_ctx=False):
    """Forward (z_cache not written; with use_ctx the context-writing forward),
    then the one-call backward."""
    import torch
    import cxxgpt_attn as cx
    N = B * S
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    ctx = _ctx(dev, B, S, D, E) if use_ctx else None
    if use_ctx:
        cx.kattn_fwd_ctx(tQ, tK, tV, O, den, ctx, B, S, D, E)
    else:
        cx.kattn_fwd(tQ, tK, tV, O, den, None, None, None, B, S, D, E)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.kattn_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, D, E, ctx=ctx)
    torch.cuda.synchronize()
    return dict(O=_np(O), den=_np(den), dQ=_np(dQ), dK=_np(dK), dV=_np(dV))


def check_fused_kattn(dev, Q, K, V, dO, B, S, D, E, literal=False, tag="", use_ctx=False):
    g = fused_kattn(dev, Q, K, V, dO, B, S, D, E, use_ctx)
    tag = f"{tag}{' ctx' if use_ctx else ''}"
    rO, rden, rzc = orc.kattn_fwd(Q, K, V, B, S, D, E, nthreads=8)
    assert_close(g["O"], rO, f"{tag} O")
    assert_close(g["den"], rden, f"{tag} den")
    dnum, dden = orc.kattn_bwd_step1(g["O"], dO, g["den"], B * S, E)
    rdQ = orc.kattn_bwd_dQ(K, V, dnum, dden, rzc, Q, B, S, D, E, nthreads=8)
    rdK, rdV = orc.kattn_bwd_dKdV(Q, K, V, dnum, dden, B, S, D, E, nthreads=8)
    assert_close(g["dQ"], rdQ, f"{tag} dQ")
    assert_close(g["dK"], rdK, f"{tag} dK")
    assert_close(g["dV"], rdV, f"{tag} dV")
    if literal:
        lQ, lK, lV = orc.kattn_bwd_literal(Q, K, V, g["O"], dO, rden, B, S, D, E)
        assert_close(g["dQ"], lQ, f"{tag} dQ literal")
        assert_close(g["dK"], lK, f"{tag} dK literal")
        assert_close(g["dV"], lV, f"{tag} dV literal")


@pytest.mark.parametrize("block", ["stage2", "flat", "chunk"])
def test_kernel_test_blocks(dev, block):
    blk = kernel_test_inputs()[block]
    check_fused_kattn(dev, blk["Q"], blk["K"], blk["V"], blk["dO"], blk["B"], blk["S"],
                      blk["D"], blk["E"], literal=True, tag=block)


@pytest.mark.parametrize("use_ctx", [False, True])
@pytest.mark.parametrize("S", [256, 4096])
def test_config3_elu(dev, S, use_ctx):
    """C3 (B' = 96, D = E = 64): several segments per sequence at S4096."""
    B, D, E = 96, 64, 64
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 300 + S)
    check_fused_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"fused C3 S{S}", use_ctx=use_ctx)


@pytest.mark.parametrize("B,S,D,E", [
    (1, 1, 64, 64), (3, 15, 64, 64), (2, 17, 32, 48), (2, 100, 64, 64), (1, 1000, 64, 64),
    (5, 333, 16, 8), (2, 40, 64, 1), (300, 16, 64, 64), (1, 4099, 64, 64), (2, 3000, 60, 64),
    (1, 50, 128, 64), (2, 20, 64, 96),   # wider than 64: the split kernels inside the call
])
def test_ragged_shapes(dev, B, S, D, E):
    """Partial last chunks, one and many segments, narrow and non-multiple-of-4 widths;
    each with and without the forward's context."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 17 * S + D + E)
    for use_ctx in (False, True):
        check_fused_kattn(dev, Q, K, V, dO, B, S, D, E, literal=(S <= 40),
                          tag=f"B{B}S{S}D{D}E{E}", use_ctx=use_ctx)


def test_unaligned_rows(dev):
    """Tensors starting 4 bytes past a 16-byte boundary take the scalar-load variant."""
    import torch
    import cxxgpt_attn as cx
    B, S, D, E = 2, 300, 64, 64
    N = B * S
    Q, K, V, dO = normal_inputs((N, D), (N, E), 5)

    def off(a):
        buf = torch.zeros(a.size + 1, device=dev)
        buf[1:] = _t(a, dev).reshape(-1)
        return buf[1:]

    def offz(n):
        return torch.full((n + 1,), float("nan"), device=dev)[1:]

    tQ, tK, tV, tdO = off(Q), off(K), off(V), off(dO)
    O, den = offz(N * E), offz(N)
    cx.kattn_fwd(tQ, tK, tV, O, den, None, None, None, B, S, D, E)
    dQ, dK, dV = offz(N * D), offz(N * D), offz(N * E)
    cx.kattn_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, D, E)
    torch.cuda.synchronize()
    gO, gden = _np(O).reshape(N, E), _np(den)
    _, _, rzc = orc.kattn_fwd(Q, K, V, B, S, D, E, nthreads=8)
    dnum, dden = orc.kattn_bwd_step1(gO, dO, gden, N, E)
    assert_close(_np(dQ).reshape(N, D), orc.kattn_bwd_dQ(K, V, dnum, dden, rzc, Q, B, S, D, E),
                 "unaligned dQ")
    rdK, rdV = orc.kattn_bwd_dKdV(Q, K, V, dnum, dden, B, S, D, E)
    assert_close(_np(dK).reshape(N, D), rdK, "unaligned dK")
    assert_close(_np(dV).reshape(N, E), rdV, "unaligned dV")


def test_matches_split_chain(dev):
    """The fused backward and the three-call chain agree on the same forward outputs."""
    import torch
    import cxxgpt_attn as cx
    B, S, D, E = 8, 2048, 64, 64
    N = B * S
    Q, K, V, dO = normal_inputs((N, D), (N, E), 77)
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O, den, zc = _nan(dev, N, E), _nan(dev, N), _nan(dev, N, D)
    cx.kattn_fwd(tQ, tK, tV, O, den, zc, None, None, B, S, D, E)
    dnum, dden = _nan(dev, N, E), _nan(dev, N)
    cx.kattn_bwd_step1(O, tdO, den, dnum, dden, N, E)
    sQ, sK, sV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.kattn_bwd_dQ(tK, tV, dnum, dden, zc, tQ, sQ, None, B, S, D, E)
    cx.kattn_bwd_dKdV(tQ, tK, tV, dnum, dden, sK, sV, B, S, D, E)
    fQ, fK, fV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.kattn_bwd(tQ, tK, tV, O, tdO, den, fQ, fK, fV, B, S, D, E)
    torch.cuda.synchronize()
    assert_close(_np(fQ), _np(sQ), "dQ fused vs split")
    assert_close(_np(fK), _np(sK), "dK fused vs split")
    assert_close(_np(fV), _np(sV), "dV fused vs split")


def fused_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag, use_ctx=False):
    import torch
    import cxxgpt_attn as cx
    N = B * S
    tQ, tK, tV, tdO = _t(Qp, dev), _t(Kp, dev), _t(V, dev), _t(dO, dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    ctx = _ctx(dev, B, S, D, E) if use_ctx else None
    if use_ctx:
        cx.lin_fwd_ctx(tQ, tK, tV, O, den, ctx, B, S, D, E)
    else:
        cx.lin_fwd(tQ, tK, tV, O, den, None, None, None, B, S, D, E)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.lin_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, D, E, ctx=ctx)
    torch.cuda.synchronize()
    rO, rden, rzc, _, _ = orc.lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=8)
    assert_close(_np(O), rO, f"{tag} O")
    assert_close(_np(den), rden, f"{tag} den_cache")
    dnum, dden = orc.lcu_bwd_step1(_np(O), dO, _np(den), N, E)
    assert_close(_np(dQ), orc.lcu_bwd_dQ(Kp, V, dnum, dden, rzc, B, S, D, E, nthreads=8),
                 f"{tag} dQ_phi")
    rdK, rdV = orc.lcu_bwd_dKdV(Qp, Kp, V, dnum, dden, B, S, D, E, nthreads=8)
    assert_close(_np(dK), rdK, f"{tag} dK_phi")
    assert_close(_np(dV), rdV, f"{tag} dV")


@pytest.mark.parametrize("B,S,E", [(2, 64, 64), (3, 77, 48), (2, 500, 20)])
def test_linear_cuda_elu(dev, B, S, E):
    """LinearGPT's path with phi outside (D = next_pow2(E), zero-padded columns)."""
    D = 1 << (E - 1).bit_length()
    Xq, Xk, V, dO = normal_inputs((B * S, E), (B * S, E), 7 + E)
    Qp, Kp = orc.phi_elu_forward(Xq, D, E), orc.phi_elu_forward(Xk, D, E)
    fused_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag=f"lcu fused E{E}")
    fused_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag=f"lcu fused ctx E{E}", use_ctx=True)


@pytest.mark.parametrize("B,S,E", [(96, 256, 64), (96, 250, 64), (2, 64, 64), (3, 77, 48),
                                   (2, 500, 20), (1, 3000, 64), (2, 30, 100)])
@pytest.mark.parametrize("use_ctx", [False, True])
def test_linear_gpt_fused(dev, B, S, E, use_ctx):
    """cxg_lin_elu_fwd / _bwd against LinearGPT's own chain (linear_gpt.hpp:100-172):
    phi_elu_forward x2 -> causal_linear_attention_fwd; step1 -> dQ -> dKdV ->
    phi_elu_backward x2, with D = next_pow2(E) zero-padded feature columns.  B96 S250:
    four backward segments of four chunks a sequence, the last ending in a partial chunk."""
    import torch
    import cxxgpt_attn as cx
    D = 1 << (E - 1).bit_length()
    N = B * S
    Xq, Xk, V, dO = normal_inputs((N, E), (N, E), 5 * S + E)
    tq, tk, tv, tdo = _t(Xq, dev), _t(Xk, dev), _t(V, dev), _t(dO, dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    ctx = _ctx(dev, B, S, E, E) if use_ctx else None
    cx.lin_elu_fwd(tq, tk, tv, O, den, ctx, B, S, E)
    dXq, dXk, dV = _nan(dev, N, E), _nan(dev, N, E), _nan(dev, N, E)
    cx.lin_elu_bwd(tq, tk, tv, O, tdo, den, dXq, dXk, dV, B, S, E, ctx=ctx)
    torch.cuda.synchronize()
    Qp, Kp = orc.phi_elu_forward(Xq, D, E), orc.phi_elu_forward(Xk, D, E)
    rO, rden, rzc, _, _ = orc.lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=8)
    tag = f"lin_elu B{B}S{S}E{E}{' ctx' if use_ctx else ''}"
    assert_close(_np(O), rO, f"{tag} O")
    assert_close(_np(den), rden, f"{tag} den_cache")
    dnum, dden = orc.lcu_bwd_step1(_np(O), dO, _np(den), N, E)
    rdQp = orc.lcu_bwd_dQ(Kp, V, dnum, dden, rzc, B, S, D, E, nthreads=8)
    rdKp, rdV = orc.lcu_bwd_dKdV(Qp, Kp, V, dnum, dden, B, S, D, E, nthreads=8)
    assert_close(_np(dXq), orc.phi_elu_backward(rdQp, Xq, D, E), f"{tag} dXq")
    assert_close(_np(dXk), orc.phi_elu_backward(rdKp, Xk, D, E), f"{tag} dXk")
    assert_close(_np(dV), rdV, f"{tag} dV")


@pytest.mark.parametrize("B,S", [(96, 1024), (3, 100)])
def test_config4_hadamard_exp(dev, B, S):
    """C4: Hadamard+Exp features (phi outside), Q, K ~ N(0, 0.25), V, dO ~ N(0, 1)."""
    D = E = 64
    N = B * S
    Q, K, _, _ = normal_inputs((N, D), (N, E), 400, q_std=0.5)
    _, _, V, dO = normal_inputs((N, D), (N, E), 400)
    Qp, Kp = orc.phi_hexp_forward(Q, D, D), orc.phi_hexp_forward(K, D, D)
    fused_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag="C4 fused", use_ctx=True)


def test_error_paths(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(64, device=dev)
    P = cx._ptr
    st = cx._stream(None)
    p = [P(t)] * 10
    for fn in ("cxg_kattn_bwd", "cxg_lin_bwd"):
        assert cx.call_status(fn, *p, 1, 4, 0, 8, st) == cx.CXG_ERR_DIMS
        assert cx.call_status(fn, *p, 1, 4, 8, 0, st) == cx.CXG_ERR_DIMS
        assert cx.call_status(fn, *([None] + p[1:]), 1, 4, 8, 8, st) == cx.CXG_ERR_NULL
        assert cx.call_status(fn, *p[:5], None, *p[6:], 1, 4, 8, 8, st) == cx.CXG_ERR_NULL
        assert cx.call_status(fn, *([None] * 10), 0, 4, 8, 8, st) == cx.CXG_OK   # empty
    # the context: none for narrow heads on sequences short enough for the
    # quadratic form or for wide heads whose widths are not multiples of 16;
    # the chunked scan's records, or the block-score path's features and score
    # blocks, otherwise; a short buffer is refused
    assert cx.lin_ctx_size(2, 100, 64, 64) == 0
    assert cx.lin_ctx_size(2, 300, 100, 64) == 0
    for D in (64, 128):
        n = cx.lin_ctx_size(2, 300, D, 64)
        assert n > 0
        for fn in ("cxg_kattn_fwd_ctx", "cxg_lin_fwd_ctx"):
            assert cx.call_status(fn, *[P(t)] * 5, P(t), n - 4, 2, 300, D, 64, st) == \
                cx.CXG_ERR_WORKSPACE
            assert cx.call_status(fn, *[P(t)] * 5, None, n, 2, 300, D, 64, st) == \
                cx.CXG_ERR_NULL


# ---------------------------------------------------------------------------
# Inputs with a mean: |S| then grows like t, which is where recovering the
# prefix state by subtraction loses precision (test_lin_bwd_numerics.py models
# it on the CPU).  The GPU runs the whole batch; the oracle checks a sample of
# sequences (each sequence is independent).
# ---------------------------------------------------------------------------
def _seq_rows(a, seqs, S):
    return np.concatenate([a[s * S:(s + 1) * S] for s in seqs])


def _check_sampled(g, ref_fn, seqs, S, tag):
    ref = ref_fn(seqs)
    for name, r in ref.items():
        assert_close(_seq_rows(g[name], seqs, S), r, f"{tag} {name}")


@pytest.mark.parametrize("api", ["kattn", "lin", "lin_elu"])
@pytest.mark.parametrize("use_ctx", [False, True])
@pytest.mark.parametrize("B,v_mean,k_mean", [(96, 1.0, 0.0), (96, 3.0, 0.0), (96, 3.0, 1.0),
                                             (300, 3.0, 0.0)])
def test_mean_shifted_inputs(dev, api, use_ctx, B, v_mean, k_mean):
    """C3 S4096 shapes with V ~ N(mu, 1) (and K shifted): B' = 96 has several
    backward segments per sequence; B' = 300 fills every resident slot, so each
    sequence is one 4096-row segment."""
    import torch
    import cxxgpt_attn as cx
    S, D, E = 4096, 64, 64
    N = B * S
    Q, K, V, dO = normal_inputs((N, D), (N, E), 900 + int(10 * v_mean + k_mean),
                                k_mean=k_mean, v_mean=v_mean)
    if api == "lin":
        Q, K = orc.phi_elu_forward(Q, D, D), orc.phi_elu_forward(K, D, D)
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    ctx = _ctx(dev, B, S, D, E) if use_ctx else None
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    if api == "kattn":
        if use_ctx:
            cx.kattn_fwd_ctx(tQ, tK, tV, O, den, ctx, B, S, D, E)
        else:
            cx.kattn_fwd(tQ, tK, tV, O, den, None, None, None, B, S, D, E)
        cx.kattn_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, D, E, ctx=ctx)
    elif api == "lin":
        if use_ctx:
            cx.lin_fwd_ctx(tQ, tK, tV, O, den, ctx, B, S, D, E)
        else:
            cx.lin_fwd(tQ, tK, tV, O, den, None, None, None, B, S, D, E)
        cx.lin_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, D, E, ctx=ctx)
    else:
        cx.lin_elu_fwd(tQ, tK, tV, O, den, ctx, B, S, E)
        cx.lin_elu_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, E, ctx=ctx)
    torch.cuda.synchronize()
    g = dict(O=_np(O), den=_np(den), dQ=_np(dQ), dK=_np(dK), dV=_np(dV))
    del tQ, tK, tV, tdO, O, den, dQ, dK, dV, ctx
    seqs = [0, 1, B // 2, B - 1]
    n = len(seqs)

    def ref(sq):
        q, k, v, do = (_seq_rows(a, sq, S) for a in (Q, K, V, dO))
        gO, gden = _seq_rows(g["O"], sq, S), _seq_rows(g["den"], sq, S)
        if api == "kattn":
            rO, rden, rzc = orc.kattn_fwd(q, k, v, n, S, D, E, nthreads=8)
            dnum, dden = orc.kattn_bwd_step1(gO, do, gden, n * S, E)
            rdQ = orc.kattn_bwd_dQ(k, v, dnum, dden, rzc, q, n, S, D, E, nthreads=8)
            rdK, rdV = orc.kattn_bwd_dKdV(q, k, v, dnum, dden, n, S, D, E, nthreads=8)
        else:
            qp, kp = (q, k) if api == "lin" else (orc.phi_elu_forward(q, D, E),
                                                  orc.phi_elu_forward(k, D, E))
            rO, rden, rzc, _, _ = orc.lcu_fwd(qp, kp, v, n, S, D, E, nthreads=8)
            dnum, dden = orc.lcu_bwd_step1(gO, do, gden, n * S, E)
            rdQ = orc.lcu_bwd_dQ(kp, v, dnum, dden, rzc, n, S, D, E, nthreads=8)
            rdK, rdV = orc.lcu_bwd_dKdV(qp, kp, v, dnum, dden, n, S, D, E, nthreads=8)
            if api == "lin_elu":
                rdQ, rdK = orc.phi_elu_backward(rdQ, q, D, E), orc.phi_elu_backward(rdK, k, D, E)
        return dict(O=rO, den=rden, dQ=rdQ, dK=rdK, dV=rdV)

    _check_sampled(g, ref, seqs, S,
                   f"{api} B{B} muV{v_mean} muK{k_mean}{' ctx' if use_ctx else ''}")


def test_context_pairing_is_checked(dev):
    """The fused backward refuses a context the matching forward did not write:
    another shape, another API's forward (another feature map), or a pointer
    no forward wrote.  Nothing is launched for a refused call."""
    import torch
    import cxxgpt_attn as cx
    B, S, D, E = 2, 300, 64, 64
    N = B * S
    Q, K, V, dO = (_t(a, dev) for a in normal_inputs((N, D), (N, E), 41))
    O, den = _nan(dev, N, E), _nan(dev, N)
    n = cx.lin_ctx_size(B, S, D, E)
    ctx = torch.empty(n // 4, device=dev)
    cx.kattn_fwd_ctx(Q, K, V, O, den, ctx, B, S, D, E)
    P, st = cx._ptr, cx._stream(None)
    outs = [_nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)]
    args = [P(Q), P(K), P(V), P(O), P(dO), P(den)]
    # the matching call is accepted
    assert cx.call_status("cxg_kattn_bwd", *args, P(ctx), *map(P, outs), B, S, D, E, st) == cx.CXG_OK
    # another sequence length over the same rows
    assert cx.call_status("cxg_kattn_bwd", *args, P(ctx), *map(P, outs), 4, S // 2, D, E, st) \
        == cx.CXG_ERR_WORKSPACE
    # the phi-outside API's backward with the ELU+1 forward's context
    assert cx.call_status("cxg_lin_bwd", *args, P(ctx), *map(P, outs), B, S, D, E, st) \
        == cx.CXG_ERR_WORKSPACE
    # a buffer no forward wrote
    other = torch.empty(n // 4, device=dev)
    assert cx.call_status("cxg_kattn_bwd", *args, P(other), *map(P, outs), B, S, D, E, st) \
        == cx.CXG_ERR_WORKSPACE
    torch.cuda.synchronize()
