"""GPU parity tests of the Hadamard+Exp attention block (cxg_lin_hexp_fwd / _bwd).

The entry points take the raw projections Xq, Xk and apply the feature map
phi(x) = exp(H x / 8) (H the 64x64 Sylvester Hadamard matrix) inside the
fused pair's kernels.  The benchmark configuration (96 sequences, S = 1024,
D = E = 64) runs the map as separate passes around the linear_cuda calls
(linear_cuda_kernels.cu:10-298);
the oracle here is that chain: phi_hexp_forward x2 -> lcu_fwd; lcu_bwd_step1
-> lcu_bwd_dQ -> lcu_bwd_dKdV -> phi_hexp_backward x2.  Each case also runs
the library's own unfused path (cxg_phi_hexp_fwd, cxg_lin_fwd(_ctx),
cxg_lin_bwd, cxg_phi_hexp_bwd) on the same inputs: the fused kernels form the
same feature values with the same operations, so the two agree to a few
units in the last place.
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


def _ctx(dev, B, S):
    import torch
    import cxxgpt_attn as cx
    n = cx.lin_ctx_size(B, S, 64, 64)
    return torch.full((max(1, n // 4),), float("nan"), device=dev) if n else None


def fused(dev, Xq, Xk, V, dO, B, S, use_ctx):
    import torch
    import cxxgpt_attn as cx
    N, E = B * S, 64
    tq, tk, tv, tdo = _t(Xq, dev), _t(Xk, dev), _t(V, dev), _t(dO, dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    ctx = _ctx(dev, B, S) if use_ctx else None
    cx.lin_hexp_fwd(tq, tk, tv, O, den, ctx, B, S, E)
    dXq, dXk, dV = _nan(dev, N, E), _nan(dev, N, E), _nan(dev, N, E)
    cx.lin_hexp_bwd(tq, tk, tv, O, tdo, den, dXq, dXk, dV, B, S, E, ctx=ctx)
    torch.cuda.synchronize()
    return dict(O=_np(O), den=_np(den), dXq=_np(dXq), dXk=_np(dXk), dV=_np(dV))


def unfused(dev, Xq, Xk, V, dO, B, S, use_ctx):
    """The same step through the library's separate feature-map passes."""
    import torch
    import cxxgpt_attn as cx
    N, D = B * S, 64
    tq, tk, tv, tdo = _t(Xq, dev), _t(Xk, dev), _t(V, dev), _t(dO, dev)
    pq, pk = _nan(dev, N, D), _nan(dev, N, D)
    cx.phi_hexp_fwd(tq, pq, N, D, D)
    cx.phi_hexp_fwd(tk, pk, N, D, D)
    O, den = _nan(dev, N, D), _nan(dev, N)
    ctx = _ctx(dev, B, S) if use_ctx else None
    if ctx is not None:
        cx.lin_fwd_ctx(pq, pk, tv, O, den, ctx, B, S, D, D)
    else:
        cx.lin_fwd(pq, pk, tv, O, den, None, None, None, B, S, D, D)
    dpq, dpk, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, D)
    cx.lin_bwd(pq, pk, tv, O, tdo, den, dpq, dpk, dV, B, S, D, D, ctx=ctx)
    dXq, dXk = _nan(dev, N, D), _nan(dev, N, D)
    cx.phi_hexp_bwd(dpq, tq, dXq, N, D, D)
    cx.phi_hexp_bwd(dpk, tk, dXk, N, D, D)
    torch.cuda.synchronize()
    return dict(O=_np(O), den=_np(den), dXq=_np(dXq), dXk=_np(dXk), dV=_np(dV))


def check(dev, B, S, seed, use_ctx):
    D = E = 64
    N = B * S
    Xq, Xk, _, _ = normal_inputs((N, D), (N, E), seed, q_std=0.5)
    _, _, V, dO = normal_inputs((N, D), (N, E), seed)
    g = fused(dev, Xq, Xk, V, dO, B, S, use_ctx)
    tag = f"hexp B{B}S{S}{' ctx' if use_ctx else ''}"
    Qp, Kp = orc.phi_hexp_forward(Xq, D, E), orc.phi_hexp_forward(Xk, D, E)
    rO, rden, rzc, _, _ = orc.lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=8)
    assert_close(g["O"], rO, f"{tag} O")
    assert_close(g["den"], rden, f"{tag} den_cache")
    dnum, dden = orc.lcu_bwd_step1(g["O"], dO, g["den"], N, E)
    rdQp = orc.lcu_bwd_dQ(Kp, V, dnum, dden, rzc, B, S, D, E, nthreads=8)
    rdKp, rdV = orc.lcu_bwd_dKdV(Qp, Kp, V, dnum, dden, B, S, D, E, nthreads=8)
    assert_close(g["dXq"], orc.phi_hexp_backward(rdQp, Xq, D, E), f"{tag} dXq")
    assert_close(g["dXk"], orc.phi_hexp_backward(rdKp, Xk, D, E), f"{tag} dXk")
    assert_close(g["dV"], rdV, f"{tag} dV")
    u = unfused(dev, Xq, Xk, V, dO, B, S, use_ctx)
    for k in ("O", "den", "dXq", "dXk", "dV"):
        assert_close(g[k], u[k], f"{tag} {k} fused vs unfused", atol=1e-6, rtol=2e-6)


@pytest.mark.parametrize("use_ctx", [False, True])
@pytest.mark.parametrize("B,S", [(96, 1024), (2, 4099), (5, 333), (2, 129), (4, 256)])
def test_hexp_block(dev, B, S, use_ctx):
    """C4 (B' = 96, S1024: several segments per sequence), a long ragged
    sequence, and short ones that take the one-launch forward records."""
    check(dev, B, S, 500 + S + B, use_ctx)


@pytest.mark.parametrize("B,S", [(3, 100), (1, 1), (2, 128)])
def test_hexp_short_sequences(dev, B, S):
    """S <= 128: the feature maps through scratch around the quadratic-form kernels."""
    check(dev, B, S, 600 + S, use_ctx=False)
    check(dev, B, S, 600 + S, use_ctx=True)


def test_hexp_context_pairing(dev):
    """A context written by another feature map's forward is refused; the
    matching one is accepted."""
    import torch
    import cxxgpt_attn as cx
    B, S, E = 2, 512, 64
    N = B * S
    X = _t(np.zeros((N, E), np.float32), dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    ctx = _ctx(dev, B, S)
    nbytes = ctx.numel() * 4
    P, st = cx._ptr, cx._stream(None)
    outs = [_nan(dev, N, E), _nan(dev, N, E), _nan(dev, N, E)]
    bwd = [P(X), P(X), P(X), P(O), P(X), P(den), P(ctx), *map(P, outs), B, S, E, st]
    cx.lin_elu_fwd(X, X, X, O, den, ctx, B, S, E)
    assert cx.call_status("cxg_lin_hexp_bwd", *bwd) == cx.CXG_ERR_WORKSPACE
    assert cx.call_status("cxg_lin_hexp_fwd", P(X), P(X), P(X), P(O), P(den), P(ctx), nbytes,
                          B, S, E, st) == cx.CXG_OK
    assert cx.call_status("cxg_lin_hexp_bwd", *bwd) == cx.CXG_OK
    torch.cuda.synchronize()


def test_hexp_error_paths(dev):
    import torch
    import cxxgpt_attn as cx
    B, S = 2, 300
    N = B * S
    x = torch.zeros(N * 96 + 4, device=dev)
    O, den = _nan(dev, N, 64), _nan(dev, N)
    P, st = cx._ptr, cx._stream(None)
    # E must be 64
    assert cx.call_status("cxg_lin_hexp_fwd", P(x), P(x), P(x), P(O), P(den), None, 0, B, S, 96,
                          st) == cx.CXG_ERR_DIMS
    # rows must be 16-byte aligned
    assert cx.call_status("cxg_lin_hexp_fwd", P(x[1:]), P(x), P(x), P(O), P(den), None, 0, B, S,
                          64, st) == cx.CXG_ERR_ALIGN
    assert cx.call_status("cxg_lin_hexp_fwd", None, P(x), P(x), P(O), P(den), None, 0, B, S, 64,
                          st) == cx.CXG_ERR_NULL
    torch.cuda.synchronize()
