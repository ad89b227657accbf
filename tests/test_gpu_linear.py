"""GPU parity tests of the causal linear attention (both APIs) through the C ABI.

two_stage_cuda API (phi = ELU+1 fused): mirrors the reference kernel test's
stage-2 blocks (src/TwoStage/kernel_test.cpp:253-298, :335-374, :410-441) -
forward O/den against ref_kernel_attn_fwd, step1 against its closed form,
dQ/dK/dV against ref_kernel_attn_bwd - plus the benchmark configurations.

linear_cuda API (phi outside, den includes eps) and the Hadamard+Exp feature
map: each entry point against its oracle restatement on the GPU's own
upstream outputs, and the whole chain end to end.
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


def kattn_chain(dev, Q, K, V, dO, B, S, D, E):
    """two_stage chain: fwd -> step1 -> dQ -> dKdV on the GPU."""
    import torch
    import cxxgpt_attn as cx
    N = B * S
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O, den, zc = _nan(dev, N, E), _nan(dev, N), _nan(dev, N, D)
    Sb, zb = _nan(dev, B * E, D), _nan(dev, B, D)
    cx.kattn_fwd(tQ, tK, tV, O, den, zc, Sb, zb, B, S, D, E)
    dnum, dden = _nan(dev, N, E), _nan(dev, N)
    cx.kattn_bwd_step1(O, tdO, den, dnum, dden, N, E)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.kattn_bwd_dQ(tK, tV, dnum, dden, zc, tQ, dQ, Sb, B, S, D, E)
    cx.kattn_bwd_dKdV(tQ, tK, tV, dnum, dden, dK, dV, B, S, D, E)
    torch.cuda.synchronize()
    return dict(O=_np(O), den=_np(den), zc=_np(zc), dnum=_np(dnum), dden=_np(dden),
                dQ=_np(dQ), dK=_np(dK), dV=_np(dV))


def check_kattn(dev, Q, K, V, dO, B, S, D, E, literal=False, tag=""):
    g = kattn_chain(dev, Q, K, V, dO, B, S, D, E)
    rO, rden, rzc = orc.kattn_fwd(Q, K, V, B, S, D, E, nthreads=8)
    assert_close(g["O"], rO, f"{tag} O")
    assert_close(g["den"], rden, f"{tag} den")
    assert_close(g["zc"], rzc, f"{tag} z_cache")
    # backward stages on the GPU's own upstream outputs (kernel_test.cpp:276-292)
    rdnum, rdden = orc.kattn_bwd_step1(g["O"], dO, g["den"], B * S, E)
    assert_close(g["dnum"], rdnum, f"{tag} dnum")
    assert_close(g["dden"], rdden, f"{tag} dden")
    rdQ = orc.kattn_bwd_dQ(K, V, g["dnum"], g["dden"], g["zc"], Q, B, S, D, E, nthreads=8)
    assert_close(g["dQ"], rdQ, f"{tag} dQ")
    rdK, rdV = orc.kattn_bwd_dKdV(Q, K, V, g["dnum"], g["dden"], B, S, D, E, nthreads=8)
    assert_close(g["dK"], rdK, f"{tag} dK")
    assert_close(g["dV"], rdV, f"{tag} dV")
    if literal:
        # the reference's own backward oracle (kernel_test.cpp:128-193), end to end
        lQ, lK, lV = orc.kattn_bwd_literal(Q, K, V, g["O"], dO, rden, B, S, D, E)
        assert_close(g["dQ"], lQ, f"{tag} dQ literal")
        assert_close(g["dK"], lK, f"{tag} dK literal")
        assert_close(g["dV"], lV, f"{tag} dV literal")
    return g


@pytest.mark.parametrize("block", ["stage2", "flat", "chunk"])
def test_kernel_test_blocks(dev, block):
    blk = kernel_test_inputs()[block]
    check_kattn(dev, blk["Q"], blk["K"], blk["V"], blk["dO"], blk["B"], blk["S"], blk["D"],
                blk["E"], literal=True, tag=block)


@pytest.mark.parametrize("S", [256, 4096])
def test_config3_elu(dev, S):
    """C3: ELU+1, B' = B*H = 96 sequences, D = E = 64, N(0,1) inputs."""
    B, D, E = 96, 64, 64
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 300 + S)
    check_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"C3 S{S}")


@pytest.mark.parametrize("B,S,D,E", [
    (1, 1, 64, 64), (3, 15, 64, 64), (2, 17, 32, 48), (2, 100, 64, 64), (1, 1000, 64, 64),
    (5, 333, 16, 8), (2, 40, 64, 1), (300, 16, 64, 64), (1, 50, 128, 64), (2, 20, 64, 96),
    (24, 2040, 64, 64), (7, 3001, 64, 64), (96, 632, 64, 64),
])
def test_ragged_shapes(dev, B, S, D, E):
    """Partial chunks, single and multi-segment plans, narrow D/E (the chunked scan) and
    widths in (64, 512] (the quadratic form); widths above 512 are in test_gpu_lingeneric.
    The last three: multi-chunk segments whose sequence ends in a partial chunk.  At
    B96 S632 (8 segments of 5 chunks on 256 compute units) the last segment holds 4.5
    chunks, so the second half of its segment sum ends in a partial chunk that must keep
    its row masks (its record feeds every earlier segment's dK/dV)."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 13 * S + D + E)
    check_kattn(dev, Q, K, V, dO, B, S, D, E, literal=(S <= 40), tag=f"B{B}S{S}D{D}E{E}")


def test_state_outputs(dev):
    """linear_cuda fwd writes the final state [d][e] into S_buf and z into z_buf."""
    import torch
    import cxxgpt_attn as cx
    B, S, D, E = 3, 150, 64, 48
    Q, K, V, _ = normal_inputs((B * S, D), (B * S, E), 99)
    Qp, Kp = orc.phi_elu_forward(Q[:, :E], D, E), orc.phi_elu_forward(K[:, :E], D, E)
    N = B * S
    O, den, zc, Sb, zb = _nan(dev, N, E), _nan(dev, N), _nan(dev, N, D), _nan(dev, B * D, E), \
        _nan(dev, B, D)
    cx.lin_fwd(_t(Qp, dev), _t(Kp, dev), _t(V, dev), O, den, zc, Sb, zb, B, S, D, E)
    torch.cuda.synchronize()
    rO, rden, rzc, rSb, rzb = orc.lcu_fwd(Qp, Kp, V, B, S, D, E)
    assert_close(_np(O), rO, "O")
    assert_close(_np(den), rden, "den_cache")
    assert_close(_np(zc), rzc, "z_cache")
    assert_close(_np(Sb), rSb, "S_buf")
    assert_close(_np(zb), rzb, "z_buf")


def lcu_chain(dev, Qp, Kp, V, dO, B, S, D, E):
    import torch
    import cxxgpt_attn as cx
    N = B * S
    tQ, tK, tV, tdO = _t(Qp, dev), _t(Kp, dev), _t(V, dev), _t(dO, dev)
    O, den, zc = _nan(dev, N, E), _nan(dev, N), _nan(dev, N, D)
    cx.lin_fwd(tQ, tK, tV, O, den, zc, None, None, B, S, D, E)
    dnum, dden = _nan(dev, N, E), _nan(dev, N)
    cx.lin_bwd_step1(O, tdO, den, dnum, dden, N, E)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.lin_bwd_dQ(tK, tV, dnum, dden, zc, dQ, None, B, S, D, E)
    cx.lin_bwd_dKdV(tQ, tK, tV, dnum, dden, dK, dV, B, S, D, E)
    torch.cuda.synchronize()
    return dict(O=_np(O), den=_np(den), zc=_np(zc), dnum=_np(dnum), dden=_np(dden), dQ=_np(dQ),
                dK=_np(dK), dV=_np(dV))


def check_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag):
    g = lcu_chain(dev, Qp, Kp, V, dO, B, S, D, E)
    rO, rden, rzc, _, _ = orc.lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=8)
    assert_close(g["O"], rO, f"{tag} O")
    assert_close(g["den"], rden, f"{tag} den_cache")
    assert_close(g["zc"], rzc, f"{tag} z_cache")
    rdnum, rdden = orc.lcu_bwd_step1(g["O"], dO, g["den"], B * S, E)
    assert_close(g["dnum"], rdnum, f"{tag} dnum")
    assert_close(g["dden"], rdden, f"{tag} dden")
    rdQ = orc.lcu_bwd_dQ(Kp, V, g["dnum"], g["dden"], g["zc"], B, S, D, E, nthreads=8)
    assert_close(g["dQ"], rdQ, f"{tag} dQ_phi")
    rdK, rdV = orc.lcu_bwd_dKdV(Qp, Kp, V, g["dnum"], g["dden"], B, S, D, E, nthreads=8)
    assert_close(g["dK"], rdK, f"{tag} dK_phi")
    assert_close(g["dV"], rdV, f"{tag} dV")
    return g


@pytest.mark.parametrize("B,S,E", [(2, 64, 64), (3, 77, 48), (2, 40, 100)])
def test_linear_cuda_elu_chain(dev, B, S, E):
    """LinearGPT's path: phi_elu_forward -> linear attention -> phi_elu_backward,
    with D = next_pow2(E) zero-padded columns (linear_gpt.hpp:33-45, :100-172)."""
    import torch
    import cxxgpt_attn as cx
    D = 1 << (E - 1).bit_length()
    Xq, Xk, V, dO = normal_inputs((B * S, E), (B * S, E), 7 + E)
    N = B * S
    tq, tk = _t(Xq, dev), _t(Xk, dev)
    pq, pk = _nan(dev, N, D), _nan(dev, N, D)
    cx.phi_elu_fwd(tq, pq, N, D, E)
    cx.phi_elu_fwd(tk, pk, N, D, E)
    torch.cuda.synchronize()
    Qp, Kp = _np(pq), _np(pk)
    assert_close(Qp, orc.phi_elu_forward(Xq, D, E), "phi_elu(Q)")
    assert_close(Kp, orc.phi_elu_forward(Xk, D, E), "phi_elu(K)")
    g = check_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag=f"lcu E{E}")
    dx = _nan(dev, N, E)
    cx.phi_elu_bwd(_t(g["dQ"], dev), tq, dx, N, D, E)
    torch.cuda.synchronize()
    assert_close(_np(dx), orc.phi_elu_backward(g["dQ"], Xq, D, E), "phi_elu_backward")


@pytest.mark.parametrize("B,S", [(96, 1024), (3, 100)])
def test_config4_hadamard_exp(dev, B, S):
    """C4: Hadamard+Exp feature map, phi(x) = exp(H_64 x / 8), Q,K ~ N(0, 0.25),
    V, dO ~ N(0, 1), through the linear_cuda API."""
    import torch
    import cxxgpt_attn as cx
    D = E = 64
    N = B * S
    Q, K, _, _ = normal_inputs((N, D), (N, E), 400, q_std=0.5)
    _, _, V, dO = normal_inputs((N, D), (N, E), 400)
    tq, tk = _t(Q, dev), _t(K, dev)
    pq, pk = _nan(dev, N, D), _nan(dev, N, D)
    cx.phi_hexp_fwd(tq, pq, N, D, D)
    cx.phi_hexp_fwd(tk, pk, N, D, D)
    torch.cuda.synchronize()
    Qp, Kp = _np(pq), _np(pk)
    assert_close(Qp, orc.phi_hexp_forward(Q, D, D), "phi_hexp(Q)")
    assert_close(Kp, orc.phi_hexp_forward(K, D, D), "phi_hexp(K)")
    g = check_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag="C4")
    dq, dk = _nan(dev, N, D), _nan(dev, N, D)
    cx.phi_hexp_bwd(_t(g["dQ"], dev), tq, dq, N, D, D)
    cx.phi_hexp_bwd(_t(g["dK"], dev), tk, dk, N, D, D)
    torch.cuda.synchronize()
    assert_close(_np(dq), orc.phi_hexp_backward(g["dQ"], Q, D, D), "phi_hexp_backward(Q)")
    assert_close(_np(dk), orc.phi_hexp_backward(g["dK"], K, D, D), "phi_hexp_backward(K)")


def test_error_paths(dev):
    import torch
    import cxxgpt_attn as cx
    x = torch.zeros(256, device=dev)
    p = cx._ptr(x)
    st = cx._stream(None)
    assert cx.call_status("cxg_kattn_fwd", p, p, p, p, p, p, None, None, 1, 4, 0, 4, st) == \
        cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_kattn_fwd", p, p, p, None, p, p, None, None, 1, 4, 4, 4, st) == \
        cx.CXG_ERR_NULL
    assert cx.call_status("cxg_kattn_fwd", p, p, p, p, p, p, None, None, 0, 4, 4, 4, st) == \
        cx.CXG_OK
    assert cx.call_status("cxg_phi_hexp_fwd", p, p, 1, 64, 32, st) == cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_phi_elu_fwd", p, p, 1, 4, 8, st) == cx.CXG_ERR_DIMS
    torch.cuda.synchronize()


@pytest.mark.parametrize("N,D,E", [(1001, 64, 64), (77, 128, 128), (130, 128, 64), (5, 192, 128)])
def test_hexp_vector_and_scalar_paths(dev, N, D, E):
    """The 16-byte-load feature-map kernels (aligned rows, D % 64 == 0) against
    the one-element-per-lane kernels (taken by an unaligned view), bit for
    bit, and both against the oracle; columns E..D of phi are zero."""
    import torch
    import cxxgpt_attn as cx
    x, _, _, _ = normal_inputs((N, E), (N, E), 31 + N, q_std=0.5)
    g = orc.normal(7 + N, N * D).reshape(N, D)

    def view(a, off):
        buf = torch.zeros(a.size + off, device=dev)
        buf[off:] = _t(a, dev).reshape(-1)
        return buf[off:]

    out = {}
    for off in (0, 1):
        tx, tg = view(x, off), view(g, off)
        phi = torch.full((N * D + off,), float("nan"), device=dev)[off:]
        dx = torch.full((N * E + off,), float("nan"), device=dev)[off:]
        cx.phi_hexp_fwd(tx, phi, N, D, E)
        cx.phi_hexp_bwd(tg, tx, dx, N, D, E)
        torch.cuda.synchronize()
        out[off] = (_np(phi).reshape(N, D), _np(dx).reshape(N, E))
    assert np.array_equal(out[0][0], out[1][0]), "phi: vector and scalar kernels differ"
    assert np.array_equal(out[0][1], out[1][1]), "dx: vector and scalar kernels differ"
    assert_close(out[0][0], orc.phi_hexp_forward(x, D, E), f"phi_hexp N{N}D{D}E{E}")
    assert np.all(out[0][0][:, (E // 64) * 64:] == 0.0)
    assert_close(out[0][1], orc.phi_hexp_backward(g, x, D, E), f"phi_hexp_bwd N{N}D{D}E{E}")


def test_long_sequence_row_offsets(dev):
    """One sequence of 2^23 + 40 rows, past where 32-bit byte offsets from the
    sequence's first 256-byte row would wrap: the chunked kernels address
    each chunk from its own first row.  With every Q row equal and every K
    row equal, c = phi(q).phi(k) factors out of every sum, which gives closed
    forms (float64, on the device) for the whole chain:
      O_t = c cumV_t / (c (t+1) + 1e-8), den_t = c (t+1), z_t = (t+1) phi(k),
      dQ_t = phi(k) (cumV_t . dnum_t + (t+1) dden_t) phi'(q),
      dK_s = phi(q) (A_s . V_s + B_s) phi'(k), dV_s = c A_s,
    with cumV the prefix sums of V and A, B the suffix sums of the step-1
    outputs dnum, dden (the GPU's own, as the chain passes them on)."""
    import torch
    import cxxgpt_attn as cx
    S, D, E = (1 << 23) + 40, 64, 64
    gen = torch.Generator().manual_seed(23)
    q = (0.5 * torch.randn(D, generator=gen)).to(dev)
    k = (0.5 * torch.randn(D, generator=gen)).to(dev)
    Q, K = q.expand(S, D).contiguous(), k.expand(S, D).contiguous()
    t = torch.arange(S, device=dev, dtype=torch.float32)[:, None]
    col = torch.arange(E, device=dev, dtype=torch.float32)[None, :]
    V = 1.0 + 0.5 * torch.sin(t * 1e-3 + col)
    dO = torch.cos(t * 7e-4 + 0.3 * col)
    del t, col
    O, den, zc = _nan(dev, S, E), _nan(dev, S), _nan(dev, S, D)
    Sb, zb = _nan(dev, E, D), _nan(dev, 1, D)
    cx.kattn_fwd(Q, K, V, O, den, zc, Sb, zb, 1, S, D, E)
    dnum, dden = _nan(dev, S, E), _nan(dev, S)
    cx.kattn_bwd_step1(O, dO, den, dnum, dden, S, E)
    dQ, dK, dV = _nan(dev, S, D), _nan(dev, S, D), _nan(dev, S, E)
    cx.kattn_bwd_dQ(K, V, dnum, dden, zc, Q, dQ, Sb, 1, S, D, E)
    cx.kattn_bwd_dKdV(Q, K, V, dnum, dden, dK, dV, 1, S, D, E)
    torch.cuda.synchronize()

    def phi(x):
        return torch.where(x > 0, x + 1.0, torch.exp(x))

    def dphi(x):
        return torch.where(x > 0, torch.ones_like(x), torch.exp(x))

    def check(got, ref, name):
        assert torch.isfinite(got).all(), f"{name}: non-finite values"
        err = (got.double() - ref).abs()
        excess = err - (1e-5 + 1e-4 * ref.abs())
        worst = int(torch.argmax(excess.reshape(-1)))
        assert float(excess.reshape(-1)[worst]) <= 0.0, (
            f"{name}: {int((excess > 0).sum())} elements out of tolerance; worst flat index "
            f"{worst}: got {float(got.reshape(-1)[worst])!r} ref {float(ref.reshape(-1)[worst])!r}")

    pq, pk = phi(q.double()), phi(k.double())
    c = float((pq * pk).sum())
    n = torch.arange(1, S + 1, device=dev, dtype=torch.float64)[:, None]
    cum = torch.cumsum(V.double(), 0)
    check(O, cum * c / (c * n + 1e-8), "O")
    check(den, c * n[:, 0], "den")
    check(zc, n * pk[None, :], "z_cache")
    dn, dd = dnum.double(), dden.double()[:, None]
    check(dQ, ((cum * dn).sum(1, keepdim=True) + n * dd) * pk[None, :] * dphi(q.double())[None, :],
          "dQ")
    del cum
    A = torch.flip(torch.cumsum(torch.flip(dn, [0]), 0), [0])
    Bs = torch.flip(torch.cumsum(torch.flip(dd, [0]), 0), [0])
    check(dV, c * A, "dV")
    check(dK, ((A * V.double()).sum(1, keepdim=True) + Bs) * pq[None, :] * dphi(k.double())[None, :],
          "dK")
