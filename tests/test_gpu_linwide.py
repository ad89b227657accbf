"""GPU parity tests of linear attention with wide heads (64 < D, E <= 512).

These widths take the quadratic-form kernels (linwide.hip).  The reference's
callers run them at D = E = n_embd = 512, S = 256: TwoStageGPT's stage 2
through the two_stage API with B = 32 (two_stage_train.cpp:168-170, 193;
two_stage_gpt.hpp:115-157) and LinearGPT through the linear_cuda API with
phi_elu outside and B = 8 (linear_train.cpp:168-191; linear_gpt.hpp:100-172).
Every output is checked against the oracle's recurrent restatement
(kernel_test.cpp:96-193, linear_cuda_kernels.cu math), which sums in the
other order, and the small shapes against the reference's literal quadratic
backward oracle as well.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, normal_inputs
from test_gpu_linear import _nan, _np, _t, check_kattn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,S,D,E", [
    (2, 256, 512, 512),   # the stage-2 shape, two sequences
    (3, 77, 256, 256), (2, 300, 128, 128), (1, 33, 100, 200), (2, 16, 512, 300),
    (4, 1, 96, 96), (1, 700, 192, 192), (2, 40, 65, 64), (1, 19, 512, 8),
    # batches of 8 and more that are not multiples of 8 (sequences dealt to
    # XCDs unevenly by the block-score kernels), one and two row blocks
    (9, 48, 128, 128), (20, 17, 96, 64), (11, 16, 64, 96),
    # a batch large enough for one wave per product unit, an odd block count
    (48, 240, 256, 256),
])
def test_two_stage_chain_wide(dev, B, S, D, E):
    """fwd (O, den, z_cache) -> step1 -> dQ -> dKdV through the two_stage API."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 7 * S + D + 3 * E)
    check_kattn(dev, Q, K, V, dO, B, S, D, E, literal=(S <= 40 and D * E <= 65536),
                tag=f"wide B{B}S{S}D{D}E{E}")


@pytest.mark.parametrize("B,S,D", [
    (32, 256, 512),   # the training shape
    (70, 240, 512),   # one wave per product unit in every pass, an odd block count
])
def test_two_stage_reference_shape(dev, B, S, D):
    """TwoStageGPT stage 2 at its training shape, B = 32, S = 256, D = E = 512,
    and at a batch large enough that the block-score forward, like the
    backward, runs one wave per product unit (the oracle checks a sample of
    sequences; each is independent)."""
    import torch
    import cxxgpt_attn as cx
    N = B * S
    Q, K, V, dO = normal_inputs((N, D), (N, D), 4242)
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O, den, zc = _nan(dev, N, D), _nan(dev, N), _nan(dev, N, D)
    Sb, zb = _nan(dev, B * D, D), _nan(dev, B, D)
    cx.kattn_fwd(tQ, tK, tV, O, den, zc, Sb, zb, B, S, D, D)
    dnum, dden = _nan(dev, N, D), _nan(dev, N)
    cx.kattn_bwd_step1(O, tdO, den, dnum, dden, N, D)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, D)
    cx.kattn_bwd_dQ(tK, tV, dnum, dden, zc, tQ, dQ, Sb, B, S, D, D)
    cx.kattn_bwd_dKdV(tQ, tK, tV, dnum, dden, dK, dV, B, S, D, D)
    fQ, fK, fV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, D)
    cx.kattn_bwd(tQ, tK, tV, O, tdO, den, fQ, fK, fV, B, S, D, D)
    torch.cuda.synchronize()
    g = {k: _np(v) for k, v in dict(O=O, den=den, zc=zc, dnum=dnum, dden=dden, dQ=dQ, dK=dK,
                                    dV=dV, fQ=fQ, fK=fK, fV=fV).items()}
    for s in (0, 17, B - 1):
        sl = slice(s * S, (s + 1) * S)
        q, k, v = Q[sl], K[sl], V[sl]
        rO, rden, rzc = orc.kattn_fwd(q, k, v, 1, S, D, D)
        assert_close(g["O"][sl], rO, f"seq{s} O")
        assert_close(g["den"][sl], rden, f"seq{s} den")
        assert_close(g["zc"][sl], rzc, f"seq{s} z_cache")
        rdQ = orc.kattn_bwd_dQ(k, v, g["dnum"][sl], g["dden"][sl], g["zc"][sl], q, 1, S, D, D)
        rdK, rdV = orc.kattn_bwd_dKdV(q, k, v, g["dnum"][sl], g["dden"][sl], 1, S, D, D)
        for name, ref in (("dQ", rdQ), ("dK", rdK), ("dV", rdV)):
            assert_close(g[name][sl], ref, f"seq{s} {name}")
            assert_close(g["f" + name[1]][sl], ref, f"seq{s} fused {name}")


def _state_bound_check(got, phiK, V, name, transpose=False):
    """S_buf against the float64 sum over s of phi(K_s) V_s^T.  S_buf is the
    reference's scratch state, a sum of S products of both signs that can
    cancel to near zero, so besides the parity bar the bound admits the float32
    summation error of the kernel's order (16-row MFMA partials added in
    sequence: depth S/16 + 16), gamma * sum_s |phi(K_s)| |V_s|^T.  A wrong layout
    or index is off by O(1) and fails it."""
    ref = phiK.T.astype(np.float64) @ V.astype(np.float64)
    absum = np.abs(phiK.astype(np.float64)).T @ np.abs(V.astype(np.float64))
    depth = phiK.shape[0] / 16 + 16
    if transpose:
        ref, absum = ref.T, absum.T
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - ref)
    bound = 1e-5 + 1e-4 * np.abs(ref) + depth * 2.0 ** -24 * absum
    assert np.all(err <= bound), f"{name}: worst err {err.max():.3e}, {int((err > bound).sum())} over"


def test_state_outputs_wide(dev):
    """The forwards leave each sequence's final state in S_buf ([d][e] for
    linear_cuda, [e][d] for two_stage) and its z in z_buf."""
    import torch
    import cxxgpt_attn as cx
    B, S, D, E = 3, 150, 256, 160
    N = B * S
    Q, K, V, _ = normal_inputs((N, D), (N, E), 98)
    Qp, Kp = orc.phi_elu_forward(Q, D, D), orc.phi_elu_forward(K, D, D)
    O, den, zc, Sb, zb = _nan(dev, N, E), _nan(dev, N), _nan(dev, N, D), _nan(dev, B * D, E), \
        _nan(dev, B, D)
    cx.lin_fwd(_t(Qp, dev), _t(Kp, dev), _t(V, dev), O, den, zc, Sb, zb, B, S, D, E)
    O2, den2, zc2, Sb2, zb2 = _nan(dev, N, E), _nan(dev, N), _nan(dev, N, D), \
        _nan(dev, B * E, D), _nan(dev, B, D)
    cx.kattn_fwd(_t(Q, dev), _t(K, dev), _t(V, dev), O2, den2, zc2, Sb2, zb2, B, S, D, E)
    torch.cuda.synchronize()
    rO, rden, rzc, rSb, rzb = orc.lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=8)
    assert_close(_np(O), rO, "lcu O")
    assert_close(_np(den), rden, "lcu den_cache")
    assert_close(_np(zc), rzc, "lcu z_cache")
    assert_close(_np(zb), rzb, "lcu z_buf")
    # two_stage: the same state transposed ([e][d]) from phi = ELU+1 fused
    pK = np.where(K > 0, K + 1.0, np.exp(K.astype(np.float64)))
    for b in range(B):
        sl = slice(b * S, (b + 1) * S)
        _state_bound_check(_np(Sb)[b * D:(b + 1) * D], Kp[sl],
                           V[sl], f"lcu S_buf [d][e] seq{b}")
        _state_bound_check(_np(Sb2)[b * E:(b + 1) * E], pK[sl], V[sl],
                           f"two_stage S_buf [e][d] seq{b}", transpose=True)
        assert_close(_np(zb2)[b], pK[sl].sum(0), f"two_stage z_buf seq{b}")


@pytest.mark.parametrize("B,S,E", [(8, 256, 512), (2, 100, 300), (3, 31, 96),
                                   (2, 60, 768)])   # above 512: the recurrence kernels
def test_linear_gpt_wide(dev, B, S, E):
    """LinearGPT's attention at its width (D = next_pow2(E), zero-padded phi):
    the linear_cuda chain and the fused block (cxg_lin_elu_*) on raw inputs."""
    import torch
    import cxxgpt_attn as cx
    D = 1 << (E - 1).bit_length()
    N = B * S
    Xq, Xk, V, dO = normal_inputs((N, E), (N, E), 3 * S + E)
    Qp, Kp = orc.phi_elu_forward(Xq, D, E), orc.phi_elu_forward(Xk, D, E)
    tq, tk, tv, tdo = _t(Qp, dev), _t(Kp, dev), _t(V, dev), _t(dO, dev)
    O, den, zc = _nan(dev, N, E), _nan(dev, N), _nan(dev, N, D)
    Sb, zb = _nan(dev, B * D, E), _nan(dev, B, D)
    cx.lin_fwd(tq, tk, tv, O, den, zc, Sb, zb, B, S, D, E)
    dnum, dden = _nan(dev, N, E), _nan(dev, N)
    cx.lin_bwd_step1(O, tdo, den, dnum, dden, N, E)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.lin_bwd_dQ(tk, tv, dnum, dden, zc, dQ, Sb, B, S, D, E)
    cx.lin_bwd_dKdV(tq, tk, tv, dnum, dden, dK, dV, B, S, D, E)
    # the fused block on the raw projections (phi_elu inside, D = E there)
    eO, eden = _nan(dev, N, E), _nan(dev, N)
    cx.lin_elu_fwd(_t(Xq, dev), _t(Xk, dev), tv, eO, eden, None, B, S, E)
    dXq, dXk, edV = _nan(dev, N, E), _nan(dev, N, E), _nan(dev, N, E)
    cx.lin_elu_bwd(_t(Xq, dev), _t(Xk, dev), tv, eO, tdo, eden, dXq, dXk, edV, B, S, E)
    # with the forward's context (block-score path: features and score blocks
    # kept): the same kernels on the same values, so the same bits
    nctx = cx.lin_ctx_size(B, S, E, E)
    if nctx:
        ctx = torch.full((nctx // 4,), float("nan"), device=dev)
        cO, cden = _nan(dev, N, E), _nan(dev, N)
        cx.lin_elu_fwd(_t(Xq, dev), _t(Xk, dev), tv, cO, cden, ctx, B, S, E)
        cdXq, cdXk, cdV = _nan(dev, N, E), _nan(dev, N, E), _nan(dev, N, E)
        cx.lin_elu_bwd(_t(Xq, dev), _t(Xk, dev), tv, cO, tdo, cden, cdXq, cdXk, cdV, B, S, E,
                       ctx=ctx)
        torch.cuda.synchronize()
        for name, a, b in (("O", cO, eO), ("den", cden, eden), ("dXq", cdXq, dXq),
                           ("dXk", cdXk, dXk), ("dV", cdV, edV)):
            assert np.array_equal(_np(a), _np(b)), f"lin_elu with context: {name}"
    torch.cuda.synchronize()
    seqs = [0, B - 1] if B > 2 else list(range(B))
    for s in seqs:
        sl = slice(s * S, (s + 1) * S)
        rO, rden, rzc, _, _ = orc.lcu_fwd(Qp[sl], Kp[sl], V[sl], 1, S, D, E)
        assert_close(_np(O)[sl], rO, f"lcu seq{s} O")
        assert_close(_np(den)[sl], rden, f"lcu seq{s} den")
        assert_close(_np(zc)[sl], rzc, f"lcu seq{s} z_cache")
        rdn, rdd = orc.lcu_bwd_step1(_np(O)[sl], dO[sl], _np(den)[sl], S, E)
        rdQ = orc.lcu_bwd_dQ(Kp[sl], V[sl], rdn, rdd, rzc, 1, S, D, E)
        rdK, rdV = orc.lcu_bwd_dKdV(Qp[sl], Kp[sl], V[sl], rdn, rdd, 1, S, D, E)
        assert_close(_np(dQ)[sl], rdQ, f"lcu seq{s} dQ_phi")
        assert_close(_np(dK)[sl], rdK, f"lcu seq{s} dK_phi")
        assert_close(_np(dV)[sl], rdV, f"lcu seq{s} dV")
        # fused block: phi_elu_backward(dQ_phi) etc. on its own O and den
        assert_close(_np(eO)[sl], rO, f"lin_elu seq{s} O")
        assert_close(_np(eden)[sl], rden, f"lin_elu seq{s} den")
        edn, edd = orc.lcu_bwd_step1(_np(eO)[sl], dO[sl], _np(eden)[sl], S, E)
        edQ = orc.lcu_bwd_dQ(Kp[sl], V[sl], edn, edd, rzc, 1, S, D, E)
        edK, edV2 = orc.lcu_bwd_dKdV(Qp[sl], Kp[sl], V[sl], edn, edd, 1, S, D, E)
        assert_close(_np(dXq)[sl], orc.phi_elu_backward(edQ, Xq[sl], D, E), f"lin_elu seq{s} dXq")
        assert_close(_np(dXk)[sl], orc.phi_elu_backward(edK, Xk[sl], D, E), f"lin_elu seq{s} dXk")
        assert_close(_np(edV)[sl], edV2, f"lin_elu seq{s} dV")


@pytest.mark.parametrize("v_mean", [0.0, 3.0])
def test_wide_fused_backward_mean_shift(dev, v_mean):
    """One-call backward (cxg_kattn_bwd) at a wide shape with V ~ N(mu, 1)."""
    import torch
    import cxxgpt_attn as cx
    B, S, D, E = 2, 256, 256, 256
    N = B * S
    Q, K, V, dO = normal_inputs((N, D), (N, E), 77, v_mean=v_mean)
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O, den = _nan(dev, N, E), _nan(dev, N)
    cx.kattn_fwd(tQ, tK, tV, O, den, None, None, None, B, S, D, E)
    dQ, dK, dV = _nan(dev, N, D), _nan(dev, N, D), _nan(dev, N, E)
    cx.kattn_bwd(tQ, tK, tV, O, tdO, den, dQ, dK, dV, B, S, D, E)
    torch.cuda.synchronize()
    rO, rden, rzc = orc.kattn_fwd(Q, K, V, B, S, D, E, nthreads=8)
    assert_close(_np(O), rO, "O")
    dnum, dden = orc.kattn_bwd_step1(_np(O), dO, _np(den), N, E)
    assert_close(_np(dQ), orc.kattn_bwd_dQ(K, V, dnum, dden, rzc, Q, B, S, D, E, nthreads=8), "dQ")
    rdK, rdV = orc.kattn_bwd_dKdV(Q, K, V, dnum, dden, B, S, D, E, nthreads=8)
    assert_close(_np(dK), rdK, "dK")
    assert_close(_np(dV), rdV, "dV")


def _launches(name):
    import cxxgpt_attn as cx
    return cx.prof_query(name)[1]


# Widths multiples of 16 take the block-score kernels (linquad.hip); others
# above 128 the one-workgroup-per-block kernels, whose forward splits the keys
# of each query block when the jobs would leave resident workgroups idle (at
# most a few hundred jobs: one or two resident workgroups per CU).
@pytest.mark.parametrize("B,S,D,E,path", [
    (1, 256, 512, 512, "qs"), (8, 256, 512, 512, "qs"), (6, 200, 512, 512, "qs"),
    (4, 333, 256, 192, "qs"), (2, 17, 512, 512, "qs"),
    (1, 256, 508, 508, "split"), (8, 256, 500, 500, "split"), (4, 333, 260, 196, "split"),
    (2, 17, 504, 504, "split")])
def test_forward_paths(dev, B, S, D, E, path):
    """Forwards with and without z_cache, both APIs (two_stage with phi inside,
    linear_cuda with phi outside), against the oracle.  Block-score path: the
    launches are the score and product kernels, and O, den do not depend on
    whether z_cache is requested (its columns are separate jobs).  Key-split
    path: without z_cache the keys are split and the parts added in a second
    launch, which changes only the order of the key sums."""
    import torch
    import cxxgpt_attn as cx
    N = B * S
    Q, K, V, _ = normal_inputs((N, D), (N, E), 11 * S + B + D)
    Qp, Kp = orc.phi_elu_forward(Q, D, D), orc.phi_elu_forward(K, D, D)
    tQ, tK, tV, tQp, tKp = _t(Q, dev), _t(K, dev), _t(V, dev), _t(Qp, dev), _t(Kp, dev)
    out = {}
    for api in ("kattn", "lcu"):
        fn = cx.kattn_fwd if api == "kattn" else cx.lin_fwd
        q, k = (tQ, tK) if api == "kattn" else (tQp, tKp)
        for split in (True, False):
            O, den = _nan(dev, N, E), _nan(dev, N)
            zc = None if split else _nan(dev, N, D)
            torch.cuda.synchronize()
            cx.prof_reset()
            cx.prof_enable(True)
            fn(q, k, tV, O, den, zc, None, None, B, S, D, E)
            torch.cuda.synchronize()
            fin = _launches("lin_wide_fin")
            qs = _launches("lin_qs_out")
            old = _launches("lin_wide_fwd")
            cx.prof_enable(False)
            cx.prof_reset()
            if path == "qs":
                assert qs == 1 and old == 0 and fin == 0, f"{api}: B{B} S{S} D{D} E{E} path"
            elif not split:
                assert fin == 0 and qs == 0
            elif S > 16:
                assert fin == 1, f"{api}: the keys of B{B} S{S} were not split"
            out[api, split] = (_np(O), _np(den))
    rO, rden, _ = orc.kattn_fwd(Q, K, V, B, S, D, E, nthreads=8)
    lO, lden, _, _, _ = orc.lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=8)
    for api, (ro, rd) in (("kattn", (rO, rden)), ("lcu", (lO, lden))):
        for split in (True, False):
            o, d = out[api, split]
            assert_close(o, ro, f"{api} split={split} O")
            assert_close(d, rd, f"{api} split={split} den")
        if path == "qs":
            assert (out[api, True][0] == out[api, False][0]).all(), f"{api} O with z_cache"
            assert (out[api, True][1] == out[api, False][1]).all(), f"{api} den with z_cache"
        else:
            assert_close(out[api, True][0], out[api, False][0], f"{api} O split vs whole",
                         atol=1e-6, rtol=1e-5)
            assert_close(out[api, True][1], out[api, False][1], f"{api} den split vs whole",
                         atol=1e-6, rtol=1e-5)
