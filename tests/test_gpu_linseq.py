"""GPU parity tests of the one-launch segment records for short sequences.

Sequences of a few hundred rows take the segment records of the forward,
dQ and dK/dV scans (the prefix or suffix state each segment of the chunked
scan starts from) from one pass with two workgroups per sequence
(lin_seqrec) instead of the aggregate + scan launch pair.  These tests run
every API whose scans use those records at shapes that take that path
(asserted through the library's per-launch hook) and compare the outputs
with the oracle: the two_stage chain (kernel_attn_fwd -> step1 -> dQ ->
dKdV, two_stage_cuda_kernels.cu:1133-1809), the fused pair (its forward) with
and without the forward's context, and the linear_cuda pair (phi applied
outside, linear_cuda_kernels.cu:10-298).  At D = E = 64 and S <= 256 the
whole forward (records, outputs and context) is one launch (lin_seqfwd).  Shapes cover one and two chunks per
wave, partial last chunks and segments, widths below 64, and mean-shifted V
at S = 256.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, normal_inputs
from test_gpu_linbwd import check_fused_kattn, fused_lcu
from test_gpu_linear import check_kattn

pytestmark = pytest.mark.gpu

# (B', S, D, E): chunks per wave 1 (S <= 256) or 2 (S 384, 512); S = 129 and
# 200 end in a partial chunk and a partial segment
SHAPES = [(96, 256, 64, 64), (5, 200, 64, 64), (2, 129, 64, 64), (7, 384, 64, 64),
          (3, 512, 48, 40), (4, 256, 20, 64)]


def _one_launch_fwd(S, D, E):
    """The forward's records and outputs in one launch (lin_seqfwd): D = E =
    64, at most 16 chunks."""
    return D == 64 and E == 64 and S <= 256


def _count(name):
    import cxxgpt_attn as cx
    return cx.prof_query(name)[1]


class _Launches:
    """Counts the launches recorded under each name while the block runs."""

    def __enter__(self):
        import cxxgpt_attn as cx
        cx.prof_reset()
        cx.prof_enable(True)
        return self

    def __exit__(self, *exc):
        import torch
        import cxxgpt_attn as cx
        torch.cuda.synchronize()
        self.n = {k: _count(k) for k in ("lin_seqrec", "lin_seqfwd", "lin_agg", "lin_scan")}
        cx.prof_enable(False)
        cx.prof_reset()
        return False


@pytest.mark.parametrize("B,S,D,E", SHAPES)
def test_chain(dev, B, S, D, E):
    """two_stage chain: the forward, dQ and dK/dV passes each take one records launch."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 40 * S + D + E)
    with _Launches() as L:
        check_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"chain B{B}S{S}D{D}E{E}")
    one = _one_launch_fwd(S, D, E)
    assert L.n["lin_seqrec"] == 3 - one and L.n["lin_seqfwd"] == one, L.n
    assert L.n["lin_agg"] == 0 and L.n["lin_scan"] == 0, L.n


@pytest.mark.parametrize("use_ctx", [False, True])
@pytest.mark.parametrize("B,S,D,E", SHAPES)
def test_fused(dev, B, S, D, E, use_ctx):
    """Fused pair: the forward's records in one launch; the backward on them
    (through the context's prefix records, or its own)."""
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 41 * S + D + E)
    with _Launches() as L:
        check_fused_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"fused B{B}S{S}D{D}E{E}",
                          use_ctx=use_ctx)
    one = _one_launch_fwd(S, D, E)
    assert L.n["lin_seqrec"] == 1 - one and L.n["lin_seqfwd"] == one, L.n
    assert L.n["lin_agg"] == 0 and L.n["lin_scan"] == 0, L.n


@pytest.mark.parametrize("B,S,D,E", [(96, 256, 64, 64), (5, 200, 64, 64), (3, 512, 48, 40)])
def test_linear_cuda_pair(dev, B, S, D, E):
    """linear_cuda's API (phi outside): cxg_lin_fwd(_ctx) -> cxg_lin_bwd."""
    Xq, Xk, V, dO = normal_inputs((B * S, D), (B * S, E), 42 * S + D + E)
    Qp, Kp = orc.phi_elu_forward(Xq, D, D), orc.phi_elu_forward(Xk, D, D)
    for use_ctx in (False, True):
        with _Launches() as L:
            fused_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag=f"lcu B{B}S{S}", use_ctx=use_ctx)
        one = _one_launch_fwd(S, D, E)
        assert L.n["lin_seqrec"] == 1 - one and L.n["lin_seqfwd"] == one, L.n


@pytest.mark.parametrize("use_ctx", [False, True])
@pytest.mark.parametrize("v_mean,k_mean", [(3.0, 0.0), (3.0, 1.0)])
def test_mean_shifted(dev, v_mean, k_mean, use_ctx):
    """V ~ N(3, 1) (and K shifted) at C3 S256, where the forward's records come
    from the one-launch pass and the backward's state near each sequence start
    from the anchors (the forward's context, or lin_bagg's)."""
    B, S, D, E = 96, 256, 64, 64
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 950 + int(10 * v_mean + k_mean),
                                k_mean=k_mean, v_mean=v_mean)
    check_fused_kattn(dev, Q, K, V, dO, B, S, D, E,
                      tag=f"S256 muV{v_mean} muK{k_mean}", use_ctx=use_ctx)


def test_records_match_two_launch_path(dev):
    """The records one launch forms equal, to rounding, those of the aggregate +
    scan pair: the dQ pass at a shape where both paths exist gives the same dQ.
    At S = 1024 and B' = 1 the plan has 32 segments of 2 chunks (64 chunks: too
    many for one workgroup, so the pair runs); the same rows as 4 sequences of
    256 (records launch) must agree with the oracle per sequence, and the
    scans' agreement shows in dQ of the first 256 rows, whose state does not
    depend on the split."""
    D = E = 64
    Q, K, V, dO = normal_inputs((4 * 256, D), (4 * 256, E), 77)
    outs = []
    for B, S in ((1, 1024), (4, 256)):
        with _Launches() as L:
            g = check_kattn(dev, Q, K, V, dO, B, S, D, E, tag=f"B{B}S{S}")
        outs.append(g)
        if S == 256:
            assert L.n["lin_seqrec"] == 2 and L.n["lin_seqfwd"] == 1, L.n
        else:
            assert L.n["lin_seqrec"] == 0 and L.n["lin_agg"] == 3, L.n
    # rows 0..255 are the first sequence in both splits: dQ of a row depends
    # only on the rows up to it
    np.testing.assert_allclose(outs[0]["dQ"][:256], outs[1]["dQ"][:256], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("S", [256, 200, 137])
def test_state_outputs_one_launch(dev, S):
    """The one-launch forward's final-state outputs: S_buf ([d][e] for
    linear_cuda, [e][d] for two_stage) and z_buf, with O, den and z_cache,
    at D = E = 64 (full, partial-chunk and partial-segment lengths)."""
    import torch
    import cxxgpt_attn as cx
    from test_gpu_linwide import _state_bound_check
    B, D, E = 3, 64, 64
    N = B * S
    Q, K, V, _ = normal_inputs((N, D), (N, E), 1200 + S)
    Qp, Kp = orc.phi_elu_forward(Q, D, D), orc.phi_elu_forward(K, D, D)

    def nan(*shape):
        return torch.full(shape, float("nan"), device=dev)

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)

    O, den, zc, Sb, zb = nan(N, E), nan(N), nan(N, D), nan(B * D, E), nan(B, D)
    O2, den2, zc2, Sb2, zb2 = nan(N, E), nan(N), nan(N, D), nan(B * E, D), nan(B, D)
    with _Launches() as L:
        cx.lin_fwd(t(Qp), t(Kp), t(V), O, den, zc, Sb, zb, B, S, D, E)
        cx.kattn_fwd(t(Q), t(K), t(V), O2, den2, zc2, Sb2, zb2, B, S, D, E)
    assert L.n["lin_seqfwd"] == 2 and L.n["lin_seqrec"] == 0, L.n
    rO, rden, rzc, rSb, rzb = orc.lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=8)
    np_ = lambda x: x.cpu().numpy()   # noqa: E731
    assert_close(np_(O), rO, "lcu O")
    assert_close(np_(den), rden, "lcu den_cache")
    assert_close(np_(zc), rzc, "lcu z_cache")
    assert_close(np_(zb), rzb, "lcu z_buf")
    kO, kden, kzc = orc.kattn_fwd(Q, K, V, B, S, D, E, nthreads=8)
    assert_close(np_(O2), kO, "two_stage O")
    assert_close(np_(den2), kden, "two_stage den")
    assert_close(np_(zc2), kzc, "two_stage z_cache")
    pK = np.where(K > 0, K + 1.0, np.exp(K.astype(np.float64)))
    for b in range(B):
        sl = slice(b * S, (b + 1) * S)
        _state_bound_check(np_(Sb)[b * D:(b + 1) * D], Kp[sl], V[sl], f"lcu S_buf seq{b}")
        _state_bound_check(np_(Sb2)[b * E:(b + 1) * E], pK[sl], V[sl],
                           f"two_stage S_buf [e][d] seq{b}", transpose=True)
        assert_close(np_(zb2)[b], pK[sl].sum(0), f"two_stage z_buf seq{b}")
