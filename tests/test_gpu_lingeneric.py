"""GPU parity tests of linear attention at feature widths above 512.

Widths up to 512 take the quadratic-form kernels (linwide.hip, or the
block-score kernels of linquad.hip for widths that are multiples of 16) or the
chunked scan.  D or E above 512 take the block-score kernels when both widths
are multiples of 16 and their scratch fits the path's budget (the first shape
below), and otherwise the one-workgroup-per-sequence recurrence kernels
(lin_fwd_generic / lin_dq_generic / lin_dkdv_generic in linattn.hip: the
other shapes).
LinearGPT reaches them for any n_embd above 512: it runs the linear_cuda API
at D = next_pow2(n_embd) (linear_gpt.hpp:232), and n_embd comes from the
checkpoint's metadata.  Each API is checked against its oracle restatement:
the two_stage chain (kernel_attn_fwd -> bwd_step1 -> bwd_dQ -> bwd_dKdV,
two_stage_cuda_kernels.cu:1133-1809), the one-call fused backward with and
without a context (none is written at these widths), and the linear_cuda
chain with phi_elu outside (linear_cuda_kernels.cu:10-378).
"""
import pytest

import oracle as orc
from helpers import normal_inputs
from test_gpu_linbwd import check_fused_kattn
from test_gpu_linear import check_kattn, check_lcu

pytestmark = pytest.mark.gpu

SHAPES = [
    (2, 100, 1024, 768),   # LinearGPT at n_embd 768: D = next_pow2(768)
    (1, 64, 600, 520),     # both widths above 512, neither a power of two
    (3, 17, 520, 64),      # only D above 512
    (1, 40, 64, 513),      # only E above 512, not a multiple of 4
]


@pytest.mark.parametrize("B,S,D,E", SHAPES)
def test_two_stage_chain_generic(dev, B, S, D, E):
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 29 * S + D + E)
    check_kattn(dev, Q, K, V, dO, B, S, D, E, literal=(S <= 20), tag=f"generic B{B}S{S}D{D}E{E}")


@pytest.mark.parametrize("B,S,D,E", SHAPES)
def test_fused_backward_generic(dev, B, S, D, E):
    Q, K, V, dO = normal_inputs((B * S, D), (B * S, E), 31 * S + D + E)
    for use_ctx in (False, True):
        check_fused_kattn(dev, Q, K, V, dO, B, S, D, E, literal=(S <= 20),
                          tag=f"fused generic B{B}S{S}D{D}E{E}", use_ctx=use_ctx)


@pytest.mark.parametrize("B,S,E", [(2, 100, 768), (1, 33, 600)])
def test_linear_cuda_chain_generic(dev, B, S, E):
    """phi_elu_forward outside (D = next_pow2(E) zero-padded columns), then the
    linear_cuda forward, step 1, dQ and dKdV."""
    D = 1 << (E - 1).bit_length()
    Xq, Xk, V, dO = normal_inputs((B * S, E), (B * S, E), 37 * S + E)
    Qp, Kp = orc.phi_elu_forward(Xq, D, E), orc.phi_elu_forward(Xk, D, E)
    check_lcu(dev, Qp, Kp, V, dO, B, S, D, E, tag=f"lcu generic B{B}S{S}D{D}E{E}")
