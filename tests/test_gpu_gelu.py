"""GPU parity tests of the exact GELU (cxg_gelu_exact, cxg_gelu_exact_deriv).

two_stage_cuda::gelu_exact / gelu_exact_deriv (two_stage_cuda_kernels.cu:
1888-1924) against the C oracle's restatement: N(0, 3) values plus the
special points (0, large |x|, where erf saturates and the derivative's
Gaussian term underflows), odd lengths (the 4-wide path's tail), an
unaligned view (the scalar path), in place, and the expander FFN
activation size of two_stage_gpt.hpp:86-99 at the C2 shape.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close

pytestmark = pytest.mark.gpu


def _vals(n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 3.0).astype(np.float32)
    special = np.array([0.0, -0.0, 1.0, -1.0, 5.0, -5.0, 10.0, -10.0, 30.0, -30.0, 1e-20,
                        -1e-20, 3.4e38, -3.4e38], dtype=np.float32)
    x[:min(n, special.size)] = special[:min(n, special.size)]
    return x


@pytest.mark.parametrize("n", [1, 7, 4096, 100003, 2048 * 3072])
def test_gelu(dev, n):
    import torch
    import cxxgpt_attn as cx
    x = _vals(n, n)
    t = torch.from_numpy(x).to(dev)
    y, d = torch.empty_like(t), torch.empty_like(t)
    cx.gelu_exact(t, y, n)
    cx.gelu_exact_deriv(t, d, n)
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), orc.gelu_exact(x), f"gelu n={n}")
    assert_close(d.cpu().numpy(), orc.gelu_exact_deriv(x), f"gelu' n={n}")


def test_gelu_unaligned_and_in_place(dev):
    import torch
    import cxxgpt_attn as cx
    n = 1001
    x = _vals(n, 3)
    buf = torch.zeros(n + 1, device=dev)
    buf[1:] = torch.from_numpy(x).to(dev)
    view = buf[1:]
    out = torch.empty(n + 1, device=dev)[1:]
    cx.gelu_exact_deriv(view, out, n)
    cx.gelu_exact(view, view, n)   # C == A
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), orc.gelu_exact_deriv(x), "gelu' unaligned")
    assert_close(view.cpu().numpy(), orc.gelu_exact(x), "gelu in place, unaligned")


def test_gelu_errors(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(8, device=dev)
    st = cx._stream(None)
    assert cx.call_status("cxg_gelu_exact", None, cx._ptr(t), 8, st) == cx.CXG_ERR_NULL
    assert cx.call_status("cxg_gelu_exact_deriv", None, None, 0, st) == cx.CXG_OK
