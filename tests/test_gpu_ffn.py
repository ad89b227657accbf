"""GPU parity tests of the expander FFN (cxg_ffn_fwd / cxg_ffn_bwd).

The two-stage block's q/k/v expanders and final FFN (two_stage_gpt.hpp:86-99,
:126-129 forward; :138-144, :177-195 backward) are two bias-free Linear layers
(gpt_gpt.hpp:86-112) with gelu_exact between them.  Small and ragged shapes
are checked against the C oracle (orc_ffn_*: products accumulated in double,
rounded once); the C2 shape (B*S = 2048 rows, n_embd 768, F = 4*2*768) is
checked against the same formulas in float64 on the GPU (torch).  Inputs at
the reference's initialisation scale (kaiming weights, gpt_gpt.hpp:79).
Tolerance: |gpu - ref| <= 1e-5 + 1e-4 |ref| for every output (tests/helpers.py).
The weight gradients are scaled as a mean loss's are (dY / M), since
Linear accumulates them over all M rows.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close

pytestmark = pytest.mark.gpu


def _inputs(M, E, F, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((M, E)).astype(np.float32)
    W1 = (rng.standard_normal((F, E)) * np.sqrt(2.0 / E)).astype(np.float32)
    W2 = (rng.standard_normal((E, F)) * np.sqrt(2.0 / F)).astype(np.float32)
    dY = (rng.standard_normal((M, E)) / M).astype(np.float32)
    return X, W1, W2, dY


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _run(dev, X, W1, W2, dY, M, E, F, g_is_act, dW0=0.0, with_ws=True, keep_pre=True):
    import torch
    import cxxgpt_attn as cx
    tX, tW1, tW2, tdY = (_t(a, dev) for a in (X, W1, W2, dY))
    nan = float("nan")
    pre = torch.full((M, F), nan, device=dev) if keep_pre else None
    act = torch.full((M, F), nan, device=dev)
    Y = torch.full((M, E), nan, device=dev)
    ws = None
    if with_ws:
        nb = cx.ffn_workspace_size(M, E, F)
        ws = torch.empty(max(nb, 4) // 4, device=dev)
    cx.ffn_fwd(tX, tW1, tW2, pre, act, Y, M, E, F, workspace=ws)
    G = act if (g_is_act or pre is None) else pre
    dX = torch.full((M, E), nan, device=dev)
    dW1 = torch.full((F, E), dW0, device=dev)
    dW2 = torch.full((E, F), dW0, device=dev)
    cx.ffn_bwd(tX, tW1, tW2, act, G, tdY, dX, dW1, dW2, M, E, F, workspace=ws)
    torch.cuda.synchronize()
    out = {k: (None if v is None else v.cpu().numpy())
           for k, v in dict(pre=pre, act=act, Y=Y, dX=dX, dW1=dW1, dW2=dW2).items()}
    return out


@pytest.mark.parametrize("M,E,F,g_is_act", [
    (256, 128, 1024, True),    # gpt_gpt.hpp:322 n_embd 128, N = 2: F = 4*2*128
    (256, 128, 1024, False),   # the final FFN's form: gelu' at the pre-activation
    (200, 64, 512, True),      # ragged M
    (130, 132, 260, False),    # no dimension a multiple of the 128 tile
    (1, 4, 4, True),           # one row
    (5, 8, 1000, True),
    (64, 512, 128, False),     # F < E
])
def test_ffn_vs_oracle(dev, M, E, F, g_is_act):
    X, W1, W2, dY = _inputs(M, E, F, M + E + F)
    got = _run(dev, X, W1, W2, dY, M, E, F, g_is_act)
    pre, act, Y = orc.ffn_fwd(X, W1, W2, M, E, F)
    tag = f"ffn M{M}E{E}F{F}"
    assert_close(got["pre"], pre, tag + " pre")
    assert_close(got["act"], act, tag + " act")
    assert_close(got["Y"], Y, tag + " Y")
    # backward from the GPU's own act / pre (the tensors a caller keeps)
    G = got["act"] if g_is_act else got["pre"]
    dX, dW1, dW2 = orc.ffn_bwd(X, W1, W2, got["act"], G, dY, M, E, F)
    assert_close(got["dX"], dX, tag + " dX")
    assert_close(got["dW1"], dW1, tag + " dW1")
    assert_close(got["dW2"], dW2, tag + " dW2")


def test_ffn_accumulates_and_scratch(dev):
    """Weight gradients add onto what dW1/dW2 hold (Linear's W.grad += dW);
    results are the same with stream-ordered scratch and without pre."""
    M, E, F = 96, 64, 256
    X, W1, W2, dY = _inputs(M, E, F, 17)
    a = _run(dev, X, W1, W2, dY, M, E, F, True, dW0=0.0)
    b = _run(dev, X, W1, W2, dY, M, E, F, True, dW0=0.5, with_ws=False, keep_pre=False)
    assert b["pre"] is None
    for k in ("act", "Y", "dX"):
        assert np.array_equal(a[k], b[k]), k
    assert_close(b["dW1"], a["dW1"] + 0.5, "dW1 accumulate")
    assert_close(b["dW2"], a["dW2"] + 0.5, "dW2 accumulate")


def test_ffn_c2_shape(dev):
    """B*S = 2048 rows, n_embd 768, F = 6144 (the MHA benchmark shape B8 S256
    with the reference's expansion N = 2): against float64 products on the GPU."""
    import torch
    M, E, F = 2048, 768, 6144
    X, W1, W2, dY = _inputs(M, E, F, 2048)
    got = _run(dev, X, W1, W2, dY, M, E, F, True)
    d = torch.float64
    tX, tW1, tW2, tdY = (_t(a, dev).to(d) for a in (X, W1, W2, dY))
    pre = tX @ tW1.T
    assert_close(got["pre"], pre.cpu().numpy(), "c2 pre")
    act64 = 0.5 * pre * (1 + torch.erf(pre / np.sqrt(2.0)))
    assert_close(got["act"], act64.cpu().numpy(), "c2 act")
    act = torch.from_numpy(got["act"]).to(dev).to(d)
    assert_close(got["Y"], (act @ tW2.T).cpu().numpy(), "c2 Y")
    gd = 0.5 * (1 + torch.erf(act / np.sqrt(2.0))) + act * torch.exp(-0.5 * act * act) / \
        np.sqrt(2 * np.pi)
    dact = (tdY @ tW2) * gd
    assert_close(got["dX"], (dact @ tW1).cpu().numpy(), "c2 dX")
    assert_close(got["dW1"], (dact.T @ tX).cpu().numpy(), "c2 dW1")
    assert_close(got["dW2"], (tdY.T @ act).cpu().numpy(), "c2 dW2")


def test_ffn_errors(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(4096, device=dev)
    P = cx._ptr
    st = cx._stream(None)
    ok = [P(t)] * 6
    assert cx.call_status("cxg_ffn_fwd", *ok, 4, 6, 8, None, 0, st) == cx.CXG_ERR_ALIGN
    assert cx.call_status("cxg_ffn_fwd", *ok, 4, 8, 0, None, 0, st) == cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_ffn_fwd", None, *ok[1:], 4, 8, 8, None, 0, st) == cx.CXG_ERR_NULL
    assert cx.call_status("cxg_ffn_fwd", *ok, 0, 8, 8, None, 0, st) == cx.CXG_OK
    mis = ctypes_offset(t, 1)
    assert cx.call_status("cxg_ffn_fwd", *ok[:5], mis, 4, 8, 8, None, 0, st) == cx.CXG_ERR_ALIGN
    need = cx.ffn_workspace_size(256, 128, 1024)
    assert need > 0
    assert cx.call_status("cxg_ffn_bwd", *[P(t)] * 9, 256, 128, 1024, P(t), need - 256, st) == \
        cx.CXG_ERR_WORKSPACE
    assert cx.ffn_workspace_size(4, 6, 8) == 0


def ctypes_offset(t, floats):
    import ctypes
    return ctypes.c_void_p(t.data_ptr() + 4 * floats)
