"""GPU parity tests of GPT's attention through cxg_gpt_attn_fwd / cxg_gpt_attn_bwd.

The reference GPT block (src/GPT/gpt_gpt.hpp:365-380, :420-438) computes its
attention with whole-matrix TensorN calls: scores = Q K^T / sqrt(E) over all
B*S rows, gpt_cuda::attention_mask (gpt_cuda_kernels.cu:458-480: -1e10 on
cross-batch and future entries), softmax, times V; the backward goes through
gpt_cuda::softmax_backward (:131-173) and three products.  The entry points
compute it as causal attention with H = 1, Dh = E (above E = 512 with the
scores in memory: causal 16x16 score blocks when E is a multiple of 16, else
each sequence's S x S scores and FP32 MFMA GEMMs).  Each case is checked
against the C oracle's MHA (ref_mha_fwd / ref_mha_bwd restated, H = 1) and,
for small B*S, against a float64 restatement of the reference's whole-matrix
formulation itself (mask value -1e10, row softmax, softmax_backward's
s * (ds - sum(s * ds)) form), which pins the equivalence the routing relies on.
TensorN's own matmul/softmax numerics are not available here (the library is
not vendored), so that part of the parity stays unpinned beyond this float64
restatement.
"""
import numpy as np
import pytest

import oracle as orc
from helpers import assert_close, normal_inputs

pytestmark = pytest.mark.gpu


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _np(t):
    return t.cpu().numpy()


def gpt_whole_matrix(Q, K, V, dO, B, S, E):
    """float64 restatement of gpt_gpt.hpp:365-380 and :420-438."""
    Q, K, V, dO = (a.astype(np.float64) for a in (Q, K, V, dO))
    dim = B * S
    scale = 1.0 / np.sqrt(E)
    scores = (Q @ K.T) * scale
    i = np.arange(dim)
    same_b = (i[:, None] // S) == (i[None, :] // S)
    causal = (i[:, None] % S) >= (i[None, :] % S)
    scores = np.where(same_b & causal, scores, -1e10)
    w = np.exp(scores - scores.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    O = w @ V
    d_w = dO @ V.T
    d_scores = w * (d_w - (w * d_w).sum(axis=1, keepdims=True)) * scale
    return O, d_scores @ K, d_scores.T @ Q, w.T @ dO


@pytest.mark.parametrize("B,S,E", [
    (2, 64, 128),     # gpt_gpt.hpp:322 default n_embd (the fused MHA kernels, H = 1)
    (2, 100, 512),    # gpt_train.cpp:139 n_embd: causal score blocks
    (1, 257, 384),    # ragged S, a mid width
    (3, 33, 260),     # just past 256
    (1, 16, 512),     # one tile
    (2, 50, 258),     # width not a multiple of 4 (scalar loads)
    (1, 130, 258),    # chunked backward and split-KV forward with scalar stores
    (4, 128, 512),
    (2, 64, 768),     # wider than 512, a multiple of 16: causal score blocks in memory
    (3, 100, 516),    # not a multiple of 16: S x S scores and FP32 MFMA GEMMs
    (1, 256, 1024),
    (2, 12, 2048),
    # generate()'s pattern (gpt_gpt.hpp:672-693): every context length, so S
    # is not a multiple of 4 (score rows padded)
    (1, 1, 768),
    (1, 7, 768),
    (1, 255, 768),
    (2, 130, 1024),
    (3, 3, 516),
    (9, 40, 384),     # score blocks with a batch of 8 and more, not a multiple of 8
    (20, 200, 768),   # a large batch, an odd block count
])
def test_gpt_attention(dev, B, S, E):
    import torch
    import cxxgpt_attn as cx
    N = B * S
    Q, K, V, dO = normal_inputs((N, E), (N, E), 7 * S + E)
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O = torch.full((N, E), float("nan"), device=dev)
    lse = torch.full((B * S,), float("nan"), device=dev)
    cx.gpt_attn_fwd(tQ, tK, tV, O, B, S, E, lse=lse)
    torch.cuda.synchronize()
    rO, rlse = orc.mha_fwd(Q, K, V, B, S, 1, E, nthreads=8, want_lse=True)
    assert_close(_np(O), rO, f"gpt O B{B}S{S}E{E}")
    assert_close(_np(lse), rlse, f"gpt lse B{B}S{S}E{E}")
    gO = _np(O)
    rdQ, rdK, rdV = orc.mha_bwd(Q, K, V, gO, dO, B, S, 1, E, nthreads=8)
    for use_lse in (True, False):
        outs = [torch.full((N, E), float("nan"), device=dev) for _ in range(3)]
        cx.gpt_attn_bwd(tQ, tK, tV, O, tdO, *outs, B, S, E, lse=lse if use_lse else None)
        torch.cuda.synchronize()
        dQ, dK, dV = (_np(t) for t in outs)
        assert_close(dQ, rdQ, f"gpt dQ B{B}S{S}E{E} lse={use_lse}")
        assert_close(dK, rdK, f"gpt dK B{B}S{S}E{E} lse={use_lse}")
        assert_close(dV, rdV, f"gpt dV B{B}S{S}E{E} lse={use_lse}")
    if N <= 300:
        wO, wdQ, wdK, wdV = gpt_whole_matrix(Q, K, V, dO, B, S, E)
        assert_close(_np(O), wO, f"gpt O vs whole-matrix form B{B}S{S}E{E}")
        assert_close(dQ, wdQ, f"gpt dQ vs whole-matrix form B{B}S{S}E{E}")
        assert_close(dK, wdK, f"gpt dK vs whole-matrix form B{B}S{S}E{E}")
        assert_close(dV, wdV, f"gpt dV vs whole-matrix form B{B}S{S}E{E}")


@pytest.mark.parametrize("B,S,E,budget", [
    (3, 64, 768, 64 * 64),          # one sequence per group
    (3, 7, 768, 2 * 7 * 8),         # forward groups of 2 and 1, backward of 1
    (5, 33, 516, 3 * 33 * 36),      # groups of 3 and 2 forward, 1 backward
])
def test_gpt_attention_groups(dev, B, S, E, budget, monkeypatch):
    """Above E = 512 the score matrices of a group of sequences are held at
    once; a small CXXGPT_GPT_SCORE_FLOATS forces several groups, so the
    later groups' row offsets (Q/K/V/dO/O/dQ/dK/dV + b0*S*E, lse + b0*S) and
    the batched GEMM's sequence strides are exercised, with and without lse."""
    import torch
    import cxxgpt_attn as cx
    monkeypatch.setenv("CXXGPT_GPT_PATH", "mat")   # the GEMM path, not the score blocks
    monkeypatch.setenv("CXXGPT_GPT_SCORE_FLOATS", str(budget))
    N = B * S
    Q, K, V, dO = normal_inputs((N, E), (N, E), 11 * S + E + B)
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    O = torch.full((N, E), float("nan"), device=dev)
    lse = torch.full((N,), float("nan"), device=dev)
    cx.gpt_attn_fwd(tQ, tK, tV, O, B, S, E, lse=lse)
    torch.cuda.synchronize()
    rO, rlse = orc.mha_fwd(Q, K, V, B, S, 1, E, nthreads=8, want_lse=True)
    assert_close(_np(O), rO, f"gpt groups O B{B}S{S}E{E}")
    assert_close(_np(lse), rlse, f"gpt groups lse B{B}S{S}E{E}")
    rdQ, rdK, rdV = orc.mha_bwd(Q, K, V, _np(O), dO, B, S, 1, E, nthreads=8)
    for use_lse in (True, False):
        nws = cx.lib().cxg_gpt_attn_bwd_workspace_size(B, S, E)
        ws = torch.empty(nws // 4 + 1, device=dev)
        outs = [torch.full((N, E), float("nan"), device=dev) for _ in range(3)]
        cx.gpt_attn_bwd(tQ, tK, tV, O, tdO, *outs, B, S, E, lse=lse if use_lse else None,
                        workspace=ws)
        torch.cuda.synchronize()
        for name, g, r in zip(("dQ", "dK", "dV"), outs, (rdQ, rdK, rdV)):
            assert_close(_np(g), r, f"gpt groups {name} B{B}S{S}E{E} lse={use_lse}")
    cx.release_scratch()


@pytest.mark.parametrize("B,S,E", [(2, 100, 512), (1, 77, 384), (2, 64, 768)])
def test_gpt_attention_without_blocks(dev, B, S, E, monkeypatch):
    """Widths above 256 that are multiples of 16 take the causal score blocks;
    with CXXGPT_GPT_PATH=mat the same shapes run the wide-head kernels (up to
    512) or the S x S scores and GEMMs, which other widths still use.  Both
    against the oracle, and against each other."""
    import torch
    import cxxgpt_attn as cx
    N = B * S
    Q, K, V, dO = normal_inputs((N, E), (N, E), 13 * S + E + B)
    tQ, tK, tV, tdO = _t(Q, dev), _t(K, dev), _t(V, dev), _t(dO, dev)
    res = {}
    for path in ("blocks", "mat"):
        if path == "mat":
            monkeypatch.setenv("CXXGPT_GPT_PATH", "mat")
        O = torch.full((N, E), float("nan"), device=dev)
        lse = torch.full((N,), float("nan"), device=dev)
        cx.gpt_attn_fwd(tQ, tK, tV, O, B, S, E, lse=lse)
        outs = [torch.full((N, E), float("nan"), device=dev) for _ in range(3)]
        cx.gpt_attn_bwd(tQ, tK, tV, O, tdO, *outs, B, S, E, lse=lse)
        torch.cuda.synchronize()
        res[path] = [_np(O), _np(lse)] + [_np(t) for t in outs]
    rO, rlse = orc.mha_fwd(Q, K, V, B, S, 1, E, nthreads=8, want_lse=True)
    rdQ, rdK, rdV = orc.mha_bwd(Q, K, V, res["blocks"][0], dO, B, S, 1, E, nthreads=8)
    for path, (gO, glse, gdQ, gdK, gdV) in res.items():
        assert_close(gO, rO, f"gpt {path} O B{B}S{S}E{E}")
        assert_close(glse, rlse, f"gpt {path} lse B{B}S{S}E{E}")
        assert_close(gdQ, rdQ, f"gpt {path} dQ B{B}S{S}E{E}")
        assert_close(gdK, rdK, f"gpt {path} dK B{B}S{S}E{E}")
        assert_close(gdV, rdV, f"gpt {path} dV B{B}S{S}E{E}")
    for k, (a, b) in enumerate(zip(res["blocks"], res["mat"])):
        assert_close(a, b, f"gpt blocks vs mat output {k}", atol=2e-5, rtol=2e-4)
    cx.release_scratch()


def test_gpt_attention_errors(dev):
    import torch
    import cxxgpt_attn as cx
    t = torch.zeros(64, device=dev)
    P = cx._ptr
    st = cx._stream(None)
    # above 512 the scores-in-memory path needs E a multiple of 4 (any S)
    assert cx.call_status("cxg_gpt_attn_fwd", P(t), P(t), P(t), P(t), None, 1, 4, 513, st) == \
        cx.CXG_ERR_ALIGN
    assert cx.call_status("cxg_gpt_attn_fwd", P(t), P(t), P(t), P(t), None, 1, 20000, 516, st) \
        == cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_gpt_attn_fwd", P(t), P(t), P(t), P(t), None, 1, 4, 0, st) == \
        cx.CXG_ERR_DIMS
    assert cx.call_status("cxg_gpt_attn_fwd", None, P(t), P(t), P(t), None, 1, 4, 300, st) == \
        cx.CXG_ERR_NULL
    assert cx.call_status("cxg_gpt_attn_fwd", None, None, None, None, None, 0, 4, 300, st) == \
        cx.CXG_OK
    assert cx.call_status("cxg_gpt_attn_bwd", *[P(t)] * 5, None, *[P(t)] * 3, 1, 4, 601, None, 0,
                          st) == cx.CXG_ERR_ALIGN
