"""GPU tests: the C ABI entry points under HIP graph capture.

A caller may capture a training step's attention calls into a graph and
replay it.  Each test captures a forward+backward chain on a side stream,
then replays it several times with new inputs written into the captured
buffers between replays (eager torch work and synchronisations in between),
and checks every replay against the same chain run eagerly on the same
inputs: bit-identical where the kernels are deterministic, and for the MHA
dQ (float atomics, whose order of arrival varies) within the parity
tolerance.  No entry point records a memset; the linear chain's segment
scratch comes from stream-ordered allocation, which capture records as graph
memory nodes.
"""
import numpy as np
import pytest

from helpers import assert_close

pytestmark = pytest.mark.gpu


def _capture(torch, fn):
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=s):
        fn(s.cuda_stream)
    torch.cuda.synchronize()
    return g


def _refill(torch, gen, tensors, std=1.0):
    for t in tensors:
        t.copy_(torch.randn(t.shape, device=t.device, generator=gen) * std)


def test_mha_fwd_bwd_graph_replay(dev):
    import torch
    import cxxgpt_attn as cx
    B, S, H, Dh = 2, 200, 4, 64
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    shp = (B * S, H * Dh)
    Q, K, V, dO = [torch.empty(shp, device=dev) for _ in range(4)]
    ws = torch.empty(max(1, cx.mha_bwd_workspace_size(B, S, H, Dh) // 4), device=dev)

    def outs():
        return ([torch.empty(shp, device=dev) for _ in range(4)],
                torch.empty(B * H * S, device=dev))

    def chain(O, dQ, dK, dV, lse, stream):
        cx.mha_fwd(Q, K, V, O, B, S, H, Dh, lse=lse, stream=stream)
        cx.mha_bwd(Q, K, V, O, dO, dQ, dK, dV, B, S, H, Dh, lse=lse, workspace=ws, stream=stream)

    _refill(torch, gen, (Q, K, V, dO))
    (gO, gdQ, gdK, gdV), glse = outs()
    graph = _capture(torch, lambda s: chain(gO, gdQ, gdK, gdV, glse, s))
    (eO, edQ, edK, edV), e_lse = outs()
    for rep in range(3):
        _refill(torch, gen, (Q, K, V, dO))
        torch.cuda.synchronize()
        chain(eO, edQ, edK, edV, e_lse, None)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b, name in ((gO, eO, "O"), (glse, e_lse, "lse"), (gdK, edK, "dK"), (gdV, edV, "dV")):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager run"
        assert_close(gdQ.cpu().numpy(), edQ.cpu().numpy(), f"replay {rep}: dQ")


@pytest.mark.parametrize("use_lse", [True, False])
def test_mha_narrow_graph_replay(dev, use_lse):
    """Narrow heads (one workgroup per head, no atomics): every output of every
    replay bit-identical to the eager run, with the forward's lse and with
    the reference's signature (statistics recomputed in the backward), RoPE
    fused."""
    import torch
    import cxxgpt_attn as cx
    B, S, H, Dh = 3, 200, 8, 8
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    shp = (B * S, H * Dh)
    Q, K, V, dO = [torch.empty(shp, device=dev) for _ in range(4)]

    def outs():
        return ([torch.empty(shp, device=dev) for _ in range(4)],
                torch.empty(B * H * S, device=dev))

    def chain(O, dQ, dK, dV, lse, stream):
        cx.mha_rope_fwd(Q, K, V, O, B, S, H, Dh, lse=lse, stream=stream)
        cx.mha_rope_bwd(Q, K, V, O, dO, dQ, dK, dV, B, S, H, Dh,
                        lse=lse if use_lse else None, stream=stream)

    _refill(torch, gen, (Q, K, V, dO))
    (gO, gdQ, gdK, gdV), glse = outs()
    graph = _capture(torch, lambda s: chain(gO, gdQ, gdK, gdV, glse, s))
    (eO, edQ, edK, edV), e_lse = outs()
    for rep in range(3):
        _refill(torch, gen, (Q, K, V, dO))
        torch.cuda.synchronize()
        chain(eO, edQ, edK, edV, e_lse, None)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b, name in ((gO, eO, "O"), (glse, e_lse, "lse"), (gdQ, edQ, "dQ"),
                           (gdK, edK, "dK"), (gdV, edV, "dV")):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager run"


def test_linear_two_stage_graph_replay(dev):
    import torch
    import cxxgpt_attn as cx
    Bq, S, D, E = 4, 1000, 64, 64   # several segments per sequence: segment scratch in use
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    N = Bq * S
    Q, K = torch.empty(N, D, device=dev), torch.empty(N, D, device=dev)
    V, dO = torch.empty(N, E, device=dev), torch.empty(N, E, device=dev)

    def outs():
        return dict(O=torch.empty(N, E, device=dev), den=torch.empty(N, device=dev),
                    zc=torch.empty(N, D, device=dev), S_buf=torch.empty(Bq * E, D, device=dev),
                    z_buf=torch.empty(Bq, D, device=dev), dnum=torch.empty(N, E, device=dev),
                    dden=torch.empty(N, device=dev), dQ=torch.empty(N, D, device=dev),
                    dK=torch.empty(N, D, device=dev), dV=torch.empty(N, E, device=dev))

    def chain(o, stream):
        cx.kattn_fwd(Q, K, V, o["O"], o["den"], o["zc"], o["S_buf"], o["z_buf"], Bq, S, D, E,
                     stream=stream)
        cx.kattn_bwd_step1(o["O"], dO, o["den"], o["dnum"], o["dden"], N, E, stream=stream)
        cx.kattn_bwd_dQ(K, V, o["dnum"], o["dden"], o["zc"], Q, o["dQ"], o["S_buf"], Bq, S, D, E,
                        stream=stream)
        cx.kattn_bwd_dKdV(Q, K, V, o["dnum"], o["dden"], o["dK"], o["dV"], Bq, S, D, E,
                          stream=stream)

    _refill(torch, gen, (Q, K, V, dO))
    go = outs()
    graph = _capture(torch, lambda s: chain(go, s))
    eo = outs()
    for rep in range(3):
        _refill(torch, gen, (Q, K, V, dO))
        torch.cuda.synchronize()
        chain(eo, None)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name in ("O", "den", "zc", "dnum", "dden", "dQ", "dK", "dV"):
            assert torch.equal(go[name], eo[name]), f"replay {rep}: {name} differs from the eager run"
        assert np.all(np.isfinite(go["dK"].cpu().numpy()))
