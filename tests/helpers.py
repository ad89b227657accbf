"""Shared test helpers: input generators and the parity check.

The parity bar for every fp32 output is elementwise
    |gpu - cpu| <= ATOL + RTOL * |cpu|,  ATOL = 1e-5, RTOL = 1e-4
(the tolerance the benchmark configuration fixes for this path).
"""
import numpy as np

import oracle as orc

ATOL = 1e-5
RTOL = 1e-4


def assert_close(got, ref, name, atol=ATOL, rtol=RTOL):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(
            f"{name}: {bad.sum()} of {bad.size} elements out of tolerance; worst at {i}: "
            f"got {got[i]!r} ref {ref[i]!r} (max abs err {err.max():.3e})")
    return float(err.max())


def kernel_test_inputs():
    """The exact input blocks of the reference kernel_test, in draw order.

    src/TwoStage/kernel_test.cpp:12-14 draws every input from one
    std::mt19937(1234) stream, uniform[-1, 1], block after block; the shapes
    are those of the test's blocks (:216-441).  Returns a dict name -> dict of
    arrays and dims.
    """
    g = orc.MT19937(1234)
    out = {}

    def mha_block(name, B, S, H, Dh):
        n = B * S * H * Dh
        shp = (B * S, H * Dh)
        Q = g.frand(n).reshape(shp)
        K = g.frand(n).reshape(shp)
        V = g.frand(n).reshape(shp)
        dO = g.frand(n).reshape(shp)
        out[name] = dict(Q=Q, K=K, V=V, dO=dO, B=B, S=S, H=H, Dh=Dh)

    def lin_block(name, B, S, D, E):
        dim = B * S
        Q = g.frand(dim * D).reshape(dim, D)
        K = g.frand(dim * D).reshape(dim, D)
        V = g.frand(dim * E).reshape(dim, E)
        dO = g.frand(dim * E).reshape(dim, E)
        out[name] = dict(Q=Q, K=K, V=V, dO=dO, B=B, S=S, D=D, E=E)

    mha_block("stage1", 2, 6, 2, 8)        # :216-250
    lin_block("stage2", 2, 6, 8, 8)        # :253-298
    mha_block("fallback", 2, 300, 1, 128)  # :301-334
    lin_block("flat", 2, 5, 7, 6)          # :335-374
    mha_block("bigS", 2, 256, 2, 64)       # :377-409
    lin_block("chunk", 2, 32, 256, 256)    # :410-441
    # :443-489 RoPE: Q, K then dQ, dK, each (B*S, D)
    B, S, D, hd = 2, 6, 16, 8
    n = B * S * D
    out["rope"] = dict(Q=g.frand(n).reshape(B * S, D), K=g.frand(n).reshape(B * S, D),
                       B=B, S=S, D=D, hd=hd)
    out["rope"]["dQ"] = g.frand(n).reshape(B * S, D)
    out["rope"]["dK"] = g.frand(n).reshape(B * S, D)
    return out


def normal_inputs(shape_q, shape_v, seed, q_std=1.0, v_std=1.0, d_shape=None, k_mean=0.0,
                  v_mean=0.0):
    """Benchmark-style inputs: one splitmix64/Box-Muller stream per tensor,
    seeds base+{Q:0, K:1, V:2, dO:3}; K and V may carry a mean."""
    nq = int(np.prod(shape_q))
    nv = int(np.prod(shape_v))
    Q = orc.normal(seed + 0, nq, 0.0, q_std).reshape(shape_q)
    K = orc.normal(seed + 1, nq, k_mean, q_std).reshape(shape_q)
    V = orc.normal(seed + 2, nv, v_mean, v_std).reshape(shape_v)
    dO = orc.normal(seed + 3, nv, 0.0, v_std).reshape(d_shape or shape_v)
    return Q, K, V, dO
