"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP attention path.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module; the product never does.  Each function forwards to the C
restatement in attn_oracle.c, which cites the reference routine it follows.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


def build():
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_mt_next.restype = ctypes.c_uint32
        _lib.orc_mt_frand.restype = ctypes.c_float
        _lib.orc_phi_elu.restype = ctypes.c_float
        _lib.orc_phi_elu.argtypes = [ctypes.c_float]
        _lib.orc_phi_elu_der.restype = ctypes.c_float
        _lib.orc_phi_elu_der.argtypes = [ctypes.c_float]
        _lib.orc_hadamard_entry.restype = ctypes.c_float
        _lib.orc_hadamard_entry.argtypes = [ctypes.c_int, ctypes.c_int]
        _lib.orc_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_float, ctypes.c_float,
                                         _f, _sz]
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "oracle wants contiguous float32"
    return a.ctypes.data_as(_f)


def _z(*shape):
    return np.zeros(shape, dtype=np.float32)


def _c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- generators
class MT19937:
    """std::mt19937 restated in C (kernel_test.cpp:12-14 draws from mt19937(1234))."""

    class _State(ctypes.Structure):
        _fields_ = [("mt", ctypes.c_uint32 * 624), ("idx", ctypes.c_int)]

    def __init__(self, seed):
        self.st = self._State()
        lib().orc_mt_seed(ctypes.byref(self.st), ctypes.c_uint32(seed))

    def next_u32(self):
        return lib().orc_mt_next(ctypes.byref(self.st))

    def frand(self, n):
        out = np.empty(n, dtype=np.float32)
        lib().orc_mt_fill_frand(ctypes.byref(self.st), _p(out), _sz(n))
        return out


def normal(seed, n, mean=0.0, std=1.0):
    """splitmix64 + Box-Muller stream: mean + std * N(0,1), float32."""
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(ctypes.c_uint64(seed), ctypes.c_float(mean), ctypes.c_float(std),
                          _p(out), _sz(n))
    return out


# ---------------------------------------------------------------- softmax MHA
def mha_fwd_literal(Q, K, V, B, S, H, Dh):
    Q, K, V = _c(Q), _c(K), _c(V)
    O = _z(B * S, H * Dh)
    lib().orc_mha_fwd_literal(_p(Q), _p(K), _p(V), _p(O), _sz(B), _sz(S), _sz(H), _sz(Dh))
    return O


def mha_fwd(Q, K, V, B, S, H, Dh, nthreads=1, want_lse=False):
    Q, K, V = _c(Q), _c(K), _c(V)
    O = _z(B * S, H * Dh)
    lse = _z(B * H * S) if want_lse else None
    lib().orc_mha_fwd(_p(Q), _p(K), _p(V), _p(O), _p(lse), _sz(B), _sz(S), _sz(H), _sz(Dh),
                      ctypes.c_int(nthreads))
    return (O, lse) if want_lse else O


def mha_bwd(Q, K, V, O, dO, B, S, H, Dh, nthreads=1):
    Q, K, V, O, dO = _c(Q), _c(K), _c(V), _c(O), _c(dO)
    dQ, dK, dV = _z(B * S, H * Dh), _z(B * S, H * Dh), _z(B * S, H * Dh)
    lib().orc_mha_bwd(_p(Q), _p(K), _p(V), _p(O), _p(dO), _p(dQ), _p(dK), _p(dV),
                      _sz(B), _sz(S), _sz(H), _sz(Dh), ctypes.c_int(nthreads))
    return dQ, dK, dV


def mha_fwd_heads(Q, K, V, B, S, H, Dh, heads, nthreads=1):
    """Forward for the listed (b*H+h) heads only; other entries are NaN."""
    Q, K, V = _c(Q), _c(K), _c(V)
    O = np.full((B * S, H * Dh), np.nan, dtype=np.float32)
    hs = np.ascontiguousarray(heads, dtype=np.uintp)
    lib().orc_mha_fwd_heads(_p(Q), _p(K), _p(V), _p(O), _sz(B), _sz(S), _sz(H), _sz(Dh),
                            hs.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t)), _sz(len(hs)),
                            ctypes.c_int(nthreads))
    return O


def mha_bwd_heads(Q, K, V, O, dO, B, S, H, Dh, heads, nthreads=1):
    Q, K, V, O, dO = _c(Q), _c(K), _c(V), _c(O), _c(dO)
    dQ = np.full((B * S, H * Dh), np.nan, dtype=np.float32)
    dK, dV = dQ.copy(), dQ.copy()
    hs = np.ascontiguousarray(heads, dtype=np.uintp)
    lib().orc_mha_bwd_heads(_p(Q), _p(K), _p(V), _p(O), _p(dO), _p(dQ), _p(dK), _p(dV),
                            _sz(B), _sz(S), _sz(H), _sz(Dh),
                            hs.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t)), _sz(len(hs)),
                            ctypes.c_int(nthreads))
    return dQ, dK, dV


# ---------------------------------------------------------------- ELU+1 (two_stage API)
def phi_elu(x):
    return np.array([lib().orc_phi_elu(float(v)) for v in np.ravel(x)],
                    dtype=np.float32).reshape(np.shape(x))


def kattn_fwd(Q, K, V, B, S, D, E, nthreads=1):
    Q, K, V = _c(Q), _c(K), _c(V)
    O, den, zc = _z(B * S, E), _z(B * S), _z(B * S, D)
    lib().orc_kattn_fwd(_p(Q), _p(K), _p(V), _p(O), _p(den), _p(zc),
                        _sz(B), _sz(S), _sz(D), _sz(E), ctypes.c_int(nthreads))
    return O, den, zc


def kattn_bwd_literal(Q, K, V, O, dO, den, B, S, D, E):
    args = [_c(a) for a in (Q, K, V, O, dO, den)]
    dQ, dK, dV = _z(B * S, D), _z(B * S, D), _z(B * S, E)
    lib().orc_kattn_bwd_literal(*[_p(a) for a in args], _p(dQ), _p(dK), _p(dV),
                                _sz(B), _sz(S), _sz(D), _sz(E))
    return dQ, dK, dV


def kattn_bwd_step1(O, dO, den, N, E):
    O, dO, den = _c(O), _c(dO), _c(den)
    dnum, dden = _z(N, E), _z(N)
    lib().orc_kattn_bwd_step1(_p(O), _p(dO), _p(den), _p(dnum), _p(dden), _sz(N), _sz(E))
    return dnum, dden


def kattn_bwd_dQ(K, V, dnum, dden, zc, Q, B, S, D, E, nthreads=1):
    args = [_c(a) for a in (K, V, dnum, dden, zc, Q)]
    dQ = _z(B * S, D)
    lib().orc_kattn_bwd_dQ(*[_p(a) for a in args], _p(dQ), _sz(B), _sz(S), _sz(D), _sz(E),
                           ctypes.c_int(nthreads))
    return dQ


def kattn_bwd_dKdV(Q, K, V, dnum, dden, B, S, D, E, nthreads=1):
    args = [_c(a) for a in (Q, K, V, dnum, dden)]
    dK, dV = _z(B * S, D), _z(B * S, E)
    lib().orc_kattn_bwd_dKdV(*[_p(a) for a in args], _p(dK), _p(dV),
                             _sz(B), _sz(S), _sz(D), _sz(E), ctypes.c_int(nthreads))
    return dK, dV


# ---------------------------------------------------------------- linear_cuda API
def lcu_fwd(Qp, Kp, V, B, S, D, E, nthreads=1):
    Qp, Kp, V = _c(Qp), _c(Kp), _c(V)
    O, den, zc = _z(B * S, E), _z(B * S), _z(B * S, D)
    Sb, zb = _z(B * D, E), _z(B, D)
    lib().orc_lcu_fwd(_p(Qp), _p(Kp), _p(V), _p(O), _p(den), _p(zc), _p(Sb), _p(zb),
                      _sz(B), _sz(S), _sz(D), _sz(E), ctypes.c_int(nthreads))
    return O, den, zc, Sb, zb


def lcu_bwd_step1(O, dO, den, N, E):
    O, dO, den = _c(O), _c(dO), _c(den)
    dnum, dden = _z(N, E), _z(N)
    lib().orc_lcu_bwd_step1(_p(O), _p(dO), _p(den), _p(dnum), _p(dden), _sz(N), _sz(E))
    return dnum, dden


def lcu_bwd_dQ(Kp, V, dnum, dden, zc, B, S, D, E, nthreads=1):
    args = [_c(a) for a in (Kp, V, dnum, dden, zc)]
    dQ = _z(B * S, D)
    lib().orc_lcu_bwd_dQ(*[_p(a) for a in args], _p(dQ), _sz(B), _sz(S), _sz(D), _sz(E),
                         ctypes.c_int(nthreads))
    return dQ


def lcu_bwd_dKdV(Qp, Kp, V, dnum, dden, B, S, D, E, nthreads=1):
    args = [_c(a) for a in (Qp, Kp, V, dnum, dden)]
    dK, dV = _z(B * S, D), _z(B * S, E)
    lib().orc_lcu_bwd_dKdV(*[_p(a) for a in args], _p(dK), _p(dV),
                           _sz(B), _sz(S), _sz(D), _sz(E), ctypes.c_int(nthreads))
    return dK, dV


def phi_elu_forward(x, D, E):
    x = _c(x)
    N = x.size // E
    phi = _z(N, D)
    lib().orc_phi_elu_forward(_p(x), _p(phi), _sz(N), _sz(D), _sz(E))
    return phi


def phi_elu_backward(dphi, x, D, E):
    dphi, x = _c(dphi), _c(x)
    N = x.size // E
    dx = _z(N, E)
    lib().orc_phi_elu_backward(_p(dphi), _p(x), _p(dx), _sz(N), _sz(D), _sz(E))
    return dx


# ---------------------------------------------------------------- Hadamard+Exp
def hadamard64():
    return np.array([[lib().orc_hadamard_entry(i, j) for j in range(64)] for i in range(64)],
                    dtype=np.float32)


def phi_hexp_forward(x, D, E):
    x = _c(x)
    N = x.size // E
    phi = _z(N, D)
    lib().orc_phi_hexp_forward(_p(x), _p(phi), _sz(N), _sz(D), _sz(E))
    return phi


def phi_hexp_backward(dphi, x, D, E):
    dphi, x = _c(dphi), _c(x)
    N = x.size // E
    dx = _z(N, E)
    lib().orc_phi_hexp_backward(_p(dphi), _p(x), _p(dx), _sz(N), _sz(D), _sz(E))
    return dx


def rope(X, B, S, D, head_dim, sign):
    """kernel_test.cpp:451-471 ref_rope: returns the rotated copy of X (B*S, D)."""
    Y = np.array(X, dtype=np.float32, copy=True, order="C")
    lib().orc_rope(_p(Y), _sz(B), _sz(S), _sz(D), _sz(head_dim), ctypes.c_float(sign))
    return Y


def gelu_exact(A):
    """two_stage_cuda_kernels.cu:1888-1895 (gelu_exact_kernel)."""
    A = _c(A)
    C = np.zeros_like(A)
    lib().orc_gelu_exact(_p(A), _p(C), _sz(A.size))
    return C


def ffn_fwd(X, W1, W2, M, E, F, nthreads=8):
    """Expander FFN forward (two_stage_gpt.hpp:86-89): returns pre, act, Y."""
    X, W1, W2 = _c(X), _c(W1), _c(W2)
    pre = np.zeros((M, F), np.float32)
    act = np.zeros((M, F), np.float32)
    Y = np.zeros((M, E), np.float32)
    lib().orc_ffn_fwd(_p(X), _p(W1), _p(W2), _p(pre), _p(act), _p(Y), _sz(M), _sz(E), _sz(F),
                      ctypes.c_int(nthreads))
    return pre, act, Y


def ffn_bwd(X, W1, W2, act, G, dY, M, E, F, dW1=None, dW2=None, nthreads=8):
    """Expander FFN backward (two_stage_gpt.hpp:177-183): returns dX, dW1, dW2
    (the weight gradients accumulate onto dW1 / dW2 when given)."""
    X, W1, W2, act, G, dY = (_c(a) for a in (X, W1, W2, act, G, dY))
    dX = np.zeros((M, E), np.float32)
    dW1 = np.zeros((F, E), np.float32) if dW1 is None else _c(dW1).copy()
    dW2 = np.zeros((E, F), np.float32) if dW2 is None else _c(dW2).copy()
    lib().orc_ffn_bwd(_p(X), _p(W1), _p(W2), _p(act), _p(G), _p(dY), _p(dX), _p(dW1), _p(dW2),
                      _sz(M), _sz(E), _sz(F), ctypes.c_int(nthreads))
    return dX, dW1, dW2


def gelu_exact_deriv(A):
    """two_stage_cuda_kernels.cu:1906-1914 (gelu_exact_deriv_kernel)."""
    A = _c(A)
    C = np.zeros_like(A)
    lib().orc_gelu_exact_deriv(_p(A), _p(C), _sz(A.size))
    return C
