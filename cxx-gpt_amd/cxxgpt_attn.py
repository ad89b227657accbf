"""ctypes binding of libcxxgpt_attn.so (the C ABI in include/cxxgpt_attn.h).

Every call goes through the C ABI with raw device pointers, exactly as a C++
or FFI caller would; torch is used only to own device memory and to supply
the current HIP stream.  There is no fallback: if the library is missing
or a call fails, an exception is raised.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libcxxgpt_attn.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "cxxgpt_attn.h")

CXG_OK = 0
CXG_ERR_NULL = 1
CXG_ERR_DIMS = 2
CXG_ERR_HEAD_DIM = 3
CXG_ERR_HIP = 4
CXG_ERR_WORKSPACE = 5
CXG_ERR_ALIGN = 6

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# name -> argument types (all return int unless listed in _RESTYPES)
SIGNATURES = {
    "cxg_status_str": [ctypes.c_int],
    "cxg_last_hip_error": [],
    "cxg_version": [],
    "cxg_release_scratch": [_vp],
    "cxg_wait_timeouts": [_vp, ctypes.POINTER(ctypes.c_uint)],
    "cxg_mha_fwd": [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp],
    "cxg_mha_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz,
                    _vp],
    "cxg_mha_bwd_workspace_size": [_sz, _sz, _sz, _sz],
    "cxg_mha_bwd_noalloc": [_vp] * 9 + [_sz] * 4 + [_vp],
    "cxg_mha_rope_fwd": [_vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp],
    "cxg_mha_rope_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _sz, _sz, _vp,
                         _sz, _vp],
    "cxg_gpt_attn_fwd": [_vp] * 5 + [_sz] * 3 + [_vp],
    "cxg_gpt_attn_bwd": [_vp] * 9 + [_sz] * 3 + [_vp, _sz, _vp],
    "cxg_gpt_attn_bwd_workspace_size": [_sz] * 3,
    "cxg_kattn_fwd": [_vp] * 8 + [_sz] * 4 + [_vp],
    "cxg_kattn_bwd_step1": [_vp] * 5 + [_sz] * 2 + [_vp],
    "cxg_kattn_bwd_dQ": [_vp] * 8 + [_sz] * 4 + [_vp],
    "cxg_kattn_bwd_dKdV": [_vp] * 7 + [_sz] * 4 + [_vp],
    "cxg_kattn_bwd": [_vp] * 10 + [_sz] * 4 + [_vp],
    "cxg_kattn_fwd_ctx": [_vp] * 6 + [_sz] * 5 + [_vp],
    "cxg_kattn_rope_fwd": [_vp] * 6 + [_sz] * 5 + [_vp],
    "cxg_kattn_rope_bwd": [_vp] * 10 + [_sz] * 4 + [_vp],
    "cxg_lin_ctx_size": [_sz] * 4,
    "cxg_lin_fwd": [_vp] * 8 + [_sz] * 4 + [_vp],
    "cxg_lin_bwd_step1": [_vp] * 5 + [_sz] * 2 + [_vp],
    "cxg_lin_bwd_dQ": [_vp] * 7 + [_sz] * 4 + [_vp],
    "cxg_lin_bwd_dKdV": [_vp] * 7 + [_sz] * 4 + [_vp],
    "cxg_lin_bwd": [_vp] * 10 + [_sz] * 4 + [_vp],
    "cxg_lin_fwd_ctx": [_vp] * 6 + [_sz] * 5 + [_vp],
    "cxg_lin_elu_fwd": [_vp] * 6 + [_sz] * 4 + [_vp],
    "cxg_lin_elu_bwd": [_vp] * 10 + [_sz] * 3 + [_vp],
    "cxg_lin_hexp_fwd": [_vp] * 6 + [_sz] * 4 + [_vp],
    "cxg_lin_hexp_bwd": [_vp] * 10 + [_sz] * 3 + [_vp],
    "cxg_phi_elu_fwd": [_vp, _vp, _sz, _sz, _sz, _vp],
    "cxg_phi_elu_bwd": [_vp, _vp, _vp, _sz, _sz, _sz, _vp],
    "cxg_phi_hexp_fwd": [_vp, _vp, _sz, _sz, _sz, _vp],
    "cxg_phi_hexp_bwd": [_vp, _vp, _vp, _sz, _sz, _sz, _vp],
    "cxg_gelu_exact": [_vp, _vp, _sz, _vp],
    "cxg_gelu_exact_deriv": [_vp, _vp, _sz, _vp],
    "cxg_ffn_workspace_size": [_sz] * 3,
    "cxg_ffn_fwd": [_vp] * 6 + [_sz] * 3 + [_vp, _sz, _vp],
    "cxg_ffn_bwd": [_vp] * 9 + [_sz] * 3 + [_vp, _sz, _vp],
    "cxg_rope_fwd": [_vp, _vp, _sz, _sz, _sz, _sz, _vp],
    "cxg_rope_bwd": [_vp, _vp, _sz, _sz, _sz, _sz, _vp],
    "cxg_prof_enable": [ctypes.c_int],
    "cxg_prof_reset": [],
    "cxg_prof_query": [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                       ctypes.POINTER(ctypes.c_int)],
}
_RESTYPES = {
    "cxg_status_str": ctypes.c_char_p,
    "cxg_version": ctypes.c_char_p,
    "cxg_mha_bwd_workspace_size": ctypes.c_size_t,
    "cxg_lin_ctx_size": ctypes.c_size_t,
    "cxg_gpt_attn_bwd_workspace_size": ctypes.c_size_t,
    "cxg_ffn_workspace_size": ctypes.c_size_t,
    "cxg_prof_enable": None,
    "cxg_prof_reset": None,
}

_lib = None


class CxgError(RuntimeError):
    def __init__(self, fn, status, hip_err):
        self.status = status
        self.hip_error = hip_err
        msg = lib().cxg_status_str(status).decode()
        super().__init__(f"{fn} failed: status {status} ({msg}), hip error {hip_err}")


def lib():
    """Load the library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built: run __graft_entry__.build() or "
                               f"make -C {_HERE}")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            if not hasattr(L, name):
                continue  # reported by missing_symbols(); calling it raises
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, ctypes.c_int)
        _lib = L
    return _lib


def missing_symbols():
    """Entry points of the binding table that the built library lacks."""
    L = lib()
    return [n for n in SIGNATURES if not hasattr(L, n)]


def _ptr(t):
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is not None:
        return ctypes.c_void_p(stream)
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _call(name, *args):
    st = getattr(lib(), name)(*args)
    if st != CXG_OK:
        raise CxgError(name, st, lib().cxg_last_hip_error())
    return st


def call_status(name, *args):
    """Raw call returning the status code (for error-path tests)."""
    return getattr(lib(), name)(*args)


# ------------------------------------------------------------------ softmax MHA
def mha_fwd(Q, K, V, O, B, S, H, Dh, lse=None, stream=None):
    _call("cxg_mha_fwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(lse), B, S, H, Dh,
          _stream(stream))


def mha_bwd(Q, K, V, O, dO, dQ, dK, dV, B, S, H, Dh, lse=None, workspace=None, stream=None):
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _call("cxg_mha_bwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(lse), _ptr(dQ),
          _ptr(dK), _ptr(dV), B, S, H, Dh, _ptr(workspace), ws_bytes, _stream(stream))


def mha_bwd_noalloc(Q, K, V, O, dO, dQ, dK, dV, B, S, H, Dh, lse=None, stream=None):
    """cxg_mha_bwd without a workspace or any allocation (static device scratch)."""
    _call("cxg_mha_bwd_noalloc", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(lse),
          _ptr(dQ), _ptr(dK), _ptr(dV), B, S, H, Dh, _stream(stream))


MHA_BWD_NOALLOC_MAX_ROWS = 1 << 19


def mha_rope_fwd(Q, K, V, O, B, S, H, Dh, lse=None, stream=None):
    _call("cxg_mha_rope_fwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(lse), B, S, H, Dh,
          _stream(stream))


def mha_rope_bwd(Q, K, V, O, dO, dQ, dK, dV, B, S, H, Dh, lse=None, workspace=None,
                 stream=None):
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _call("cxg_mha_rope_bwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(lse),
          _ptr(dQ), _ptr(dK), _ptr(dV), B, S, H, Dh, _ptr(workspace), ws_bytes,
          _stream(stream))


def mha_bwd_workspace_size(B, S, H, Dh):
    return lib().cxg_mha_bwd_workspace_size(B, S, H, Dh)


# ------------------------------------------------------------------ GPT's attention (H = 1)
def wait_timeouts(stream=None):
    """Count of the backward's in-kernel waits that gave up on this stream (0 normally)."""
    n = ctypes.c_uint(0)
    _call("cxg_wait_timeouts", _stream(stream), ctypes.byref(n))
    return n.value


def release_scratch(stream=None):
    """Free the library's cached scratch buffer of (current device, stream)."""
    _call("cxg_release_scratch", _stream(stream))


def gpt_attn_fwd(Q, K, V, O, B, S, E, lse=None, stream=None):
    _call("cxg_gpt_attn_fwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(lse), B, S, E,
          _stream(stream))


def gpt_attn_bwd(Q, K, V, O, dO, dQ, dK, dV, B, S, E, lse=None, workspace=None, stream=None):
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _call("cxg_gpt_attn_bwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(lse), _ptr(dQ),
          _ptr(dK), _ptr(dV), B, S, E, _ptr(workspace), nbytes, _stream(stream))


# ------------------------------------------------------------------ ELU+1, two_stage API
def kattn_fwd(Q, K, V, O, den, zc, S_buf, z_buf, B, S, D, E, stream=None):
    _call("cxg_kattn_fwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(den), _ptr(zc),
          _ptr(S_buf), _ptr(z_buf), B, S, D, E, _stream(stream))


def kattn_bwd_step1(O, dO, den, dnum, dden, N, E, stream=None):
    _call("cxg_kattn_bwd_step1", _ptr(O), _ptr(dO), _ptr(den), _ptr(dnum), _ptr(dden), N, E,
          _stream(stream))


def kattn_bwd_dQ(K, V, dnum, dden, zc, Q, dQ, S_buf, B, S, D, E, stream=None):
    _call("cxg_kattn_bwd_dQ", _ptr(K), _ptr(V), _ptr(dnum), _ptr(dden), _ptr(zc), _ptr(Q),
          _ptr(dQ), _ptr(S_buf), B, S, D, E, _stream(stream))


def kattn_bwd_dKdV(Q, K, V, dnum, dden, dK, dV, B, S, D, E, stream=None):
    _call("cxg_kattn_bwd_dKdV", _ptr(Q), _ptr(K), _ptr(V), _ptr(dnum), _ptr(dden), _ptr(dK),
          _ptr(dV), B, S, D, E, _stream(stream))


def kattn_bwd(Q, K, V, O, dO, den, dQ, dK, dV, B, S, D, E, ctx=None, stream=None):
    """Fused step1 + dQ + dKdV (no z_cache, no dnum/dden round trip); ctx from kattn_fwd_ctx."""
    _call("cxg_kattn_bwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(den), _ptr(ctx),
          _ptr(dQ), _ptr(dK), _ptr(dV), B, S, D, E, _stream(stream))


def lin_ctx_size(B, S, D, E):
    """Bytes of the forward-to-backward context of the fused pair (0: not used)."""
    return lib().cxg_lin_ctx_size(B, S, D, E)


def kattn_fwd_ctx(Q, K, V, O, den, ctx, B, S, D, E, stream=None):
    nbytes = 0 if ctx is None else ctx.numel() * ctx.element_size()
    _call("cxg_kattn_fwd_ctx", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(den), _ptr(ctx), nbytes,
          B, S, D, E, _stream(stream))


def kattn_rope_fwd(Q, K, V, O, den, B, S, D, E, ctx=None, stream=None):
    """Stage 2 with RoPE fused: Q, K unrotated (rotated over width D as loaded)."""
    nbytes = 0 if ctx is None else ctx.numel() * ctx.element_size()
    _call("cxg_kattn_rope_fwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(den), _ptr(ctx), nbytes,
          B, S, D, E, _stream(stream))


def kattn_rope_bwd(Q, K, V, O, dO, den, dQ, dK, dV, B, S, D, E, ctx=None, stream=None):
    """Backward of kattn_rope_fwd: dQ, dK with respect to the unrotated Q, K."""
    _call("cxg_kattn_rope_bwd", _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(den),
          _ptr(ctx), _ptr(dQ), _ptr(dK), _ptr(dV), B, S, D, E, _stream(stream))


# ------------------------------------------------------------------ linear_cuda API
def lin_fwd(Qp, Kp, V, O, den, zc, S_buf, z_buf, B, S, D, E, stream=None):
    _call("cxg_lin_fwd", _ptr(Qp), _ptr(Kp), _ptr(V), _ptr(O), _ptr(den), _ptr(zc),
          _ptr(S_buf), _ptr(z_buf), B, S, D, E, _stream(stream))


def lin_bwd_step1(O, dO, den, dnum, dden, N, E, stream=None):
    _call("cxg_lin_bwd_step1", _ptr(O), _ptr(dO), _ptr(den), _ptr(dnum), _ptr(dden), N, E,
          _stream(stream))


def lin_bwd_dQ(Kp, V, dnum, dden, zc, dQp, S_buf, B, S, D, E, stream=None):
    _call("cxg_lin_bwd_dQ", _ptr(Kp), _ptr(V), _ptr(dnum), _ptr(dden), _ptr(zc), _ptr(dQp),
          _ptr(S_buf), B, S, D, E, _stream(stream))


def lin_bwd_dKdV(Qp, Kp, V, dnum, dden, dKp, dV, B, S, D, E, stream=None):
    _call("cxg_lin_bwd_dKdV", _ptr(Qp), _ptr(Kp), _ptr(V), _ptr(dnum), _ptr(dden), _ptr(dKp),
          _ptr(dV), B, S, D, E, _stream(stream))


def lin_bwd(Qp, Kp, V, O, dO, den, dQp, dKp, dV, B, S, D, E, ctx=None, stream=None):
    """Fused step1 + dQ + dKdV of the linear_cuda API; ctx from lin_fwd_ctx."""
    _call("cxg_lin_bwd", _ptr(Qp), _ptr(Kp), _ptr(V), _ptr(O), _ptr(dO), _ptr(den), _ptr(ctx),
          _ptr(dQp), _ptr(dKp), _ptr(dV), B, S, D, E, _stream(stream))


def lin_fwd_ctx(Qp, Kp, V, O, den, ctx, B, S, D, E, stream=None):
    nbytes = 0 if ctx is None else ctx.numel() * ctx.element_size()
    _call("cxg_lin_fwd_ctx", _ptr(Qp), _ptr(Kp), _ptr(V), _ptr(O), _ptr(den), _ptr(ctx), nbytes,
          B, S, D, E, _stream(stream))


def lin_elu_fwd(Xq, Xk, V, O, den, ctx, B, S, E, stream=None):
    """LinearGPT attention forward with phi_elu fused (raw projections in)."""
    nbytes = 0 if ctx is None else ctx.numel() * ctx.element_size()
    _call("cxg_lin_elu_fwd", _ptr(Xq), _ptr(Xk), _ptr(V), _ptr(O), _ptr(den), _ptr(ctx), nbytes,
          B, S, E, _stream(stream))


def lin_elu_bwd(Xq, Xk, V, O, dO, den, dXq, dXk, dV, B, S, E, ctx=None, stream=None):
    """LinearGPT attention backward: step1 + dQ + dKdV + phi_elu_backward, fused."""
    _call("cxg_lin_elu_bwd", _ptr(Xq), _ptr(Xk), _ptr(V), _ptr(O), _ptr(dO), _ptr(den),
          _ptr(ctx), _ptr(dXq), _ptr(dXk), _ptr(dV), B, S, E, _stream(stream))


def lin_hexp_fwd(Xq, Xk, V, O, den, ctx, B, S, E, stream=None):
    """Hadamard+Exp attention forward with the feature map fused (raw projections in)."""
    nbytes = 0 if ctx is None else ctx.numel() * ctx.element_size()
    _call("cxg_lin_hexp_fwd", _ptr(Xq), _ptr(Xk), _ptr(V), _ptr(O), _ptr(den), _ptr(ctx), nbytes,
          B, S, E, _stream(stream))


def lin_hexp_bwd(Xq, Xk, V, O, dO, den, dXq, dXk, dV, B, S, E, ctx=None, stream=None):
    """Hadamard+Exp attention backward: step1 + dQ + dKdV + the feature map's backward, fused."""
    _call("cxg_lin_hexp_bwd", _ptr(Xq), _ptr(Xk), _ptr(V), _ptr(O), _ptr(dO), _ptr(den),
          _ptr(ctx), _ptr(dXq), _ptr(dXk), _ptr(dV), B, S, E, _stream(stream))


def gelu_exact(A, C, n, stream=None):
    _call("cxg_gelu_exact", _ptr(A), _ptr(C), n, _stream(stream))


def gelu_exact_deriv(A, C, n, stream=None):
    _call("cxg_gelu_exact_deriv", _ptr(A), _ptr(C), n, _stream(stream))


def ffn_workspace_size(M, E, F):
    return lib().cxg_ffn_workspace_size(M, E, F)


def ffn_fwd(X, W1, W2, pre, act, Y, M, E, F, workspace=None, stream=None):
    """Expander FFN forward: pre = X W1^T (if pre is not None), act = gelu(pre),
    Y = act W2^T."""
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _call("cxg_ffn_fwd", _ptr(X), _ptr(W1), _ptr(W2), _ptr(pre), _ptr(act), _ptr(Y), M, E, F,
          _ptr(workspace), nbytes, _stream(stream))


def ffn_bwd(X, W1, W2, act, G, dY, dX, dW1, dW2, M, E, F, workspace=None, stream=None):
    """Expander FFN backward: dact = (dY W2) * gelu'(G); dW2 += dY^T act;
    dX = dact W1; dW1 += dact^T X."""
    nbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    _call("cxg_ffn_bwd", _ptr(X), _ptr(W1), _ptr(W2), _ptr(act), _ptr(G), _ptr(dY), _ptr(dX),
          _ptr(dW1), _ptr(dW2), M, E, F, _ptr(workspace), nbytes, _stream(stream))


def phi_elu_fwd(x, phi, N, D, E, stream=None):
    _call("cxg_phi_elu_fwd", _ptr(x), _ptr(phi), N, D, E, _stream(stream))


def phi_elu_bwd(dphi, x, dx, N, D, E, stream=None):
    _call("cxg_phi_elu_bwd", _ptr(dphi), _ptr(x), _ptr(dx), N, D, E, _stream(stream))


def phi_hexp_fwd(x, phi, N, D, E, stream=None):
    _call("cxg_phi_hexp_fwd", _ptr(x), _ptr(phi), N, D, E, _stream(stream))


def phi_hexp_bwd(dphi, x, dx, N, D, E, stream=None):
    _call("cxg_phi_hexp_bwd", _ptr(dphi), _ptr(x), _ptr(dx), N, D, E, _stream(stream))


# ------------------------------------------------------------------ RoPE
def rope_fwd(Q, K, B, S, D, head_dim, stream=None):
    _call("cxg_rope_fwd", _ptr(Q), _ptr(K), B, S, D, head_dim, _stream(stream))


def rope_bwd(dQ, dK, B, S, D, head_dim, stream=None):
    _call("cxg_rope_bwd", _ptr(dQ), _ptr(dK), B, S, D, head_dim, _stream(stream))


# ------------------------------------------------------------------ timing hook
def prof_enable(on=True):
    lib().cxg_prof_enable(1 if on else 0)


def prof_reset():
    lib().cxg_prof_reset()


def prof_query(name):
    """(total_ms, count) of the kernel launches recorded under `name`."""
    tot = ctypes.c_double(0.0)
    n = ctypes.c_int(0)
    lib().cxg_prof_query(name.encode(), ctypes.byref(tot), ctypes.byref(n))
    return tot.value, n.value
