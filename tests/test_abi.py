"""CPU checks of the C ABI boundary (no GPU calls).

The HIP library must load, export every entry point include/*.h declares,
and the ctypes binding must know all of them; argument checks that fail
before any HIP call (status codes) are exercised with NULL device pointers.
"""
import glob
import os
import re
import subprocess

import pytest

import cxxgpt_attn as cx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(cxg_[A-Za-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    for n in ("cxg_mha_fwd", "cxg_mha_bwd", "cxg_kattn_fwd", "cxg_kattn_bwd_step1",
              "cxg_kattn_bwd_dQ", "cxg_kattn_bwd_dKdV", "cxg_lin_fwd", "cxg_lin_bwd_step1",
              "cxg_lin_bwd_dQ", "cxg_lin_bwd_dKdV", "cxg_phi_elu_fwd", "cxg_phi_elu_bwd",
              "cxg_phi_hexp_fwd", "cxg_phi_hexp_bwd"):
        assert n in names, n


def test_library_exports_every_declared_symbol():
    L = cx.lib()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(L, n)]
    assert not missing, missing
    assert not cx.missing_symbols()
    out = subprocess.run(["nm", "-D", "--defined-only", cx.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (cxg_[A-Za-z0-9_]+)", out))
    assert declared_symbols() <= exported


def test_binding_covers_header():
    assert declared_symbols() <= set(cx.SIGNATURES)


def test_status_strings_and_version():
    L = cx.lib()
    assert L.cxg_status_str(cx.CXG_OK) == b"ok"
    assert b"256" in L.cxg_status_str(cx.CXG_ERR_HEAD_DIM)
    assert L.cxg_version().startswith(b"cxxgpt-attn")


@pytest.mark.parametrize("call,args,want", [
    # Dh > 256 is rejected before any launch (the reference aborts,
    # two_stage_cuda_kernels.cu:316-321)
    ("cxg_mha_fwd", (None, None, None, None, None, 1, 4, 1, 300, None), cx.CXG_ERR_HEAD_DIM),
    ("cxg_mha_fwd", (None, None, None, None, None, 1, 4, 1, 0, None), cx.CXG_ERR_DIMS),
    ("cxg_mha_fwd", (None, None, None, None, None, 1, 4, 1, 64, None), cx.CXG_ERR_NULL),
    ("cxg_mha_fwd", (None, None, None, None, None, 0, 4, 1, 64, None), cx.CXG_OK),
    ("cxg_mha_bwd", (None,) * 9 + (1, 4, 1, 257, None, 0, None), cx.CXG_ERR_HEAD_DIM),
    ("cxg_kattn_fwd", (None,) * 8 + (1, 4, 0, 4, None), cx.CXG_ERR_DIMS),
    ("cxg_kattn_fwd", (None,) * 8 + (1, 4, 4, 4, None), cx.CXG_ERR_NULL),
    ("cxg_kattn_fwd", (None,) * 8 + (0, 4, 4, 4, None), cx.CXG_OK),
    ("cxg_kattn_bwd_step1", (None,) * 5 + (4, 0, None), cx.CXG_ERR_DIMS),
    ("cxg_kattn_bwd_step1", (None,) * 5 + (0, 4, None), cx.CXG_OK),
    ("cxg_lin_bwd_dKdV", (None,) * 7 + (1, 4, 4, 4, None), cx.CXG_ERR_NULL),
    ("cxg_phi_hexp_fwd", (None, None, 2, 64, 32, None), cx.CXG_ERR_DIMS),
    ("cxg_phi_elu_fwd", (None, None, 2, 4, 8, None), cx.CXG_ERR_DIMS),
    # the allocation-free backward's capacity check precedes its pointer checks
    ("cxg_mha_bwd_noalloc", (None,) * 9 + (1, cx.MHA_BWD_NOALLOC_MAX_ROWS + 1, 1, 64, None),
     cx.CXG_ERR_WORKSPACE),
    ("cxg_mha_bwd_noalloc", (None,) * 9 + (1, cx.MHA_BWD_NOALLOC_MAX_ROWS, 1, 64, None),
     cx.CXG_ERR_NULL),
])
def test_argument_checks_without_gpu(call, args, want):
    assert cx.call_status(call, *args) == want


ERR_BIN = os.path.join(ROOT, "tests", "cpp", "dropin_errors")


@pytest.fixture(scope="module")
def dropin_errors():
    """tests/cpp/dropin_errors, built by build() (made here if missing)."""
    if not os.path.exists(ERR_BIN):
        subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "cpp"), ERR_BIN], check=True,
                       capture_output=True)
    return ERR_BIN


@pytest.mark.parametrize("mode,fn,dh", [("abort_fwd", "fused_mha_fwd", 300),
                                        ("abort_bwd", "fused_mha_bwd", 257)])
def test_dropin_aborts_above_256(dropin_errors, mode, fn, dh):
    """The C++ wrappers keep the reference's fprintf + std::abort() for head_dim
    > 256 (two_stage_cuda_kernels.cu:316-321, :867-872); the check happens
    before any HIP call, so this runs without a GPU."""
    r = subprocess.run([dropin_errors, mode], capture_output=True, text=True, timeout=60)
    assert r.returncode == -6, (r.returncode, r.stdout, r.stderr)   # SIGABRT
    assert f"two_stage_cuda::{fn}: head_dim {dh} > 256" in r.stderr
    assert "returned without aborting" not in r.stdout


@pytest.mark.parametrize("mode", ["throw_null", "macros"])
def test_dropin_throws_and_shim_macros(dropin_errors, mode):
    """Other failures throw std::runtime_error (the reference's CHECK_CUDA_ERROR);
    the stand-in defines TENSORN_CUDA_AVAILABLE and CHECK_CUDA_ERROR."""
    r = subprocess.run([dropin_errors, mode], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert r.stdout.startswith("caught: ")
