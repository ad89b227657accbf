#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Headline step ("c2", the headline metric's configuration): causal softmax MHA forward +
backward, FP32, B=8 H=12 S=256 Dh=64, through the C ABI of
libcxxgpt_attn.so -- cxg_mha_fwd (writes O and the row log-sum-exp) then
cxg_mha_bwd (consumes it); these replace the reference's two_stage_cuda::
fused_mha_fwd / fused_mha_bwd (src/TwoStage/two_stage_gpt.hpp:106, :171).
value = algorithmic TFLOP/s of the step, counting 4*Dh*P (fwd) + 8*Dh*P
(bwd) FLOPs per (b,h) with P = S(S+1)/2 causal pairs; recomputation is not
credited.

Other workloads (run after the headline unless --no-secondary; any one of
them can be made the reported workload with --workload NAME):
  c2legacy  C2 through the legacy signatures (no lse: the backward recomputes it)
  c2dropin  c2legacy with a null workspace (the C++ drop-in wrappers' calls:
            the library's cached per-stream scratch)
  c2graph   c2 captured once in a HIP graph and replayed (not in the default run)
  mhats     TwoStageGPT's stage-1 shape, B32 H64 S256 Dh8, legacy signatures
            (two_stage_train.cpp:168-170); mhatsrope with its RoPE fused
            (cxg_mha_rope_fwd/bwd), mhatsropesep with RoPE as separate passes
  gen1, gen64, gen256
            generate()'s forward at B = 1, S = 1 / 64 / 256, probe heads H8 Dh32
            (two_stage_gpt.hpp:453-470), latency per call
  c3        ELU+1 linear attention fwd+bwd, B' = 96 sequences, S=4096, D=E=64,
            two_stage API chain kernel_attn_fwd -> bwd_step1 -> bwd_dQ ->
            bwd_dKdV; GB/s of compulsory I/O, (12*S*D + 2*S)*4 bytes/sequence
  c3s256    the same at S=256
  c3fused   c3 through the fused pair: cxg_kattn_fwd_ctx (O, den and a segment-
            state context instead of z_cache) -> cxg_kattn_bwd (step1 + dQ + dKdV
            in one pass, prefix state from the context); c3fuseds256 at S=256
  c3lgpt    c3's shape through LinearGPT's block with phi_elu fused as well
            (cxg_lin_elu_fwd -> cxg_lin_elu_bwd on the raw q/k projections)
  c4        Hadamard+Exp linear attention (S=1024) through the linear_cuda API
            (phi_hexp fwd x2, linear fwd/step1/dQ/dKdV, phi_hexp bwd x2)
  c4fused   c4 with the linear part through the fused pair (cxg_lin_fwd_ctx ->
            cxg_lin_bwd) between the feature-map passes
  c4hexp    c4 with the feature map inside the fused pair's kernels
            (cxg_lin_hexp_fwd -> cxg_lin_hexp_bwd on the raw projections)
  c3wide    TwoStageGPT's stage-2 shape, 32 sequences of S256 with D=E=512
            (two_stage_train.cpp:168-170), two_stage API chain; c3widefused
            through the fused pair; lgptwide LinearGPT's shape (8 sequences,
            S256, D=E=512, linear_train.cpp:168-172) through cxg_lin_elu_*
  c3widerope, c3wideropesep
            c3wide's shape with stage 2's RoPE (two_stage_gpt.hpp:113, :160) fused
            into the kernels (cxg_kattn_rope_fwd/bwd) / as separate passes around
            the fused pair; c3rope, c3ropesep the same at C3's S4096 D=E=64 shape
  c5        long-sequence MHA, B2 H12 S4096 Dh64, fwd+bwd
  rope      RoPE fwd + bwd on the stage-1 q/k heads at the C2 shape (in place),
            GB/s of compulsory I/O (each tensor read and written once)
  c2rope    C2 with RoPE fused into the MHA kernels (cxg_mha_rope_fwd/bwd)
  c2ropesep C2 with RoPE as separate passes, the reference's call sequence
  gpt       GPT's attention at its training shape (B8 S256, one head of E=512,
            gpt_train.cpp:139/156): cxg_gpt_attn_fwd -> cxg_gpt_attn_bwd
  gpt768    the same at E=768 (causal score blocks kept in memory)
  gelu      exact GELU + derivative over the q/k/v expander FFN activations at
            the C2 shape (3 x 2048 x 6144 floats; two_stage_gpt.hpp:86-99), GB/s
  ffn       one expander FFN fwd+bwd (X [2048][768], W1 [6144][768], W2
            [768][6144]; two_stage_gpt.hpp:86-89,177-183), six FP32 GEMMs, TFLOP/s
  copy      256 MiB device copy: HBM counter calibration for the profiles

Inputs are synthetic N(0,1) tensors generated on the GPU from fixed seeds and
resident in HBM before timing starts.  Timing: W warmup steps, then K steps
between two HIP events on the launch stream; the reported workload repeats
that window HEADLINE_WINDOWS times back to back and reports the median
window (every window's figure is in `timing`).  The roofline object is
measured live: after the timed region the same steps run again with the
library's timing hook on (each launch records the start and end of its own
dispatch into HIP events on the launch stream), giving each kernel's mean
duration; the dominant kernel's
algorithmic FLOPs (or bytes) per launch divided by that duration is
`achieved`.  The CPU baseline times the C oracle (the restated CPU reference,
test infrastructure) on the host cores over a bounded sample of the same
workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2]
                       [--no-secondary] [--no-cpu] [--cpu-budget SECONDS]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cxx-gpt_amd"))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 MFMA
METRIC = "attn fwd+bwd TFLOP/s (% MFMA peak) B8H12S256D64 fp32; lin-attn HBM GB/s"

# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE, scaled by
# the same counters' reading on a copy kernel of known size; written from the
# committed counter summaries (profiles/).  Key "<workload>/<kernel tag>".
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def mha_flops(B, S, H, Dh, fwd=True, bwd=True):
    P = S * (S + 1) // 2
    return ((4 * Dh * P if fwd else 0) + (8 * Dh * P if bwd else 0)) * B * H


def lin_bytes(Bq, S, D):
    """Compulsory fused I/O of linear attention fwd+bwd (12 S D + 2 S floats/sequence)."""
    return (12 * S * D + 2 * S) * 4 * Bq


def lin_kernel_bytes(Bq, S, D, fused=False):
    """Per-launch bytes each linear-attention entry point must move through its
    own signature: inputs read once, outputs written once.  fused: the forward
    without z_cache and the one-call backward."""
    T, r = Bq * S * D * 4, Bq * S * 4   # one (rows x 64) tensor, one per-row vector
    # quadratic-form kernels (short sequences): the one-call backward is step 1
    # then lin_wide_bwd
    quad = {"lin_step1": 2 * T + r + T + r,      # O, dO, den -> dnum, dden
            "lin_wide_dq": 4 * T + r + T,        # K, V, dnum, dden, Q (phi') -> dQ
            "lin_wide_dkdv": 4 * T + r + 2 * T,  # Q, K, V, dnum, dden -> dK, dV
            "lin_wide_bwd": 4 * T + r + 3 * T}   # Q, K, V, dnum, dden -> dQ, dK, dV
    if fused:
        return {"lin_fwd": 3 * T + T + r,        # Q,K,V -> O, den
                "lin_seqfwd": 3 * T + T + r,     # the same forward in one launch (S <= 256)
                "lin_bwd": 5 * T + r + 3 * T,    # Q,K,V,O,dO, den -> dQ, dK, dV
                "lin_wide_fwd": 3 * T + T + r, **quad}
    return {"lin_fwd": 3 * T + 2 * T + r,        # Q,K,V -> O, z_cache, den
            "lin_seqfwd": 3 * T + 2 * T + r,
            "lin_step1": 2 * T + r + T + r,      # O, dO, den -> dnum, dden
            "lin_dq": 5 * T + r + T,             # K, V, dnum, z_cache, Q, dden -> dQ
            "lin_dkdv": 4 * T + r + 2 * T,       # Q, K, V, dnum, dden -> dK, dV
            "lin_wide_fwd": 3 * T + 2 * T + r, **quad}


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


class Stepper:
    """Pre-bound C-ABI calls, so the timed loop pays one ctypes call per entry point."""

    def __init__(self, lib, calls):
        self.calls = [(getattr(lib, name), name, args) for name, args in calls]

    def __call__(self):
        for f, name, args in self.calls:
            st = f(*args)
            if st != 0:
                raise RuntimeError(f"{name} returned status {st}")


def timed(step, steps, warmup, stream, windows=1, spread=None):
    """ms per step: `windows` back-to-back windows of exactly `steps` steps,
    each bracketed by a synchronize and two HIP events on the launch stream;
    the median window's mean is returned (one window: its mean).  `spread`, a
    list, receives every window's ms per step."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    per = []
    for _ in range(windows):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / steps)
    if spread is not None:
        spread.extend(per)
    return sorted(per)[len(per) // 2]


# Windows of K steps the reported workload is timed over (the median is
# reported): a 20-step window of C2 is about 1 ms, short enough that one
# window can catch a clock ramp or a neighbour's interference.
HEADLINE_WINDOWS = 9


# Seconds of GPU work per secondary workload's timed region and per kernel
# attribution pass: long enough for a sampler polling the GPU every few seconds
# to see it busy, short enough for the whole run to stay within minutes.
SUSTAIN_S = 0.4


def steps_for(ms_per_step, floor, seconds=SUSTAIN_S, cap=20000):
    """Steps that fill about `seconds` of GPU time at ms_per_step (at least floor)."""
    return int(max(floor, min(cap, seconds * 1e3 / max(ms_per_step, 1e-4))))


def attribute(cx, step, steps):
    """Mean device duration (ms) and launch count per kernel tag, from the
    library's timing hook: the launches record their dispatches' start and end
    into HIP events on the launch stream (rocprofv3's kernel trace is the
    cross-check; they agree within about 1%).  `steps`: a count, or
    ("seconds", ms_per_step) for a time-based pass."""
    import torch
    if isinstance(steps, tuple):
        steps = steps_for(steps[1], 10)
    torch.cuda.synchronize()
    cx.prof_reset()
    cx.prof_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    cx.prof_enable(False)
    out = {}
    for n in ("mha_fwd", "mha_stats", "mha_bwd_prep", "mha_bwd", "mha_nar_fwd", "mha_nar_stats",
              "mha_nar_bwd", "mha_nar_rope_fwd", "mha_nar_rope_bwd", "lin_agg", "lin_scan",
              "lin_seqrec", "lin_seqfwd", "lin_fwd", "lin_step1", "lin_dq", "lin_dkdv", "lin_bagg", "lin_bscan", "lin_bwd",
              "lin_wide_fwd", "lin_wide_fin", "lin_wide_dq", "lin_wide_dkdv", "lin_wide_bwd",
              "lin_wide_state", "lin_qs_feat", "lin_qs_score", "lin_qs_bscore", "lin_qs_out",
              "lin_qs_grad", "lin_qs_zc", "gpt_qs_score", "gpt_qs_softmax", "gpt_qs_out",
              "gpt_qs_bscore", "gpt_qs_grad",
              "phi_hexp_fwd", "phi_hexp_bwd", "lin_rope_feat",
              "rope_fwd", "rope_bwd", "mha_rope_fwd", "mha_rope_bwd", "mha_wide_fwd",
              "mha_wide_stats", "mha_wide_bwd", "mha_wide_merge", "mha_wide_bsum", "gelu", "gelu_deriv", "ffn_gemm",
              "ffn_fixup"):
        tot, cnt = cx.prof_query(n)
        if cnt:
            out[n] = (tot / cnt, cnt / steps)
    cx.prof_reset()
    return out


def load_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    # the GPU box grants one GPU's share of the host (OMP_NUM_THREADS = 16 there)
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


# ---------------------------------------------------------------------------- workloads
class Ctx:
    def __init__(self, cx, torch, steps, warmup):
        self.cx, self.torch, self.steps, self.warmup = cx, torch, steps, warmup
        self.dev = torch.device("cuda:0")
        self.stream = torch.cuda.current_stream(self.dev)
        self.sp = ctypes.c_void_p(self.stream.cuda_stream)
        self.traffic = load_traffic()
        self.windows, self.spread = 1, None   # set for the reported workload only

    def randn(self, g, *shape, std=1.0):
        t = self.torch.randn(*shape, device=self.dev, generator=g)
        return t * std if std != 1.0 else t

    def gen(self, seed):
        g = self.torch.Generator(device=self.dev)
        g.manual_seed(seed)
        return g

    def empty(self, *shape):
        return self.torch.empty(*shape, device=self.dev)


class GraphStep:
    """A step captured once into a HIP graph (torch.cuda.CUDAGraph on a side
    stream) and replayed: the same kernels with their launch overheads and
    inter-kernel gaps reduced, as a caller that captures its training step
    runs them.  `make(stream_handle)` builds the step's C-ABI calls on the
    capture stream."""

    def __init__(self, torch, make):
        self.g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            warm = make(ctypes.c_void_p(s.cuda_stream))
            warm()   # scratch allocations and first-call set-up happen outside capture
        torch.cuda.synchronize()
        with torch.cuda.graph(self.g, stream=s):
            make(ctypes.c_void_p(s.cuda_stream))()
        torch.cuda.synchronize()

    def __call__(self):
        self.g.replay()


def _mha(c, name, B, S, H, Dh, use_lse, seed, steps, warmup, rope=None, fwd_only=False,
         null_ws=False, graph=False):
    """rope: None (plain MHA), "fused" (cxg_mha_rope_fwd/bwd) or "separate"
    (cxg_rope_fwd, cxg_mha_fwd, cxg_mha_bwd, cxg_rope_bwd: the reference's call
    sequence at two_stage_gpt.hpp:102-106, :171-174).  fwd_only: the forward
    alone (inference: generate() re-runs it per token, two_stage_gpt.hpp:453-470)."""
    g = c.gen(seed)
    shp = (B * S, H * Dh)
    Q, K, V, dO = [c.randn(g, *shp) for _ in range(4)]
    O, dQ, dK, dV = c.empty(*shp), c.empty(*shp), c.empty(*shp), c.empty(*shp)
    lse = c.empty(B * H * S) if use_lse else None
    ws_bytes = c.cx.mha_bwd_workspace_size(B, S, H, Dh)
    ws = c.empty(max(1, ws_bytes // 4))
    if null_ws:   # as the drop-in wrappers call it: stream-ordered scratch per call
        ws, ws_bytes = None, 0
    P = _ptr
    fwd, bwd = ("cxg_mha_rope_fwd", "cxg_mha_rope_bwd") if rope == "fused" else \
        ("cxg_mha_fwd", "cxg_mha_bwd")
    calls = [
        (fwd, (P(Q), P(K), P(V), P(O), P(lse), B, S, H, Dh, c.sp)),
        (bwd, (P(Q), P(K), P(V), P(O), P(dO), P(lse), P(dQ), P(dK), P(dV),
               B, S, H, Dh, P(ws), ws_bytes, c.sp)),
    ]
    if rope == "separate":
        calls = [("cxg_rope_fwd", (P(Q), P(K), B, S, H * Dh, Dh, c.sp))] + calls + \
                [("cxg_rope_bwd", (P(dQ), P(dK), B, S, H * Dh, Dh, c.sp))]
    if fwd_only:
        calls = calls[:1]
    step = Stepper(c.cx.lib(), calls)
    eager = step
    if graph:
        def make(sp):
            return Stepper(c.cx.lib(), [(n, tuple(sp if a is c.sp else a for a in args))
                                        for n, args in calls])
        step = GraphStep(c.torch, make)
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    # per-kernel durations from the eager calls (the hook's events are not
    # recorded inside a graph)
    att = attribute(c.cx, eager, ("seconds", ms))
    flops = mha_flops(B, S, H, Dh, bwd=not fwd_only)
    value = flops / (ms * 1e-3) / 1e12
    kflops = {"mha_fwd": mha_flops(B, S, H, Dh, bwd=False),
              "mha_bwd": mha_flops(B, S, H, Dh, fwd=False),
              "mha_nar_fwd": mha_flops(B, S, H, Dh, bwd=False),
              "mha_nar_bwd": mha_flops(B, S, H, Dh, fwd=False),
              "mha_nar_rope_fwd": mha_flops(B, S, H, Dh, bwd=False),
              "mha_nar_rope_bwd": mha_flops(B, S, H, Dh, fwd=False),
              "mha_rope_fwd": mha_flops(B, S, H, Dh, bwd=False),
              "mha_rope_bwd": mha_flops(B, S, H, Dh, fwd=False)}
    dom = max((k for k in att if k in kflops), key=lambda k: att[k][0])
    ach = kflops[dom] / (att[dom][0] * 1e-3) / 1e12
    roof = {"bound": "mfma", "kernel": dom, "achieved": round(ach, 3),
            "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(ach / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": c.traffic.get(f"{name}/{dom}"),
            "flops_per_launch": kflops[dom],
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()}}
    return dict(value=value, unit="TFLOP/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: causal softmax MHA "
                                    + ("forward only (" if fwd_only else "fwd+bwd (")
                                    + ("replayed as a captured HIP graph: " if graph else "")
                                    + {None: ("cxg_mha_fwd with lse -> cxg_mha_bwd" if use_lse
                                              else "legacy signatures, no lse" +
                                              (", no workspace (the drop-in wrappers' call)"
                                               if null_ws else ", caller workspace")),
                                       "fused": "RoPE fused: cxg_mha_rope_fwd -> "
                                                "cxg_mha_rope_bwd",
                                       "separate": "RoPE as separate passes: cxg_rope_fwd, "
                                                   "cxg_mha_fwd, cxg_mha_bwd, cxg_rope_bwd"}[rope]
                                    + ")",
                        "B": B, "H": H, "S": S, "Dh": Dh, "flops_per_step": flops,
                        "us_per_step": round(ms * 1e3, 2)},
                frac=value / FP32_MFMA_PEAK_TFLOPS,
                cpu_inputs=(Q, K, V, dO, B, S, H, Dh))


def _gelu(c, name, rows, cols, seed, steps, warmup):
    """Exact GELU and its derivative as the two-stage block's q/k/v expander
    FFNs apply them (two_stage_gpt.hpp:86-99 forward, :177-195 backward):
    per expander gelu_exact(f, act) then gelu_exact_deriv(act, g), on three
    separate [rows, cols] tensors, so the 450 MiB footprint exceeds the
    last-level cache.  GB/s of compulsory I/O (each call reads and writes its
    tensor once)."""
    g = c.gen(seed)
    n = rows * cols
    P = _ptr
    calls = []
    keep = []
    for _ in range(3):
        f = c.randn(g, n)
        act, gd = c.empty(n), c.empty(n)
        keep += [f, act, gd]
        calls += [("cxg_gelu_exact", (P(f), P(act), n, c.sp)),
                  ("cxg_gelu_exact_deriv", (P(act), P(gd), n, c.sp))]
    step = Stepper(c.cx.lib(), calls)
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    total = len(calls) * 2 * n * 4
    value = total / (ms * 1e-3) / 1e9
    kb = {"gelu": 2 * n * 4, "gelu_deriv": 2 * n * 4}
    dom = max((k for k in att if k in kb), key=lambda k: att[k][0])
    ach = kb[dom] / (att[dom][0] * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": c.traffic.get(f"{name}/{dom}"), "bytes_per_launch": kb[dom],
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()}}
    return dict(value=value, unit="GB/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: exact GELU + derivative over the q/k/v expander "
                                    f"FFN activations (two_stage_gpt.hpp:86-99, :177-195) at "
                                    f"the C2 shape",
                        "rows": rows, "cols": cols, "tensors": 3, "bytes_per_step": total},
                frac=value / HBM_PEAK_GBS, cpu_inputs=None)


def _ffn(c, name, M, E, F, seed, steps, warmup):
    """One expander FFN forward + backward (two_stage_gpt.hpp:86-89, :177-183)
    through cxg_ffn_fwd / cxg_ffn_bwd: six FP32 GEMMs of 2*M*E*F flops each,
    GELU in the first's epilogue and gelu' in the first backward one's."""
    import torch
    g = c.gen(seed)
    X = c.randn(g, M * E)
    W1 = c.randn(g, F * E, std=(2.0 / E) ** 0.5)
    W2 = c.randn(g, E * F, std=(2.0 / F) ** 0.5)
    dY = c.randn(g, M * E, std=1.0 / M)
    act, Y = c.empty(M * F), c.empty(M * E)
    dX = c.empty(M * E)
    dW1 = torch.zeros(F * E, device=X.device)
    dW2 = torch.zeros(E * F, device=X.device)
    nb = c.cx.lib().cxg_ffn_workspace_size(M, E, F)
    ws = c.empty(max(nb, 4) // 4)
    P = _ptr
    step = Stepper(c.cx.lib(), [
        ("cxg_ffn_fwd", (P(X), P(W1), P(W2), None, P(act), P(Y), M, E, F, P(ws), nb, c.sp)),
        ("cxg_ffn_bwd", (P(X), P(W1), P(W2), P(act), P(act), P(dY), P(dX), P(dW1), P(dW2),
                         M, E, F, P(ws), nb, c.sp))])
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    flops = 12.0 * M * E * F
    value = flops / (ms * 1e-3) / 1e12
    per_launch = 2.0 * M * E * F
    ach = per_launch / (att["ffn_gemm"][0] * 1e-3) / 1e12
    roof = {"bound": "mfma", "kernel": "ffn_gemm", "achieved": round(ach, 2),
            "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(ach / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": c.traffic.get(f"{name}/ffn_gemm"), "flops_per_launch": per_launch,
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()},
            "launches_per_step": {k: round(v[1], 2) for k, v in att.items()}}
    return dict(value=value, unit="TFLOP/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: one expander FFN (Linear -> exact GELU -> Linear, "
                                    f"no bias) forward + backward at the C2 shape, "
                                    f"two_stage_gpt.hpp:86-89,177-183",
                        "rows": M, "n_embd": E, "hidden": F, "flops_per_step": flops},
                frac=value / FP32_MFMA_PEAK_TFLOPS, cpu_inputs=None)


def _gpt(c, name, B, S, E, seed, steps, warmup):
    """GPT's attention (one head over the embedding) through cxg_gpt_attn_fwd
    (with lse) -> cxg_gpt_attn_bwd: the reference GPT training shape."""
    g = c.gen(seed)
    N = B * S
    Q, K, V, dO = [c.randn(g, N, E) for _ in range(4)]
    O, dQ, dK, dV = c.empty(N, E), c.empty(N, E), c.empty(N, E), c.empty(N, E)
    lse = c.empty(B * S)
    ws_bytes = c.cx.lib().cxg_gpt_attn_bwd_workspace_size(B, S, E)
    ws = c.empty(max(1, ws_bytes // 4))
    P = _ptr
    step = Stepper(c.cx.lib(), [
        ("cxg_gpt_attn_fwd", (P(Q), P(K), P(V), P(O), P(lse), B, S, E, c.sp)),
        ("cxg_gpt_attn_bwd", (P(Q), P(K), P(V), P(O), P(dO), P(lse), P(dQ), P(dK), P(dV),
                              B, S, E, P(ws), ws_bytes, c.sp)),
    ])
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    flops = mha_flops(B, S, 1, E)
    value = flops / (ms * 1e-3) / 1e12
    kflops = {"mha_wide_fwd": mha_flops(B, S, 1, E, bwd=False),
              "mha_wide_bwd": mha_flops(B, S, 1, E, fwd=False),
              "mha_fwd": mha_flops(B, S, 1, E, bwd=False),
              "mha_bwd": mha_flops(B, S, 1, E, fwd=False),
              # E > 512: each GEMM launch is one S x S x E product for every
              # sequence of a group (as many as keep two S x S score
              # matrices per sequence within 2^25 floats), credited with its
              # causal half (S^2 E of the 2 S^2 E executed)
              "ffn_gemm": 1.0 * min(B, max(1, (1 << 25) // (2 * S * S))) * S * S * E}
    if any(k.startswith("gpt_qs") for k in att):
        # causal score blocks: credit per step (P = S(S+1)/2 causal pairs per
        # sequence): QK^T and PV forward, dP (S recomputed, not credited) and
        # dQ, dK, dV backward
        P2 = S * (S + 1) // 2 * B * 2 * E
        roof = wide_roofline(c, name, att, {"gpt_qs_score": P2, "gpt_qs_out": P2,
                                            "gpt_qs_bscore": P2, "gpt_qs_grad": 3 * P2})
    else:
        dom = max((k for k in att if k in kflops), key=lambda k: att[k][0])
        ach = kflops[dom] / (att[dom][0] * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": dom, "achieved": round(ach, 3),
                "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(ach / FP32_MFMA_PEAK_TFLOPS, 4),
                "traffic": c.traffic.get(f"{name}/{dom}"), "flops_per_launch": kflops[dom],
                "kernel_ms": {k: round(v[0], 5) for k, v in att.items()}}
    return dict(value=value, unit="TFLOP/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: GPT attention (one head over the embedding, "
                                    "gpt_gpt.hpp:365-438) via cxg_gpt_attn_fwd -> "
                                    "cxg_gpt_attn_bwd",
                        "B": B, "S": S, "E": E, "flops_per_step": flops},
                frac=value / FP32_MFMA_PEAK_TFLOPS, cpu_inputs=None)


def _kattn(c, name, Bq, S, D, seed, steps, warmup, fused=False, lgpt=False):
    """fused: the fused pair (context-writing forward, one-call backward);
    otherwise the reference's four-call chain.  lgpt: LinearGPT's block with
    phi_elu fused too (cxg_lin_elu_fwd / _bwd on the raw projections)."""
    g = c.gen(seed)
    E, N = D, Bq * S
    Q, K, V, dO = c.randn(g, N, D), c.randn(g, N, D), c.randn(g, N, E), c.randn(g, N, E)
    O, den = c.empty(N, E), c.empty(N)
    dQ, dK, dV = c.empty(N, D), c.empty(N, D), c.empty(N, E)
    P = _ptr
    if lgpt:
        nctx = c.cx.lin_ctx_size(Bq, S, D, E)
        ctx = c.empty(max(1, nctx // 4))
        step = Stepper(c.cx.lib(), [
            ("cxg_lin_elu_fwd", (P(Q), P(K), P(V), P(O), P(den), P(ctx), nctx, Bq, S, E, c.sp)),
            ("cxg_lin_elu_bwd", (P(Q), P(K), P(V), P(O), P(dO), P(den), P(ctx), P(dQ), P(dK),
                                 P(dV), Bq, S, E, c.sp)),
        ])
    elif fused:
        nctx = c.cx.lin_ctx_size(Bq, S, D, E)
        ctx = c.empty(max(1, nctx // 4))
        step = Stepper(c.cx.lib(), [
            ("cxg_kattn_fwd_ctx", (P(Q), P(K), P(V), P(O), P(den), P(ctx), nctx, Bq, S, D, E,
                                   c.sp)),
            ("cxg_kattn_bwd", (P(Q), P(K), P(V), P(O), P(dO), P(den), P(ctx), P(dQ), P(dK),
                               P(dV), Bq, S, D, E, c.sp)),
        ])
    else:
        zc, dnum, dden = c.empty(N, D), c.empty(N, E), c.empty(N)
        step = Stepper(c.cx.lib(), [
            ("cxg_kattn_fwd", (P(Q), P(K), P(V), P(O), P(den), P(zc), None, None, Bq, S, D, E,
                               c.sp)),
            ("cxg_kattn_bwd_step1", (P(O), P(dO), P(den), P(dnum), P(dden), N, E, c.sp)),
            ("cxg_kattn_bwd_dQ", (P(K), P(V), P(dnum), P(dden), P(zc), P(Q), P(dQ), None,
                                  Bq, S, D, E, c.sp)),
            ("cxg_kattn_bwd_dKdV", (P(Q), P(K), P(V), P(dnum), P(dden), P(dK), P(dV),
                                    Bq, S, D, E, c.sp)),
        ])
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    total = lin_bytes(Bq, S, D)
    value = total / (ms * 1e-3) / 1e9
    kb = lin_kernel_bytes(Bq, S, D, fused or lgpt)
    dom = max((k for k in att if k in kb), key=lambda k: att[k][0])
    ach = kb[dom] / (att[dom][0] * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": c.traffic.get(f"{name}/{dom}"), "bytes_per_launch": kb[dom],
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()}}
    return dict(value=value, unit="GB/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: ELU+1 linear attention fwd+bwd, " + (
                            "LinearGPT block, phi_elu fused (cxg_lin_elu_fwd -> cxg_lin_elu_bwd)"
                            if lgpt else
                            "fused pair (cxg_kattn_fwd_ctx -> cxg_kattn_bwd with the context)"
                            if fused else "two_stage API chain (fwd, step1, dQ, dKdV)"),
                        "B_seq": Bq, "S": S, "D": D, "E": E, "bytes_per_step": total},
                frac=value / HBM_PEAK_GBS, cpu_inputs=(Q, K, V, dO, Bq, S, D, E))


def lin_wide_flops(Bq, S, D, E):
    """Algorithmic FLOPs of the quadratic form per kernel, P = S(S+1)/2 causal
    pairs per sequence: forward A = phi(Q)phi(K)^T and A V; dQ needs
    X = dnum V^T and G phi(K); dK, dV need G^T phi(Q) and A^T dnum (A and X
    recomputed there, not credited)."""
    P = S * (S + 1) // 2
    f = 2 * P * (D + E) * Bq
    # per step: the one-workgroup-per-block kernels (one launch of each a step),
    # and the block-score kernels, whose credit is summed over a step's launches
    # (forward: scores A, products A V; backward: X = dnum V^T in the score
    # launches, the three gradient products in the product launches)
    return {"lin_wide_fwd": f, "lin_wide_dq": f, "lin_wide_dkdv": f, "lin_wide_bwd": 2 * f,
            "lin_qs_score": 2 * P * D * Bq, "lin_qs_out": 2 * P * E * Bq,
            "lin_qs_bscore": 2 * P * E * Bq, "lin_qs_grad": (4 * P * D + 2 * P * E) * Bq}


def wide_roofline(c, name, att, kf):
    """MFMA roofline of the quadratic form's dominant kernel tag (most time per
    step): its credited FLOPs per step over its time per step."""
    dom = max((k for k in att if k in kf), key=lambda k: att[k][0] * att[k][1])
    per_step_ms = att[dom][0] * att[dom][1]
    ach = kf[dom] / (per_step_ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": dom, "achieved": round(ach, 3),
            "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(ach / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": c.traffic.get(f"{name}/{dom}"),
            "flops_per_launch": int(round(kf[dom] / att[dom][1])),
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()},
            "launches_per_step": {k: round(v[1], 2) for k, v in att.items() if v[1] != 1}}


def _linwide(c, name, Bq, S, D, seed, steps, warmup, mode):
    """Linear attention with wide heads at the reference's training shapes.
    mode "chain": the two_stage API's four calls (TwoStageGPT stage 2,
    two_stage_gpt.hpp:115-157); "fused": kernel_attn_fwd then the one-call
    backward; "lgpt": LinearGPT's block with phi_elu fused (cxg_lin_elu_*)."""
    g = c.gen(seed)
    E, N = D, Bq * S
    Q, K, V, dO = c.randn(g, N, D), c.randn(g, N, D), c.randn(g, N, E), c.randn(g, N, E)
    O, den = c.empty(N, E), c.empty(N)
    dQ, dK, dV = c.empty(N, D), c.empty(N, D), c.empty(N, E)
    P = _ptr
    # the forward-to-backward context (the block-score path keeps its features
    # and score blocks there; 0 bytes for shapes that write none)
    nctx = c.cx.lin_ctx_size(Bq, S, D, E)
    ctx = c.empty(max(1, nctx // 4)) if nctx else None
    if mode == "lgpt":
        step = Stepper(c.cx.lib(), [
            ("cxg_lin_elu_fwd", (P(Q), P(K), P(V), P(O), P(den), P(ctx), nctx, Bq, S, E, c.sp)),
            ("cxg_lin_elu_bwd", (P(Q), P(K), P(V), P(O), P(dO), P(den), P(ctx), P(dQ), P(dK),
                                 P(dV), Bq, S, E, c.sp)),
        ])
        desc = ("LinearGPT block, phi_elu fused (cxg_lin_elu_fwd -> cxg_lin_elu_bwd with the "
                "context)")
    elif mode == "fused":
        step = Stepper(c.cx.lib(), [
            ("cxg_kattn_fwd_ctx", (P(Q), P(K), P(V), P(O), P(den), P(ctx), nctx, Bq, S, D, E,
                                   c.sp)),
            ("cxg_kattn_bwd", (P(Q), P(K), P(V), P(O), P(dO), P(den), P(ctx), P(dQ), P(dK),
                               P(dV), Bq, S, D, E, c.sp)),
        ])
        desc = "two_stage fused pair (cxg_kattn_fwd_ctx -> cxg_kattn_bwd with the context)"
    else:
        zc, dnum, dden = c.empty(N, D), c.empty(N, E), c.empty(N)
        step = Stepper(c.cx.lib(), [
            ("cxg_kattn_fwd", (P(Q), P(K), P(V), P(O), P(den), P(zc), None, None, Bq, S, D, E,
                               c.sp)),
            ("cxg_kattn_bwd_step1", (P(O), P(dO), P(den), P(dnum), P(dden), N, E, c.sp)),
            ("cxg_kattn_bwd_dQ", (P(K), P(V), P(dnum), P(dden), P(zc), P(Q), P(dQ), None,
                                  Bq, S, D, E, c.sp)),
            ("cxg_kattn_bwd_dKdV", (P(Q), P(K), P(V), P(dnum), P(dden), P(dK), P(dV),
                                    Bq, S, D, E, c.sp)),
        ])
        desc = "two_stage API chain (fwd with z_cache, step1, dQ, dKdV)"
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    total = lin_bytes(Bq, S, D)
    value = total / (ms * 1e-3) / 1e9
    kf = lin_wide_flops(Bq, S, D, E)
    roof = wide_roofline(c, name, att, kf)
    step_flops = 3 * kf["lin_wide_fwd"]
    return dict(value=value, unit="GB/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: ELU+1 linear attention fwd+bwd, wide heads "
                                    f"(quadratic form), {desc}",
                        "B_seq": Bq, "S": S, "D": D, "E": E, "bytes_per_step": total,
                        "algorithmic_flops_per_step": step_flops,
                        "step_tflops": round(step_flops / (ms * 1e-3) / 1e12, 3)},
                frac=value / HBM_PEAK_GBS, cpu_inputs=(Q, K, V, dO, Bq, S, D, E))


def _kattn_rope(c, name, Bq, S, D, seed, steps, warmup, fused):
    """TwoStageGPT's stage 2 with its RoPE (two_stage_gpt.hpp:113-122, :149-160):
    fused, cxg_kattn_rope_fwd -> cxg_kattn_rope_bwd (q, k rotated inside the
    kernels); otherwise RoPE as separate in-place passes around the fused pair
    (cxg_rope_fwd, cxg_kattn_fwd_ctx, cxg_kattn_bwd, cxg_rope_bwd).  GB/s of the
    compulsory linear-attention I/O, as c3."""
    g = c.gen(seed)
    E, N = D, Bq * S
    Q, K, V, dO = c.randn(g, N, D), c.randn(g, N, D), c.randn(g, N, E), c.randn(g, N, E)
    O, den = c.empty(N, E), c.empty(N)
    dQ, dK, dV = c.empty(N, D), c.empty(N, D), c.empty(N, E)
    nctx = c.cx.lin_ctx_size(Bq, S, D, E)
    ctx = c.empty(max(1, nctx // 4)) if nctx else None
    P = _ptr
    if fused:
        calls = [("cxg_kattn_rope_fwd", (P(Q), P(K), P(V), P(O), P(den), P(ctx), nctx, Bq, S, D,
                                         E, c.sp)),
                 ("cxg_kattn_rope_bwd", (P(Q), P(K), P(V), P(O), P(dO), P(den), P(ctx), P(dQ),
                                         P(dK), P(dV), Bq, S, D, E, c.sp))]
        desc = "RoPE fused (cxg_kattn_rope_fwd -> cxg_kattn_rope_bwd)"
    else:
        calls = [("cxg_rope_fwd", (P(Q), P(K), Bq, S, D, D, c.sp)),
                 ("cxg_kattn_fwd_ctx", (P(Q), P(K), P(V), P(O), P(den), P(ctx), nctx, Bq, S, D,
                                        E, c.sp)),
                 ("cxg_kattn_bwd", (P(Q), P(K), P(V), P(O), P(dO), P(den), P(ctx), P(dQ), P(dK),
                                    P(dV), Bq, S, D, E, c.sp)),
                 ("cxg_rope_bwd", (P(dQ), P(dK), Bq, S, D, D, c.sp))]
        desc = "RoPE as separate passes around the fused pair (cxg_rope_fwd, " \
               "cxg_kattn_fwd_ctx, cxg_kattn_bwd, cxg_rope_bwd)"
    step = Stepper(c.cx.lib(), calls)
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    total = lin_bytes(Bq, S, D)
    value = total / (ms * 1e-3) / 1e9
    kt = {k: round(v[0], 5) for k, v in att.items()}
    if D > 64 or S <= 128:   # the quadratic form: MFMA-bound
        roof = wide_roofline(c, name, att, lin_wide_flops(Bq, S, D, E))
    else:
        kb = lin_kernel_bytes(Bq, S, D, True)
        dom = max((k for k in att if k in kb), key=lambda k: att[k][0])
        ach = kb[dom] / (att[dom][0] * 1e-3) / 1e9
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                "traffic": c.traffic.get(f"{name}/{dom}"), "bytes_per_launch": kb[dom],
                "kernel_ms": kt}
    return dict(value=value, unit="GB/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: stage-2 ELU+1 linear attention fwd+bwd with RoPE "
                                    f"over the full width, {desc}",
                        "B_seq": Bq, "S": S, "D": D, "E": E, "bytes_per_step": total},
                frac=value / HBM_PEAK_GBS, cpu_inputs=None)


def _hexp(c, name, Bq, S, seed, steps, warmup, fused=False, inside=False):
    """fused: the feature maps around the fused pair (cxg_lin_fwd_ctx ->
    cxg_lin_bwd with the context) instead of the four-call linear_cuda chain;
    inside: the feature map inside the fused pair's kernels (cxg_lin_hexp_fwd
    -> cxg_lin_hexp_bwd on the raw projections)."""
    g = c.gen(seed)
    D = E = 64
    N = Bq * S
    Xq, Xk = c.randn(g, N, D, std=0.5), c.randn(g, N, D, std=0.5)
    V, dO = c.randn(g, N, E), c.randn(g, N, E)
    e = c.empty
    pq, pk, O, den, zc = e(N, D), e(N, D), e(N, E), e(N), e(N, D)
    dnum, dden, dpq, dpk, dV, dxq, dxk = e(N, E), e(N), e(N, D), e(N, D), e(N, E), e(N, D), \
        e(N, D)
    P, sp = _ptr, c.sp
    if fused:
        nctx = c.cx.lin_ctx_size(Bq, S, D, E)
        ctx = c.empty(max(1, nctx // 4))
        mid = [
            ("cxg_lin_fwd_ctx", (P(pq), P(pk), P(V), P(O), P(den), P(ctx), nctx, Bq, S, D, E,
                                 sp)),
            ("cxg_lin_bwd", (P(pq), P(pk), P(V), P(O), P(dO), P(den), P(ctx), P(dpq), P(dpk),
                             P(dV), Bq, S, D, E, sp)),
        ]
    else:
        mid = [
            ("cxg_lin_fwd", (P(pq), P(pk), P(V), P(O), P(den), P(zc), None, None, Bq, S, D, E,
                             sp)),
            ("cxg_lin_bwd_step1", (P(O), P(dO), P(den), P(dnum), P(dden), N, E, sp)),
            ("cxg_lin_bwd_dQ", (P(pk), P(V), P(dnum), P(dden), P(zc), P(dpq), None, Bq, S, D, E,
                                sp)),
            ("cxg_lin_bwd_dKdV", (P(pq), P(pk), P(V), P(dnum), P(dden), P(dpk), P(dV), Bq, S, D,
                                  E, sp)),
        ]
    if inside:
        nctx = c.cx.lin_ctx_size(Bq, S, D, E)
        ctx = c.empty(max(1, nctx // 4))
        step = Stepper(c.cx.lib(), [
            ("cxg_lin_hexp_fwd", (P(Xq), P(Xk), P(V), P(O), P(den), P(ctx), nctx, Bq, S, E, sp)),
            ("cxg_lin_hexp_bwd", (P(Xq), P(Xk), P(V), P(O), P(dO), P(den), P(ctx), P(dxq),
                                  P(dxk), P(dV), Bq, S, E, sp)),
        ])
    else:
        step = Stepper(c.cx.lib(), [
            ("cxg_phi_hexp_fwd", (P(Xq), P(pq), N, D, E, sp)),
            ("cxg_phi_hexp_fwd", (P(Xk), P(pk), N, D, E, sp)),
        ] + mid + [
            ("cxg_phi_hexp_bwd", (P(dpq), P(Xq), P(dxq), N, D, E, sp)),
            ("cxg_phi_hexp_bwd", (P(dpk), P(Xk), P(dxk), N, D, E, sp)),
        ])
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    total = lin_bytes(Bq, S, D)
    value = total / (ms * 1e-3) / 1e9
    kb = lin_kernel_bytes(Bq, S, D, fused or inside)
    dom = max((k for k in att if k in kb), key=lambda k: att[k][0])
    ach = kb[dom] / (att[dom][0] * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": c.traffic.get(f"{name}/{dom}"), "bytes_per_launch": kb[dom],
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()}}
    how = ("feature map inside the fused pair's kernels (cxg_lin_hexp_fwd -> cxg_lin_hexp_bwd)"
           if inside else
           "feature maps around the fused pair (cxg_lin_fwd_ctx -> cxg_lin_bwd)" if fused else
           "linear_cuda API chain incl. feature map")
    return dict(value=value, unit="GB/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: Hadamard+Exp linear attention fwd+bwd, " + how,
                        "B_seq": Bq, "S": S, "D": D, "E": E, "bytes_per_step": total},
                frac=value / HBM_PEAK_GBS, cpu_inputs=None)


def _copy(c, steps, warmup):
    """Calibration workload: a plain device-to-device copy of a 256 MiB fp32
    tensor (torch's copy kernel).  Its rocprofv3 FETCH_SIZE / WRITE_SIZE
    readings against the known 256 MiB read + 256 MiB write give the scale
    factor for the counters of the attention kernels (profiles/)."""
    n = 64 << 20
    src, dst = c.empty(n), c.empty(n)
    src.fill_(1.0)

    def step():
        dst.copy_(src)
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    nbytes = 2 * n * 4
    value = nbytes / (ms * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": "copy", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4), "traffic": nbytes,
            "bytes_per_launch": nbytes}
    return dict(value=value, unit="GB/s", ms=ms, roofline=roof,
                config={"workload": "copy: 256 MiB fp32 device-to-device copy (HBM "
                                    "calibration, not an attention workload)",
                        "bytes_per_step": nbytes},
                frac=value / HBM_PEAK_GBS, cpu_inputs=None)


def _rope(c, name, B, S, H, Dh, seed, steps, warmup):
    """RoPE on the stage-1 q/k heads of two_stage_gpt.hpp (:102 forward, :174
    backward) at the C2 shape: cxg_rope_fwd on (Q, K) then cxg_rope_bwd on
    (dQ, dK), all (B*S, H*Dh), in place.  Compulsory I/O: each tensor read and
    written once per call."""
    g = c.gen(seed)
    shp = (B * S, H * Dh)
    Q, K, dQ, dK = [c.randn(g, *shp) for _ in range(4)]
    P = _ptr
    D = H * Dh
    step = Stepper(c.cx.lib(), [
        ("cxg_rope_fwd", (P(Q), P(K), B, S, D, Dh, c.sp)),
        ("cxg_rope_bwd", (P(dQ), P(dK), B, S, D, Dh, c.sp)),
    ])
    ms = timed(step, steps, warmup, c.stream, c.windows, c.spread)
    att = attribute(c.cx, step, ("seconds", ms))
    per_call = 2 * 2 * B * S * D * 4        # two tensors, read + write
    total = 2 * per_call
    value = total / (ms * 1e-3) / 1e9
    dom = max(att, key=lambda k: att[k][0])
    ach = per_call / (att[dom][0] * 1e-3) / 1e9
    roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
            "traffic": c.traffic.get(f"{name}/{dom}"), "bytes_per_launch": per_call,
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()}}
    return dict(value=value, unit="GB/s", ms=ms, roofline=roof,
                config={"workload": f"{name}: RoPE forward + backward on the stage-1 q/k heads "
                                    f"(two_stage_cuda::rope_fwd/rope_bwd), in place",
                        "B": B, "S": S, "H": H, "Dh": Dh, "bytes_per_step": total},
                frac=value / HBM_PEAK_GBS, cpu_inputs=[Q, K, dQ, dK, B, S, D, Dh])


def run_workload(c, name, steps, warmup):
    if name == "copy":
        return _copy(c, steps, warmup)
    if name == "rope":
        return _rope(c, name, 8, 256, 12, 64, 81, steps, warmup)
    if name == "c2rope":
        return _mha(c, name, 8, 256, 12, 64, True, 1234, steps, warmup, rope="fused")
    if name == "c2ropesep":
        return _mha(c, name, 8, 256, 12, 64, True, 1234, steps, warmup, rope="separate")
    if name == "c2":
        return _mha(c, name, 8, 256, 12, 64, True, 1234, steps, warmup)
    if name == "c2legacy":
        return _mha(c, name, 8, 256, 12, 64, False, 1234, steps, warmup)
    if name == "c2graph":
        return _mha(c, name, 8, 256, 12, 64, True, 1234, steps, warmup, graph=True)
    if name == "c2dropin":
        return _mha(c, name, 8, 256, 12, 64, False, 1234, steps, warmup, null_ws=True)
    if name == "c5":
        return _mha(c, name, 2, 4096, 12, 64, True, 555, max(10, steps // 10),
                    max(3, warmup // 4))
    if name == "mhats":      # TwoStageGPT stage 1 (two_stage_train.cpp:168-170, 193): legacy calls
        return _mha(c, name, 32, 256, 64, 8, False, 1301, steps, warmup)
    if name == "mhatsrope":   # stage 1 with its RoPE (two_stage_gpt.hpp:102-106, :171-174) fused
        return _mha(c, name, 32, 256, 64, 8, False, 1303, steps, warmup, rope="fused")
    if name == "mhatsropesep":   # the same as the reference's four calls
        return _mha(c, name, 32, 256, 64, 8, False, 1303, steps, warmup, rope="separate")
    if name in ("gen1", "gen64", "gen256"):   # generate() forward at B = 1 (probe shape H8 Dh32)
        return _mha(c, name, 1, int(name[3:]), 8, 32, True, 1302, steps, warmup, fwd_only=True)
    if name == "c3":
        return _kattn(c, name, 96, 4096, 64, 77, max(20, steps // 4), max(5, warmup // 2))
    if name == "c3s256":
        return _kattn(c, name, 96, 256, 64, 78, steps, warmup)
    if name == "c3fused":
        return _kattn(c, name, 96, 4096, 64, 77, max(20, steps // 4), max(5, warmup // 2),
                      fused=True)
    if name == "c3fuseds256":
        return _kattn(c, name, 96, 256, 64, 78, steps, warmup, fused=True)
    if name == "ffn":
        return _ffn(c, name, 8 * 256, 768, 4 * 2 * 768, 97, steps, warmup)
    if name == "gelu":
        return _gelu(c, name, 8 * 256, 8 * 768, 93, steps, warmup)
    if name == "gpt":
        return _gpt(c, name, 8, 256, 512, 91, steps, warmup)
    if name == "gpt768":     # a GPT-2-small width: the scores-in-memory path
        return _gpt(c, name, 8, 256, 768, 92, steps, warmup)
    if name == "c3lgpt":
        return _kattn(c, name, 96, 4096, 64, 77, max(20, steps // 4), max(5, warmup // 2),
                      lgpt=True)
    if name == "c4":
        return _hexp(c, name, 96, 1024, 79, max(20, steps // 2), warmup)
    if name == "c4fused":
        return _hexp(c, name, 96, 1024, 79, max(20, steps // 2), warmup, fused=True)
    if name == "c4hexp":
        return _hexp(c, name, 96, 1024, 79, max(20, steps // 2), warmup, inside=True)
    if name == "c3wide":     # TwoStageGPT stage 2 (two_stage_train.cpp:168-170, 193)
        return _linwide(c, name, 32, 256, 512, 83, steps, warmup, "chain")
    if name == "c3widefused":
        return _linwide(c, name, 32, 256, 512, 83, steps, warmup, "fused")
    if name == "c3widerope":   # stage 2 with its RoPE fused (two_stage_gpt.hpp:113, :160)
        return _kattn_rope(c, name, 32, 256, 512, 85, steps, warmup, True)
    if name == "c3wideropesep":
        return _kattn_rope(c, name, 32, 256, 512, 85, steps, warmup, False)
    if name == "c3rope":
        return _kattn_rope(c, name, 96, 4096, 64, 86, max(20, steps // 4), max(5, warmup // 2),
                           True)
    if name == "c3ropesep":
        return _kattn_rope(c, name, 96, 4096, 64, 86, max(20, steps // 4), max(5, warmup // 2),
                           False)
    if name == "lgptwide":   # LinearGPT (linear_train.cpp:168-172, 191)
        return _linwide(c, name, 8, 256, 512, 84, steps, warmup, "lgpt")
    raise ValueError(f"unknown workload {name}")


# ---------------------------------------------------------------------------- CPU baseline
def cpu_baseline(name, inputs, nthreads, budget_s):
    """Time the C oracle (restated reference CPU math) on the host cores over
    whole fwd+bwd passes of the workload, repeated until budget_s is used."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as orc
    host = [np.ascontiguousarray(t.float().cpu().numpy()) for t in inputs[:4]]
    Q, K, V, dO = host
    dims = inputs[4:]
    reps, t0 = 0, time.perf_counter()
    while True:
        if name == "rope":
            B, S, D, hd = dims
            for X, sign in ((Q, 1.0), (K, 1.0), (V, -1.0), (dO, -1.0)):
                orc.rope(X, B, S, D, hd, sign)
        elif name.startswith("c2") or name == "c5":
            B, S, H, Dh = dims
            O = orc.mha_fwd(Q, K, V, B, S, H, Dh, nthreads=nthreads)
            orc.mha_bwd(Q, K, V, O, dO, B, S, H, Dh, nthreads=nthreads)
        else:
            Bq, S, D, E = dims
            O, den, zc = orc.kattn_fwd(Q, K, V, Bq, S, D, E, nthreads=nthreads)
            dnum, dden = orc.kattn_bwd_step1(O, dO, den, Bq * S, E)
            orc.kattn_bwd_dQ(K, V, dnum, dden, zc, Q, Bq, S, D, E, nthreads=nthreads)
            orc.kattn_bwd_dKdV(Q, K, V, dnum, dden, Bq, S, D, E, nthreads=nthreads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            break
    per = el / reps
    if name == "rope":
        B, S, D, hd = dims
        return dict(value=round(2 * 2 * 2 * B * S * D * 4 / per / 1e9, 4), unit="GB/s", cores=1,
                    kind="port",
                    sample=f"{reps} rope fwd+bwd passes (B{B} S{S} D{D} head_dim {hd}) through "
                           f"the C oracle's ref_rope restatement, one thread; {el:.1f} s wall, "
                           f"{per * 1e3:.1f} ms/pass")
    if name.startswith("c2") or name == "c5":
        B, S, H, Dh = dims
        return dict(value=round(mha_flops(B, S, H, Dh) / per / 1e12, 6), unit="TFLOP/s",
                    cores=nthreads, kind="port",
                    sample=f"{reps} complete fwd+bwd passes of {name} (B{B} H{H} S{S} Dh{Dh}) "
                           f"through the C oracle (row-form ref_mha_fwd + literal ref_mha_bwd "
                           f"restatement), {nthreads} threads over (b,h); {el:.1f} s wall, "
                           f"{per * 1e3:.1f} ms/pass")
    Bq, S, D, E = dims
    return dict(value=round(lin_bytes(Bq, S, D) / per / 1e9, 4), unit="GB/s", cores=nthreads,
                kind="port",
                sample=f"{reps} complete fwd+bwd chains of {name} (B'{Bq} S{S} D{D} E{E}) "
                       f"through the C oracle's O(S*D*E) scans, {nthreads} threads over "
                       f"sequences; {el:.1f} s wall, {per * 1e3:.1f} ms/pass")


# ---------------------------------------------------------------------------- main
# The linear-attention half of the metric (C3 S4096: the fused pair, then the
# reference-signature chain with its CPU baseline) goes last, so that the end
# of the printed line -- what a reader of only its tail sees -- carries it.
SECONDARY = ("c2legacy", "c2dropin", "c5", "mhats", "mhatsrope", "mhatsropesep", "gen1", "gen64", "gen256", "rope", "c2rope",
             "c2ropesep", "gpt", "gpt768", "gelu", "ffn", "c3s256", "c3fuseds256", "c3lgpt",
             "c3wide", "c3widefused", "c3widerope", "c3wideropesep", "c3rope", "c3ropesep",
             "lgptwide", "c4", "c4fused", "c4hexp", "c3fused", "c3")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2",
                    choices=["c2", "c2legacy", "c2dropin", "c2graph", "c3", "c3s256", "c3fused", "c3fuseds256", "c3lgpt",
                             "c3wide", "c3widefused", "c3widerope", "c3wideropesep", "c3rope",
                             "c3ropesep", "lgptwide", "c4", "c4fused", "c4hexp", "c5",
                             "mhats", "mhatsrope", "mhatsropesep", "gen1",
                             "gen64", "gen256", "gpt768", "rope", "c2rope",
                             "c2ropesep", "gpt", "gelu", "ffn", "copy"])
    ap.add_argument("--no-secondary", action="store_true", help="only the reported workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds per CPU baseline")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the attention path has no multi-GPU leg. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import cxxgpt_attn as cx
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    cx.lib()  # raises if the HIP library is not built: there is no fallback
    c = Ctx(cx, torch, args.steps, args.warmup)

    c.windows, c.spread = HEADLINE_WINDOWS, []
    r = run_workload(c, args.workload, args.steps, args.warmup)
    windows_ms = c.spread
    c.windows, c.spread = 1, None
    out = {
        "metric": METRIC,
        "value": round(r["value"], 3),
        "unit": r["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) tensors from a seeded GPU generator, resident in HBM",
        "config": r["config"],
        "roofline": r["roofline"],
        "step_frac_of_peak": round(r["frac"], 4),
        "timing": {"windows": len(windows_ms), "steps_per_window": args.steps,
                   "reported": "median window",
                   "window_ms_per_step": [round(w, 5) for w in windows_ms]},
    }
    out["roofline"]["duration_source"] = (
        "mean dispatch duration from the start/stop HIP events each launch records itself "
        "(hipExtLaunchKernelGGL through the library's timing hook, on the launch stream), "
        f"over about {SUSTAIN_S} s of steps; rocprofv3 kernel-trace averages are in profiles/")
    out["roofline"]["traffic_source"] = (
        "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE per dispatch, scaled by the same counters "
        "on a 256 MiB copy (profiles/hbm_traffic.md, run of the date given there)")
    sec = {}
    if not args.no_secondary and args.workload == "c2":
        for name in SECONDARY:
            # a short probe fixes the step count that fills SUSTAIN_S of GPU time
            probe = run_workload(c, name, 3, 1)
            n = steps_for(probe["ms"], args.steps)
            s = run_workload(c, name, n, args.warmup)
            sec[name] = {"value": round(s["value"], 3), "unit": s["unit"], "steps": n,
                         "ms_per_step": round(s["ms"], 5), "frac_of_peak": round(s["frac"], 4),
                         "roofline": s["roofline"], "config": s["config"]}
            if name == "c3":
                c3_inputs = s["cpu_inputs"]
    if not args.no_cpu:
        nth = cpu_threads()
        out["cpu_baseline"] = cpu_baseline(args.workload, r["cpu_inputs"], nth, args.cpu_budget) \
            if r["cpu_inputs"] is not None else None
        if "c3" in sec:
            sec["c3"]["cpu_baseline"] = cpu_baseline("c3", c3_inputs, nth, args.cpu_budget)
    else:
        out["cpu_baseline"] = None
    if sec:
        out["secondary"] = sec   # last key: its last entries are c3fused and c3
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
