#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (one GPU).

Headline step ("C2"): causal softmax MHA forward +
backward, FP32, B=8 H=12 S=256 Dh=64, through the C ABI of
libcxxgpt_attn.so -- cxg_mha_fwd (writes O and the row log-sum-exp) then
cxg_mha_bwd (consumes it), the pair the reference's two_stage_cuda::
fused_mha_fwd / fused_mha_bwd replace (src/TwoStage/two_stage_gpt.hpp:106,
:171).  value = algorithmic TFLOP/s of the step, counting
4*Dh*P (fwd) + 8*Dh*P (bwd) FLOPs per (b,h) with P = S(S+1)/2 causal pairs;
recomputation is not credited.

Secondary lines (same JSON object, key "secondary"):
  * C2 through the legacy signatures (no lse: the backward recomputes it),
  * C3 ELU+1 linear attention fwd+bwd at S=4096 (B' = 96, D = E = 64) through
    the two_stage API chain kernel_attn_fwd -> bwd_step1 -> bwd_dQ ->
    bwd_dKdV, metered in GB/s of compulsory I/O (12*S*D + 2*S floats per
    sequence),
  * C4 Hadamard+Exp linear attention (S=1024) through the linear_cuda API,
  * C5 long-sequence MHA (B2 H12 S4096 Dh64) fwd+bwd.

Inputs are synthetic N(0,1) tensors generated on the GPU from a fixed seed
and resident in HBM before timing starts.  The roofline object is measured
live: after the timed region the same steps run again with the library's
per-launch HIP-event hook on (events recorded on the launch stream), which
gives each kernel's mean duration.  The CPU baseline times the C oracle
(the restated CPU reference, test infrastructure) on the host cores over a
bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       [--no-secondary]
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

# Traffic factors from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (KiB per
# dispatch), scaled by the same counters' reading on a plain copy kernel of
# known size.  Keys: kernel tag -> HBM bytes per launch.  Filled from the
# committed counter summary when present.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")


def mha_flops(B, S, H, Dh, fwd=True, bwd=True):
    P = S * (S + 1) // 2
    per = (4 * Dh * P if fwd else 0) + (8 * Dh * P if bwd else 0)
    return per * B * H


def lin_bytes(Bq, S, D):
    return (12 * S * D + 2 * S) * 4 * Bq


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


def timed(step, steps, warmup, stream):
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    return e0.elapsed_time(e1) / steps, wall


def attribute(cx, step, steps, names):
    """Mean device duration (ms) per launch of each kernel tag, from the
    library's per-launch HIP events on the launch stream."""
    import torch
    torch.cuda.synchronize()
    cx.prof_reset()
    cx.prof_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    cx.prof_enable(False)
    out = {}
    for n in names:
        tot, cnt = cx.prof_query(n)
        if cnt:
            out[n] = (tot / cnt, cnt)
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
    # the GPU box grants one GPU's share of the host (16 threads)
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


# ----------------------------------------------------------------------------
def bench_mha(cx, torch, dev, stream, B, S, H, Dh, steps, warmup, use_lse, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    shp = (B * S, H * Dh)
    Q, K, V, dO = [torch.randn(shp, device=dev, generator=g) for _ in range(4)]
    O = torch.empty(shp, device=dev)
    dQ, dK, dV = torch.empty_like(O), torch.empty_like(O), torch.empty_like(O)
    lse = torch.empty(B * H * S, device=dev) if use_lse else None
    ws_bytes = cx.mha_bwd_workspace_size(B, S, H, Dh)
    ws = torch.empty(max(1, ws_bytes // 4), device=dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    calls = [
        ("cxg_mha_fwd", (_ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(lse), B, S, H, Dh, sp)),
        ("cxg_mha_bwd", (_ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(lse), _ptr(dQ),
                         _ptr(dK), _ptr(dV), B, S, H, Dh, _ptr(ws), ws_bytes, sp)),
    ]
    step = Stepper(cx.lib(), calls)
    ms, wall = timed(step, steps, warmup, stream)
    att = attribute(cx, step, max(10, min(steps, 100)),
                    ["mha_fwd", "mha_stats", "mha_bwd_prep", "mha_bwd"])
    return dict(ms=ms, wall=wall, att=att,
                tensors=dict(Q=Q, K=K, V=V, dO=dO, O=O))


def bench_kattn(cx, torch, dev, stream, Bq, S, D, E, steps, warmup, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    N = Bq * S
    Q = torch.randn(N, D, device=dev, generator=g)
    K = torch.randn(N, D, device=dev, generator=g)
    V = torch.randn(N, E, device=dev, generator=g)
    dO = torch.randn(N, E, device=dev, generator=g)
    O, den, zc = torch.empty(N, E, device=dev), torch.empty(N, device=dev), \
        torch.empty(N, D, device=dev)
    dnum, dden = torch.empty(N, E, device=dev), torch.empty(N, device=dev)
    dQ, dK, dV = torch.empty(N, D, device=dev), torch.empty(N, D, device=dev), \
        torch.empty(N, E, device=dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    calls = [
        ("cxg_kattn_fwd", (_ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(den), _ptr(zc), None, None,
                           Bq, S, D, E, sp)),
        ("cxg_kattn_bwd_step1", (_ptr(O), _ptr(dO), _ptr(den), _ptr(dnum), _ptr(dden), N, E, sp)),
        ("cxg_kattn_bwd_dQ", (_ptr(K), _ptr(V), _ptr(dnum), _ptr(dden), _ptr(zc), _ptr(Q),
                              _ptr(dQ), None, Bq, S, D, E, sp)),
        ("cxg_kattn_bwd_dKdV", (_ptr(Q), _ptr(K), _ptr(V), _ptr(dnum), _ptr(dden), _ptr(dK),
                                _ptr(dV), Bq, S, D, E, sp)),
    ]
    step = Stepper(cx.lib(), calls)
    ms, wall = timed(step, steps, warmup, stream)
    return dict(ms=ms, wall=wall, tensors=dict(Q=Q, K=K, V=V, dO=dO))


def bench_hexp(cx, torch, dev, stream, Bq, S, steps, warmup, seed):
    """C4: phi_hexp_fwd x2 -> linear_cuda fwd -> step1 -> dQ -> dKdV -> phi_hexp_bwd x2."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    D = E = 64
    N = Bq * S
    Xq = 0.5 * torch.randn(N, D, device=dev, generator=g)
    Xk = 0.5 * torch.randn(N, D, device=dev, generator=g)
    V = torch.randn(N, E, device=dev, generator=g)
    dO = torch.randn(N, E, device=dev, generator=g)
    e = lambda *s: torch.empty(*s, device=dev)  # noqa: E731
    pq, pk, O, den, zc = e(N, D), e(N, D), e(N, E), e(N), e(N, D)
    dnum, dden, dpq, dpk, dV, dxq, dxk = e(N, E), e(N), e(N, D), e(N, D), e(N, E), e(N, D), \
        e(N, D)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = _ptr
    calls = [
        ("cxg_phi_hexp_fwd", (P(Xq), P(pq), N, D, E, sp)),
        ("cxg_phi_hexp_fwd", (P(Xk), P(pk), N, D, E, sp)),
        ("cxg_lin_fwd", (P(pq), P(pk), P(V), P(O), P(den), P(zc), None, None, Bq, S, D, E, sp)),
        ("cxg_lin_bwd_step1", (P(O), P(dO), P(den), P(dnum), P(dden), N, E, sp)),
        ("cxg_lin_bwd_dQ", (P(pk), P(V), P(dnum), P(dden), P(zc), P(dpq), None, Bq, S, D, E,
                            sp)),
        ("cxg_lin_bwd_dKdV", (P(pq), P(pk), P(V), P(dnum), P(dden), P(dpk), P(dV), Bq, S, D, E,
                              sp)),
        ("cxg_phi_hexp_bwd", (P(dpq), P(Xq), P(dxq), N, D, E, sp)),
        ("cxg_phi_hexp_bwd", (P(dpk), P(Xk), P(dxk), N, D, E, sp)),
    ]
    step = Stepper(cx.lib(), calls)
    ms, wall = timed(step, steps, warmup, stream)
    return dict(ms=ms, wall=wall)


# ----------------------------------------------------------------------------
def cpu_baseline_mha(t, B, S, H, Dh, nthreads, budget_s):
    """Time the C oracle (restated reference CPU math) on the host cores over
    whole C2 fwd+bwd passes, repeated until budget_s of wall time is used."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as orc
    Q, K, V, dO = [np.ascontiguousarray(t[k].float().cpu().numpy()) for k in ("Q", "K", "V", "dO")]
    reps = 0
    t0 = time.perf_counter()
    while True:
        O = orc.mha_fwd(Q, K, V, B, S, H, Dh, nthreads=nthreads)
        orc.mha_bwd(Q, K, V, O, dO, B, S, H, Dh, nthreads=nthreads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            break
    per = el / reps
    return dict(value=mha_flops(B, S, H, Dh) / per / 1e12, unit="TFLOP/s", cores=nthreads,
                kind="port",
                sample=f"{reps} full C2 fwd+bwd passes (B{B} H{H} S{S} Dh{Dh}) of the C oracle "
                       f"(orc_mha_fwd row form + literal ref_mha_bwd restatement), "
                       f"{nthreads} threads over (b,h), {el:.1f} s wall, {per * 1e3:.1f} ms/pass")


def cpu_baseline_kattn(t, Bq, S, D, E, nthreads, budget_s):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle as orc
    Q, K, V, dO = [np.ascontiguousarray(t[k].float().cpu().numpy()) for k in ("Q", "K", "V", "dO")]
    N = Bq * S
    reps = 0
    t0 = time.perf_counter()
    while True:
        O, den, zc = orc.kattn_fwd(Q, K, V, Bq, S, D, E, nthreads=nthreads)
        dnum, dden = orc.kattn_bwd_step1(O, dO, den, N, E)
        orc.kattn_bwd_dQ(K, V, dnum, dden, zc, Q, Bq, S, D, E, nthreads=nthreads)
        orc.kattn_bwd_dKdV(Q, K, V, dnum, dden, Bq, S, D, E, nthreads=nthreads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            break
    per = el / reps
    return dict(value=lin_bytes(Bq, S, D) / per / 1e9, unit="GB/s", cores=nthreads, kind="port",
                sample=f"{reps} full C3 fwd+bwd chains (B'{Bq} S{S} D{D} E{E}) of the C oracle "
                       f"(O(S*D*E) scans), {nthreads} threads over sequences, {el:.1f} s wall")


# ----------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="only the headline config")
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
    cx.lib()  # raises if the HIP library is not built: no fallback
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    steps, warmup = args.steps, args.warmup
    traffic = load_traffic()

    # ---------------- headline: C2 softmax MHA fwd+bwd (extended ABI with lse)
    B, S, H, Dh = 8, 256, 12, 64
    r = bench_mha(cx, torch, dev, stream, B, S, H, Dh, steps, warmup, True, 1234)
    flops = mha_flops(B, S, H, Dh)
    tflops = flops / (r["ms"] * 1e-3) / 1e12
    att = r["att"]
    dom = max(att, key=lambda k: att[k][0])
    kflops = {"mha_fwd": mha_flops(B, S, H, Dh, bwd=False),
              "mha_bwd": mha_flops(B, S, H, Dh, fwd=False)}
    dom_ms = att[dom][0]
    ach = kflops.get(dom, 0) / (dom_ms * 1e-3) / 1e12
    roof = {"bound": "mfma", "kernel": dom, "achieved": round(ach, 3),
            "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(ach / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": traffic.get(f"C2/{dom}"),
            "kernel_ms": {k: round(v[0], 5) for k, v in att.items()},
            "step_frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4)}

    out = {
        "metric": "attn fwd+bwd TFLOP/s (% MFMA peak) B8H12S256D64 fp32; lin-attn HBM GB/s",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(r["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) Q/K/V/dO, seeded, resident in HBM",
        "config": {"workload": "C2 causal softmax MHA fwd+bwd (cxg_mha_fwd with lse -> "
                               "cxg_mha_bwd)", "B": B, "H": H, "S": S, "Dh": Dh,
                   "flops_per_step": flops},
        "roofline": roof,
        "wall_s_timed": round(r["wall"], 4),
    }

    sec = {}
    if not args.no_secondary:
        # C2 through the legacy signatures (no lse)
        rl = bench_mha(cx, torch, dev, stream, B, S, H, Dh, steps, warmup, False, 1234)
        sec["C2_legacy_no_lse"] = {
            "value": round(flops / (rl["ms"] * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": round(rl["ms"], 5),
            "kernel_ms": {k: round(v[0], 5) for k, v in rl["att"].items()}}
        del rl
        # C3 ELU+1 linear attention, S=4096
        Bq, S3, D = 96, 4096, 64
        rk = bench_kattn(cx, torch, dev, stream, Bq, S3, D, D, max(20, steps // 4),
                         max(5, warmup // 2), 77)
        gbs = lin_bytes(Bq, S3, D) / (rk["ms"] * 1e-3) / 1e9
        sec["C3_elu_S4096"] = {"value": round(gbs, 1), "unit": "GB/s",
                               "ms_per_step": round(rk["ms"], 5),
                               "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                               "bytes_per_step": lin_bytes(Bq, S3, D)}
        kt = rk["tensors"]
        rk256 = bench_kattn(cx, torch, dev, stream, Bq, 256, D, D, steps, warmup, 78)
        gbs = lin_bytes(Bq, 256, D) / (rk256["ms"] * 1e-3) / 1e9
        sec["C3_elu_S256"] = {"value": round(gbs, 1), "unit": "GB/s",
                              "ms_per_step": round(rk256["ms"], 5),
                              "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        del rk256
        # C4 Hadamard+Exp, S=1024
        rh = bench_hexp(cx, torch, dev, stream, 96, 1024, max(20, steps // 2), warmup, 79)
        gbs = lin_bytes(96, 1024, 64) / (rh["ms"] * 1e-3) / 1e9
        sec["C4_hexp_S1024"] = {"value": round(gbs, 1), "unit": "GB/s",
                                "ms_per_step": round(rh["ms"], 5),
                                "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        # C5 long-sequence MHA
        B5, S5 = 2, 4096
        r5 = bench_mha(cx, torch, dev, stream, B5, S5, H, Dh, max(10, steps // 10),
                       max(3, warmup // 4), True, 555)
        f5 = mha_flops(B5, S5, H, Dh)
        t5 = f5 / (r5["ms"] * 1e-3) / 1e12
        sec["C5_mha_S4096"] = {"value": round(t5, 3), "unit": "TFLOP/s",
                               "ms_per_step": round(r5["ms"], 5),
                               "frac_mfma": round(t5 / FP32_MFMA_PEAK_TFLOPS, 4),
                               "kernel_ms": {k: round(v[0], 5) for k, v in r5["att"].items()}}
        del r5
        out["secondary"] = sec

    if not args.no_cpu:
        nth = cpu_threads()
        out["cpu_baseline"] = cpu_baseline_mha(r["tensors"], B, S, H, Dh, nth, args.cpu_budget)
        out["cpu_baseline"]["value"] = round(out["cpu_baseline"]["value"], 6)
        if not args.no_secondary:
            cb = cpu_baseline_kattn(kt, 96, 4096, 64, 64, nth, args.cpu_budget)
            cb["value"] = round(cb["value"], 3)
            sec["C3_elu_S4096"]["cpu_baseline"] = cb
    else:
        out["cpu_baseline"] = None

    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
