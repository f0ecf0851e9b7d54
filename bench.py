#!/usr/bin/env python3
"""Benchmark of the KATA-SPD hot path on one MI355X.

Workload: causal concat-SPD attention forward+backward,
B=8, H=12, T=2048, dk=dv=64, M=4 groups, bf16 inputs / fp32 accumulation,
q,k,v ~ N(0,1)/8, dO ~ N(0,1) (seed 1), synthetic data already resident in
HBM.  One step = forward (o, den) + backward (dq, dk, dv) through the C ABI
(linatt_kata_fwd, linatt_kata_bwd_dq, linatt_kata_bwd_dkdv) on the current
HIP stream, with preallocated outputs.

Before each workload's warmup steps the launches run untimed for about a
second (``--settle-seconds``) so that the GPU has left its idle clock; the
timed steps then measure sustained throughput, as a training loop sees it.

Prints ONE JSON line: tokens/s (B*T per step), per-kernel average durations
measured with HIP events recorded on the launch stream, the roofline of the
dominant kernel (algorithmic FLOPs per launch / its average duration), and
the CPU baseline: the float32 restatement of the reference math in
``oracle/kata.py`` timed on the host cores over a bounded sample of heads.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--groups M]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

METRIC = "KATA/delta fwd+bwd tokens/s & TFLOP/s (% MFMA peak) at B8 H12 T2048 D64"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


def kata_flops(B, H, T, dk, dv, M, variant="concat"):
    """Algorithmic FLOPs (FlashAttention convention, causal half, no
    recompute): one 'unit' per product over the causal triangle."""
    qk = B * H * T * T * dk * (M if variant == "sum" else 1)
    pv = B * H * T * T * dv
    fwd = qk + pv
    # backward products: S recompute (qk), dP (pv), dV (pv), dQ (qk), dK (qk)
    dkdv = qk + pv + pv + qk      # the dk/dv kernel needs S, dP, dV, dK
    dq = qk                       # the dq kernel's own product (S, dP are recompute)
    return {"fwd": fwd, "bwd_dq": dq, "bwd_dkdv": dkdv, "total": fwd + dq + dkdv}


def delta_flops(B, H, T, K, V, C=64):
    """Algorithmic FLOPs of the chunked delta rule (count once, no recompute):
    per token-head C(6K+4V) + 6KV + (2/3)C^2 (Gram, QK^T, W = 3x2C^2K; U and
    the intra A.v = 2x2C^2V; W.h, Q.h, K^T v_new = 3x2CKV; the 64x64 UT
    inverse (2/3)C^3 per chunk); backward = 2x forward.  Split by kernel:
    prep = Gram, QK^T, W, U, inverse; state pass = W.h, K^T v_new and the
    output's Q.h, intra A.v (one kernel); reverse state pass = Aqk^T dO,
    K dS, Q^T dO, W^T dVn (2CV + 8KV); the backward chunk kernel the rest of
    2x forward."""
    n = B * H * T
    prep = n * (6 * C * K + 2 * C * V + (2.0 / 3.0) * C * C)
    state = n * (4 * K * V + 2 * K * V + 2 * C * V)
    fwd = prep + state
    state_bwd = n * (2 * C * V + 8 * K * V)
    return {"prep": prep, "state_fwd": state, "fwd": fwd,
            "state_bwd": state_bwd, "bwd_chunk": 2 * fwd - state_bwd, "bwd": 2 * fwd,
            "total": 3 * fwd}


def delta_state_bytes(B, H, T, K, V, gated, h0, C=64):
    """Compulsory HBM bytes of the two state passes (bf16 tensors, fp32 g and
    states).  Forward, with the output: k, w, u, q and the chunks' Aqk
    blocks read, v_new and o written, g, the per-chunk states h (bf16), h0
    read and ht written.  Backward: q, k, w, dO read, dv_new written, g, the
    per-chunk dh (bf16), dh0 written."""
    n, NT = B * T * H, (T + C - 1) // C
    gb = 4 if gated else 0
    st = B * H * K * V * 4
    fwd = n * (2 * K + 2 * K + 2 * V + 2 * V + 2 * K + 2 * C + 2 * V + gb) + \
        B * H * NT * K * V * 2 + st * (2 if h0 else 1)
    bwd = n * (2 * K + 2 * K + 2 * K + 2 * V + 2 * V + gb) + B * H * NT * K * V * 2 + \
        (st if h0 else 0)
    return {"state_fwd": fwd, "state_bwd": bwd}


def settle(parts, seconds):
    """Run the step's launches untimed for `seconds` of wall time.  An idle
    MI355X starts a burst at a low shader clock and needs about a second of
    sustained load to reach its working clock; without this, a short warmup
    times the clock ramp (KATA config 2: 0.40 ms/step after 5 warmup steps
    from idle, 0.33 ms/step once the clock has settled)."""
    import torch
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            for _, f in parts:
                f()
        torch.cuda.synchronize()


DELTA_FWD_STAGES = (("prep", 1), ("state_fwd", 2))
DELTA_BWD_STAGES = (("state_bwd", 1), ("bwd_chunk", 2))


def bench_delta(gated, steps, warmup, settle_s, H=6, K=128):
    """BASELINE config 3 (DeltaNet) / 4 (GatedDeltaNet): B8 H6 T2048 K=V=128
    (or the given H, K = V) bf16, chunk 64, fwd + bwd through the C ABI with
    preallocated outputs,
    context and workspace.  Each kernel is launched on its own
    (linatt_delta_fwd_stages / linatt_delta_bwd_stages, which together make
    exactly the launches of linatt_delta_fwd + linatt_delta_bwd) between HIP
    events on the launch stream, so every kernel has a measured duration."""
    import torch
    from linatt_amd import _lib
    L = _lib.load()
    B, T, V = 8, 2048, K
    seed = 3 if gated else 2
    q, k, v, beta, g, h0, do = delta_inputs(B, H, T, K, V, gated, seed)
    dev = torch.device("cuda", 0)
    qd, kd, vd, bd, dod = (x.to(dev) for x in (q, k, v, beta, do))
    gd = g.to(dev) if gated else None
    h0d = h0.to(dev) if gated else None
    o = torch.empty_like(vd)
    ht = torch.empty(B, H, K, V, device=dev)
    dt = _lib.LINATT_BFLOAT16
    ctx = torch.empty(L.linatt_delta_ctx_bytes(B, T, H, K, V, dt), device=dev, dtype=torch.uint8)
    ws = torch.empty(L.linatt_delta_bwd_workspace_bytes(B, T, H, K, V, dt), device=dev,
                     dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    dbeta = torch.empty(B, T, H, device=dev)
    dg = torch.empty_like(dbeta) if gated else None
    dh0 = torch.empty_like(h0d) if gated else None
    dht = torch.zeros(B, H, K, V, device=dev)
    P = _lib.ptr
    sp = _lib.stream_of(qd)
    scale = K ** -0.5
    stream = torch.cuda.current_stream(dev)

    def fwd(stages):
        _lib.check("linatt_delta_fwd_stages", L.linatt_delta_fwd_stages(
            P(qd), P(kd), P(vd), P(bd), P(gd), P(h0d), P(o), P(ht), P(ctx), B, T, H, K, V,
            scale, stages, dt, sp))

    def bwd(stages):
        _lib.check("linatt_delta_bwd_stages", L.linatt_delta_bwd_stages(
            P(qd), P(kd), P(vd), P(bd), P(gd), P(h0d), P(dod), P(dht), P(ctx), P(ws), P(dq),
            P(dk), P(dv), P(dbeta), P(dg), P(dh0), B, T, H, K, V, scale, stages, dt, sp))

    parts = [(n, (lambda m=m: fwd(m))) for n, m in DELTA_FWD_STAGES] + \
            [(n, (lambda m=m: bwd(m))) for n, m in DELTA_BWD_STAGES]
    settle(parts, settle_s)
    for _ in range(warmup):
        for _, f in parts:
            f()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(parts) + 1)]
          for _ in range(steps)]
    for s in range(steps):
        ev[s][0].record(stream)
        for i, (_, f) in enumerate(parts):
            f()
            ev[s][i + 1].record(stream)
    torch.cuda.synchronize()
    kms = {n: sum(ev[s][i].elapsed_time(ev[s][i + 1]) for s in range(steps)) / steps
           for i, (n, _) in enumerate(parts)}
    f_ms = sum(kms[n] for n, _ in DELTA_FWD_STAGES)
    b_ms = sum(kms[n] for n, _ in DELTA_BWD_STAGES)
    fl = delta_flops(B, H, T, K, V)
    by = delta_state_bytes(B, H, T, K, V, gated, gated)
    kern = {}
    for n in kms:
        e = {"avg_ms": round(kms[n], 4)}
        if n in by:
            gbs = by[n] / (kms[n] * 1e-3) / 1e9
            e.update({"bound": "hbm", "alg_mb": round(by[n] / 1e6, 1), "gbs": round(gbs, 1),
                      "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)})
        tf = fl[n] / (kms[n] * 1e-3) / 1e12
        e.update({"alg_gflop": round(fl[n] / 1e9, 2), "tflops": round(tf, 1),
                  "frac_mfma_peak": round(tf / PEAK_BF16_TFLOPS, 4)})
        if n not in by:
            e["bound"] = "mfma"
        kern[n] = e
    tot = f_ms + b_ms
    tf = fl["total"] / (tot * 1e-3) / 1e12
    return {"config": {"B": B, "H": H, "T": T, "K": K, "V": V, "chunk": 64, "gated": gated,
                       "seed": seed, "h0": gated},
            "fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4), "ms": round(tot, 4),
            "tokens_per_s": round(B * T / (tot * 1e-3), 1),
            "alg_gflop": round(fl["total"] / 1e9, 2), "tflops": round(tf, 1),
            "frac_mfma_peak": round(tf / PEAK_BF16_TFLOPS, 4), "kernels": kern}


def _time_parts(parts, steps, settle_s, warmup=2):
    """Average ms per part and per step of `parts` (name, fn) launched in
    order on the current stream, bracketed by HIP events."""
    import torch
    settle(parts, settle_s)
    for _ in range(warmup):
        for _, f in parts:
            f()
    stream = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(parts) + 1)]
          for _ in range(steps)]
    torch.cuda.synchronize()
    for s in range(steps):
        ev[s][0].record(stream)
        for i, (_, f) in enumerate(parts):
            f()
            ev[s][i + 1].record(stream)
    torch.cuda.synchronize()
    per = {name: sum(ev[s][i].elapsed_time(ev[s][i + 1]) for s in range(steps)) / steps
           for i, (name, _) in enumerate(parts)}
    return per, sum(per.values())


def bench_kata_variant(steps, settle_s, B, H, T, dk, dv, M, variant, decay, seed):
    """KATA fwd + bwd through the C ABI at a trained mixer's shape: the sum
    score (kata_quadratic_sum) or the decayed concat score at the offset-gated
    width (dk = 128 packs two 32-wide groups padded to 64,
    kataconv_cat_l2_gdn_340m.yaml).  The decayed backward is one call
    (linatt_kata_bwd_decay: dq pass, then dk/dv pass)."""
    import torch
    from linatt_amd import _lib
    L = _lib.load()
    g = torch.Generator().manual_seed(seed)
    dev = torch.device("cuda", 0)
    q, k = ((torch.randn(B, T, H, dk, generator=g) / 8).to(torch.bfloat16).to(dev) for _ in range(2))
    v = (torch.randn(B, T, H, dv, generator=g) / 8).to(torch.bfloat16).to(dev)
    do = torch.randn(B, T, H, dv, generator=g).to(torch.bfloat16).to(dev)
    c = None
    if decay:
        c = (-(torch.rand(B, T, H, generator=g) * 0.05)).cumsum(1).to(dev)
    o = torch.empty_like(v)
    den = torch.empty(B, T, H, device=dev)
    dq, dk_, dv_ = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dc = torch.empty_like(c) if decay else None
    ws = torch.empty(L.linatt_kata_bwd_workspace_bytes(B, T, H, dv, _lib.LINATT_BFLOAT16),
                     device=dev, dtype=torch.uint8)
    P, bt, sp = _lib.ptr, _lib.LINATT_BFLOAT16, _lib.stream_of(q)
    scale = 1.0 / math.sqrt(dk // M)
    var = 1 if variant == "sum" else 0

    def fwd():
        _lib.check("linatt_kata_fwd", L.linatt_kata_fwd(
            P(q), P(k), P(v), P(c), P(o), P(den), B, T, H, H, dk, dv, M, scale, var, bt, sp))

    def bwd():
        if decay:
            _lib.check("linatt_kata_bwd_decay", L.linatt_kata_bwd_decay(
                P(q), P(k), P(v), P(c), P(o), P(den), P(do), P(dq), P(dk_), P(dv_), P(dc), P(ws),
                B, T, H, H, dk, dv, M, scale, bt, sp))
        else:
            _lib.check("linatt_kata_bwd", L.linatt_kata_bwd(
                P(q), P(k), P(v), P(o), P(den), P(do), P(dq), P(dk_), P(dv_), P(ws),
                B, T, H, H, dk, dv, M, scale, var, bt, sp))

    per, ms = _time_parts([("fwd", fwd), ("bwd", bwd)], steps, settle_s)
    fl = kata_flops(B, H, T, dk, dv, M, variant)
    out = {"config": {"B": B, "H": H, "T": T, "dk": dk, "dv": dv, "num_groups": M,
                      "variant": variant, "decay": decay, "dtype": "bf16", "seed": seed},
           "fwd_ms": round(per["fwd"], 4), "bwd_ms": round(per["bwd"], 4), "ms": round(ms, 4),
           "tokens_per_s": round(B * T / (ms * 1e-3), 1), "alg_gflop": round(fl["total"] / 1e9, 2)}
    out["tflops"] = round(fl["total"] / (ms * 1e-3) / 1e12, 1)
    out["frac_mfma_peak"] = round(out["tflops"] / PEAK_BF16_TFLOPS, 4)
    out["fwd_frac_mfma_peak"] = round(fl["fwd"] / (per["fwd"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
    out["bwd_frac_mfma_peak"] = round((fl["bwd_dq"] + fl["bwd_dkdv"]) / (per["bwd"] * 1e-3) / 1e12
                                      / PEAK_BF16_TFLOPS, 4)
    return out


def bench_kata_onorm(steps, settle_s, M=4):
    """The mixer's output RMSNorm fused into the KATA kernels against the
    two-step chain (KATA, then the RMSNorm kernels) at config 2 (B8 H12
    T2048 D64, bf16): forward y and backward dq, dk, dv, dnorm_weight."""
    import torch
    from linatt_amd import _lib
    L = _lib.load()
    B, H, T, D = 8, 12, 2048, 64
    g = torch.Generator().manual_seed(8)
    dev = torch.device("cuda", 0)
    q, k, v = ((torch.randn(B, T, H, D, generator=g) / 8).to(torch.bfloat16).to(dev) for _ in range(3))
    dy = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16).to(dev)
    w = (0.75 + 0.5 * torch.rand(D, generator=g)).to(dev)
    o, y, dO, dq, dk, dv = (torch.empty_like(q) for _ in range(6))
    den, rstd = (torch.empty(B, T, H, device=dev) for _ in range(2))
    dw = torch.empty(D, device=dev)
    bt = _lib.LINATT_BFLOAT16
    n = B * T * H
    ws = torch.empty(L.linatt_kata_bwd_onorm_workspace_bytes(B, T, H, D, bt), device=dev, dtype=torch.uint8)
    rws = torch.empty(L.linatt_rmsnorm_bwd_workspace_bytes(n, D), device=dev, dtype=torch.uint8)
    P, sp, scale = _lib.ptr, _lib.stream_of(q), 1.0 / math.sqrt(D // M)

    def f_fwd():
        _lib.check("linatt_kata_fwd_onorm", L.linatt_kata_fwd_onorm(
            P(q), P(k), P(v), None, P(o), P(den), P(w), 1e-5, P(y), P(rstd), B, T, H, H, D, D, M,
            scale, 0, bt, sp))

    def f_bwd():
        _lib.check("linatt_kata_bwd_onorm", L.linatt_kata_bwd_onorm(
            P(q), P(k), P(v), None, P(o), P(den), P(rstd), P(w), P(dy), P(dq), P(dk), P(dv), None,
            P(dw), P(ws), B, T, H, H, D, D, M, scale, 0, bt, sp))

    def u_fwd():
        _lib.check("linatt_kata_fwd", L.linatt_kata_fwd(
            P(q), P(k), P(v), None, P(o), P(den), B, T, H, H, D, D, M, scale, 0, bt, sp))
        _lib.check("linatt_rmsnorm_fwd", L.linatt_rmsnorm_fwd(
            P(o), P(w), P(y), P(rstd), n, D, 1e-5, bt, sp))

    def u_bwd():
        _lib.check("linatt_rmsnorm_bwd", L.linatt_rmsnorm_bwd(
            P(o), P(w), P(rstd), P(dy), P(dO), P(dw), P(rws), n, D, bt, sp))
        _lib.check("linatt_kata_bwd", L.linatt_kata_bwd(
            P(q), P(k), P(v), P(o), P(den), P(dO), P(dq), P(dk), P(dv), P(ws),
            B, T, H, H, D, D, M, scale, 0, bt, sp))

    pf, msf = _time_parts([("fwd", f_fwd), ("bwd", f_bwd)], steps, settle_s)
    pu, msu = _time_parts([("fwd", u_fwd), ("bwd", u_bwd)], steps, settle_s / 2)
    return {"config": {"B": B, "H": H, "T": T, "D": D, "num_groups": M, "dtype": "bf16", "seed": 8},
            "fused_fwd_ms": round(pf["fwd"], 4), "fused_bwd_ms": round(pf["bwd"], 4),
            "fused_ms": round(msf, 4), "unfused_fwd_ms": round(pu["fwd"], 4),
            "unfused_bwd_ms": round(pu["bwd"], 4), "unfused_ms": round(msu, 4),
            "speedup": round(msu / msf, 3)}


def bench_delta_kata(steps, settle_s):
    """The SPD delta rule (DeltaKata, kata/spd/flash_delta.py:1060-1116)
    forward (the training variant, which keeps what the backward reads) and
    backward at the KATA bench shape with the mixer's settings
    (configs/model/kata_delta_m1_340m.yaml: M=1, delta_scale 0.5, l2-normalised
    q, k, beta = sigmoid): B8 H12 T2048 D64 bf16 through linatt_dkata_fwd.
    Algorithmic FLOPs, causal pairs T^2/2 per head: the Gram kappa(k, k)
    (2 M D) and the Ec product (2 dv) of the solve, the readout kappa(q, k)
    (2 M D) and its product (2 dv)."""
    import torch
    from linatt_amd import _lib
    L = _lib.load()
    B, H, T, D, M, scale = 8, 12, 2048, 64, 1, 0.5
    g = torch.Generator().manual_seed(6)
    nrm = lambda x: x * torch.rsqrt((x * x).sum(-1, keepdim=True))  # noqa: E731
    q = nrm(torch.randn(B, T, H, D, generator=g)).to(torch.bfloat16)
    k = nrm(torch.randn(B, T, H, D, generator=g)).to(torch.bfloat16)
    v = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    dev = torch.device("cuda", 0)
    qd, kd, vd, bd = (x.to(dev) for x in (q, k, v, beta))
    o = torch.empty(B, T, H, D, device=dev)
    den = torch.empty(B, T, H, device=dev)
    dt = _lib.LINATT_BFLOAT16
    ws = torch.empty(L.linatt_dkata_workspace_bytes(B, T, H, D, D, dt), device=dev,
                     dtype=torch.uint8)
    P, sp = _lib.ptr, _lib.stream_of(qd)

    U = None  # the training forward keeps no float32 U (as flash_delta's autograd does)
    do = torch.randn(B, T, H, D, generator=g).to(dev)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    dbeta = torch.empty(B, T, H, device=dev)
    bws = torch.empty(L.linatt_dkata_bwd_workspace_bytes(B, T, H, D, D, dt), device=dev,
                      dtype=torch.uint8)

    def timed(norm):
        """(fwd ms, bwd ms) with normalize = norm: o = num / (den + eps), whose
        backward also reads o."""
        def fwd():
            _lib.check("linatt_dkata_fwd_train", L.linatt_dkata_fwd_train(
                P(qd), P(kd), P(vd), P(bd), P(U), P(o), P(den), P(ws), B, T, H, D, D, M, scale,
                norm, 1e-5, dt, sp))

        def bwd():
            _lib.check("linatt_dkata_bwd", L.linatt_dkata_bwd(
                P(qd), P(kd), P(vd), P(bd), P(U), P(o) if norm else None, P(den), P(do), P(dq),
                P(dk), P(dv), P(dbeta), P(ws), P(bws), B, T, H, D, D, M, scale, norm, 1e-5, dt, sp))

        settle([("fwd", fwd), ("bwd", bwd)], settle_s)
        stream = torch.cuda.current_stream(dev)
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
        torch.cuda.synchronize()
        for s_ in range(steps):
            ev[s_][0].record(stream)
            fwd()
            ev[s_][1].record(stream)
            bwd()
            ev[s_][2].record(stream)
        torch.cuda.synchronize()
        return (sum(e[0].elapsed_time(e[1]) for e in ev) / steps,
                sum(e[1].elapsed_time(e[2]) for e in ev) / steps)

    # the mixer's setting (delta_normalize defaults to False, kata/layer.py:59)
    # first, then the normalised form
    f_ms, b_ms = timed(0)
    fn_ms, bn_ms = timed(1)
    flops = B * H * T * T / 2 * (4 * M * D + 4 * D)
    tf = flops / (f_ms * 1e-3) / 1e12
    return {"config": {"B": B, "H": H, "T": T, "D": D, "num_groups": M, "scale": scale,
                       "normalize": False, "seed": 6},
            "fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4),
            "tokens_per_s_fwd_bwd": round(B * T / ((f_ms + b_ms) * 1e-3), 1),
            "fwd_alg_gflop": round(flops / 1e9, 2), "fwd_tflops": round(tf, 1),
            "fwd_frac_mfma_peak": round(tf / PEAK_BF16_TFLOPS, 4),
            "normalize_fwd_ms": round(fn_ms, 4), "normalize_bwd_ms": round(bn_ms, 4)}


def bench_mixer(steps, settle_s):
    """The mixer's non-GEMM ops at the 200M KATA shape (B8 T2048, hidden 768,
    12 heads of 64; configs/model/200m/kata_quadratic_200m.yaml: short conv 4
    with SiLU on q, k, v, output RMSNorm): linatt_short_conv_fwd/bwd on one
    (B, T, 768) bf16 tensor, linatt_rmsnorm_fwd/bwd on (B*T*12, 64) bf16 and
    linatt_rope forward / inverse (interleaved, the full head), each against
    HBM with its compulsory bytes (inputs read once, outputs written once);
    then the fused q/k prologue linatt_qk_prologue_fwd/bwd (the same three
    steps with the RMSNorm over each head, one kernel each way) beside the sum
    of the three unfused kernels."""
    import torch
    from linatt_amd import _lib
    L = _lib.load()
    B, T, C, W, H, D = 8, 2048, 768, 4, 12, 64
    g = torch.Generator().manual_seed(7)
    dev = torch.device("cuda", 0)
    x = torch.randn(B, T, C, generator=g).bfloat16().to(dev)
    dy = torch.randn(B, T, C, generator=g).bfloat16().to(dev)
    w = (torch.randn(C, W, generator=g) / W).to(dev)
    y, dx = torch.empty_like(x), torch.empty_like(x)
    dw = torch.empty(C, W, device=dev)
    cws = torch.empty(L.linatt_short_conv_bwd_workspace_bytes(B, T, C, W), device=dev,
                      dtype=torch.uint8)
    n = B * T * H
    rw = torch.ones(D, device=dev)
    rstd = torch.empty(n, device=dev)
    rdw = torch.empty(D, device=dev)
    rws = torch.empty(L.linatt_rmsnorm_bwd_workspace_bytes(n, D), device=dev, dtype=torch.uint8)
    qws = torch.empty(L.linatt_qk_prologue_bwd_workspace_bytes(B, T, H, D, W), device=dev,
                      dtype=torch.uint8)
    P, sp, bf = _lib.ptr, _lib.stream_of(x), _lib.LINATT_BFLOAT16
    parts = [
        ("short_conv_fwd", lambda: _lib.check("linatt_short_conv_fwd", L.linatt_short_conv_fwd(
            P(x), P(w), None, None, P(y), None, B, T, C, W, 1, bf, sp))),
        ("short_conv_bwd", lambda: _lib.check("linatt_short_conv_bwd", L.linatt_short_conv_bwd(
            P(x), P(w), None, None, P(dy), P(dx), P(dw), None, P(cws), B, T, C, W, 1, bf, sp))),
        ("rmsnorm_fwd", lambda: _lib.check("linatt_rmsnorm_fwd", L.linatt_rmsnorm_fwd(
            P(x), P(rw), P(y), P(rstd), n, D, 1e-5, bf, sp))),
        ("rmsnorm_bwd", lambda: _lib.check("linatt_rmsnorm_bwd", L.linatt_rmsnorm_bwd(
            P(x), P(rw), P(rstd), P(dy), P(dx), P(rdw), P(rws), n, D, bf, sp))),
        ("rope_fwd", lambda: _lib.check("linatt_rope", L.linatt_rope(
            P(x), P(y), B, T, H, D, D, 10000.0, 0, 1, 0, bf, sp))),
        ("rope_bwd", lambda: _lib.check("linatt_rope", L.linatt_rope(
            P(dy), P(dx), B, T, H, D, D, 10000.0, 0, 1, 1, bf, sp))),
        ("qk_prologue_fwd", lambda: _lib.check("linatt_qk_prologue_fwd", L.linatt_qk_prologue_fwd(
            P(x), P(w), None, None, P(rw), P(y), None, B, T, H, D, W, 1, 1, 1e-5, D, D, 10000.0,
            0, 1, bf, sp))),
        ("qk_prologue_bwd", lambda: _lib.check("linatt_qk_prologue_bwd", L.linatt_qk_prologue_bwd(
            P(x), P(w), None, None, P(rw), P(dy), P(dx), P(dw), None, P(rdw), P(qws), B, T, H, D,
            W, 1, 1, 1e-5, D, D, 10000.0, 0, 1, bf, sp))),
    ]
    settle(parts, settle_s)
    stream = torch.cuda.current_stream(dev)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(parts) + 1)] for _ in range(steps)]
    for s_ in range(steps):
        ev[s_][0].record(stream)
        for i, (_, f) in enumerate(parts):
            f()
            ev[s_][i + 1].record(stream)
    torch.cuda.synchronize()
    nb = B * T * C * 2
    alg = {"short_conv_fwd": 2 * nb, "short_conv_bwd": 3 * nb, "rmsnorm_fwd": 2 * nb + n * 4,
           "rmsnorm_bwd": 3 * nb + n * 4, "rope_fwd": 2 * nb, "rope_bwd": 2 * nb,
           "qk_prologue_fwd": 2 * nb, "qk_prologue_bwd": 3 * nb}
    out = {"config": {"B": B, "T": T, "hidden": C, "kernel_size": W, "heads": H, "head_dim": D,
                      "dtype": "bf16", "seed": 7}}
    for i, (name, _) in enumerate(parts):
        ms = sum(ev[s_][i].elapsed_time(ev[s_][i + 1]) for s_ in range(steps)) / steps
        gbs = alg[name] / (ms * 1e-3) / 1e9
        out[name] = {"avg_ms": round(ms, 4), "alg_mb": round(alg[name] / 1e6, 1),
                     "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    for d in ("fwd", "bwd"):
        chain = sum(out[f"{k}_{d}"]["avg_ms"] for k in ("short_conv", "rmsnorm", "rope"))
        out[f"qk_chain_unfused_{d}_ms"] = round(chain, 4)
        out[f"qk_fused_speedup_{d}"] = round(chain / out[f"qk_prologue_{d}"]["avg_ms"], 2)
    return out


def delta_inputs(B, H, T, K, V, gated, seed):
    """Config 3 / 4 inputs, drawn on the CPU in float32 (q, v ~ N(0,1); k
    ~ N(0,1) l2-normalised; beta = sigmoid(N(0,1)); g = logsigmoid(N(0,1)+4)/16;
    h0 ~ N(0, 0.02^2)), rounded once to bf16 where the op takes bf16."""
    import torch
    g_ = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g_).to(torch.bfloat16)
    k = torch.randn(B, T, H, K, generator=g_)
    k = (k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, generator=g_).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g_))
    g = torch.nn.functional.logsigmoid(torch.randn(B, T, H, generator=g_) + 4) / 16 if gated else None
    h0 = torch.randn(B, H, K, V, generator=g_) * 0.02 if gated else None
    do = torch.randn(B, T, H, V, generator=g_).to(torch.bfloat16)
    return q, k, v, beta, g, h0, do


def bench_state(prefill_reps, decode_steps, settle_s):
    """KATA-SPD M=4, B=1 H=12 D=64 bf16.  A T=32768 prefill
    (linatt_kata_prefill: o, den and the fp32 psi-state), then decode steps at
    batch 64 from the broadcast prefill state with fresh q, k, v ~ N(0,1)/8
    per step (seed 4000+i, all resident on the device before timing).
    Algorithmic prefill work in the O(T) form: states 2 T P dv + readout
    2 T P dv + chunk-local scores (about 105 GFLOP at this shape); decode bytes per step:
    the fp32 state read + written, 2 B H (P dv + P) 4 + inputs/outputs.  The
    same decode steps also run on the packed state (one row per unordered
    pair a <= b of each group, P' = M E (E + 1) / 2 rows: decode_packed_*)."""
    import torch
    from linatt_amd import _lib
    L = _lib.load()
    B, H, T, D, M = 1, 12, 32768, 64, 4
    P = M * (D // M) ** 2
    scale = 1.0 / math.sqrt(D // M)
    g = torch.Generator().manual_seed(4)
    q, k, v = ((torch.randn(B, T, H, D, generator=g) / 8).to(torch.bfloat16) for _ in range(3))
    dev = torch.device("cuda", 0)
    qd, kd, vd = (x.to(dev) for x in (q, k, v))
    o = torch.empty_like(vd)
    den = torch.empty(B, T, H, device=dev)
    S = torch.empty(B, H, P, D, device=dev)
    z = torch.empty(B, H, P, device=dev)
    dt = _lib.LINATT_BFLOAT16
    seg = 1024
    ws = torch.empty(L.linatt_kata_prefill_workspace_bytes(B, T, H, D, D, M, seg, dt), device=dev,
                     dtype=torch.uint8)
    Pp = _lib.ptr
    sp = _lib.stream_of(qd)
    stream = torch.cuda.current_stream(dev)

    def prefill():
        _lib.check("linatt_kata_prefill", L.linatt_kata_prefill(
            Pp(qd), Pp(kd), Pp(vd), Pp(o), Pp(den), Pp(S), Pp(z), Pp(ws), B, T, H, D, D, M, scale,
            1e-6, seg, 0, dt, sp))

    settle([("prefill", prefill)], settle_s)
    prefill()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(prefill_reps):
        prefill()
    e1.record(stream)
    torch.cuda.synchronize()
    pre_ms = e0.elapsed_time(e1) / prefill_reps

    Bd = 64
    Sd = S.expand(Bd, H, -1, -1).contiguous()
    zd = z.expand(Bd, H, -1).contiguous()
    steps = []
    for i in range(decode_steps):
        gi = torch.Generator().manual_seed(4000 + i)
        steps.append(tuple((torch.randn(Bd, H, D, generator=gi) / 8).to(torch.bfloat16).to(dev)
                           for _ in range(3)))
    od = torch.empty(Bd, H, D, device=dev, dtype=torch.bfloat16)

    def decode(x):
        _lib.check("linatt_kata_decode_step", L.linatt_kata_decode_step(
            Pp(x[0]), Pp(x[1]), Pp(x[2]), Pp(Sd), Pp(zd), Pp(od), Bd, H, D, D, M, scale, 1e-6, dt,
            sp))

    decode(steps[0])
    torch.cuda.synchronize()
    e0.record(stream)
    for x in steps:
        decode(x)
    e1.record(stream)
    torch.cuda.synchronize()
    dec_ms = e0.elapsed_time(e1) / decode_steps

    # the same steps on the packed state (one row per unordered pair a <= b
    # of each group: M E (E + 1) / 2 rows instead of M E^2)
    from linatt_amd import spd_state
    PT = spd_state.state_rows(D, M, True)
    Sp1, zp1 = spd_state.pack_state(S, z, M)
    Sp = Sp1.expand(Bd, H, -1, -1).contiguous()
    zp = zp1.expand(Bd, H, -1).contiguous()

    def decode_packed(x):
        _lib.check("linatt_kata_decode_step_packed", L.linatt_kata_decode_step_packed(
            Pp(x[0]), Pp(x[1]), Pp(x[2]), Pp(Sp), Pp(zp), Pp(od), Bd, H, D, D, M, scale, 1e-6, dt,
            sp))

    decode_packed(steps[0])
    torch.cuda.synchronize()
    e0.record(stream)
    for x in steps:
        decode_packed(x)
    e1.record(stream)
    torch.cuda.synchronize()
    decp_ms = e0.elapsed_time(e1) / decode_steps
    pre_flops = 2 * (2 * T * P * D) * B * H + B * H * T * 32 * 2 * D  # states, readout, chunk scores
    pre_bytes = B * H * T * D * 2 * 4 + B * H * T * 4 + B * H * (P * D + P) * 4
    dec_bytes = 2 * Bd * H * (P * D + P) * 4 + Bd * H * 4 * D * 2
    decp_bytes = 2 * Bd * H * (PT * D + PT) * 4 + Bd * H * 4 * D * 2
    return {"config": {"B": B, "H": H, "T": T, "D": D, "num_groups": M, "seg_len": seg,
                       "decode_batch": Bd, "decode_steps": decode_steps, "seed": 4},
            "prefill_ms": round(pre_ms, 4),
            "prefill_tokens_per_s": round(B * T / (pre_ms * 1e-3), 1),
            "prefill_alg_gflop": round(pre_flops / 1e9, 2),
            "prefill_tflops": round(pre_flops / (pre_ms * 1e-3) / 1e12, 1),
            "prefill_hbm_frac": round(pre_bytes / (pre_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "decode_ms_per_step": round(dec_ms, 4),
            "decode_steps_per_s": round(1e3 / dec_ms, 1),
            "decode_bytes_per_step": dec_bytes,
            "decode_gbs": round(dec_bytes / (dec_ms * 1e-3) / 1e9, 1),
            "decode_hbm_frac": round(dec_bytes / (dec_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "decode_packed_ms_per_step": round(decp_ms, 4),
            "decode_packed_bytes_per_step": decp_bytes,
            "decode_packed_gbs": round(decp_bytes / (decp_ms * 1e-3) / 1e9, 1),
            "decode_packed_hbm_frac": round(decp_bytes / (decp_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}


def bench_gen_decode(decode_steps):
    """Decode steps of the generic state kernels (linatt_kata_gen_decode: the
    flash scores outside the MFMA state form) at batch 64, 12 heads, bf16,
    from a fixed random fp32 state, in the full layout (P rows) and the
    packed one (P' rows, one per pair a <= b: variant | LINATT_KATA_PACKED_STATE).
    Fresh q, k, v ~ N(0,1)/8 per step, resident before timing.  Bytes per step:
    the state read + written, 2 B H (P dv + P) 4, + inputs/outputs."""
    import torch
    from linatt_amd import _lib
    from linatt_amd.kata_cache import state_rows
    L = _lib.load()
    dev = torch.device("cuda", 0)
    B, H, dv = 64, 12, 64
    dt = _lib.LINATT_BFLOAT16
    out = {}
    for name, dk, M, variant, decay in (("concat_m1_d64", 64, 1, "concat", False),
                                        ("sum_m4_d64", 64, 4, "sum", False),
                                        ("decay_m2_dk128", 128, 2, "concat", True)):
        g = torch.Generator().manual_seed(21)
        steps = [tuple((torch.randn(B, H, w, generator=g) / 8).to(torch.bfloat16).to(dev)
                       for w in (dk, dk, dv)) for _ in range(decode_steps)]
        c = torch.full((B, H), -0.01, device=dev) if decay else None
        od = torch.empty(B, H, dv, device=dev, dtype=torch.bfloat16)
        scale = 1.0 / math.sqrt(dk // M)
        var0 = 1 if variant == "sum" else 0
        res = {"dk": dk, "num_groups": M, "variant": variant, "decay": decay}
        for tag, packed in (("full", False), ("packed", True)):
            P = state_rows(dk, M, variant, packed)
            S = (torch.randn(B, H, P, dv, generator=g) * 0.01).to(dev)
            z = (1.0 + torch.rand(B, H, P, generator=g)).to(dev)
            var = var0 | (_lib.LINATT_KATA_PACKED_STATE if packed else 0)

            def dec(x):
                _lib.check("linatt_kata_gen_decode", L.linatt_kata_gen_decode(
                    _lib.ptr(x[0]), _lib.ptr(x[1]), _lib.ptr(x[2]), _lib.ptr(c), _lib.ptr(S),
                    _lib.ptr(z), _lib.ptr(od), B, H, dk, dv, M, var, scale, 1e-6, dt,
                    _lib.stream_of(od)))

            dec(steps[0])
            torch.cuda.synchronize()
            stream = torch.cuda.current_stream(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for x in steps:
                dec(x)
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / decode_steps
            nbytes = 2 * B * H * (P * dv + P) * 4 + B * H * (2 * dk + 2 * dv) * 2
            res[tag] = {"rows": P, "ms_per_step": round(ms, 4), "bytes_per_step": nbytes,
                        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
            del S, z
        out[name] = res
    out["config"] = {"B": B, "H": H, "dv": dv, "decode_steps": decode_steps, "seed": 21}
    return out


def bench_gen_prefill(reps):
    """Cached prefill of the flash scores outside the MFMA state form
    (``kata_cache.parallel_kata_attn_cached``: the flash forward, then the
    generic state kernels) at B8 H12 T2048 bf16: from an empty cache
    (forward + state update) and continued from a state of 2048 tokens
    (forward + readout + update).  The update's and readout's products are
    2 B H T P dv FLOP each (P the packed state rows)."""
    import torch
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    from linatt_amd.parallel_kata_attn import _fwd as kata_fwd
    dev = torch.device("cuda", 0)
    B, H, T, dv = 8, 12, 2048, 64
    stream = torch.cuda.current_stream(dev)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    out = {}
    for name, dk, M, variant, decay in (("concat_m1_d64", 64, 1, "concat", False),
                                        ("sum_m4_d64", 64, 4, "sum", False),
                                        ("sum_m2_d64", 64, 2, "sum", False),
                                        ("decay_m2_dk128", 128, 2, "concat", True)):
        g = torch.Generator().manual_seed(31)
        q, k = ((torch.randn(B, T, H, dk, generator=g) * 0.5).to(torch.bfloat16).to(dev)
                for _ in range(2))
        v = torch.randn(B, T, H, dv, generator=g).to(torch.bfloat16).to(dev)
        c = -(torch.rand(B, T, H, generator=g) * 0.05).cumsum(1).to(dev) if decay else None
        sc = 1.0 / math.sqrt(dk // M)
        fwd_ms = timed(lambda: kata_fwd(q, k, v, M, sc, variant, c))
        pre_ms = timed(lambda: parallel_kata_attn_cached(q, k, v, None, M, None, variant=variant,
                                                         c=c))
        _, st = parallel_kata_attn_cached(q, k, v, None, M, None, variant=variant, c=c)
        S0, z0 = st.S.clone(), st.z.clone()

        def restore():
            st.S.copy_(S0)
            st.z.copy_(z0)

        def cont():
            restore()
            parallel_kata_attn_cached(q, k, v, st, M, None, variant=variant, c=c)

        cont_ms = timed(cont) - timed(restore)
        P = st.S.shape[2]
        flop = 2 * B * H * T * P * dv
        upd_ms = pre_ms - fwd_ms
        out[name] = {"state_rows": P, "forward_ms": round(fwd_ms, 4),
                     "prefill_from_empty_ms": round(pre_ms, 4),
                     "continued_prefill_ms": round(cont_ms, 4),
                     "update_ms": round(upd_ms, 4), "readout_ms": round(cont_ms - pre_ms, 4),
                     "update_tflops": round(flop / (upd_ms * 1e-3) / 1e12, 1),
                     "readout_tflops": round(flop / ((cont_ms - pre_ms) * 1e-3) / 1e12, 1)}
        del st, S0, z0
    out["config"] = {"B": B, "H": H, "T": T, "dv": dv, "dtype": "bf16", "reps": reps, "seed": 31}
    return out


def bench_cache_serving(decode_steps):
    """The decode cache end to end through its public call
    (``kata_cache.parallel_kata_attn_cached``), as a serving loop drives it:
    a B8 H12 T2048 bf16 prompt into an empty cache, then single-token decode
    steps (fresh q, k, v ~ N(0,1)/8 per step, resident before timing) on the
    state it left.  Per score: the prompt's ms and the decode step's ms
    (tokens/s = B / step), called eagerly and replayed from a HIP graph of 16
    steps."""
    import torch
    from linatt_amd.kata_cache import parallel_kata_attn_cached
    dev = torch.device("cuda", 0)
    B, H, T, dv = 8, 12, 2048, 64
    stream = torch.cuda.current_stream(dev)
    out = {}
    for name, dk, M, variant, decay in (("concat_m4_d64", 64, 4, "concat", False),
                                        ("concat_m1_d64", 64, 1, "concat", False),
                                        ("sum_m4_d64", 64, 4, "sum", False),
                                        ("decay_m2_dk128", 128, 2, "concat", True)):
        g = torch.Generator().manual_seed(41)
        q, k = ((torch.randn(B, T, H, dk, generator=g) / 8).to(torch.bfloat16).to(dev)
                for _ in range(2))
        v = (torch.randn(B, T, H, dv, generator=g) / 8).to(torch.bfloat16).to(dev)
        c = -(torch.rand(B, T, H, generator=g) * 0.05).cumsum(1).to(dev) if decay else None
        steps = [tuple((torch.randn(B, 1, H, w, generator=g) / 8).to(torch.bfloat16).to(dev)
                       for w in (dk, dk, dv)) for _ in range(decode_steps)]
        cs = torch.full((B, 1, H), -0.01, device=dev) if decay else None
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        parallel_kata_attn_cached(q, k, v, None, M, None, variant=variant, c=c)  # warm
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(3):
            _, st = parallel_kata_attn_cached(q, k, v, None, M, None, variant=variant, c=c)
        e1.record(stream)
        torch.cuda.synchronize()
        pre_ms = e0.elapsed_time(e1) / 3
        parallel_kata_attn_cached(*steps[0], st, M, None, variant=variant, c=cs)
        torch.cuda.synchronize()
        e0.record(stream)
        for x in steps:
            _, st = parallel_kata_attn_cached(*x, st, M, None, variant=variant, c=cs)
        e1.record(stream)
        torch.cuda.synchronize()
        dec_ms = e0.elapsed_time(e1) / decode_steps
        # the same steps replayed from a HIP graph (the calls are capturable:
        # no memsets, no host synchronisation), which removes the host side
        # of each call
        ng = 16

        def loop():
            s_ = st
            for x in steps[:ng]:
                _, s_ = parallel_kata_attn_cached(*x, s_, M, None, variant=variant, c=cs)
            return s_

        side = torch.cuda.Stream(dev)
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            loop()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            loop()
        graph.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(4):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        gr_ms = e0.elapsed_time(e1) / (4 * ng)
        out[name] = {"state_rows": st.S.shape[2], "prompt_ms": round(pre_ms, 4),
                     "prompt_tokens_per_s": round(B * T / (pre_ms * 1e-3), 1),
                     "decode_ms_per_step": round(dec_ms, 4),
                     "decode_tokens_per_s": round(B / (dec_ms * 1e-3), 1),
                     "decode_graph_ms_per_step": round(gr_ms, 4),
                     "decode_graph_tokens_per_s": round(B / (gr_ms * 1e-3), 1)}
        del st, graph
    out["config"] = {"B": B, "H": H, "T": T, "dv": dv, "dtype": "bf16",
                     "decode_steps": decode_steps, "seed": 41}
    return out


def _cpu_threads():
    """Threads for the CPU baselines: every core the host reports, capped at
    the 16 CPUs the GPU box allots to one GPU."""
    import torch
    n = os.cpu_count() or 1
    torch.set_num_threads(min(n, 16))
    return {"cores": torch.get_num_threads(), "os_cpu_count": n, "cpu_model": _cpu_model()}


def _oracle():
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import delta as D, kata as K
    return K, D


def cpu_baseline(q, k, v, do, M, seconds):
    """Time the float32 restatement of the reference path (dense forward +
    explicit backward, kata/parallel_kata_attn.py:49-146) head by head on the
    host until `seconds` elapse; return tokens/s scaled to the full step."""
    import torch
    K, _ = _oracle()
    th = _cpu_threads()
    B, T, H, D = q.shape
    heads = [(b, h) for b in range(B) for h in range(H)]
    done = 0
    t0 = time.perf_counter()
    for b, h in heads:
        sl = lambda x: x[b:b + 1, :, h:h + 1]  # noqa: E731
        o, den = K.kata_fwd(sl(q), sl(k), sl(v), M, work_dtype=torch.float32)
        K.kata_bwd(sl(q), sl(k), sl(v), o, den, sl(do), M, work_dtype=torch.float32)
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    tokens = done / len(heads) * B * T
    return {"value": tokens / el, "unit": "tokens/s", **th, "kind": "port",
            "sample": f"{done} of {len(heads)} (batch, head) slices of config 2 "
                      f"(T={T}, M={M}), float32 dense fwd + explicit bwd, {el:.1f} s"}


def cpu_baseline_config1(qkv, M, seconds):
    """Config 1 (forward only, (1, 4, 512, 64) fp32, M groups): the float32
    dense forward of the reference (kata/parallel_kata_attn.py:49-75) on the
    whole input, repeated until `seconds` elapse."""
    import torch
    K, _ = _oracle()
    th = _cpu_threads()
    q, k, v = qkv
    B, T, H, D = q.shape
    reps = 0
    t0 = time.perf_counter()
    while True:
        K.kata_fwd(q, k, v, M, work_dtype=torch.float32)
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    return {"value": reps * B * T / el, "unit": "tokens/s", **th, "kind": "port",
            "sample": f"{reps} full config-1 forwards (B={B} T={T} H={H} M={M}), float32, "
                      f"{el:.1f} s"}


def cpu_baseline_delta(gated, seconds):
    """Config 3 / 4: the chunked WY/UT restatement (oracle/delta.py) in float32
    with autograd for the backward, (batch, head) slice by slice until
    `seconds` elapse; tokens/s scaled to the full config."""
    import torch
    _, Dm = _oracle()
    th = _cpu_threads()
    B, H, T, Kd, Vd = 8, 6, 2048, 128, 128
    q, k, v, beta, g, h0, do = delta_inputs(B, H, T, Kd, Vd, gated, 3 if gated else 2)
    heads = [(b, h) for b in range(B) for h in range(H)]
    done = 0
    t0 = time.perf_counter()
    for b, h in heads:
        sl = lambda x: x[b:b + 1, :, h:h + 1].float().requires_grad_(True)  # noqa: E731
        leaves = [sl(q), sl(k), sl(v), beta[b:b + 1, :, h:h + 1].clone().requires_grad_(True)]
        gg = g[b:b + 1, :, h:h + 1].clone().requires_grad_(True) if gated else None
        hh = h0[b:b + 1, h:h + 1].clone().requires_grad_(True) if gated else None
        o, ht = Dm.delta_rule_chunked(*leaves, g=gg, scale=Kd ** -0.5, initial_state=hh)
        (o * do[b:b + 1, :, h:h + 1].float()).sum().backward()
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    return {"value": done / len(heads) * B * T / el, "unit": "tokens/s", **th, "kind": "port",
            "sample": f"{done} of {len(heads)} (batch, head) slices of config "
                      f"{4 if gated else 3}, float32 chunked fwd + autograd bwd, {el:.1f} s"}


def bench_config1(steps):
    """Config 1 on the GPU: the fp32 KATA forward at (1, 512, 4, 64), M=4,
    q, k, v i.i.d. N(0,1) (seed 0), through linatt_kata_fwd."""
    import torch
    from linatt_amd import _lib
    L = _lib.load()
    B, T, H, D, M = 1, 512, 4, 64, 4
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, T, H, D, generator=g) for _ in range(3))
    dev = torch.device("cuda", 0)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    o = torch.empty_like(qd)
    den = torch.empty(B, T, H, device=dev)
    sp = _lib.stream_of(qd)
    P = _lib.ptr

    def fwd():
        _lib.check("linatt_kata_fwd", L.linatt_kata_fwd(
            P(qd), P(kd), P(vd), None, P(o), P(den), B, T, H, H, D, D, M, 1.0 / math.sqrt(D // M),
            0, _lib.LINATT_FLOAT32, sp))

    for _ in range(3):
        fwd()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        fwd()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    return (q, k, v), {"config": {"B": B, "T": T, "H": H, "D": D, "num_groups": M, "dtype": "f32",
                          "seed": 0},
               "fwd_ms": round(ms, 4), "tokens_per_s": round(B * T / (ms * 1e-3), 1)}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# HBM bytes per launch of the config-2 kernels (FETCH_SIZE x 1024 x 2.0 +
# WRITE_SIZE x 1024 x 1.0, the factors a 512 MiB device copy gives the two
# counters), from the rocprofv3 --pmc runs summarised in
# profiles/hbm_traffic_bench_all_workloads.md.  Counters cannot be read from
# inside the timed run, so the figure is carried here and refreshed with the
# profile.
MEASURED_TRAFFIC_BYTES = {
    "fwd": int((121.7 + 30.5) * 1e6),
    "bwd_dq": int((182.1 + 61.1) * 1e6),
    "bwd_dkdv": int((170.9 + 50.3) * 1e6),
}


def copy_calibration():
    """A plain device copy of known size (512 MiB bf16, 3 launches), the
    reference against which the rocprofv3 FETCH_SIZE / WRITE_SIZE counters are
    scaled into bytes."""
    import torch
    n = 256 * 1024 * 1024
    src = torch.empty(n, device="cuda", dtype=torch.bfloat16).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n * 2, "launches": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--groups", type=int, default=4)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-delta", action="store_true")
    ap.add_argument("--no-state", action="store_true")
    ap.add_argument("--no-kata", action="store_true",
                    help="skip the KATA config-2 timing (profiling the other workloads)")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--settle-seconds", type=float, default=1.5,
                    help="untimed sustained load before each workload's warmup steps")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 512 MiB device copy (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; multi-GPU runs are not part of "
              "it. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration()
        return

    import torch
    from linatt_amd import _lib
    L = _lib.load()

    B, H, T, D, M = 8, 12, 2048, 64, args.groups
    scale = 1.0 / math.sqrt(D // M)
    g = torch.Generator().manual_seed(1)
    q, k, v = ((torch.randn(B, T, H, D, generator=g) / 8).to(torch.bfloat16) for _ in range(3))
    do = torch.randn(B, T, H, D, generator=g).to(torch.bfloat16)
    dev = torch.device("cuda", 0)
    qd, kd, vd, dod = (x.to(dev) for x in (q, k, v, do))
    o = torch.empty_like(vd)
    den = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
    ws = torch.empty(L.linatt_kata_bwd_workspace_bytes(B, T, H, D, _lib.LINATT_BFLOAT16) // 4, device=dev,
                     dtype=torch.float32)
    P = _lib.ptr
    dt = _lib.LINATT_BFLOAT16
    stream = torch.cuda.current_stream(dev)
    sp = _lib.stream_of(qd)
    bargs = (P(qd), P(kd), P(vd), P(o), P(den), P(dod), P(dq), P(dk), P(dv), P(ws),
             B, T, H, H, D, D, M, scale, 0, dt, sp)

    def fwd():
        _lib.check("linatt_kata_fwd", L.linatt_kata_fwd(
            P(qd), P(kd), P(vd), None, P(o), P(den), B, T, H, H, D, D, M, scale, 0, dt, sp))

    def bwd_dq():
        _lib.check("linatt_kata_bwd_dq", L.linatt_kata_bwd_dq(*bargs))

    def bwd_dkdv():
        _lib.check("linatt_kata_bwd_dkdv", L.linatt_kata_bwd_dkdv(*bargs))

    parts = [("fwd", fwd), ("bwd_dq", bwd_dq), ("bwd_dkdv", bwd_dkdv)]
    if args.no_kata:
        args.steps, args.warmup = 1, 0
    else:
        settle(parts, args.settle_seconds)
    for _ in range(args.warmup):
        for _, f in parts:
            f()
    torch.cuda.synchronize()

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(parts) + 1)]
          for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for s in range(args.steps):
        ev[s][0].record(stream)
        for i, (_, f) in enumerate(parts):
            f()
            ev[s][i + 1].record(stream)
    stop.record(stream)
    torch.cuda.synchronize()
    ms_total = start.elapsed_time(stop)
    ms_step = ms_total / args.steps
    kern_ms = {name: sum(ev[s][i].elapsed_time(ev[s][i + 1]) for s in range(args.steps)) / args.steps
               for i, (name, _) in enumerate(parts)}

    fl = kata_flops(B, H, T, D, D, M)
    kern = {n: {"avg_ms": round(kern_ms[n], 4), "alg_gflop": fl[n] / 1e9,
                "tflops": fl[n] / (kern_ms[n] * 1e-3) / 1e12} for n in kern_ms}
    for n in kern:
        kern[n]["tflops"] = round(kern[n]["tflops"], 1)
        kern[n]["frac_mfma_peak"] = round(kern[n]["tflops"] / PEAK_BF16_TFLOPS, 4)
    dom = max(kern_ms, key=kern_ms.get)
    ach = fl[dom] / (kern_ms[dom] * 1e-3) / 1e12
    step_tflops = fl["total"] / (ms_step * 1e-3) / 1e12
    tokens_per_s = B * T / (ms_step * 1e-3)

    delta = None
    if not args.no_delta:
        st = args.settle_seconds / 2
        ds = max(3, args.steps // 2)
        delta = {"deltanet_config3": bench_delta(False, ds, 2, st),
                 "gated_deltanet_config4": bench_delta(True, ds, 2, st),
                 # the 200M models' own shape (configs/model/200m/gated_deltanet_200m.yaml:
                 # 12 heads of 64) and the north star's B8 H12 T2048 D64
                 "deltanet_h12_d64": bench_delta(False, ds, 2, st / 2, H=12, K=64),
                 "gated_deltanet_h12_d64": bench_delta(True, ds, 2, st / 2, H=12, K=64)}

    state = gen_decode = gen_prefill = serving = None
    if not args.no_state:
        state = bench_state(3, args.decode_steps, args.settle_seconds / 3)
        gen_decode = bench_gen_decode(max(16, args.decode_steps // 4))
        gen_prefill = bench_gen_prefill(5)
        serving = bench_cache_serving(64)

    q1, config1 = bench_config1(max(10, args.steps))
    delta_kata = None if args.no_delta else bench_delta_kata(max(3, args.steps // 2),
                                                             args.settle_seconds / 3)
    mixer = bench_mixer(max(5, args.steps), args.settle_seconds / 3)
    vs = max(5, args.steps // 2)
    variants = {
        # kata_quadratic_sum_m4_200m.yaml: 12 heads of 64, four groups
        "sum_m4_h12_d64": bench_kata_variant(vs, args.settle_seconds / 3, 8, 12, 2048, 64, 64, 4,
                                             "sum", False, 9),
        # kata_quadratic_sum_m2_200m.yaml: the same heads, two groups
        "sum_m2_h12_d64": bench_kata_variant(vs, args.settle_seconds / 3, 8, 12, 2048, 64, 64, 2,
                                             "sum", False, 11),
        # kataconv_cat_l2_gdn_340m.yaml: 16 heads, decayed concat score over
        # offset-packed groups (dk = 128, dv = 64, two groups)
        "decay_m2_h16_dk128": bench_kata_variant(vs, args.settle_seconds / 3, 8, 16, 2048, 128, 64,
                                                 2, "concat", True, 10),
    }
    onorm = bench_kata_onorm(vs, args.settle_seconds / 3, M)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(q, k, v, do, M, args.cpu_seconds)
        config1["cpu_baseline"] = cpu_baseline_config1(q1, 4, args.cpu_seconds / 3)
        if delta is not None:
            delta["deltanet_config3"]["cpu_baseline"] = cpu_baseline_delta(False, args.cpu_seconds / 3)
            delta["gated_deltanet_config4"]["cpu_baseline"] = cpu_baseline_delta(
                True, args.cpu_seconds / 3)

    out = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "kata_concat_fwd_bwd (BASELINE config 2)", "B": B, "H": H,
                   "T": T, "dk": D, "dv": D, "num_groups": M, "chunk": 64, "causal": True,
                   "seed": 1},
        "tflops": round(step_tflops, 1),
        "frac_mfma_peak": round(step_tflops / PEAK_BF16_TFLOPS, 4),
        "alg_gflop_per_step": round(fl["total"] / 1e9, 2),
        "kernels": kern,
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(ach, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ach / PEAK_BF16_TFLOPS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES.get(dom)},
        "cpu_baseline": cpu,
        "delta_rule": delta,
        "kata_state_config5": state,
        "kata_state_decode_generic": gen_decode,
        "kata_state_prefill_generic": gen_prefill,
        "kata_cache_serving": serving,
        "kata_config1": config1,
        "delta_kata_fwd_bwd": delta_kata,
        "mixer_ops": mixer,
        "kata_variants": variants,
        "kata_output_norm_config2": onorm,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
