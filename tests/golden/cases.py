"""Golden fixture recipes for the hot path: seeded inputs (drawn in float32
on the CPU, rounded once to the case's 16-bit dtype) and the float64 oracle
outputs computed from them.

The fixtures are regression vectors generated from the oracle, not vectors
taken from the reference (the reference's tests hold none for these
operators).  They guard two things: the oracle cannot drift without the CPU
test of the stored outputs failing, and the HIP path is checked against
fixed vectors on the GPU box without running the oracle there.

``CASES[name] = (inputs(seed) -> dict, outputs(inputs) -> dict, seed)``;
``inputs`` returns CPU tensors plus JSON-ready scalars under ``"params"``.
Shapes are small but cross the kernels' tile and chunk boundaries
(64-row tiles, 64-token chunks, 128-token prefill segments).
"""

from __future__ import annotations

import torch

from oracle import delta as D
from oracle import delta_kata as DK
from oracle import kata as K
from oracle import mixer as X

BF16 = torch.bfloat16


def _gen(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std


# --- KATA flash scores (parallel_kata_attn*, kata/parallel_kata_attn.py) ---

def _kata_in(seed, T, HQ, H, M, variant):
    dk = 64
    return {"q": _gen((1, T, HQ, dk), seed, 0.25).to(BF16), "k": _gen((1, T, H, dk), seed + 1, 0.25).to(BF16),
            "v": _gen((1, T, H, 64), seed + 2, 0.25).to(BF16), "do": _gen((1, T, HQ, 64), seed + 3).to(BF16),
            "params": {"M": M, "variant": variant, "scale": K.default_scale(dk, M)}}


def kata_out(x):
    p = x["params"]
    o, den = K.kata_fwd(x["q"], x["k"], x["v"], p["M"], p["scale"], p["variant"])
    dq, dk, dv = K.kata_bwd(x["q"], x["k"], x["v"], o, den, x["do"], p["M"], p["scale"], p["variant"])
    return {"o": o, "den": den, "dq": dq, "dk": dk, "dv": dv}


def kata_decay_in(seed):
    T, dk = 40, 128
    c = -torch.cumsum(torch.rand(1, T, 1, generator=torch.Generator().manual_seed(seed + 4)) * 0.1, 1)
    return {"q": _gen((1, T, 1, dk), seed, 0.125).to(BF16), "k": _gen((1, T, 1, dk), seed + 1, 0.125).to(BF16),
            "v": _gen((1, T, 1, 64), seed + 2, 0.125).to(BF16), "c": c,
            "do": _gen((1, T, 1, 64), seed + 3).to(BF16), "params": {"M": 2, "scale": K.default_scale(dk, 2)}}


def kata_decay_out(x):
    p = x["params"]
    o, dq, dk, dv, dc = K.kata_decay_fwd_bwd(x["q"], x["k"], x["v"], x["c"], x["do"], p["M"], p["scale"])
    return {"o": o, "dq": dq, "dk": dk, "dv": dv, "dc": dc}


# --- chunked (gated) delta rule (chunk_[gated_]delta_rule) ----------------

def _delta_in(seed, T, Kd, V, gated, h0):
    x = {"q": _gen((1, T, 1, Kd), seed).to(BF16), "k": D.l2norm(_gen((1, T, 1, Kd), seed + 1)).to(BF16),
         "v": _gen((1, T, 1, V), seed + 2).to(BF16), "beta": torch.sigmoid(_gen((1, T, 1), seed + 3)),
         "do": _gen((1, T, 1, V), seed + 6).to(BF16), "params": {"scale": Kd ** -0.5}}
    if gated:
        x["g"] = torch.nn.functional.logsigmoid(_gen((1, T, 1), seed + 4) + 4) / 16
    if h0:
        x["h0"] = _gen((1, 1, Kd, V), seed + 5, 0.02)
        x["dht"] = _gen((1, 1, Kd, V), seed + 7)
    return x


def delta_out(x):
    r = D.delta_rule_fwd_bwd(x["q"], x["k"], x["v"], x["beta"], x.get("g"), x["params"]["scale"],
                             x.get("h0"), x["do"], x.get("dht"))
    return {n: r[n] for n in ("o", "ht", "dq", "dk", "dv", "dbeta", "dg", "dh0") if n in r}


# --- KATA state form: config 5's prefill, then one decode step -------------

def kata_state_in(seed):
    T = 130
    return {"q": _gen((1, T + 1, 1, 64), seed).to(BF16), "k": _gen((1, T + 1, 1, 64), seed + 1).to(BF16),
            "v": _gen((1, T + 1, 1, 64), seed + 2).to(BF16),
            "params": {"M": 4, "T": T, "seg_len": 128, "eps": 1e-6}}


def kata_state_out(x):
    p = x["params"]
    M, T, eps = p["M"], p["T"], p["eps"]
    q, k, v = x["q"], x["k"], x["v"]
    o, den, S, z = K.kata_prefill_fwd_state_form(q[:, :T], k[:, :T], v[:, :T], M, eps=eps)
    o1, S1, z1 = K.kata_decode_step(S, z, q[:, T], k[:, T], v[:, T], M, eps=eps)
    return {"o": o, "den": den, "S": S, "z": z, "o_decode": o1, "z_decode": z1}


# --- SPD delta rule (flash_delta, kata/spd/flash_delta.py) -----------------

def flash_delta_in(seed):
    T, Dd = 70, 64
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(1, T, 1, Dd, generator=g), dim=-1).to(BF16)
    k = torch.nn.functional.normalize(torch.randn(1, T, 1, Dd, generator=g), dim=-1).to(BF16)
    v = torch.randn(1, T, 1, Dd, generator=g).to(BF16)
    beta = torch.sigmoid(torch.randn(1, T, 1, generator=g))
    do = torch.randn(1, T, 1, Dd, generator=g)
    return {"q": q, "k": k, "v": v, "beta": beta, "do": do, "params": {"M": 2, "scale": 0.5}}


def flash_delta_out(x):
    p = x["params"]
    o, dq, dk, dv, db = DK.flash_delta_fwd_bwd(x["q"], x["k"], x["v"], x["beta"], p["M"], x["do"], p["scale"])
    return {"o": o, "dq": dq, "dk": dk, "dv": dv, "dbeta": db}


# --- mixer prologue / epilogue (short_conv, rms_norm) ----------------------

def mixer_in(seed):
    T, C, W, Dh = 40, 128, 4, 64
    return {"x": _gen((1, T, C), seed).to(BF16), "w": _gen((C, 1, W), seed + 1, 0.5).to(BF16),
            "b": _gen((C,), seed + 2, 0.1).to(BF16), "dy": _gen((1, T, C), seed + 3).to(BF16),
            "nw": 1.0 + _gen((Dh,), seed + 4, 0.1), "params": {"head_dim": Dh, "eps": 1e-5}}


def mixer_out(x):
    y, (dx, dw, db) = X.fwd_bwd(lambda xx, ww, bb: X.short_conv(xx, ww, bb, "silu"),
                                [x["x"], x["w"], x["b"]], x["dy"])
    Dh, eps = x["params"]["head_dim"], x["params"]["eps"]
    B, T, C = x["x"].shape
    n, (dn, dnw) = X.fwd_bwd(lambda xx, ww: X.rmsnorm(xx, ww, eps),
                             [x["x"].reshape(B, T, C // Dh, Dh), x["nw"]], x["dy"].reshape(B, T, C // Dh, Dh))
    return {"conv_y": y, "conv_dx": dx, "conv_dw": dw, "conv_db": db,
            "norm_y": n, "norm_dx": dn, "norm_dw": dnw}


CASES = {
    "kata_concat_m4_gqa": (lambda s: _kata_in(s, 70, 2, 1, 4, "concat"), kata_out, 101),
    "kata_sum_m2": (lambda s: _kata_in(s, 37, 1, 1, 2, "sum"), kata_out, 102),
    "kata_decay_dk128_m2": (kata_decay_in, kata_decay_out, 103),
    "delta_gated_h0": (lambda s: _delta_in(s, 80, 64, 64, True, True), delta_out, 104),
    "delta_k128": (lambda s: _delta_in(s, 70, 128, 128, False, False), delta_out, 105),
    "kata_state_m4": (kata_state_in, kata_state_out, 106),
    "flash_delta_m2": (flash_delta_in, flash_delta_out, 107),
    "mixer": (mixer_in, mixer_out, 108),
}
