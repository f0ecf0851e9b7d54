"""KATA-SPD in psi-state form on MI355X: O(T) long-context prefill and the
recurrent decode step.

* ``spd_chunk_scan_cat(q, k, v, M, scale=None, C=32, eps=1e-6, ...)`` keeps
  the signature of the reference's concat tree-scan
  (``kata/spd/chunk_scan_cat.py:219-345``): head-major ``(B, H, T, D)``
  inputs, returns ``(o, den)`` with ``o = num / max(den, eps)``.  ``C``,
  ``warps`` and ``stages`` are accepted and ignored.  ``feature="quad"`` (the
  SPD kernel) runs the state-form prefill below; ``feature="linear"``
  (psi(x) = x, kappa = scale q.k) runs ``linatt_linear_scan_fwd``, a chunked
  linear-attention state pass (d = dv = 64).
* ``kata_prefill(q, k, v, num_groups=4, scale=None, eps=1e-6, seg_len=1024,
  initial_state=None)`` takes the time-major ``(B, T, H, D)`` layout of the
  flash path, optionally continues from a state ``(S0, z0)``, and also
  returns the state after the last token: ``S = sum_s psi(sqrt(scale) k_s)
  v_s^T`` ``(B, H, M*E*E, dv)`` and ``z = sum_s psi(sqrt(scale) k_s)``
  ``(B, H, M*E*E)``, float32, ``psi(x) = vec(x_g x_g^T)`` per group.
* ``kata_decode_step(S, z, q, k, v, num_groups=4, scale=None, eps=1e-6)``
  appends one token per ``(b, h)`` (``q, k, v`` of shape ``(B, H, D)``),
  updating ``S`` and ``z`` in place, and returns ``o (B, H, dv)``.  The
  reference's flash path keeps no decode state (``kata/layer.py:492``); this
  is the state the ``past_key_values`` cache would hold.
* The state also comes in a packed layout (``kata_prefill(...,
  packed_state=True)``; ``kata_decode_step`` takes either): psi(x) is
  symmetric in each group's (a, b), so one row per unordered pair a <= b
  holds all of it, ``M E (E + 1) / 2`` rows instead of ``M E^2`` (136 of 256
  per group at M = 4), and a decode step streams about half the bytes.
  ``pack_state`` / ``unpack_state`` convert between the layouts.

All three run in ``liblinatt_hip.so`` (``linatt_kata_prefill_state[_packed]``,
``linatt_linear_scan_fwd``, ``linatt_kata_decode_step[_packed]``); unsupported
shapes raise.
"""

from __future__ import annotations

import functools
import math

import torch

from . import _lib

_lib.load()

__all__ = ["spd_chunk_scan_cat", "kata_prefill", "kata_decode_step"]


def _scale(dk, num_groups, scale):
    return 1.0 / math.sqrt(dk // num_groups) if scale is None else float(scale)


def _check(dtype, dk, dv, M):
    L = _lib.load()
    if not L.linatt_kata_state_supported(_lib.dtype_code(dtype), dk, dv, M):
        raise NotImplementedError(
            f"linatt_amd state form: no kernel for {dtype}, dk={dk}, dv={dv}, num_groups={M}")
    return L


def state_rows(dk, num_groups, packed=False):
    """State rows per (b, h): M E^2 in the full layout, M E (E + 1) / 2 in the
    packed one (one row per unordered pair a <= b of each group)."""
    E = dk // num_groups
    return num_groups * E * (E + 1) // 2 if packed else num_groups * E * E


def _pair_index(dk, num_groups, device):
    """(full rows of the packed rows, packed row of every full row)."""
    E, M = dk // num_groups, num_groups
    full_of, tri_of = [], [0] * (M * E * E)
    for g in range(M):
        for a in range(E):
            for b in range(a, E):
                t = len(full_of)
                full_of.append(g * E * E + a * E + b)
                tri_of[g * E * E + a * E + b] = t
                tri_of[g * E * E + b * E + a] = t
    return (torch.tensor(full_of, device=device, dtype=torch.long),
            torch.tensor(tri_of, device=device, dtype=torch.long))


def pack_state(S, z, num_groups):
    """Full-layout state ``S (B, H, M E^2, dv)``, ``z (B, H, M E^2)`` to the
    packed layout (the rows a <= b; linatt_kata_decode_step_packed)."""
    dk = round((S.shape[2] // num_groups) ** 0.5) * num_groups
    full_of, _ = _pair_index(dk, num_groups, S.device)
    return S.index_select(2, full_of).contiguous(), z.index_select(2, full_of).contiguous()


def unpack_state(S, z, num_groups):
    """Packed state to the full layout (each pair's row to both of its rows)."""
    E = next(e for e in range(1, 257) if num_groups * e * (e + 1) // 2 == S.shape[2])
    _, tri_of = _pair_index(E * num_groups, num_groups, S.device)
    return S.index_select(2, tri_of).contiguous(), z.index_select(2, tri_of).contiguous()


def _prefill(q, k, v, M, scale, eps, seg_len, head_major, want_state, initial_state=None,
             in_place=False, packed=False):
    _lib.require_device(q, k, v)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    if head_major:
        B, H, T, dk = q.shape
    else:
        B, T, H, dk = q.shape
    dv = v.shape[-1]
    if k.shape != q.shape or v.shape[:-1] != q.shape[:-1]:
        raise ValueError("q, k, v shapes do not match")
    if dk % M:
        raise ValueError(f"d_k={dk} not divisible by M={M}")
    L = _check(q.dtype, dk, dv, M)
    sc = _scale(dk, M, scale)
    dt = _lib.dtype_code(q.dtype)
    P = state_rows(dk, M, packed)
    o = torch.empty_like(v)
    den = torch.empty(q.shape[:-1], device=q.device, dtype=torch.float32)
    S0 = z0 = None
    if initial_state is not None:
        S0, z0 = initial_state
        _lib.require_device(S0, z0)
        if (S0.shape != (B, H, P, dv) or z0.shape != (B, H, P) or S0.dtype != torch.float32
                or z0.dtype != torch.float32 or S0.device != q.device or z0.device != q.device):
            raise ValueError(f"initial_state must be float32 S {(B, H, P, dv)}, z {(B, H, P)} "
                             f"on {q.device}")
        S0, z0 = S0.contiguous(), z0.contiguous()
    S = z = None
    if in_place and S0 is not None:
        if not (initial_state[0].is_contiguous() and initial_state[1].is_contiguous()):
            raise ValueError("an in-place state must be contiguous")
        S, z = S0, z0  # the scan reads each state element before it writes it
    elif want_state:
        S = torch.empty(B, H, P, dv, device=q.device, dtype=torch.float32)
        z = torch.empty(B, H, P, device=q.device, dtype=torch.float32)
    ws = torch.empty(L.linatt_kata_prefill_workspace_bytes(B, T, H, dk, dv, M, seg_len, dt),
                     device=q.device, dtype=torch.uint8)
    name = "linatt_kata_prefill_state_packed" if packed else "linatt_kata_prefill_state"
    _lib.check(name, getattr(L, name)(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(den), _lib.ptr(S0),
        _lib.ptr(z0), _lib.ptr(S), _lib.ptr(z), _lib.ptr(ws), B, T, H, dk, dv, M, sc, float(eps),
        seg_len, 1 if head_major else 0, dt, _lib.stream_of(q)))
    return o, den, S, z


def spd_chunk_scan_cat(q, k, v, M, scale=None, C=32, eps=1e-6, warps=4, stages=None,
                       feature="quad"):
    """Concat-SPD causal forward in state form, head-major ``(B, H, T, D)``
    (reference ``kata/spd/chunk_scan_cat.py:219-345``).  Returns ``(o, den)``."""
    if feature == "linear":
        return _linear_scan(q, k, v, M, scale, eps)
    if feature != "quad":
        raise ValueError(f"spd_chunk_scan_cat: feature must be 'quad' or 'linear', got {feature!r}")
    o, den, _, _ = _prefill(q, k, v, M, scale, eps, 1024, True, False)
    return o, den


def _linear_scan(q, k, v, M, scale, eps):
    """``feature="linear"`` of the tree-scan (``kata/spd/chunk_scan_cat.py:
    90-92, 219-235``): kappa = scale q.k, head-major ``(B, H, T, D)``."""
    _lib.require_device(q, k, v)
    B, H, T, D = q.shape
    dv = v.shape[-1]
    if k.shape != q.shape or v.shape[:3] != (B, H, T):
        raise ValueError(f"q, k must be (B, H, T, D) and v (B, H, T, dv); got q {tuple(q.shape)}, "
                         f"k {tuple(k.shape)}, v {tuple(v.shape)}")
    if D % M:
        raise ValueError(f"D={D} not divisible by M={M}")
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in (torch.bfloat16, torch.float16):
        raise NotImplementedError(f"linatt_amd linear scan: bfloat16 / float16 only, got {q.dtype}")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    o = torch.empty(B, H, T, dv, device=q.device, dtype=q.dtype)
    den = torch.empty(B, H, T, device=q.device, dtype=torch.float32)
    L = _lib.load()
    _lib.check("linatt_linear_scan_fwd", L.linatt_linear_scan_fwd(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(den), B, H, T, D, dv,
        _scale(D, M, scale), float(eps), _lib.dtype_code(q.dtype), _lib.stream_of(q)))
    return o, den


def kata_prefill(q, k, v, num_groups=4, scale=None, eps=1e-6, seg_len=1024, initial_state=None,
                 in_place=False, packed_state=False):
    """Time-major ``(B, T, H, D)`` prefill: ``(o, den, S, z)``.  With
    ``initial_state=(S0, z0)`` (the state after earlier tokens) the outputs and
    the returned state also cover those tokens; ``in_place=True`` writes that
    state back into ``S0, z0`` (returned as ``S, z``).  ``packed_state``: the
    state (returned and initial) in the packed layout, one row per unordered
    pair a <= b of each group (``state_rows``, ``pack_state`` /
    ``unpack_state``), which ``kata_decode_step`` takes as well and streams in
    about half the bytes."""
    return _prefill(q, k, v, num_groups, scale, eps, seg_len, False, True, initial_state,
                    in_place, packed_state)


def kata_decode_step(S, z, q, k, v, num_groups=4, scale=None, eps=1e-6):
    """One token per ``(b, h)``: updates ``S``, ``z`` in place and returns ``o``.
    The state may be in the full or the packed layout (told apart by its row
    count, ``state_rows``)."""
    if q.dim() != 3 or v.dim() != 3:
        raise ValueError(f"q, k must be (B, H, dk) and v (B, H, dv); got q {tuple(q.shape)}, "
                         f"v {tuple(v.shape)}")
    B, H, dk = q.shape
    dv = v.shape[-1]
    if k.shape != q.shape or v.shape[:2] != (B, H):
        raise ValueError(f"k must be {tuple(q.shape)} and v (B, H, dv) = {(B, H)} + (dv,); "
                         f"got k {tuple(k.shape)}, v {tuple(v.shape)}")
    _lib.require_device(S, z, q, k, v)
    devs = {t.device for t in (S, z, q, k, v)}
    if len(devs) != 1:
        raise ValueError(f"S, z, q, k, v must be on one device, got {sorted(map(str, devs))}")
    M = num_groups
    if dk % M:
        raise ValueError(f"d_k={dk} not divisible by M={M}")
    P, PT = state_rows(dk, M), state_rows(dk, M, True)
    packed = S.dim() == 4 and S.shape[2] == PT
    R = PT if packed else P
    if S.shape != (B, H, R, dv) or z.shape != (B, H, R):
        raise ValueError(f"state must be S {(B, H, P, dv)}, z {(B, H, P)} (full layout) or "
                         f"S {(B, H, PT, dv)}, z {(B, H, PT)} (packed)")
    if S.dtype != torch.float32 or z.dtype != torch.float32 or not (S.is_contiguous() and z.is_contiguous()):
        raise ValueError("S and z must be contiguous float32 (updated in place)")
    L = _check(q.dtype, dk, dv, M)
    q, k, v = q.contiguous(), k.to(q.dtype).contiguous(), v.to(q.dtype).contiguous()
    o = torch.empty(B, H, dv, device=q.device, dtype=q.dtype)
    # a small batch splits each (b, h)'s rows over several workgroups
    nws = _decode_workspace_bytes(B, H, dk, M, int(packed))
    if nws and _lib.split_decode_pays(R):
        ws = _lib.stream_scratch(q.device, nws)
        _lib.check("linatt_kata_decode_step_split", L.linatt_kata_decode_step_split(
            _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(S), _lib.ptr(z), _lib.ptr(o),
            _lib.ptr(ws), nws, B, H, dk, dv, M, int(packed), _scale(dk, M, scale), float(eps),
            _lib.dtype_code(q.dtype), _lib.stream_of(q)))
        return o
    name = "linatt_kata_decode_step_packed" if packed else "linatt_kata_decode_step"
    _lib.check(name, getattr(L, name)(
        _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(S), _lib.ptr(z), _lib.ptr(o), B, H, dk,
        dv, M, _scale(dk, M, scale), float(eps), _lib.dtype_code(q.dtype), _lib.stream_of(q)))
    return o


@functools.lru_cache(maxsize=64)
def _decode_workspace_bytes(B, H, dk, M, packed):
    return _lib.load().linatt_kata_decode_workspace_bytes(B, H, dk, M, packed)
