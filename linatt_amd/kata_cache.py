"""Recurrent decode state for the KATA flash mixer: the ``past_key_values``
entry the reference's flash path never fills.

The reference's flash branch sets ``final_state = None`` (``kata/layer.py:492``)
and hands it to ``update_layer_cache`` (``:532-537``), so incremental decoding
makes each new token attend only to itself; its evaluation forces
``use_cache=False`` for KATA to stay correct (``eval_recall.py:133-144``).
Every flash score has an exact O(1)-per-token state form, kept here per layer:

    S = sum_s psi(sqrt(scale) k_s) v_s^T   (B, H, P, dv) float32
    z = sum_s psi(sqrt(scale) k_s)         (B, H, P)     float32
    o_t = psi(sqrt(scale) q_t)^T S / max(psi(.) . z, eps)

with psi(x) = vec(x_g x_g^T) per group for the concat score (P = M E^2),
vec(sum_g x_g x_g^T) for the sum score (P = E^2), and, for the decayed
score, S and z scaled by exp(c_t - c_{t-1}) before each token's term.
Since x_g x_g^T is symmetric, a new state keeps only the rows a <= b of each
group (P = M E (E + 1) / 2, or E (E + 1) / 2 for the sum score), which about
halves a decode step's bytes and the cache's memory.

The concat score without decay at the MFMA state-form shapes
(``linatt_kata_state_supported``) takes a chunk of T > 1 tokens through the
state-form prefill continued from the current state
(``linatt_kata_prefill_state``; a short prompt into an empty cache, where the
flash forward is faster, goes the generic way below) and a single token
through ``linatt_kata_decode_step``.  Every other flash score (M = 1, the sum
score, the decayed score, the offset gate's padded width dk = 128) takes a
chunk through the flash forward plus the stored state's readout and a state
update, and a single token through ``linatt_kata_gen_decode``.

The cache contract is fla's (``fla.layers.utils.get_layer_cache`` /
``update_layer_cache``, imported at ``kata/layer.py:19`` from the third-party
package ``flash-linear-attention==0.5.0``, absent here): a per-layer dict with a
``"recurrent_state"`` entry, looked up by ``layer.layer_idx``, and
``past_key_values.update(recurrent_state=..., layer_idx=..., offset=...)``.
``LayerStateCache`` is a minimal object with that interface, and
``get_layer_cache`` / ``update_layer_cache`` follow fla's helpers, so the
mixer's flash branch can keep a real state:

    last_state = get_layer_cache(self, past_key_values)
    rec = last_state["recurrent_state"] if last_state is not None else None
    o, final_state = parallel_kata_attn_cached(q_in, k_in, v, rec, self.spd_num_groups, scale_in)
    update_layer_cache(self, past_key_values, recurrent_state=final_state, offset=q.shape[1])

Scope: dv = 64, dk <= 128 with a power-of-two group width of at least 16
(every flash configuration of the reference); other shapes raise.
"""

from __future__ import annotations

import functools
import math
from typing import NamedTuple

import torch

from . import _lib, spd_state
from .parallel_kata_attn import _fwd as _kata_fwd

__all__ = ["KataState", "state_rows", "parallel_kata_attn_cached", "LayerStateCache", "get_layer_cache",
           "update_layer_cache"]


class KataState(NamedTuple):
    """A layer's recurrent state: ``S (B, H, P, dv)``, ``z (B, H, P)`` float32,
    the number of tokens it covers, and the score it belongs to (``variant``
    "concat" or "sum", ``num_groups``).  A new state is kept in the packed
    layout (one row per unordered pair a <= b of each group: ``state_rows(dk,
    M, variant, packed=True)`` rows; ``spd_state.unpack_state(S, z, G)`` with
    G = M for the concat score, 1 for the sum score, gives the full one); a
    full-layout state given to a call is continued as such."""

    S: torch.Tensor
    z: torch.Tensor
    offset: int
    variant: str = "concat"
    num_groups: int = 0


def state_rows(dk, M, variant="concat", packed=False):
    """State rows per (b, h) of a score: M E^2 (concat) or E^2 (sum) in the
    full layout, M E (E + 1) / 2 or E (E + 1) / 2 packed."""
    E = dk // M
    return (1 if variant == "sum" else M) * (E * (E + 1) // 2 if packed else E * E)


def parallel_kata_attn_cached(q, k, v, state=None, num_groups=4, scale=None, eps=1e-6,
                              variant="concat", c=None):
    """KATA causal attention of ``q, k, v`` (time-major ``(B, T, H, D)``)
    continued from ``state`` (a :class:`KataState`, or ``None`` for an empty
    cache).  Returns ``(o, new_state)``: ``o (B, T, H, dv)`` in v's dtype
    equals rows ``offset .. offset + T - 1`` of the flash forward over every
    token so far (``kata/parallel_kata_attn.py:357-361``, ``:539-576`` for
    ``variant="sum"``, ``:291-354`` with the decay ``c``), up to the
    ``max(den, eps)`` guard of the state form.  ``c (B, T, H)`` is the decay's
    cumulative log-decay over this call's tokens (non-increasing; the mixer's
    ``cumsum`` over the call).  An existing state's tensors are updated in
    place and returned in ``new_state``.

    The concat score without decay at the shapes of
    ``linatt_kata_state_supported`` runs the MFMA state-form prefill
    (``spd_state.kata_prefill``), except for a call of at most 1024 tokens
    (2048 with two groups) into an empty cache and a continued chunk of at
    most 1024 tokens over at least 96 (batch, head) pairs; every other call
    runs the flash forward over the call's tokens plus the generic state
    kernels (``linatt_kata_gen_*``: dk <= 128, dv = 64)."""
    if q.dim() != 4 or k.shape != q.shape or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"q, k must be (B, T, H, dk) and v (B, T, H, dv); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    if variant not in ("concat", "sum"):
        raise ValueError(f"variant must be 'concat' or 'sum', got {variant!r}")
    if c is not None and variant != "concat":
        raise NotImplementedError("decay is only defined for the concat score")
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    M = num_groups
    if state is not None:
        if state.S.shape[:2] != (B, H) or state.z.shape[:2] != (B, H):
            raise ValueError(f"state is for (B, H) = {tuple(state.S.shape[:2])}, inputs are {(B, H)}")
        if state.variant != variant or (state.num_groups and state.num_groups != M):
            raise ValueError(f"state is for the {state.variant} score with {state.num_groups} groups, "
                             f"the call is {variant} with {M}")
    offset = 0 if state is None else state.offset
    L = _lib.load()
    dt = v.dtype
    fast = (variant == "concat" and c is None
            and L.linatt_kata_state_supported(_lib.dtype_code(dt), dk, dv, M))
    # a prompt of a few thousand tokens into an empty cache: the flash forward
    # plus the state update beat the state-form prefill (whose output kernel
    # repeats the flash work inside each 1024-token segment) at T <= 1024, and
    # at T <= 2048 for two groups; so do the flash forward, the state readout
    # and the update for a continued chunk of at most 1024 tokens over 96 or
    # more (batch, head) pairs (measured at B = 1 .. 16, H = 12).  Both paths
    # keep the same packed row order, so a state passes between them
    if fast and state is None and (T <= 1024 or (T <= 2048 and M == 2)):
        fast = False
    if fast and state is not None and 1 < T <= 1024 and B * H >= 96:
        fast = False
    if fast:
        if T == 1 and state is not None:
            o = spd_state.kata_decode_step(state.S, state.z, q[:, 0], k[:, 0], v[:, 0], M,
                                           scale, eps)
            return o[:, None], KataState(state.S, state.z, offset + 1, variant, M)
        # a new state is packed (a decode step then streams about half the
        # bytes); an existing one keeps its layout
        packed = state is None or state.S.shape[2] == spd_state.state_rows(dk, M, True)
        init = None if state is None else (state.S, state.z)
        o, _, S, z = spd_state.kata_prefill(q, k, v, M, scale, eps, initial_state=init,
                                            in_place=state is not None, packed_state=packed)
        return o, KataState(S, z, offset + T, variant, M)
    return _generic(q, k, v, state, M, scale, eps, variant, c, offset)


@functools.lru_cache(maxsize=64)
def _decode_workspace_bytes(B, H, dk, M, var):
    return _lib.load().linatt_kata_gen_decode_workspace_bytes(B, H, dk, M, var)


def _generic(q, k, v, state, M, scale, eps, variant, c, offset):
    _lib.require_device(q, k, v)
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    if dk % M:
        raise ValueError(f"d_k={dk} not divisible by M={M}")
    sc = 1.0 / math.sqrt(dk // M) if scale is None else float(scale)
    var = _lib.LINATT_KATA_SUM if variant == "sum" else _lib.LINATT_KATA_CONCAT
    dt = v.dtype
    q, k, v = q.to(dt).contiguous(), k.to(dt).contiguous(), v.contiguous()
    # a new state is packed (a decode step streams about half the bytes); an
    # existing one keeps its layout
    packed = state is None or state.S.shape[2] == state_rows(dk, M, variant, True)
    if packed:
        var |= _lib.LINATT_KATA_PACKED_STATE
    P = state_rows(dk, M, variant, packed)
    cf = None
    if c is not None:
        _lib.require_device(c)
        cf = c.float().contiguous()
        if cf.shape != (B, T, H):
            raise ValueError(f"c must be (B, T, H) = {(B, T, H)}, got {tuple(cf.shape)}")
    if state is not None:
        S, z = state.S, state.z
        if S.shape != (B, H, P, dv) or z.shape != (B, H, P) or S.dtype != torch.float32 \
                or not (S.is_contiguous() and z.is_contiguous()):
            Pf, Pp = state_rows(dk, M, variant), state_rows(dk, M, variant, True)
            raise ValueError(f"state must be contiguous float32 S {(B, H, Pf, dv)}, z {(B, H, Pf)} "
                             f"or packed S {(B, H, Pp, dv)}, z {(B, H, Pp)}")
    L = _lib.load()
    code, sp = _lib.dtype_code(dt), _lib.stream_of(q)
    if T == 1 and state is not None:
        o = torch.empty(B, H, dv, device=q.device, dtype=dt)
        # a small batch splits each (b, h)'s rows over several workgroups
        nws = _decode_workspace_bytes(B, H, dk, M, var)
        if nws and _lib.split_decode_pays(P):
            ws = _lib.stream_scratch(q.device, nws)
            _lib.check("linatt_kata_gen_decode_split", L.linatt_kata_gen_decode_split(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(cf), _lib.ptr(S), _lib.ptr(z),
                _lib.ptr(o), _lib.ptr(ws), nws, B, H, dk, dv, M, var, sc, float(eps), code, sp))
        else:
            _lib.check("linatt_kata_gen_decode", L.linatt_kata_gen_decode(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(cf), _lib.ptr(S), _lib.ptr(z),
                _lib.ptr(o), B, H, dk, dv, M, var, sc, float(eps), code, sp))
        return o[:, None], KataState(S, z, offset + 1, variant, M)
    # the call's own tokens by the flash forward, then the stored state's part
    o, den = _kata_fwd(q, k, v, M, sc, variant, cf)
    if state is not None:
        _lib.check("linatt_kata_gen_readout", L.linatt_kata_gen_readout(
            _lib.ptr(q), _lib.ptr(cf), _lib.ptr(S), _lib.ptr(z), _lib.ptr(o), _lib.ptr(den),
            B, T, H, dk, dv, M, var, sc, float(eps), code, sp))
    else:
        S = torch.empty(B, H, P, dv, device=q.device, dtype=torch.float32)
        z = torch.empty(B, H, P, device=q.device, dtype=torch.float32)
    _lib.check("linatt_kata_gen_update", L.linatt_kata_gen_update(
        _lib.ptr(k), _lib.ptr(v), _lib.ptr(cf), _lib.ptr(S), _lib.ptr(z),
        1 if state is not None else 0, B, T, H, dk, dv, M, var, sc, code, sp))
    return o, KataState(S, z, offset + T, variant, M)


class LayerStateCache:
    """Per-layer state store with the interface of fla's ``Cache`` that the
    mixer uses: ``cache[layer_idx]`` is a dict with ``"recurrent_state"``,
    ``"attn_state"``, ``"conv_state"`` and ``"ffn_state"``;
    ``update(..., layer_idx=i, offset=n)`` replaces the given entries of layer
    ``i`` (creating it) and, for layer 0, advances the sequence length."""

    def __init__(self):
        self.states: list[dict] = []
        self._seen_tokens = 0

    def __getitem__(self, layer_idx: int) -> dict:
        return self.states[layer_idx]

    def __len__(self) -> int:
        return len(self.states)

    def update(self, recurrent_state=None, attn_state=None, conv_state=None, ffn_state=None,
               layer_idx: int = 0, offset: int = 1, cache_kwargs=None) -> dict:
        new = {"recurrent_state": recurrent_state, "attn_state": attn_state,
               "conv_state": conv_state, "ffn_state": ffn_state}
        if layer_idx == 0:
            self._seen_tokens += offset
        if layer_idx < len(self.states):
            for key, val in new.items():
                if val is not None:
                    self.states[layer_idx][key] = val
        elif layer_idx == len(self.states):
            self.states.append(new)
        else:
            raise IndexError(f"layer {layer_idx} updated before layer {len(self.states)}")
        return self.states[layer_idx]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self._seen_tokens if layer_idx < len(self.states) else 0


def get_layer_cache(layer, past_key_values):
    """The layer's entry of ``past_key_values`` (by ``layer.layer_idx``), or
    ``None`` when there is no cache or the layer has none yet."""
    if past_key_values is None or len(past_key_values) <= layer.layer_idx:
        return None
    return past_key_values[layer.layer_idx]


def update_layer_cache(layer, past_key_values, **kwargs):
    """``past_key_values.update(layer_idx=layer.layer_idx, **kwargs)``; a no-op
    without a cache."""
    if past_key_values is None:
        return None
    return past_key_values.update(layer_idx=layer.layer_idx, **kwargs)
