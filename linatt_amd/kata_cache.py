"""Recurrent decode state for the KATA flash mixer: the ``past_key_values``
entry the reference's flash path never fills.

The reference's flash branch sets ``final_state = None`` (``kata/layer.py:492``)
and hands it to ``update_layer_cache`` (``:532-537``), so incremental decoding
makes each new token attend only to itself; its evaluation forces
``use_cache=False`` for KATA to stay correct (``eval_recall.py:133-144``).  The
concat-SPD score has an exact O(1)-per-token state form, kept here per layer:

    S = sum_s psi(sqrt(scale) k_s) v_s^T   (B, H, M*E*E, dv) float32
    z = sum_s psi(sqrt(scale) k_s)         (B, H, M*E*E)     float32
    psi(x) = vec(x_g x_g^T) per group,  o_t = psi(sqrt(scale) q_t)^T S / max(psi(.) . z, eps)

A chunk of T > 1 tokens goes through the state-form prefill continued from the
current state (``linatt_kata_prefill_state``); a single token through the
decode step (``linatt_kata_decode_step``), both in ``liblinatt_hip.so``.

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

Scope: the concat score without decay or offset gate, at the shapes the
state-form kernels are compiled for (``linatt_kata_state_supported``); other
mixers raise.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import spd_state

__all__ = ["KataState", "parallel_kata_attn_cached", "LayerStateCache", "get_layer_cache",
           "update_layer_cache"]


class KataState(NamedTuple):
    """A layer's recurrent state: ``S (B, H, P, dv)``, ``z (B, H, P)`` float32
    (``P = M E^2``) and the number of tokens it covers."""

    S: torch.Tensor
    z: torch.Tensor
    offset: int


def parallel_kata_attn_cached(q, k, v, state=None, num_groups=4, scale=None, eps=1e-6):
    """Concat-SPD causal attention of ``q, k, v`` (time-major ``(B, T, H, D)``)
    continued from ``state`` (a :class:`KataState`, or ``None`` for an empty
    cache).  Returns ``(o, new_state)``: ``o (B, T, H, dv)`` in v's dtype equals
    rows ``offset .. offset + T - 1`` of the flash forward over every token so
    far (``kata/parallel_kata_attn.py:357-361``), up to the ``max(den, eps)``
    guard of the state form.  An existing state's tensors are updated in
    place (a decode step reads and writes the state once, at HBM speed) and
    returned in ``new_state``."""
    if q.dim() != 4 or k.shape != q.shape or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"q, k must be (B, T, H, dk) and v (B, T, H, dv); got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, T, H, _ = q.shape
    if state is not None and (state.S.shape[:2] != (B, H) or state.z.shape[:2] != (B, H)):
        raise ValueError(f"state is for (B, H) = {tuple(state.S.shape[:2])}, inputs are {(B, H)}")
    offset = 0 if state is None else state.offset
    if T == 1 and state is not None:
        o = spd_state.kata_decode_step(state.S, state.z, q[:, 0], k[:, 0], v[:, 0], num_groups,
                                       scale, eps)
        return o[:, None], KataState(state.S, state.z, offset + 1)
    init = None if state is None else (state.S, state.z)
    o, _, S, z = spd_state.kata_prefill(q, k, v, num_groups, scale, eps, initial_state=init,
                                        in_place=state is not None)
    return o, KataState(S, z, offset + T)


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
