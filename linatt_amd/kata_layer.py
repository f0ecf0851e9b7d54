"""A fused ``KataAttention.forward`` for the reference mixer, on MI355X.

``kata/layer.py:284-545`` runs the mixer as a chain of modules: q/k/v
projections, three short convolutions (``:299-318``), per-head q/k norms and
RoPE (``:340-372``), the attention op (``:374-518``), the output RMSNorm and
``o_proj`` (``:539-541``).  Its flash branch stores no decode state
(``final_state = None``, ``:492``) and it never stores the convolution
states it reads (``:532-537``), so incremental decoding is wrong for KATA
and its evaluation turns the cache off (``eval_recall.py:133-144``).

``kata_attention_forward`` is a drop-in for that method (same signature and
return value ``(o, None, past_key_values)``), installed by
``linatt_amd.patch.apply_mixer()``.  On the configurations it covers it runs:

* the q and k chains (convolution + SiLU -> RMSNorm or L2 norm per head ->
  RoPE, full-head interleaved or per group) as one HIP kernel each
  (``mixer.fused_qk_prologue``), with v's convolution on its own;
* without a cache, the flash branch with the output RMSNorm inside the
  attention kernels (``parallel_kata_attn_onorm``: concat, sum, decayed;
  offset-gated inputs go through the same op); GQA natively (k and v keep
  their ``num_kv_heads`` heads, the reference repeats them);
* with a cache (``use_cache`` or a non-empty ``past_key_values``), the
  recurrent state form of the score (``kata_cache.parallel_kata_attn_cached``:
  a prefill continued from the layer's state, or one decode step; concat,
  sum, decayed, offset-gated), and the convolution states are stored with
  it, so prefill + decode equals the parallel forward over the whole
  sequence;
* the SPD delta branch through ``linatt_amd.flash_delta``.

The projections and ``o_proj`` stay library GEMMs.  Anything else (the
psi-feature maps, ``delta_state``, a cache for the delta branch or for a
shape without a state form) runs the original forward unchanged.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib

_lib.load()

from . import kata_cache  # noqa: E402
from .flash_delta import flash_delta  # noqa: E402
from .mixer import fused_qk_prologue, rms_norm, rotary, short_conv  # noqa: E402
from .parallel_kata_attn import parallel_kata_attn_onorm  # noqa: E402

__all__ = ["kata_attention_forward", "ORIGINAL_FORWARD"]

# KataAttention.forward before apply_mixer() replaced it, per class
ORIGINAL_FORWARD: dict[type, object] = {}

_FLASH_MAPS = ("kata_quadratic", "kata_quadratic_sum")


def _original(self):
    for cls in type(self).__mro__:
        if cls in ORIGINAL_FORWARD:
            return ORIGINAL_FORWARD[cls]
    raise RuntimeError("kata_attention_forward: no original forward recorded for "
                       f"{type(self).__name__} (install it with linatt_amd.patch.apply_mixer())")


def _norm_spec(self, side):
    """The q or k norm as fused_qk_prologue takes it: a module with weight and
    eps, "l2", or None."""
    if not self.qk_norm:
        return None
    kind = getattr(self, f"norm_{side}")
    if kind == "l2":
        return "l2"
    return getattr(self, f"{side}_norm")


def _apply_norm(x, spec):
    if spec is None:
        return x
    if spec == "l2":
        from .delta_rule import l2norm
        return l2norm(x)
    return rms_norm(x, spec.weight, spec.eps)


def _state_form_ok(self, q_dtype):
    """A recurrent state exists for every flash score (concat, sum, decayed,
    offset-gated) at dv = 64 and a key width (the offset gate's padded one)
    of at most 128 split into power-of-two groups of at least 16, where the
    flash forward is compiled too."""
    if self.use_delta or self.feature_map_name not in _FLASH_MAPS:
        return False
    M = self.spd_num_groups
    dk = M * self._off_Epad if self.use_offset_gate else self.head_k_dim
    E = dk // M
    if self.head_v_dim != 64 or dk > 128 or dk % M or E < 16 or E & (E - 1):
        return False
    L = _lib.load()
    variant = _lib.LINATT_KATA_SUM if self.feature_map_name == "kata_quadratic_sum" else 0
    return bool(L.linatt_kata_supported(_lib.dtype_code(q_dtype), dk, self.head_v_dim, M, variant,
                                        1 if self.use_decay else 0))


def _proj_dtype(x):
    """The dtype the projections produce: autocast's, or x's."""
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return x.dtype


def _prologue_ok(self, rot):
    """fused_qk_prologue's shapes: head dim 32, 64 or 128, kernel size 2-4,
    rotation rows of a multiple of 4 dividing the head dim (a multiple of 8
    when half-split)."""
    D = self.head_k_dim
    W = self.q_conv1d.weight.shape[-1]
    if D not in (32, 64, 128) or W not in (2, 3, 4):
        return False
    if getattr(self.q_conv1d, "activation", "silu") not in ("silu", "swish", None, "identity"):
        return False
    if rot is not None:
        rw = rot.dim
        if D % rw or rw % 4 or (not rot.interleaved and rw % 8):
            return False
    return True


def _covered(self):
    if not (self.use_delta or self.feature_map_name in _FLASH_MAPS):
        return False
    if self.use_delta and getattr(self, "delta_state", False):
        return False
    rot = getattr(self, "rotary", None) if self.use_rope else None
    if rot is not None and getattr(rot, "scale_base", None) is not None:
        return False
    return True


def kata_attention_forward(self, hidden_states, attention_mask=None, past_key_values=None,
                           use_cache=False, **kwargs):
    """Drop-in for ``KataAttention.forward`` (``kata/layer.py:284-545``)."""
    if not _covered(self):
        return _original(self)(self, hidden_states, attention_mask=attention_mask,
                               past_key_values=past_key_values, use_cache=use_cache, **kwargs)
    x = hidden_states
    B, T, _ = x.shape
    H, D, Dv = self.num_heads, self.head_k_dim, self.head_v_dim
    Hk = H // self.num_kv_groups
    M = self.spd_num_groups
    cached = bool(use_cache) or (past_key_values is not None and len(past_key_values) > 0)
    if cached and (self.use_delta or not _state_form_ok(self, _proj_dtype(x))):
        # no state form for this score: the reference's own (stateless) path
        return _original(self)(self, hidden_states, attention_mask=attention_mask,
                               past_key_values=past_key_values, use_cache=use_cache, **kwargs)

    last = kata_cache.get_layer_cache(self, past_key_values)
    conv_q = conv_k = conv_v = None
    if last is not None and last.get("conv_state") is not None:
        conv_q, conv_k, conv_v = last["conv_state"]
    offset = 0
    if past_key_values is not None and self.layer_idx is not None:
        offset = past_key_values.get_seq_length(self.layer_idx)

    rot = self.rotary if self.use_rope else None
    nq, nk = _norm_spec(self, "q"), _norm_spec(self, "k")
    q = self.q_proj(x)
    k = self.k_proj(x)
    v = self.v_proj(x)
    fused = self.use_short_conv and _prologue_ok(self, rot)
    if self.use_short_conv:
        v, conv_v = short_conv(v, self.v_conv1d.weight, self.v_conv1d.bias,
                               self.v_conv1d.activation, conv_v, cached)
    if fused:
        q, conv_q = fused_qk_prologue(q, self.q_conv1d, nq, rot, D, seqlen_offset=offset,
                                      cache=conv_q, output_final_state=cached)
        k, conv_k = fused_qk_prologue(k, self.k_conv1d, nk, rot, D, seqlen_offset=offset,
                                      cache=conv_k, output_final_state=cached)
    else:
        if self.use_short_conv:
            q, conv_q = short_conv(q, self.q_conv1d.weight, self.q_conv1d.bias,
                                   self.q_conv1d.activation, conv_q, cached)
            k, conv_k = short_conv(k, self.k_conv1d.weight, self.k_conv1d.bias,
                                   self.k_conv1d.activation, conv_k, cached)
        q = _apply_norm(q.reshape(B, T, H, D), nq)
        k = _apply_norm(k.reshape(B, T, Hk, D), nk)
        if rot is not None:
            rw = rot.dim
            q = rotary(q.reshape(B, T, -1, rw), rw, rot.base, offset, rot.interleaved).reshape(B, T, H, D)
            k = rotary(k.reshape(B, T, -1, rw), rw, rot.base, offset, rot.interleaved).reshape(B, T, Hk, D)
    if attention_mask is not None:
        v = v.mul(attention_mask[:, -T:, None])
    q = q.reshape(B, T, H, D)
    k = k.reshape(B, T, Hk, D)
    v = v.reshape(B, T, Hk, Dv)

    norm = self.norm
    has_norm = hasattr(norm, "weight") and hasattr(norm, "eps")
    final_state = None
    y = None  # normalised output, when the norm ran inside the attention op
    if self.use_delta:
        beta = torch.sigmoid(self.b_proj(x))
        if self.num_kv_groups > 1:
            k = k.repeat_interleave(self.num_kv_groups, dim=2)
            v = v.repeat_interleave(self.num_kv_groups, dim=2)
        Tp = max(64, 1 << (T - 1).bit_length())
        qh, kh, vh, bh = (t.contiguous() for t in (q, k, v, beta))
        if Tp != T:
            p = Tp - T
            qh, kh, vh = (F.pad(t, (0, 0, 0, 0, 0, p)) for t in (qh, kh, vh))
            bh = F.pad(bh, (0, 0, 0, p))
        o = flash_delta(qh.bfloat16(), kh.bfloat16(), vh.bfloat16(), bh.bfloat16(), M,
                        scale=self.delta_scale, C=64, normalize=self.delta_normalize)
        o = o[:, :T].to(v.dtype)
    else:
        q_in, k_in, scale = q, k, None
        if self.use_offset_gate:
            off = torch.sigmoid(self.a_proj(x))
            q_in, k_in = self._augment_offset(q, k, off)
            scale = self._off_scale
        variant = "sum" if self.feature_map_name == "kata_quadratic_sum" else "concat"
        c = None
        if self.use_decay:
            # the call's cumulative log-decay (a stored state sits at c = 0)
            dt_ = F.softplus(self.dt_proj(x) + self.dt_bias)
            c = (-self.A_log.float().exp() * dt_.float()).cumsum(dim=1).contiguous()
        if cached:
            if self.num_kv_groups > 1:
                k_in = k_in.repeat_interleave(self.num_kv_groups, dim=2)
                v = v.repeat_interleave(self.num_kv_groups, dim=2)
            rec = last.get("recurrent_state") if last is not None else None
            o, final_state = kata_cache.parallel_kata_attn_cached(q_in, k_in, v, rec, M, scale,
                                                                  variant=variant, c=c)
        else:
            if has_norm:
                y = parallel_kata_attn_onorm(q_in, k_in, v, norm.weight, norm.eps, M, scale,
                                             variant, c)
            else:
                from .parallel_kata_attn import (parallel_kata_attn, parallel_kata_attn_decay,
                                                 parallel_kata_attn_sum)
                if c is not None:
                    o = parallel_kata_attn_decay(q_in, k_in, v, c, M, scale)
                elif variant == "sum":
                    o = parallel_kata_attn_sum(q_in, k_in, v, M, scale)
                else:
                    o = parallel_kata_attn(q_in, k_in, v, M, scale)

    if past_key_values is not None:
        conv_state = (conv_q, conv_k, conv_v) if (cached and self.use_short_conv) else None
        kata_cache.update_layer_cache(self, past_key_values, recurrent_state=final_state,
                                      conv_state=conv_state, offset=T)
    if y is None:
        y = rms_norm(o, norm.weight, norm.eps) if has_norm else norm(o)
    out = self.o_proj(y.reshape(B, T, H * Dv))
    return out, None, past_key_values

