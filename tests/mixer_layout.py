"""Test helper: a module with the reference mixer's attribute layout
(``kata/layer.py:42-281``: parameter and flag names of ``KataAttention``), for
the tests of ``linatt_amd.kata_layer.kata_attention_forward``, and that layer
in float64 on the CPU from the oracle's functions.

The reference package needs the absent ``fla``, so its class cannot be
built here; this one carries the same names, built from linatt_amd's
drop-in modules.  Its own ``forward`` stands for the reference's method (the
hook's fallback) and only records that it ran.
"""

import math

import torch
from torch import nn

from oracle import delta as OD
from oracle import kata as K
from oracle import mixer as X

F64 = torch.float64


class KataAttentionLayout(nn.Module):
    """``KataAttention``'s attributes for the flash branch (kata_quadratic /
    kata_quadratic_sum, optional decay, offset gate, GQA) with short
    convolutions, q/k norms and RoPE."""

    def __init__(self, hidden, H, D, M, *, feature_map="kata_quadratic", num_kv_heads=None,
                 qk_norm=True, norm_q="rmsnorm", norm_k="rmsnorm", use_rope=True,
                 rope_group=False, use_short_conv=True, conv_size=4, use_decay=False,
                 use_offset_gate=False, output_norm="rmsnorm", layer_idx=0, device=None):
        super().__init__()
        from linatt_amd.mixer import RMSNorm, RotaryEmbedding, ShortConvolution
        fk = {"device": device}
        self.hidden_size, self.mode = hidden, "chunk"
        self.num_heads = H
        self.num_kv_heads = num_kv_heads or H
        self.num_kv_groups = H // self.num_kv_heads
        self.head_k_dim = self.head_v_dim = D
        self.key_dim = self.value_dim = H * D
        self.key_dim_per_group = self.value_dim_per_group = self.num_kv_heads * D
        self.layer_idx = layer_idx
        self.qk_norm, self.norm_q, self.norm_k = qk_norm, norm_q, norm_k
        if qk_norm and norm_q == "rmsnorm":
            self.q_norm = RMSNorm(D, dtype=torch.float32, **fk)
        if qk_norm and norm_k == "rmsnorm":
            self.k_norm = RMSNorm(D, dtype=torch.float32, **fk)
        self.use_rope, self.rope_group = use_rope, rope_group
        if use_rope:
            self.rotary = (RotaryEmbedding(D // M) if rope_group
                           else RotaryEmbedding(D, interleaved=True))
        self.feature_map_name = feature_map
        self.spd_num_groups = M
        self.q_proj = nn.Linear(hidden, self.key_dim, bias=False, **fk)
        self.k_proj = nn.Linear(hidden, self.key_dim_per_group, bias=False, **fk)
        self.v_proj = nn.Linear(hidden, self.value_dim_per_group, bias=False, **fk)
        self.use_short_conv, self.conv_size = use_short_conv, conv_size
        if use_short_conv:
            self.q_conv1d = ShortConvolution(self.key_dim, conv_size, activation="silu", **fk)
            self.k_conv1d = ShortConvolution(self.key_dim_per_group, conv_size, activation="silu", **fk)
            self.v_conv1d = ShortConvolution(self.value_dim_per_group, conv_size, activation="silu", **fk)
        self.norm = (RMSNorm(D, dtype=torch.float32, **fk) if output_norm == "rmsnorm"
                     else nn.Identity())
        self.o_proj = nn.Linear(self.value_dim, hidden, bias=False, **fk)
        self.use_delta, self.delta_state = False, False
        self.use_offset_gate = use_offset_gate
        if use_offset_gate:
            self._off_E = D // M
            self._off_Epad = max(16, 1 << self._off_E.bit_length())
            self._off_scale = 1.0 / math.sqrt(self._off_E)
            self.a_proj = nn.Linear(hidden, H, bias=True, **fk)
        self.use_decay = use_decay
        if use_decay:
            self.dt_proj = nn.Linear(hidden, H, bias=False, **fk)
            self.A_log = nn.Parameter(torch.log(torch.empty(H, **fk).uniform_(1, 4)))
            self.dt_bias = nn.Parameter(torch.empty(H, **fk).uniform_(-3, -1))
        with torch.no_grad():  # non-trivial norm weights
            for name in ("q_norm", "k_norm", "norm"):
                m = getattr(self, name, None)
                if getattr(m, "weight", None) is not None:
                    m.weight.uniform_(0.75, 1.25)
        self.original_calls = 0

    def _augment_offset(self, q, k, off):
        """The offset gate's packing as ``kata/layer.py:265-281`` specifies it:
        each group of q gets the gate off_t and k a 1 as an extra coordinate,
        zero-padded to a power of two."""
        B, T, H, _ = q.shape
        M, E, Ep = self.spd_num_groups, self._off_E, self._off_Epad

        def pack(x, col):
            xg = x.reshape(B, T, H, M, E)
            extra = torch.zeros(B, T, H, M, Ep - E, dtype=x.dtype, device=x.device)
            extra[..., 0] = col[..., None].to(x.dtype)
            return torch.cat([xg, extra], dim=-1).reshape(B, T, H, M * Ep)

        return pack(q, off), pack(k, torch.ones_like(off))

    def forward(self, hidden_states, attention_mask=None, past_key_values=None, use_cache=False,
                **kwargs):
        """Stands for the reference's own forward (the hook's fallback)."""
        self.original_calls += 1
        return ("original", hidden_states.shape), None, past_key_values


def _bf16_round(t):
    """t rounded to bf16, as a float64 tensor whose gradient passes through
    unchanged (the rounding autocast applies to a projection's output)."""
    return t + (t.to(torch.bfloat16).double() - t).detach()


def layout_reference(layer, x, autocast=True):
    """The layer of ``kata/layer.py:284-545`` (flash branch, no cache) in
    float64 on the CPU: oracle short convolution, q/k RMSNorm or L2 norm,
    RoPE, KATA scores (GQA by repeating k/v as the reference does), output
    RMSNorm, o_proj.  Returns ``(y, x_leaf, params)`` for autograd.

    With ``autocast`` every projection is taken as ``torch.autocast(bf16)``
    computes it -- bf16 operands, the product rounded once to bf16 -- so the
    comparison measures the kernels, not the rounding of their inputs (which
    the decay's cumulative sum and the squared scores amplify; the gradients
    still pass through the roundings unchanged)."""
    P = {n: p.detach().double().cpu().requires_grad_(True) for n, p in layer.named_parameters()}
    x = x.detach().double().cpu().requires_grad_(True)
    B, T, _ = x.shape
    H, D, M = layer.num_heads, layer.head_k_dim, layer.spd_num_groups
    Hk = layer.num_kv_heads

    def linear(inp, name, bias=None):
        w = P[f"{name}.weight"]
        if autocast:
            y = _bf16_round(_bf16_round(inp) @ _bf16_round(w).T)
            return y if bias is None else _bf16_round(y + _bf16_round(bias))
        return inp @ w.T if bias is None else inp @ w.T + bias

    def branch(name, heads):
        y = linear(x, f"{name}_proj")
        if layer.use_short_conv:
            b = P.get(f"{name}_conv1d.bias")
            y, _ = X.short_conv(y, P[f"{name}_conv1d.weight"], b, "silu")
        return y.reshape(B, T, heads, D)

    q, k, v = branch("q", H), branch("k", Hk), branch("v", Hk)
    if layer.num_kv_groups > 1:
        k = k.repeat_interleave(layer.num_kv_groups, dim=2)
        v = v.repeat_interleave(layer.num_kv_groups, dim=2)
    if layer.qk_norm:
        q = OD.l2norm(q) if layer.norm_q == "l2" else X.rmsnorm(q, P["q_norm.weight"], 1e-5)
        k = OD.l2norm(k) if layer.norm_k == "l2" else X.rmsnorm(k, P["k_norm.weight"], 1e-5)
    if layer.use_rope:
        if layer.rope_group:
            E = D // M
            q = X.rope(q.reshape(B, T, H * M, E), E).reshape(B, T, H, D)
            k = X.rope(k.reshape(B, T, H * M, E), E).reshape(B, T, H, D)
        else:
            q, k = X.rope(q, D, interleaved=True), X.rope(k, D, interleaved=True)
    scale, c = None, None
    if layer.use_offset_gate:
        off = torch.sigmoid(linear(x, "a_proj", P["a_proj.bias"]))
        q, k = layer._augment_offset(q, k, off)
        scale = layer._off_scale
    if layer.use_decay:
        dt = torch.nn.functional.softplus(linear(x, "dt_proj") + P["dt_bias"])
        c = (-P["A_log"].exp() * dt).cumsum(dim=1)
    variant = "sum" if layer.feature_map_name == "kata_quadratic_sum" else "concat"
    o, _ = K.kata_fwd(q, k, v, M, scale, variant, c)
    if "norm.weight" in P:
        o = X.rmsnorm(o, P["norm.weight"], 1e-5)
    y = linear(o.reshape(B, T, H * D), "o_proj")
    return y, x, P
