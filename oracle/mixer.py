"""Float64 CPU restatement of the token mixer's non-GEMM prologue / epilogue.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference: ``kata/layer.py`` KataAttention -- the short convolutions on the
projected q, k, v (constructed at ``:178-197``, applied at ``:299-318``) and
the output RMSNorm (``:199-205``, applied at ``:539``; the q/k RMSNorm of
``:126-128, 347`` is the same op).  Both modules are the third-party
``fla.modules.ShortConvolution`` / ``fla.modules.RMSNorm``
(flash-linear-attention==0.5.0, pinned at ``scripts/setup.sh:27``), absent
here; they are restated from their published definitions:

* ShortConvolution(hidden_size, kernel_size, bias, activation="silu") is a
  depthwise causal ``nn.Conv1d`` (weight (C, 1, W), left padding W - 1)
  followed by SiLU; its decode cache holds the last W inputs, newest last.
* RMSNorm(hidden_size, elementwise_affine, eps) is
  ``x / sqrt(mean(x^2) + eps) * weight`` in fp32.
* RotaryEmbedding(dim, base, interleaved) rotates pair p of the first
  ``dim`` dims of every head -- (2p, 2p + 1) interleaved (GPT-J), (p,
  p + dim / 2) otherwise (GPT-NeoX) -- by ``(t + offset) * base^(-2p / dim)``.

Parity against fla itself is unpinned (fla is absent and the reference holds
no outputs of these modules); the tests pin this restatement against a
library convolution, explicit loops and invariants.
"""

from __future__ import annotations

import torch

F64 = torch.float64


def short_conv(x, weight, bias=None, activation="silu", cache=None):
    """``x (B, T, C)``, ``weight (C, W)`` or ``(C, 1, W)``, ``bias (C)``,
    ``cache (B, C, W)`` (inputs before position 0, newest last, or None for
    zeros).  Returns ``(y, final_cache)`` in float64; ``final_cache`` holds
    the W inputs before position T."""
    x = x.to(F64)
    w = weight.reshape(weight.shape[0], -1).to(F64)
    B, T, C = x.shape
    W = w.shape[1]
    prev = cache.to(F64) if cache is not None else torch.zeros(B, C, W, dtype=F64)
    xp = torch.cat([prev.transpose(1, 2), x], dim=1)          # positions -W .. T-1
    z = torch.zeros(B, T, C, dtype=F64)
    for j in range(W):
        z = z + w[:, j] * xp[:, 1 + j:1 + j + T]               # position t - (W-1) + j
    if bias is not None:
        z = z + bias.to(F64)
    y = z * torch.sigmoid(z) if activation == "silu" else z
    final = xp[:, -W:].transpose(1, 2).contiguous()
    return y, final


def short_conv_loop(x, weight, bias=None, activation="silu", cache=None):
    """The same convolution as explicit per-element loops (small inputs)."""
    B, T, C = x.shape
    w = weight.reshape(C, -1)
    W = w.shape[1]
    y = torch.zeros(B, T, C, dtype=F64)
    for b in range(B):
        for t in range(T):
            for c in range(C):
                z = float(bias[c]) if bias is not None else 0.0
                for j in range(W):
                    p = t - (W - 1) + j
                    if p >= 0:
                        xv = float(x[b, p, c])
                    elif cache is not None:
                        xv = float(cache[b, c, W + p])
                    else:
                        xv = 0.0
                    z += float(w[c, j]) * xv
                if activation == "silu":
                    z = z / (1.0 + torch.exp(torch.tensor(-z, dtype=F64)).item())
                y[b, t, c] = z
    return y


def rmsnorm(x, weight=None, eps=1e-5):
    """``x / sqrt(mean(x^2, -1) + eps) * weight`` in float64."""
    x = x.to(F64)
    r = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    y = x * r
    return y * weight.to(F64) if weight is not None else y


def fwd_bwd(fn, inputs, dy, **kw):
    """float64 autograd gradients of ``<fn(*inputs), dy>`` w.r.t. the given
    tensors (None entries are passed through)."""
    leaves = [t.detach().to(F64).requires_grad_(True) if t is not None else None for t in inputs]
    with torch.enable_grad():
        out = fn(*leaves, **kw)
        y = out[0] if isinstance(out, tuple) else out
        grads = torch.autograd.grad((y * dy.to(F64)).sum(), [t for t in leaves if t is not None])
    it = iter(grads)
    return y.detach(), [next(it) if t is not None else None for t in leaves]


def rope(x, rot_dim, base=10000.0, offset=0, interleaved=False, inverse=False):
    """``x (B, T, H, D)`` rotated as fla's RotaryEmbedding does, float64."""
    x = x.to(F64)
    B, T, H, D = x.shape
    half = rot_dim // 2
    p = torch.arange(half, dtype=F64)
    inv_freq = base ** (-2.0 * p / rot_dim)
    ang = (torch.arange(T, dtype=F64) + offset)[:, None] * inv_freq[None, :]   # (T, half)
    cs, sn = torch.cos(ang)[None, :, None, :], torch.sin(ang)[None, :, None, :]
    if inverse:
        sn = -sn
    y = x.clone()
    i0 = 2 * p.long() if interleaved else p.long()
    i1 = i0 + 1 if interleaved else p.long() + half
    a, b = x[..., i0], x[..., i1]
    y[..., i0] = a * cs - b * sn
    y[..., i1] = a * sn + b * cs
    return y
