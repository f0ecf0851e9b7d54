"""Rebind the reference's hot-path operators to the HIP kernels at run time.

The reference keeps every change to installed packages in one module that
swaps module attributes once, idempotently, and applies itself on import
(``fla_patches.py:19-31, 195-200``).  This module does the same for the hot
path:

    import kata, fla            # the reference's packages
    import linatt_amd.patch     # applies on import; apply() again is a no-op

Names rebound (only in modules that are importable; the rest are skipped):

* ``kata.parallel_kata_attn``: ``parallel_kata_attn``,
  ``parallel_kata_attn_fwd``, ``parallel_kata_attn_sum``,
  ``parallel_kata_attn_sum_fwd_impl``, ``parallel_kata_attn_decay``,
  ``parallel_kata_attn_bwd`` and ``parallel_kata_attn_bwd_triton``;
* the same names in ``kata.layer``, which imports them by name
  (``kata/layer.py:29-37``), so rebinding the defining module alone would not
  reach the mixer;
* ``kata.spd.chunk_scan_cat.spd_chunk_scan_cat``;
* the mixer's ``ShortConvolution``, ``RMSNorm`` and ``RotaryEmbedding`` classes, which
  ``kata.layer`` imports from ``fla.modules`` (``kata/layer.py:20``); the
  rebinding must happen before the model is built;
* the SPD delta rule ``flash_delta`` (trainable, bf16 backward) and its
  forward pieces ``flash_delta_U``, ``flash_delta_readout``,
  ``flash_delta_den`` in ``kata.spd.flash_delta``, and ``flash_delta`` where
  the mixer imports it (``kata/layer.py:36``);
* fla's delta-rule ops where fla's layers bind them
  (``fla.layers.delta_net.chunk_delta_rule``,
  ``fla.layers.gated_deltanet.chunk_gated_delta_rule``) and where fla defines
  them (``fla.ops.delta_rule`` / ``fla.ops.gated_delta_rule``).

fla's short-sequence ``fused_recurrent_*`` ops are left alone.  ``restore()``
puts every original back (used by the tests).

``apply_mixer()`` (opt-in, not applied on import) goes one step further and
replaces ``kata.layer.KataAttention.forward`` itself with
``linatt_amd.kata_layer.kata_attention_forward``: the q/k chains as one fused
kernel each, the output RMSNorm inside the attention kernels, and a real
decode state when a cache is used (the reference's flash branch keeps none,
``kata/layer.py:492``).  Configurations it does not cover run the original
method.  ``restore()`` undoes it too.
"""

from __future__ import annotations

import importlib
import threading

__all__ = ["apply", "apply_mixer", "restore", "TARGETS"]

# (module, attribute, provider module in linatt_amd, provider attribute)
TARGETS = (
    *((mod, name, "parallel_kata_attn", name)
      for mod in ("kata.parallel_kata_attn", "kata.layer")
      for name in ("parallel_kata_attn", "parallel_kata_attn_fwd", "parallel_kata_attn_sum",
                   "parallel_kata_attn_sum_fwd_impl", "parallel_kata_attn_decay",
                   "parallel_kata_attn_bwd", "parallel_kata_attn_bwd_triton")),
    ("kata.spd.chunk_scan_cat", "spd_chunk_scan_cat", "spd_state", "spd_chunk_scan_cat"),
    ("kata.layer", "ShortConvolution", "mixer", "ShortConvolution"),
    ("kata.layer", "RMSNorm", "mixer", "RMSNorm"),
    ("kata.layer", "RotaryEmbedding", "mixer", "RotaryEmbedding"),
    *(("kata.spd.flash_delta", name, "flash_delta", name)
      for name in ("flash_delta", "flash_delta_U", "flash_delta_readout", "flash_delta_den")),
    ("kata.layer", "flash_delta", "flash_delta", "flash_delta"),
    ("fla.layers.delta_net", "chunk_delta_rule", "delta_rule", "chunk_delta_rule"),
    ("fla.ops.delta_rule", "chunk_delta_rule", "delta_rule", "chunk_delta_rule"),
    ("fla.layers.gated_deltanet", "chunk_gated_delta_rule", "delta_rule", "chunk_gated_delta_rule"),
    ("fla.ops.gated_delta_rule", "chunk_gated_delta_rule", "delta_rule", "chunk_gated_delta_rule"),
)

_lock = threading.Lock()
_originals: dict[tuple[str, str], object] = {}


def _try_import(name: str):
    try:
        return importlib.import_module(name)
    except Exception:  # absent package, or one that fails to import here
        return None


def apply() -> list[tuple[str, str]]:
    """Rebind every target whose module imports and that defines the name
    (a module that lacks the name is left as it is).  Returns the
    ``(module, name)`` pairs that now point at ``linatt_amd``.  Calling it
    again changes nothing already rebound and picks up modules imported
    since."""
    done = []
    with _lock:
        for mod_name, attr, prov_mod, prov_attr in TARGETS:
            mod = _try_import(mod_name)
            if mod is None or not hasattr(mod, attr):
                continue
            new = getattr(importlib.import_module(f"linatt_amd.{prov_mod}"), prov_attr)
            cur = getattr(mod, attr)
            if cur is not new:
                _originals.setdefault((mod_name, attr), cur)
                setattr(mod, attr, new)
            done.append((mod_name, attr))
    return done


_mixer_originals: dict[type, object] = {}


def apply_mixer() -> bool:
    """Install the fused ``KataAttention.forward`` on ``kata.layer.KataAttention``
    (its subclasses ``FlashKata``, ``ChunkedKata`` and ``DeltaKata`` inherit
    it).  Returns False when ``kata.layer`` is not importable.  Idempotent;
    ``restore()`` puts the original method back."""
    mod = _try_import("kata.layer")
    if mod is None or not hasattr(mod, "KataAttention"):
        return False
    from . import kata_layer
    cls = mod.KataAttention
    with _lock:
        if cls.forward is not kata_layer.kata_attention_forward:
            # (the class's own attribute, or None when it inherits forward)
            _mixer_originals.setdefault(cls, cls.__dict__.get("forward"))
            kata_layer.ORIGINAL_FORWARD[cls] = cls.forward
            cls.forward = kata_layer.kata_attention_forward
    return True


def restore() -> None:
    """Put back every attribute ``apply()`` replaced and the method
    ``apply_mixer()`` replaced."""
    with _lock:
        for (mod_name, attr), orig in list(_originals.items()):
            mod = _try_import(mod_name)
            if mod is not None:
                setattr(mod, attr, orig)
            del _originals[(mod_name, attr)]
        from . import kata_layer
        for cls, orig in list(_mixer_originals.items()):
            if orig is None:
                del cls.forward
            else:
                cls.forward = orig
            kata_layer.ORIGINAL_FORWARD.pop(cls, None)
            del _mixer_originals[cls]


apply()
