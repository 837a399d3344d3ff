"""The layer's weights as its forward sees them: plain, parametrized or LoRA.

The reference lets callers adapt the engine's weights in two ways
(complexity/training/lora.py):

* ``LoRALinear`` replaces a shared ``nn.Linear`` (lora.py:37-90): the module
  keeps the frozen linear as ``base`` and adds
  ``scaling * (dropout(x) @ lora_A.T) @ lora_B.T`` to its output
  (``lora_residual``).  The engine detects it by ``is_lora_adapter``
  (engine.py:333-349).
* ``LoRAExpertTensor`` is a ``torch.nn.utils.parametrize`` parametrization of
  ``expert_gate`` / ``expert_up`` / ``expert_down`` (lora.py:93-165,
  203-215): every attribute access returns a freshly materialised
  ``original + scaling * lora_A @ lora_B`` tensor.  The reference fetches each
  expert tensor once per call (engine.py:461-464).

The HIP kernels read packed copies of the weights, so the engine needs (1) a
cache key that changes whenever what a weight would materialise to changes,
without materialising it, and (2) each weight materialised at most once per
call, the same tensor feeding the pack, the autograd inputs and the backward
packs.  A shared LoRA adapter is served by its merged weight
``base.weight + scaling * lora_B @ lora_A``, which equals the adapter's
output on every input while its dropout is inactive (eval mode or p = 0);
gradients reach ``lora_A`` / ``lora_B`` through torch's autograd of the merge.
"""

from __future__ import annotations

import itertools
from typing import Optional

import torch
import torch.nn as nn
from torch.nn.utils import parametrize

SHARED_NAMES = ("shared_gate", "shared_up", "shared_down")
EXPERT_NAMES = ("expert_gate", "expert_up", "expert_down")
WEIGHT_NAMES = SHARED_NAMES + EXPERT_NAMES


def _tkey(t: torch.Tensor):
    return (t.data_ptr(), t._version, t.dtype, t.device, tuple(t.shape))


def is_lora_linear(mod: Optional[nn.Module]) -> bool:
    """True for a module with the reference's LoRALinear surface (lora.py:37-90)."""
    return (
        mod is not None
        and getattr(mod, "is_lora_adapter", False)
        and isinstance(getattr(mod, "base", None), nn.Linear)
        and isinstance(getattr(mod, "lora_A", None), torch.Tensor)
        and isinstance(getattr(mod, "lora_B", None), torch.Tensor)
        and isinstance(getattr(mod, "scaling", None), (int, float))
    )


def lora_dropout_active(mod: nn.Module) -> bool:
    """LoRALinear applies ``dropout`` to the low-rank branch's input
    (lora.py:79-87); in training mode with p > 0 no merged weight reproduces it."""
    drop = getattr(mod, "dropout", None)
    if drop is None or isinstance(drop, nn.Identity):
        return False
    return bool(drop.training and getattr(drop, "p", 0.0) > 0.0)


def shared_adapter_blocker(engine: nn.Module) -> Optional[str]:
    """Why the shared linears' adapters keep the layer off the HIP kernels
    (None when every shared module is a plain linear or a mergeable LoRALinear)."""
    for name in SHARED_NAMES:
        mod = engine._modules.get(name)
        if mod is None or not getattr(mod, "is_lora_adapter", False):
            continue
        if not is_lora_linear(mod):
            return (f"{name} is a LoRA adapter without the LoRALinear surface (base, lora_A, lora_B, scaling); "
                    "the layer runs on PYTORCH")
        if lora_dropout_active(mod):
            return (f"LoRA dropout on {name} is active (training mode, p > 0): the low-rank branch sees "
                    "dropped-out inputs, which no merged weight reproduces; the layer runs on PYTORCH")
    return None


def merged_lora_weight(mod: nn.Module) -> torch.Tensor:
    """``base.weight + scaling * lora_B @ lora_A`` in the base dtype (product and
    sum in at least fp32, one rounding), differentiable in lora_A / lora_B."""
    base = mod.base.weight
    wide = torch.promote_types(base.dtype, torch.float32)
    delta = mod.lora_B.to(wide) @ mod.lora_A.to(wide)
    return (base.to(wide) + float(mod.scaling) * delta).to(base.dtype)


def _param_key(owner: nn.Module, attr: str):
    """Key of ``owner.attr`` that changes whenever the tensor an access would
    return can change; None when it cannot be cached (a parametrization in
    training mode may draw random numbers, e.g. the reference's factor dropout,
    lora.py:150-163)."""
    if parametrize.is_parametrized(owner, attr):
        plist = owner.parametrizations[attr]
        if any(m.training for m in plist):
            return None
        tensors = itertools.chain(plist.parameters(), plist.buffers())
        return ("param", id(plist), tuple(_tkey(t) for t in tensors))
    return _tkey(getattr(owner, attr))


def weights_key(engine: nn.Module):
    """Cache key of the six weights (None: not cacheable this call)."""
    parts = []
    for name in SHARED_NAMES:
        mod = engine._modules.get(name)
        if mod is None:
            parts.append(None)
        elif is_lora_linear(mod):
            a, b = _param_key(mod, "lora_A"), _param_key(mod, "lora_B")
            base = _param_key(mod.base, "weight")
            if a is None or b is None or base is None:
                return None
            parts.append(("lora", base, a, b, float(mod.scaling)))
        else:
            k = _param_key(mod, "weight")
            if k is None:
                return None
            parts.append(k)
    for name in EXPERT_NAMES:
        k = _param_key(engine, name)
        if k is None:
            return None
        parts.append(k)
    return tuple(parts)


def materialize(engine: nn.Module) -> dict:
    """name -> the weight tensor the forward uses, each materialised once."""
    out = {}
    for name in SHARED_NAMES:
        mod = engine._modules.get(name)
        if mod is None:
            out[name] = None
        elif is_lora_linear(mod):
            out[name] = merged_lora_weight(mod)
        else:
            out[name] = mod.weight
    for name in EXPERT_NAMES:
        out[name] = getattr(engine, name)
    return out


def any_requires_grad(engine: nn.Module) -> bool:
    return any(p.requires_grad for p in engine.parameters())


def stored_dtype(engine: nn.Module, name: str) -> torch.dtype:
    """dtype of an expert weight without materialising a parametrized one."""
    if parametrize.is_parametrized(engine, name):
        return engine.parametrizations[name].original.dtype
    return getattr(engine, name).dtype
