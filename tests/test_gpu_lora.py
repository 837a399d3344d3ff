"""Adapted (LoRA) weights on the HIP backend against the oracle.

The reference adapts the layer's weights in two ways
(complexity/training/lora.py):

* a ``torch.nn.utils.parametrize`` parametrization of ``expert_gate`` /
  ``expert_up`` / ``expert_down`` that materialises
  ``original + scaling * lora_A @ lora_B`` on every access
  (``LoRAExpertTensor``, lora.py:93-165, registered at :199-215); the
  reference's contract is one materialisation per weight per call
  (tests/test_lora.py:391-440);
* a ``LoRALinear`` around each shared linear (lora.py:37-90), whose output
  ``base(x) + scaling * (dropout(x) @ A.T) @ B.T`` the engine's shared branch
  consumes (engine.py:333-349; tests/test_lora.py:267-329).

The adapters below have those two surfaces.  Expected outputs and factor
gradients are autograd of the oracle's universal forward in f64 on the CPU,
with each adapted weight written out from its factors (the f64 merge and the
two-step low-rank form agree to f64 rounding).  Bounds: normwise
max|got - ref| / max|ref| <= 1e-4 for fp32, 2e-2 for bf16.
"""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn.utils import parametrize

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

BOUND = {"fp32": 1e-4, "bf16": 2e-2}
DT = {"fp32": torch.float32, "bf16": torch.bfloat16}
EXPERTS = ("expert_gate", "expert_up", "expert_down")
SHARED = ("shared_gate", "shared_up", "shared_down")


class ExpertLoRA(nn.Module):
    """Parametrization W -> W + scaling * A @ B per expert (lora.py:93-165).
    ``calls`` counts materialisations."""

    def __init__(self, base: torch.Tensor, rank: int, alpha: float, gen: torch.Generator):
        super().__init__()
        E, fan_in, fan_out = base.shape
        self.scaling = alpha / rank
        self.lora_A = nn.Parameter((torch.randn(E, fan_in, rank, generator=gen) * 0.1).to(base.device, base.dtype))
        self.lora_B = nn.Parameter((torch.randn(E, rank, fan_out, generator=gen) * 0.02).to(base.device, base.dtype))
        self.calls = 0

    def forward(self, base: torch.Tensor) -> torch.Tensor:
        self.calls += 1
        return torch.baddbmm(base, self.lora_A, self.lora_B, beta=1.0, alpha=self.scaling)


class LinearLoRA(nn.Module):
    """LoRALinear's surface (lora.py:37-90): frozen ``base`` plus
    ``scaling * (dropout(x) A^T) B^T``."""

    is_lora_adapter = True

    def __init__(self, base: nn.Linear, rank: int, alpha: float, gen: torch.Generator, dropout: float = 0.0):
        super().__init__()
        self.base = base
        self.rank = rank
        self.scaling = alpha / rank
        self.dropout = nn.Dropout(dropout) if dropout else nn.Identity()
        w = base.weight
        self.lora_A = nn.Parameter((torch.randn(rank, base.in_features, generator=gen) * 0.1).to(w.device, w.dtype))
        self.lora_B = nn.Parameter((torch.randn(base.out_features, rank, generator=gen) * 0.02).to(w.device, w.dtype))
        self.base.requires_grad_(False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.base(x) + self.lora_residual(x)

    def lora_residual(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(F.linear(self.dropout(x), self.lora_A), self.lora_B) * self.scaling


def _engine(gpu, dtype, strategy, shared=256):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    engine = TRHashEngine(TRHashEngineConfig(hidden_size=128, vocab_size=5000, num_experts=4, top_k=2,
                                             shared_width=shared, expert_width=64,
                                             routing_strategy="token_id_multi_hash", routed_output_scale=2.0,
                                             shared_output_scale=0.5, precision=dtype, backend="hip")).to(gpu)
    if dtype == "bf16":
        engine = engine.to(torch.bfloat16)
    engine.routed_strategy = strategy
    return engine


def _adapt_experts(engine, gen):
    """Freeze the layer and parametrize its expert tensors (apply_lora, lora.py:193-215)."""
    engine.requires_grad_(False)
    adapters = {}
    for name in EXPERTS:
        a = ExpertLoRA(getattr(engine, name), rank=4, alpha=8.0, gen=gen)
        parametrize.register_parametrization(engine, name, a)
        engine.parametrizations[name].original.requires_grad_(False)
        a.calls = 0                                  # registration evaluates it once
        adapters[name] = a
    return adapters


def _adapt_shared(engine, gen, dropout=0.0):
    engine.requires_grad_(False)
    adapters = {}
    for name in SHARED:
        a = LinearLoRA(getattr(engine, name), rank=4, alpha=8.0, gen=gen, dropout=dropout)
        setattr(engine, name, a)
        adapters[name] = a
    return adapters


def _oracle(engine, x, ids, dout, expert_adapters=None, shared_adapters=None):
    """Output and gradients (x and every factor) by autograd of the oracle's
    forward in f64 on the CPU."""
    cfg = engine.config
    d = torch.float64
    leaves = {"x": x.detach().cpu().to(d).requires_grad_(True)}
    params = {}
    for name in EXPERTS:
        if expert_adapters:
            a = expert_adapters[name]
            orig = engine.parametrizations[name].original.detach().cpu().to(d)
            A = leaves[name + ".A"] = a.lora_A.detach().cpu().to(d).requires_grad_(True)
            B = leaves[name + ".B"] = a.lora_B.detach().cpu().to(d).requires_grad_(True)
            params[name] = orig + a.scaling * torch.bmm(A, B)
        else:
            params[name] = getattr(engine, name).detach().cpu().to(d)
    for name in SHARED:
        if shared_adapters:
            a = shared_adapters[name]
            A = leaves[name + ".A"] = a.lora_A.detach().cpu().to(d).requires_grad_(True)
            B = leaves[name + ".B"] = a.lora_B.detach().cpu().to(d).requires_grad_(True)
            params[name] = a.base.weight.detach().cpu().to(d) + a.scaling * (B @ A)
        else:
            params[name] = getattr(engine, name).weight.detach().cpu().to(d)
    out = O.engine_forward(leaves["x"], ids.cpu(), engine._active_route_table.cpu(), params,
                           route_weights=cfg.route_weights, shared_scale=cfg.shared_output_scale,
                           routed_scale=cfg.routed_output_scale)
    names = list(leaves)
    grads = torch.autograd.grad(out, [leaves[n] for n in names], dout.detach().cpu().to(d))
    return out.detach(), dict(zip(names, grads))


def _got_grads(xg, expert_adapters=None, shared_adapters=None):
    got = {"x": xg.grad}
    for group in (expert_adapters, shared_adapters):
        for name, a in (group or {}).items():
            got[name + ".A"], got[name + ".B"] = a.lora_A.grad, a.lora_B.grad
    return got


def _err(got, ref):
    return O.normwise_rel_err(got.float().cpu(), ref.float().cpu())


def _check_grads(got, ref, dtype):
    for name, r in ref.items():
        g = got[name]
        assert g is not None, name
        assert _err(g, r) <= BOUND[dtype], (name, _err(g, r))


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("strategy", ["dense", "grouped"])
def test_expert_lora_parametrization_follows_factor_updates(gpu, dtype, strategy):
    """Parametrized expert weights on HIP: outputs and factor gradients match
    the oracle before and after an optimizer step that changes the factors in
    place (no stale pack), and each weight is materialised once per call."""
    from complexity_amd.tr_hash import TRHashBackend

    print(f"expert LoRA parametrization {dtype} {strategy}", flush=True)
    gen = torch.Generator().manual_seed(11)
    engine = _engine(gpu, dtype, strategy)
    adapters = _adapt_experts(engine, gen)
    ids = torch.randint(0, 5000, (2, 150), generator=gen).to(gpu)      # 300 tokens: the saving path
    x = torch.randn(2, 150, 128, generator=gen).to(gpu, DT[dtype])
    dout = (torch.randn(2, 150, 128, generator=gen) * 0.1).to(gpu, DT[dtype])
    opt = torch.optim.SGD([p for a in adapters.values() for p in (a.lora_A, a.lora_B)], lr=2.0)

    for step in range(2):
        for a in adapters.values():
            a.calls = 0
        opt.zero_grad(set_to_none=True)
        xg = x.detach().clone().requires_grad_(True)
        out = engine(xg, ids)
        assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
        out.backward(dout)
        torch.cuda.synchronize()
        assert [adapters[n].calls for n in EXPERTS] == [1, 1, 1], step
        ref_out, ref = _oracle(engine, x, ids, dout, expert_adapters=adapters)
        assert _err(out, ref_out) <= BOUND[dtype], (step, _err(out, ref_out))
        _check_grads(_got_grads(xg, expert_adapters=adapters), ref, dtype)
        opt.step()                                   # changes A and B in place

    # inference: the pack is cached while the factors stay, rebuilt when one changes
    engine.eval()
    with torch.no_grad():
        first = engine(x, ids)
        pack = engine._packed
        again = engine(x, ids)
        assert engine._packed is pack and torch.equal(first, again)
        adapters["expert_down"].lora_B.mul_(-3.0)
        changed = engine(x, ids)
        assert engine._packed is not pack
    torch.cuda.synchronize()
    ref_out, _ = _oracle(engine, x, ids, dout, expert_adapters=adapters)
    assert _err(changed, ref_out) <= BOUND[dtype], _err(changed, ref_out)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("strategy", ["dense", "grouped"])
def test_shared_lora_runs_on_hip(gpu, dtype, strategy):
    """LoRALinear adapters on the shared linears stay on HIP (merged weights):
    outputs and factor gradients match the oracle across an optimizer step;
    active LoRA dropout resolves to PYTORCH with a reason."""
    from complexity_amd.tr_hash import TRHashBackend

    print(f"shared LoRA {dtype} {strategy}", flush=True)
    gen = torch.Generator().manual_seed(12)
    engine = _engine(gpu, dtype, strategy)
    adapters = _adapt_shared(engine, gen)
    ids = torch.randint(0, 5000, (2, 150), generator=gen).to(gpu)
    x = torch.randn(2, 150, 128, generator=gen).to(gpu, DT[dtype])
    dout = (torch.randn(2, 150, 128, generator=gen) * 0.1).to(gpu, DT[dtype])
    opt = torch.optim.SGD([p for a in adapters.values() for p in (a.lora_A, a.lora_B)], lr=2.0)

    engine.train()
    for step in range(2):
        opt.zero_grad(set_to_none=True)
        xg = x.detach().clone().requires_grad_(True)
        out = engine(xg, ids)
        assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
        out.backward(dout)
        torch.cuda.synchronize()
        ref_out, ref = _oracle(engine, x, ids, dout, shared_adapters=adapters)
        assert _err(out, ref_out) <= BOUND[dtype], (step, _err(out, ref_out))
        _check_grads(_got_grads(xg, shared_adapters=adapters), ref, dtype)
        opt.step()

    engine.eval()
    with torch.no_grad():
        out = engine(x, ids)
        assert engine.last_backend.selected is TRHashBackend.HIP
    torch.cuda.synchronize()
    ref_out, _ = _oracle(engine, x, ids, dout, shared_adapters=adapters)
    assert _err(out, ref_out) <= BOUND[dtype], _err(out, ref_out)

    # dropout on the low-rank branch in training mode has no merged weight
    for a in adapters.values():
        a.dropout = nn.Dropout(0.1)
    engine.train()
    with pytest.raises(RuntimeError, match="LoRA dropout"):
        engine(x, ids)
