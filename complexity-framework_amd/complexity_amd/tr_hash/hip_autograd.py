"""Differentiable HIP forward of one TR-Hash layer.

The reference keeps its Triton path differentiable with one autograd
Function per kernel (``CGGRGroupedGEMM``, ``HashCGGRGroupedGEMM``,
``PairHashReduce``..., complexity_cuda/triton_token_routed.py:1616-1833) and
nn.Linear autograd for the shared branch (engine.py:333-349).  Here the whole
layer is one Function: the forward runs the HIP kernels of
``ops.layer_forward`` and saves x and, above decode token counts, the raw
gate|up GEMM outputs and (dense strategy) the down GEMM's input h, which
the down weight gradient reads (at decode sizes the backward kernel
recomputes them);
the backward runs
``ops.layer_backward``: the SwiGLU backward kernel, the data gradient through
the down/combine kernels (the routed rows summed per token through the
inverse permutation) and the token-reduction weight-gradient GEMMs.

Gradients flow to x, to the shared linears' weights and to the expert
parameters (their active slice; rows and columns outside the active capacity
get zero, as slicing does under autograd).  token_ids and the route table
are not differentiable, as in the reference.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from .. import ops

# Token counts up to which the forward runs the decode-shape kernels and the
# backward recomputes gate|up instead of saving it.
SAVE_MIN_TOKENS = 128

_PARAM_NAMES = ("shared_gate", "shared_up", "shared_down", "expert_gate", "expert_up", "expert_down")


class _LayerPlan:
    """Non-tensor state of one differentiable call."""

    def __init__(self, packed: ops.PackedLayer, bwd_packs, token_ids: torch.Tensor, route_table: torch.Tensor,
                 route_weights: Sequence[float], shared_scale: float, routed_scale: float, order: int,
                 active: tuple):
        self.packed = packed
        self.bwd_packs = bwd_packs          # callable -> ops.BackwardPacks (built on first backward)
        self.token_ids = token_ids
        self.route_table = route_table
        self.route_weights = tuple(route_weights)
        self.shared_scale = float(shared_scale)
        self.routed_scale = float(routed_scale)
        self.order = order
        self.active = active                # (E_active, W_active)


class HIPLayerFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, plan: _LayerPlan, x: torch.Tensor, residual: Optional[torch.Tensor], *params):
        # Above the decode sizes the forward also keeps the raw gate|up outputs
        # (as the reference's autograd keeps the gate/up linear outputs), so
        # the backward runs one GEMM where it would otherwise run three.
        save = x.shape[0] > SAVE_MIN_TOKENS
        out = ops.layer_forward(x, plan.token_ids, plan.route_table, plan.packed, plan.route_weights,
                                plan.shared_scale, plan.routed_scale, order=plan.order, residual=residual,
                                save=save)
        gu = h = None
        if save:
            out, gu, h = out
        ctx.plan = plan
        ctx.has_residual = residual is not None
        ctx.param_shapes = [None if p is None else (p.shape, p.dtype) for p in params]
        ctx.save_for_backward(x, gu, h)
        return out

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        x, gu, h = ctx.saved_tensors
        plan: _LayerPlan = ctx.plan
        need_dx = ctx.needs_input_grad[1]
        need_dres = ctx.has_residual and ctx.needs_input_grad[2]
        need_params = ctx.needs_input_grad[3:]
        need_dw = any(need_params)
        dx, grads = ops.layer_backward(dout, x, plan.token_ids, plan.route_table, plan.packed, plan.bwd_packs(),
                                       plan.route_weights, plan.shared_scale, plan.routed_scale, order=plan.order,
                                       need_dx=need_dx, need_dw=need_dw, saved_gu=gu, saved_h=h)
        E, W = plan.active
        out_params = []
        for name, need, meta in zip(_PARAM_NAMES, need_params, ctx.param_shapes):
            g = grads.get(name) if need else None
            if g is None or meta is None:
                out_params.append(None)
                continue
            shape, dtype = meta
            if name.startswith("expert") and tuple(g.shape) != tuple(shape):
                full = torch.zeros(shape, dtype=g.dtype, device=g.device)
                if name == "expert_down":
                    full[:E, :W, :] = g
                else:
                    full[:E, :, :W] = g
                g = full
            out_params.append(g if g.dtype == dtype else g.to(dtype))
        return (None, dx if need_dx else None, dout if need_dres else None, *out_params)


class RMSNormFunction(torch.autograd.Function):
    """``weight * rmsnorm(x)`` (complexity/core/normalization/norms.py:46-55)
    on the HIP kernels, differentiable in x and weight: the forward saves
    x and each token's fp32 1/rms, the backward writes dx and the weight
    gradient (summed over tokens in a fixed order)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float):
        y, r = ops.rmsnorm_forward(x, weight, eps)
        ctx.save_for_backward(x, weight, r)
        return y

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x, weight, r = ctx.saved_tensors
        dx, dw = ops.rmsnorm_backward(x, weight, r, dy)
        return (dx if ctx.needs_input_grad[0] else None, dw if ctx.needs_input_grad[1] else None, None)


class RMSNormResidualFunction(torch.autograd.Function):
    """``(weight * rmsnorm(x), x)`` for the block's MLP half
    (block.py:271-278): the second output is x again (a view), the residual
    the layer adds.  Its gradient (the layer's dout) is added to dx inside
    the norm's backward kernel instead of by a separate sum over [N, H]."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float):
        y, r = ops.rmsnorm_forward(x, weight, eps)
        ctx.save_for_backward(x, weight, r)
        return y, x.view_as(x)

    @staticmethod
    def backward(ctx, dy: Optional[torch.Tensor], dres: Optional[torch.Tensor]):
        x, weight, r = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(x)
        dx, dw = ops.rmsnorm_backward(x, weight, r, dy, dres=dres)
        return (dx if ctx.needs_input_grad[0] else None, dw if ctx.needs_input_grad[1] else None, None)


def hip_layer_autograd(plan: _LayerPlan, x: torch.Tensor, residual: Optional[torch.Tensor], params) -> torch.Tensor:
    return HIPLayerFunction.apply(plan, x, residual, *params)
