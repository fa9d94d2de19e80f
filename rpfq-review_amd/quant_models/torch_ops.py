"""PyTorch operators of the packed path under the ``rpfq`` namespace.

The reference exposes its layer as one custom operator,
``torch.ops.quant.QATLinearComplexPhaseV2_forward(Tensor x, Tensor weight,
Tensor? bias) -> Tensor`` (RPFQ-ViT-main/quant_models/kernel.py:599-605,
CompositeExplicitAutograd).  The same ``(x, weight-or-packed, bias) -> y``
contract is registered here, running the HIP kernels of librpfq.so:

* ``torch.ops.rpfq.qat_linear(x, weight, bias, method_u="complex_phase_v2",
  method_w="complex_phase_v2", act_bits=8)``: called as ``(x, weight, bias)``
  it takes the reference operator's configuration -- two residual axis
  stages for U and W and 8-bit activations (kernel.py:416-445, :504-505) --
  in quant_i.py's float32 arithmetic (the Triton operator splits U / W to
  bf16 first).  It is the reference layer's training forward
  (quant_i.py:513-554) with the weight
  quantized on the GPU (rpfq_quantize_wide) and float32 activations
  fake-quantized by the act-quant kernel, ``F.linear`` on the float32 A_q;
  backward straight-through (the weight receives the A_q gradient, the input
  the gradient through A_q).  No global rotation (a module-level parameter in
  the reference, handled by QATLinearComplexPhase).
* ``torch.ops.rpfq.wide_linear(x, packed, n_complex, k_complex, codebook,
  stages, block, rotation, bias)``: a packed blob (rpfq_wide_linear),
  y = U x + W conj(x) + bias on [re | im] features; backward: the input
  gradient on the same blob (rpfq_wide_linear_grad_x, after relaying its
  codes out with rpfq_wide_pack_adjoint per call) and the bias gradient as
  the column sum (the reference operator's backward, kernel.py:585-588).
* ``torch.ops.rpfq.act_quant(x, num_bits)``: ActivationQuantSTE's forward
  (quant_i.py:438-455) on [..., 2K'] features.

Each operator has a fake (meta) implementation, so shapes propagate under
FakeTensor tracing without a GPU.  Device tensors only at run time: the
kernels have no host path.
"""
from __future__ import annotations

from typing import List, Optional

import torch
import torch.nn.functional as F

from . import _native as N

_KINDS = {
    "complex_phase_v1": ("axis", 1),
    "complex_phase_v2": ("axis", 2),
    "complex_phase_v3": ("axis", 3),
    "complex_phase_v4": ("axis", 4),
    "complex_phase_new_v2": ("sign", 2),
}


def _spec(method_u: str, method_w: str):
    if method_u not in _KINDS or method_w not in _KINDS:
        raise ValueError(f"rpfq.qat_linear supports {sorted(_KINDS)}; got U={method_u}, W={method_w}")
    return _KINDS[method_u] + _KINDS[method_w]


def _act(x: torch.Tensor, act_bits: int) -> torch.Tensor:
    from . import ops

    return ops.act_quant(x, act_bits) if act_bits > 0 else x


@torch.library.custom_op("rpfq::qat_linear", mutates_args=())
def qat_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
               method_u: str = "complex_phase_v2", method_w: str = "complex_phase_v2",
               act_bits: int = 8) -> torch.Tensor:
    from . import ops

    N.require_device(x, weight, bias)
    a_q, _, _ = ops.quantize_wide(weight.detach().float(), *_spec(method_u, method_w))
    return F.linear(_act(x, act_bits), a_q.to(x.dtype), None if bias is None else bias.to(x.dtype))


@qat_linear.register_fake
def _(x, weight, bias, method_u="complex_phase_v2", method_w="complex_phase_v2", act_bits=8):
    return x.new_empty(tuple(x.shape[:-1]) + (weight.shape[0],))


def _qat_setup(ctx, inputs, output):
    x, weight, bias, method_u, method_w, act_bits = inputs
    ctx.spec = _spec(method_u, method_w)
    ctx.act_bits = act_bits
    ctx.has_bias = bias is not None
    ctx.save_for_backward(x, weight)


def _qat_backward(ctx, grad):
    from . import ops

    x, weight = ctx.saved_tensors
    a_q, _, _ = ops.quantize_wide(weight.detach().float(), *ctx.spec)
    xq = _act(x, ctx.act_bits)
    g2 = grad.reshape(-1, grad.shape[-1])
    grad_x = (g2 @ a_q.to(g2.dtype)).reshape(x.shape)          # straight through the act quant
    grad_w = (g2.t().float() @ xq.reshape(-1, x.shape[-1]).float()).to(weight.dtype)  # and the weight quant
    grad_b = g2.sum(0) if ctx.has_bias else None
    return grad_x, grad_w, grad_b, None, None, None


qat_linear.register_autograd(_qat_backward, setup_context=_qat_setup)


@torch.library.custom_op("rpfq::wide_linear", mutates_args=())
def wide_linear(x: torch.Tensor, packed: torch.Tensor, n_complex: int, k_complex: int, codebook: int,
                stages: int, block: int, rotation: Optional[List[float]], bias: Optional[torch.Tensor]) -> torch.Tensor:
    from . import ops

    rot = None
    if rotation is not None:
        if len(rotation) != 4:
            raise ValueError("rotation is [cos_u, sin_u, cos_w, sin_w]")
        rot = ((rotation[0], rotation[1]), (rotation[2], rotation[3]))
    pw = ops.PackedWide(n_complex, k_complex, codebook, stages, block, packed, rot)
    return pw.linear(x, bias)


@wide_linear.register_fake
def _(x, packed, n_complex, k_complex, codebook, stages, block, rotation, bias):
    return x.new_empty(tuple(x.shape[:-1]) + (2 * n_complex,))


def _wide_setup(ctx, inputs, output):
    x, packed, n_complex, k_complex, codebook, stages, block, rotation, bias = inputs
    ctx.layer = (n_complex, k_complex, codebook, stages, block, rotation)
    ctx.x_dtype = x.dtype
    ctx.bias_dtype = None if bias is None else bias.dtype
    ctx.save_for_backward(packed)


def _wide_backward(ctx, grad):
    from . import ops

    (packed,) = ctx.saved_tensors
    n_complex, k_complex, codebook, stages, block, rotation = ctx.layer
    rot = None if rotation is None else ((rotation[0], rotation[1]), (rotation[2], rotation[3]))
    pw = ops.PackedWide(n_complex, k_complex, codebook, stages, block, packed, rot)
    grad_x = pw.grad_x(grad, out_dtype=ctx.x_dtype) if ctx.needs_input_grad[0] else None
    grad_b = None
    if ctx.bias_dtype is not None and ctx.needs_input_grad[8]:
        grad_b = grad.reshape(-1, grad.shape[-1]).float().sum(0).to(ctx.bias_dtype)
    return grad_x, None, None, None, None, None, None, None, grad_b


wide_linear.register_autograd(_wide_backward, setup_context=_wide_setup)


@torch.library.custom_op("rpfq::act_quant", mutates_args=())
def act_quant(x: torch.Tensor, num_bits: int) -> torch.Tensor:
    from . import ops

    return ops.act_quant(x, num_bits)


@act_quant.register_fake
def _(x, num_bits):
    return torch.empty_like(x)
