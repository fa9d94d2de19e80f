"""Complex phase-quantized linear layer, MI355X edition.

Keeps the module API of RPFQ-ViT-main/quant_models/quant_i.py (class names,
constructor signatures, attributes, state-dict keys and errors) so models and
checkpoints written against the reference load unchanged:

* ``QATLinearComplexPhase(quant_method_u, quant_method_w, enable_act_quant,
  act_num_bits, enable_rotation, quant_group_size, *args, **kwargs)``
  (quant_i.py:475-511), ``forward(x[..., in]) -> y[..., out]``;
* ``ComplexWeightQuantizer`` / ``ComplexActivationQuantizer`` and the STE
  autograd functions (quant_i.py:121-191, :374-472);
* ``SUPPORTED_QUANT_METHODS`` (quant_i.py:355-362).

Execution:
* eval mode, device tensors -> the packed HIP path: the layer is packed once
  (codes + scales, re-packed when the weight changes) and every call runs the
  gfx950 kernels of librpfq.so through the C ABI.  There is no host fallback:
  if the library is missing the call raises.
* training mode on device tensors -> the quantization-aware forward with the
  weight quantized by the rpfq_quantize_wide kernels and activations by the
  act-quant kernel, straight-through gradients, F.linear on the float32 A_q
  (RPFQ_HIP_QAT=0 selects the torch formulation below);
* host tensors (or complex_phase_next_v1) -> the same forward in torch ops,
  the reference's training semantics.
"""
from __future__ import annotations

import math
import os
from typing import Dict, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import packing as P

TensorPair = Tuple[torch.Tensor, torch.Tensor]
EPS = 1e-6


# ---------------------------------------------------------------------------
# straight-through quantizers (training semantics)
# ---------------------------------------------------------------------------
def _axis_value(re, im):
    st = P.axis_stage(re, im, P.TRAIN_MIN_SCALE)
    return st.value_re, st.value_im


def _sign_value(re, im):
    st = P.sign_stage(re, im)
    return st.value_re, st.value_im


def _residual(re, im, steps, stage_fn):
    q_re, q_im = torch.zeros_like(re), torch.zeros_like(im)
    for _ in range(steps):
        s_re, s_im = stage_fn(re, im)
        q_re, q_im = q_re + s_re, q_im + s_im
        re, im = re - s_re, im - s_im
    return q_re, q_im


def _ste(name: str, steps: int, stage_fn, doc: str):
    """Autograd function: forward = quantizer, backward = identity."""

    def forward(ctx, w_real, w_imag):
        return _residual(w_real, w_imag, steps, stage_fn)

    def backward(ctx, grad_real, grad_imag):
        return grad_real, grad_imag

    return type(name, (torch.autograd.Function,), {
        "__doc__": doc, "forward": staticmethod(forward), "backward": staticmethod(backward)})


PhaseQuantSTE = _ste("PhaseQuantSTE", 1, _axis_value, "2-bit axis quantization (quant_i.py:121-130).")
PhaseQuantSTE_V2 = _ste("PhaseQuantSTE_V2", 2, _axis_value, "Two residual axis stages (quant_i.py:133-142).")
PhaseQuantSTE_V3 = _ste("PhaseQuantSTE_V3", 3, _axis_value, "Three residual axis stages (quant_i.py:145-154).")
PhaseQuantSTE_V4 = _ste("PhaseQuantSTE_V4", 4, _axis_value, "Four residual axis stages (quant_i.py:157-166).")
NewPhaseQuantSTE = _ste("NewPhaseQuantSTE", 1, _sign_value, "Quadrant-sign quantization (quant_i.py:169-178).")
NewPhaseQuantSTE_V2 = _ste("NewPhaseQuantSTE_V2", 2, _sign_value,
                           "Two residual quadrant-sign stages (quant_i.py:181-190).")


class LearnableGroupedPhaseQuant(nn.Module):
    """Learnable grouped phase quantizer (quant_i.py:193-351): per group of
    rows an optional rotation, nearest codeword of a learnable 4-phase
    codebook by cosine similarity, a least-squares group magnitude, and one
    residual quadrant-sign step; straight-through gradient for the weight."""

    def __init__(self, n_rows: int, group_size: int = 32, n_codewords: int = 4, enable_rotation: bool = True,
                 use_residual: bool = True, init_mode: str = "quadrant"):
        super().__init__()
        self.n_rows = n_rows
        self.group_size = group_size
        self.n_codewords = n_codewords
        self.enable_rotation = enable_rotation
        self.use_residual = use_residual
        self.num_groups = math.ceil(n_rows / group_size)
        if init_mode == "quadrant":
            phases = [math.pi / 4, 3 * math.pi / 4, -3 * math.pi / 4, -math.pi / 4]
        elif init_mode == "axis":
            phases = [0.0, math.pi / 2, math.pi, -math.pi / 2]
        else:
            raise ValueError(f"Unsupported init_mode: {init_mode}")
        init = torch.tensor(phases, dtype=torch.float32)
        if n_codewords != 4:
            init = torch.linspace(-math.pi, math.pi, steps=n_codewords + 1)[:-1]
        self.phase_angles = nn.Parameter(init)
        if enable_rotation:
            self.rotation_angles = nn.Parameter(torch.zeros(self.num_groups, 1, 1))
        else:
            self.register_parameter("rotation_angles", None)

    def _fit(self, w_real, w_imag, phase_angles, rotation_angles):
        """Steps 1-5 of the reference forward (quant_i.py:286-331): grouped,
        rotated planes, chosen codeword, group magnitudes and residual signs."""
        if w_real.shape != w_imag.shape:
            raise ValueError("w_real and w_imag must have the same shape.")
        rows, cols = w_real.shape
        gs = self.group_size
        pad = (gs - rows % gs) % gs
        valid = w_real.new_ones(rows, 1)
        wr, wi = w_real, w_imag
        if pad:
            wr, wi, valid = F.pad(wr, (0, 0, 0, pad)), F.pad(wi, (0, 0, 0, pad)), F.pad(valid, (0, 0, 0, pad))
        groups = wr.shape[0] // gs
        wr = wr.reshape(groups, gs, cols)
        wi = wi.reshape(groups, gs, cols)
        valid = valid.reshape(groups, gs, 1)
        c = s = None
        if self.enable_rotation:
            c, s = torch.cos(rotation_angles), torch.sin(rotation_angles)
            rr, ri = wr * c + wi * s, wi * c - wr * s
        else:
            rr, ri = wr, wi
        inv = torch.rsqrt((rr.square() + ri.square()).clamp_min(EPS))
        book = torch.stack((torch.cos(phase_angles), torch.sin(phase_angles)), dim=-1)
        sim = (rr * inv).unsqueeze(-1) * book[:, 0].view(1, 1, 1, -1) + \
              (ri * inv).unsqueeze(-1) * book[:, 1].view(1, 1, 1, -1)
        idx = sim.argmax(dim=-1)
        chosen = book[idx]
        d_re, d_im = chosen[..., 0], chosen[..., 1]
        num = ((rr * d_re + ri * d_im) * valid).sum(dim=(1, 2), keepdim=True)
        den = (((d_re.square() + d_im.square()) * valid).sum(dim=(1, 2), keepdim=True)).clamp_min(EPS)
        alpha = num / den
        q_re, q_im = alpha * d_re, alpha * d_im
        fit = {"rows": rows, "cols": cols, "c": c, "s": s, "book": book, "idx": idx, "alpha": alpha,
               "q_re": q_re, "q_im": q_im}
        if self.use_residual:
            e_re, e_im = rr - q_re, ri - q_im
            count = (valid.sum(dim=(1, 2), keepdim=True) * e_re.shape[-1]).clamp_min(1.0)
            fit["b_re"] = (e_re.abs() * valid).sum(dim=(1, 2), keepdim=True) / count
            fit["b_im"] = (e_im.abs() * valid).sum(dim=(1, 2), keepdim=True) / count
            fit["pos_re"], fit["pos_im"] = e_re >= 0, e_im >= 0
        return fit

    def forward(self, w_real: torch.Tensor, w_imag: torch.Tensor) -> TensorPair:
        f = self._fit(w_real, w_imag, self.phase_angles, self.rotation_angles)
        q_re, q_im = f["q_re"], f["q_im"]
        if self.use_residual:
            q_re = q_re + f["b_re"] * torch.where(f["pos_re"], 1.0, -1.0).to(q_re.dtype)
            q_im = q_im + f["b_im"] * torch.where(f["pos_im"], 1.0, -1.0).to(q_im.dtype)
        if self.enable_rotation:
            c, s = f["c"], f["s"]
            q_re, q_im = q_re * c - q_im * s, q_im * c + q_re * s
        q_re = q_re.reshape(-1, f["cols"])[:f["rows"]]
        q_im = q_im.reshape(-1, f["cols"])[:f["rows"]]
        return q_re + (w_real - w_real.detach()), q_im + (w_imag - w_imag.detach())

    def table(self, w_real: torch.Tensor, w_imag: torch.Tensor):
        """Packed form of forward() on host copies of the weight and the
        learned parameters: a 4-bit index per weight (codeword |
        (residual re >= 0) << 2 | (residual im >= 0) << 3) and per row the 16
        values the indices stand for, each formed by forward()'s float32 ops
        in forward()'s order (alpha d + beta sign, rotation back, + 0), so
        table[row][index] equals forward()'s value bit for bit.
        Returns (index uint8 [rows, cols], table_re, table_im float32 [rows, 16])."""
        if self.n_codewords != 4 or not self.use_residual:
            raise NotImplementedError("packed next_v1 needs 4 codewords and the residual sign step")
        pa = self.phase_angles.detach().cpu()
        ra = self.rotation_angles.detach().cpu() if self.rotation_angles is not None else None
        f = self._fit(w_real.detach().cpu().float(), w_imag.detach().cpu().float(), pa, ra)
        rows, cols = f["rows"], f["cols"]
        idx = (f["idx"].to(torch.uint8) | (f["pos_re"].to(torch.uint8) << 2) | (f["pos_im"].to(torch.uint8) << 3))
        e = torch.arange(16)
        d = f["book"][e & 3]                                   # [16, 2]
        sg_re = torch.where(((e >> 2) & 1) == 1, 1.0, -1.0)
        sg_im = torch.where(((e >> 3) & 1) == 1, 1.0, -1.0)
        alpha = f["alpha"].reshape(-1, 1)                      # [groups, 1]
        t_re = alpha * d[:, 0].view(1, 16) + f["b_re"].reshape(-1, 1) * sg_re.view(1, 16)
        t_im = alpha * d[:, 1].view(1, 16) + f["b_im"].reshape(-1, 1) * sg_im.view(1, 16)
        if self.enable_rotation:
            c, s = f["c"].reshape(-1, 1), f["s"].reshape(-1, 1)
            t_re, t_im = t_re * c - t_im * s, t_im * c + t_re * s
        t_re, t_im = t_re + 0.0, t_im + 0.0  # forward()'s "+ (w - w.detach())" (turns -0 into +0)
        gs = self.group_size
        t_re = t_re.repeat_interleave(gs, dim=0)[:rows].contiguous()
        t_im = t_im.repeat_interleave(gs, dim=0)[:rows].contiguous()
        return idx.reshape(-1, cols)[:rows].contiguous(), t_re, t_im


SUPPORTED_QUANT_METHODS = (
    "complex_phase_v1",
    "complex_phase_v2",
    "complex_phase_v3",
    "complex_phase_v4",
    "complex_phase_new_v2",
    "complex_phase_next_v1",
)

_FUNCTION_QUANTIZERS: Dict[str, type] = {
    "complex_phase_v1": PhaseQuantSTE,
    "complex_phase_v2": PhaseQuantSTE_V2,
    "complex_phase_v3": PhaseQuantSTE_V3,
    "complex_phase_v4": PhaseQuantSTE_V4,
    "complex_phase_new_v2": NewPhaseQuantSTE_V2,
}


class ComplexWeightQuantizer(nn.Module):
    """Quantizer of one complex plane (quant_i.py:374-435)."""

    def __init__(self, quant_method: str = "complex_phase_v1", enable_rotation: bool = False,
                 n_rows: int | None = None, group_size: int = 32):
        super().__init__()
        self.quant_method = quant_method
        self.enable_rotation = enable_rotation
        self.is_module_quantizer = quant_method == "complex_phase_next_v1"
        if quant_method not in SUPPORTED_QUANT_METHODS:
            raise ValueError(f"Unsupported quantization method: {quant_method}")
        if self.is_module_quantizer:
            if n_rows is None:
                raise ValueError("complex_phase_next_v1 requires n_rows.")
            self.quant_fn = LearnableGroupedPhaseQuant(n_rows=n_rows, group_size=group_size, n_codewords=4,
                                                       enable_rotation=enable_rotation, use_residual=True,
                                                       init_mode="quadrant")
            self.register_parameter("rotation_angle", None)
            return
        self.quant_fn = _FUNCTION_QUANTIZERS[quant_method]
        if enable_rotation:
            self.rotation_angle = nn.Parameter(torch.zeros(1))
        else:
            self.register_parameter("rotation_angle", None)

    def rotation_cos_sin(self):
        """float32 (cos, sin) of the learned global rotation, evaluated on the
        host (as the reference's CPU quantization does), or None."""
        if self.is_module_quantizer or not self.enable_rotation:
            return None
        theta = self.rotation_angle.detach().cpu()
        return torch.cos(theta), torch.sin(theta)

    def forward(self, w_real: torch.Tensor, w_imag: torch.Tensor) -> TensorPair:
        if self.is_module_quantizer:
            return self.quant_fn(w_real, w_imag)
        if not self.enable_rotation:
            return self.quant_fn.apply(w_real, w_imag)
        c, s = torch.cos(self.rotation_angle), torch.sin(self.rotation_angle)
        r_re, r_im = P.rotate_for_quant(w_real, w_imag, c, s)
        q_re, q_im = self.quant_fn.apply(r_re, r_im)
        return P.rotate_back(q_re, q_im, c, s)


class ActivationQuantSTE(torch.autograd.Function):
    """Per-row symmetric fake quantization of each half (quant_i.py:438-460):
    scale = qmax / max(|x|, 1e-5), x_hat = clamp(round(x scale)) / scale,
    round half to even."""

    @staticmethod
    def forward(ctx, x_real, x_imag, num_bits: int):
        qmax = (1 << (num_bits - 1)) - 1
        qmin = -(1 << (num_bits - 1))
        out = []
        for x in (x_real, x_imag):
            scale = float(qmax) / x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-5)
            out.append((x * scale).round().clamp(qmin, qmax) / scale)
        return out[0], out[1]

    @staticmethod
    def backward(ctx, grad_real, grad_imag):
        return grad_real, grad_imag, None


class ComplexActivationQuantizer(nn.Module):
    """Activation quantizer wrapper (quant_i.py:463-472)."""

    def __init__(self, num_bits: int):
        super().__init__()
        self.num_bits = num_bits

    def forward(self, x_real: torch.Tensor, x_imag: torch.Tensor) -> TensorPair:
        return ActivationQuantSTE.apply(x_real, x_imag, self.num_bits)


# ---------------------------------------------------------------------------
# HIP training path: the same quantizers as device kernels, straight-through
# gradients (quant_i.py:128-130, :452-455)
# ---------------------------------------------------------------------------
HIP_QAT = os.environ.get("RPFQ_HIP_QAT", "1") != "0"
# eval packing on the GPU quantizer instead of the host (float64-sum scales,
# ~1 ulp from the host's torch CPU order; no host round trip of the weight)
DEVICE_PACK = os.environ.get("RPFQ_DEVICE_PACK", "0") == "1"

# Eval-mode act quant in the packed layer's own launch (the streaming
# kernel's row prologue, rpfq_act_quant_wide_linear) where that launch
# qualifies; RPFQ_FUSE_AQ_PROLOGUE=0 runs the separate act-quant pass.
FUSE_AQ_PROLOGUE = os.environ.get("RPFQ_FUSE_AQ_PROLOGUE", "1") != "0"
# The MLP's GELU in fc1's store on every kernel (default); RPFQ_FUSE_GELU=1
# keeps torch's separate GELU pass after fp16 launches on the tiled kernels
# (fused only where fc1 streams or keeps its layer resident, and for bf16).
GELU_ON_TILED = os.environ.get("RPFQ_FUSE_GELU", "2") == "2"
# bf16 rows into a layer on the DMA kernel: the preceding LayerNorm writes
# them as prescaled fp16 operand rows (forward_layer_norm); "0" keeps the
# bf16 LayerNorm output and the kernel's in-LDS conversion.
PRESCALED_LN = os.environ.get("RPFQ_PRESCALED_LN", "1") != "0"
# Input gradient of the HIP training forward on the packed blob of the
# step's own codes (rpfq_wide_linear_grad_x) instead of the library GEMM on
# A_q: "1" on (each grad_y element of a float32 step then carries one fp16
# rounding, 2^-11 relative, and the fused fp16 coefficients replace A_q),
# "0" (default) off.  Measured on ViT-B/16 bs64, MI355X: float32 steps gain
# 2-5% (the kernel is ~3x faster than the float32 library GEMM); fp16
# autocast steps lose 20% (2,042 -> 1,626 images/s: the per-step repack and
# a host read of each rotated layer's angles cost more than the kernel,
# which is slower than the library's fp16 GEMM on the decoded weight).
QAT_PACKED_GRAD = os.environ.get("RPFQ_QAT_PACKED_GRAD", "0")

_HIP_KINDS = {
    "complex_phase_v1": ("axis", 1),
    "complex_phase_v2": ("axis", 2),
    "complex_phase_v3": ("axis", 3),
    "complex_phase_v4": ("axis", 4),
    "complex_phase_new_v2": ("sign", 2),
}


def rotation_grad(grad_aq: torch.Tensor, weight: torch.Tensor, a_q: torch.Tensor):
    """d loss / d theta of the U and W rotations under the straight-through
    quantizer.  With out = q e^{+i theta}, q = Q(w e^{-i theta}) and dQ = I,
    d out / d theta = (w_im - out_im, out_re - w_re) per element, so
    grad_theta = sum(g_re (w_im - out_im) + g_im (out_re - w_re)), with g the
    gradient of the plane (G11 + G22, G21 - G12 for U; G11 - G22, G12 + G21
    for W from the 2x2 blocks of grad_aq, quant_i.py:534-544) and out the
    plane of A_q (recovered by the same split as the weight)."""
    g11, g12, g21, g22 = _blocks(grad_aq)
    gu = (g11 + g22, g21 - g12)
    gw = (g11 - g22, g12 + g21)
    u_re, u_im, w_re, w_im = P.split_blocks(weight)
    ou_re, ou_im, ow_re, ow_im = P.split_blocks(a_q)
    th_u = (gu[0] * (u_im - ou_im) + gu[1] * (ou_re - u_re)).sum()
    th_w = (gw[0] * (w_im - ow_im) + gw[1] * (ow_re - w_re)).sum()
    return th_u, th_w


def _blocks(a: torch.Tensor):
    no, ni = a.shape[0] // 2, a.shape[1] // 2
    return a[:no, :ni], a[:no, ni:], a[no:, :ni], a[no:, ni:]


class _HipWideQuantSTE(torch.autograd.Function):
    """A_q from the float32 master weight by rpfq_quantize_wide; backward:
    the weight gets the A_q gradient unchanged (split and recombination are
    inverse linear maps and the quantizer is straight-through), the rotation
    angles get rotation_grad."""

    @staticmethod
    def forward(ctx, weight, theta_u, theta_w, spec):
        from . import ops

        rot = None
        if theta_u is not None:
            tu, tw = theta_u.detach().float().reshape(1), theta_w.detach().float().reshape(1)
            rot = torch.cat((torch.cos(tu), torch.sin(tu), torch.cos(tw), torch.sin(tw)))
        a_q, _, _ = ops.quantize_wide(weight.detach(), *spec, rot=rot)
        ctx.rotated = theta_u is not None
        if ctx.rotated:
            ctx.save_for_backward(weight, a_q)
        return a_q

    @staticmethod
    def backward(ctx, grad):
        if not ctx.rotated:
            return grad, None, None, None
        weight, a_q = ctx.saved_tensors
        th_u, th_w = rotation_grad(grad.float(), weight.detach(), a_q)
        return grad, th_u.reshape(1), th_w.reshape(1), None


class _GivenWeightSTE(torch.autograd.Function):
    """_HipWideQuantSTE with the quantization already done: forward returns
    the given A_q; backward as _HipWideQuantSTE (the weight gets the A_q
    gradient, the rotation angles rotation_grad)."""

    @staticmethod
    def forward(ctx, weight, theta_u, theta_w, a_q):
        ctx.rotated = theta_u is not None
        if ctx.rotated:
            ctx.save_for_backward(weight, a_q)
        return a_q

    @staticmethod
    def backward(ctx, grad):
        if not ctx.rotated:
            return grad, None, None, None
        weight, a_q = ctx.saved_tensors
        th_u, th_w = rotation_grad(grad.float(), weight.detach(), a_q)
        return grad, th_u.reshape(1), th_w.reshape(1), None


class _LinearPackedGradX(torch.autograd.Function):
    """F.linear(x, a_q, bias) whose input gradient runs on the packed blob
    of the same codes (grad_y A16, rpfq_wide_linear_grad_x) while the weight
    and bias gradients stay the library GEMM and column sum (kernel.py:
    581-588)."""

    @staticmethod
    def forward(ctx, x, a_q, bias, pw):
        ctx.pw = pw
        ctx.has_bias = bias is not None
        ctx.save_for_backward(x)
        return F.linear(x, a_q, bias)

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        g2 = grad.reshape(-1, grad.shape[-1])
        gx = ctx.pw.grad_x(grad, out_dtype=x.dtype) if ctx.needs_input_grad[0] else None
        gw = (g2.t() @ x.reshape(-1, x.shape[-1]).to(g2.dtype)) if ctx.needs_input_grad[1] else None
        gb = g2.sum(0) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return gx, gw, gb, None


class _HipActQuantSTE(torch.autograd.Function):
    """ActivationQuantSTE (quant_i.py:438-455) by the rpfq_act_quant kernel
    for float32 activations (bit-exact); identity gradient."""

    @staticmethod
    def forward(ctx, x, num_bits):
        from . import ops

        return ops.act_quant(x, num_bits)

    @staticmethod
    def backward(ctx, grad):
        return grad, None


class _PackedLinearFn(torch.autograd.Function):
    """Eval-mode packed layer under autograd: the forward runs
    rpfq_wide_linear; the backward gives the input the gradient through the
    packed weight on the device (rpfq_wide_linear_grad_x, the reference
    operator's grad_x = grad_output @ w_quant, kernel.py:585) and the bias
    its column sum (:588).  The packed weight is frozen (it is not a
    parameter), so it receives no gradient."""

    @staticmethod
    def forward(ctx, x, bias, pw):
        ctx.pw = pw
        ctx.x_dtype = x.dtype
        ctx.bias_dtype = None if bias is None else bias.dtype
        return pw.linear(x, None if bias is None else bias.detach(), out_dtype=x.dtype)

    @staticmethod
    def backward(ctx, grad):
        gx = ctx.pw.grad_x(grad, out_dtype=ctx.x_dtype) if ctx.needs_input_grad[0] else None
        gb = None
        if ctx.needs_input_grad[1]:
            gb = grad.reshape(-1, grad.shape[-1]).float().sum(0).to(ctx.bias_dtype)
        return gx, gb, None


def records_grad(module: nn.Module, x: torch.Tensor) -> bool:
    """Autograd records a call of `module` on x: grad mode is on and x or
    one of the module's parameters requires a gradient.  The fused inference
    kernels (LayerNorm, act quant, GELU, residual stores) have no backward,
    so every caller that picks them checks this one predicate."""
    return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in module.parameters()))


def _linear(x: torch.Tensor, q_weight: torch.Tensor, bias):
    """F.linear(x, A_q, bias) (quant_i.py:554).  Reduced-precision x outside
    autocast meets A_q and the bias cast to x's dtype, as autocast casts
    them (autograd flows through the casts)."""
    if x.dtype != q_weight.dtype and not torch.is_autocast_enabled(x.device.type):
        q_weight = q_weight.to(x.dtype)
        bias = None if bias is None else bias.to(x.dtype)
    return F.linear(x, q_weight, bias)


class QATLinearComplexPhase(nn.Linear):
    """Complex-structured quantized linear layer (quant_i.py:475-554).

    The weight [out, in] acts on features laid out [real half | imag half] as
    the widely-linear map y = U x + W conj(x) + b with U and W quantized to
    phase codes.  Eval-mode device tensors run the packed HIP kernels."""

    def __init__(self, quant_method_u: str = "complex_phase_v1", quant_method_w: str = "complex_phase_v1",
                 enable_act_quant: bool = True, act_num_bits: int = 4, enable_rotation: bool = False,
                 quant_group_size: int = 32, *args, **kwargs):
        super().__init__(*args, **kwargs)
        if self.in_features % 2 != 0 or self.out_features % 2 != 0:
            raise ValueError("Complex-phase QAT requires even in/out features.")
        self.enable_act_quant = enable_act_quant
        rows = self.out_features // 2
        self.quantizer_u = ComplexWeightQuantizer(quant_method=quant_method_u, enable_rotation=enable_rotation,
                                                  n_rows=rows, group_size=quant_group_size)
        self.quantizer_w = ComplexWeightQuantizer(quant_method=quant_method_w, enable_rotation=enable_rotation,
                                                  n_rows=rows, group_size=quant_group_size)
        self.act_quantizer = ComplexActivationQuantizer(num_bits=act_num_bits) if enable_act_quant else None
        # packed HIP state (not part of the state dict)
        self.use_packed = True
        self.pack_on_device = DEVICE_PACK
        self._packed = None
        self._packed_key = None
        self._override = None

    # -- training-semantics forward (reference arithmetic, autograd STE) ----
    def quantized_weight(self) -> torch.Tensor:
        """A_q [out, in] as the reference forms it (quant_i.py:514-544)."""
        u_re, u_im, w_re, w_im = P.split_blocks(self.weight)
        uq_re, uq_im = self.quantizer_u(u_re, u_im)
        wq_re, wq_im = self.quantizer_w(w_re, w_im)
        return P.join_blocks(uq_re, uq_im, wq_re, wq_im)

    def _hip_qat_spec(self, x: torch.Tensor):
        """(kind_u, steps_u, kind_w, steps_w) when the training forward runs
        on the HIP quantizer, else None (host tensors, next_v1, disabled)."""
        if not (HIP_QAT and self.use_packed and x.is_cuda and self.weight.dtype == torch.float32):
            return None
        ku = _HIP_KINDS.get(self.quantizer_u.quant_method)
        kw = _HIP_KINDS.get(self.quantizer_w.quant_method)
        if ku is None or kw is None:
            return None
        return ku + kw

    @staticmethod
    def _packed_grad() -> bool:
        return QAT_PACKED_GRAD == "1" and torch.is_grad_enabled()

    def _qat_forward_packed_grad(self, x: torch.Tensor, spec) -> torch.Tensor:
        """The HIP training forward with the input gradient on the packed
        blob of this step's codes (QAT_PACKED_GRAD)."""
        from . import ops

        qu, qw = self.quantizer_u, self.quantizer_w
        rot, rotation = None, None
        if qu.rotation_angle is not None:
            th = torch.cat((qu.rotation_angle.detach().float().reshape(1), qw.rotation_angle.detach().float().reshape(1)))
            rot = torch.stack((torch.cos(th[0]), torch.sin(th[0]), torch.cos(th[1]), torch.sin(th[1])))
            v = rot.tolist()
            rotation = ((v[0], v[1]), (v[2], v[3]))
        a_q, scales, codes = ops.quantize_wide(self.weight.detach(), *spec, rot=rot, want_codes=True)
        q_weight = _GivenWeightSTE.apply(self.weight, qu.rotation_angle, qw.rotation_angle, a_q)
        lc = P.quantizer_codes(scales, codes, self.out_features // 2, self.in_features // 2, spec[0], spec[1],
                               rotation)
        pw = ops.pack_layer(lc.planes, lc.scale_re, lc.scale_im, lc.n_complex, lc.k_complex, lc.codebook, lc.stages,
                            0, rotation, sync=False)
        if self.act_quantizer is not None:
            if x.dtype == torch.float32:
                x = _HipActQuantSTE.apply(x, self.act_quantizer.num_bits)
            else:
                h = self.in_features // 2
                x = torch.cat(self.act_quantizer(x[..., :h], x[..., h:]), dim=-1)
        return _LinearPackedGradX.apply(x, q_weight, self.bias, pw)

    def _qat_forward(self, x: torch.Tensor) -> torch.Tensor:
        spec = self._hip_qat_spec(x)
        if spec is not None and spec[0] == spec[2] and spec[1] == spec[3] and self._packed_grad():
            return self._qat_forward_packed_grad(x, spec)
        if spec is not None:
            q_weight = _HipWideQuantSTE.apply(self.weight, self.quantizer_u.rotation_angle,
                                              self.quantizer_w.rotation_angle, spec)
            if self.act_quantizer is not None:
                if x.dtype == torch.float32:
                    x = _HipActQuantSTE.apply(x, self.act_quantizer.num_bits)
                else:  # reduced-precision activations: the reference's per-op rounding
                    h = self.in_features // 2
                    x = torch.cat(self.act_quantizer(x[..., :h], x[..., h:]), dim=-1)
            return _linear(x, q_weight, self.bias)
        q_weight = self.quantized_weight()
        if self.act_quantizer is not None:
            h = self.in_features // 2
            qr, qi = self.act_quantizer(x[..., :h], x[..., h:])
            x = torch.cat((qr, qi), dim=-1)
        return _linear(x, q_weight, self.bias)

    # -- packed HIP path ------------------------------------------------------
    def load_packed(self, codes: "P.LayerCodes") -> None:
        """Run this layer from externally supplied code planes and scales
        (e.g. an exported bundle or the benchmark's synthetic codes) instead
        of packing its own float32 weight."""
        if codes.n_complex * 2 != self.out_features or codes.k_complex * 2 != self.in_features:
            raise ValueError("packed codes do not match the layer shape")
        self._override = codes
        self._packed = None
        self._packed_key = None

    def packed(self, device: torch.device):
        """The layer's PackedWide on `device`, packing on first use and again
        whenever the float32 weight changed."""
        from .ops import pack_layer

        key = ("override", id(self._override)) if self._override is not None else \
            (self.weight.data_ptr(), self.weight._version, self._rotation_version())
        if self._packed is not None and self._packed_key == key and self._packed.device == device:
            return self._packed
        if self._override is not None:
            lc = self._override
        elif self.quantizer_u.is_module_quantizer or self.quantizer_w.is_module_quantizer:
            lc = self._table_codes()
        elif self.pack_on_device and self.weight.is_cuda:
            lc = P.quantize_layer_device(self.weight, self.quantizer_u.quant_method, self.quantizer_w.quant_method,
                                         self.quantizer_u.rotation_cos_sin(), self.quantizer_w.rotation_cos_sin())
        else:
            # offline step, on the host in float32 like the reference's
            # exporter, so codes and scales are bit-identical to the
            # reference's CPU quantization (device sums reorder float32 adds)
            rot_u = self.quantizer_u.rotation_cos_sin()
            rot_w = self.quantizer_w.rotation_cos_sin()
            lc = P.quantize_layer(self.weight.detach().cpu(), self.quantizer_u.quant_method,
                                  self.quantizer_w.quant_method, rot_u, rot_w)
        self._packed = pack_layer([p.to(device) for p in lc.planes], [s.to(device) for s in lc.scale_re],
                                  [s.to(device) for s in lc.scale_im], lc.n_complex, lc.k_complex, lc.codebook,
                                  lc.stages, lc.block, lc.rotation)
        self._packed_key = key
        return self._packed

    def _table_codes(self) -> "P.LayerCodes":
        """complex_phase_next_v1 in the TABLE codebook: 4-bit indices and the
        per-row value tables of both learned grouped quantizers (host)."""
        if not (self.quantizer_u.is_module_quantizer and self.quantizer_w.is_module_quantizer):
            raise NotImplementedError("packed HIP path needs complex_phase_next_v1 for both U and W")
        from . import _native as N

        u_re, u_im, w_re, w_im = P.split_blocks(self.weight.detach().cpu().float())
        iu, tu_re, tu_im = self.quantizer_u.quant_fn.table(u_re, u_im)
        iw, tw_re, tw_im = self.quantizer_w.quant_fn.table(w_re, w_im)
        return P.LayerCodes([P.pack4(iu), P.pack4(iw)], [tu_re, tw_re], [tu_im, tw_im], u_re.shape[0],
                            u_re.shape[1], N.CB_TABLE, 1, 0, None)

    def _rotation_version(self):
        vs = []
        for q in (self.quantizer_u, self.quantizer_w):
            params = [q.rotation_angle] if q.rotation_angle is not None else []
            if q.is_module_quantizer:
                params = [p for p in (q.quant_fn.phase_angles, q.quant_fn.rotation_angles) if p is not None]
            for p in params:
                vs.append((p.data_ptr(), p._version))
        return tuple(vs)

    def _weights_need_grad(self) -> bool:
        """A parameter the packed blob is derived from (the float32 weight,
        the rotation angles, the learned phase tables) requires a gradient.
        Codes supplied through load_packed are not derived from them, so such
        a layer's weights get no gradient from its output."""
        if self._override is not None:
            return False
        return any(p.requires_grad for name, p in self.named_parameters() if name != "bias")

    def _records_grad(self, x: torch.Tensor) -> bool:
        """Autograd records this call: x or a parameter needs a gradient
        (records_grad, shared with the model-level fused-block predicate)."""
        return records_grad(self, x)

    def _packed_forward(self, x: torch.Tensor, prequantized: bool = False) -> torch.Tensor:
        from . import ops

        if prequantized and self._records_grad(x):
            raise RuntimeError("forward_prequantized under autograd: the fused act quant has no gradient")
        if torch.is_grad_enabled() and self._weights_need_grad():
            # The reference's forward is the same straight-through formulation
            # in eval as in training (quant_i.py:513-554), so the weight and
            # rotation angles get their gradients; the packed blob is a
            # constant of the weight and could give them none.
            return self._qat_forward(x)
        pw = self.packed(x.device)
        if self._records_grad(x):
            if self.act_quantizer is not None and not prequantized:
                x = _HipActQuantSTE.apply(x, self.act_quantizer.num_bits)
            return _PackedLinearFn.apply(x, self.bias, pw)
        bias = None if self.bias is None else self.bias.detach()
        if self.act_quantizer is not None and not prequantized:
            if self._aq_fusable(pw, x):  # act quant in the layer's own launch
                return pw.act_quant_linear(x, self.act_quantizer.num_bits, bias, out_dtype=x.dtype)
            x = ops.act_quant(x, self.act_quantizer.num_bits)
        return pw.linear(x, bias, out_dtype=x.dtype)

    @staticmethod
    def _aq_fusable(pw, x: torch.Tensor) -> bool:
        """The streaming kernel's row prologue takes this launch
        (rpfq_act_quant_wide_linear: a layer at batch 1-2, K' <= 384)."""
        m = x.numel() // x.shape[-1] if x.dim() else 0
        return FUSE_AQ_PROLOGUE and hasattr(pw, "ln_fusable") and m > 0 and pw.ln_fusable(m, x.dtype)

    def packed_inference(self, x: torch.Tensor):
        """The packed layer (ops.PackedWide or a stage-group container) the
        inference path would contract x with when that path applies without
        an activation quantizer (eval mode, device tensors, no autograd
        recording), else None: what a caller fusing this layer with its
        neighbours (ops.wide_mlp) may use in its place."""
        if self.act_quantizer is not None or not (x.is_cuda and not self.training and self.use_packed) \
                or self._records_grad(x):
            return None
        return self.packed(x.device)

    def packed_act_bits(self, x: torch.Tensor) -> int:
        """Bits of the activation quantization the packed inference path would
        apply to x (0 if none, if x does not take the packed path, or if
        autograd records the call: the fused kernels have no backward)."""
        if self.act_quantizer is None or not (x.is_cuda and not self.training and self.use_packed) \
                or self._records_grad(x):
            return 0
        return self.act_quantizer.num_bits

    def forward_prequantized(self, x: torch.Tensor) -> torch.Tensor:
        """forward() for an input the caller already fake-quantized exactly as
        this layer's activation quantizer would (e.g. by
        rpfq_layer_norm_act_quant); only valid when packed_act_bits(x) > 0."""
        return self._packed_forward(x, prequantized=True)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda and not self.training and self.use_packed:
            return self._packed_forward(x)
        return self._qat_forward(x)

    def forward_gelu(self, x: torch.Tensor, prequantized: bool = False) -> torch.Tensor:
        """F.gelu(self(x)) (exact erf GELU); x already activation-quantized
        for this layer if prequantized.  On the packed HIP path the GELU runs
        in the kernel's store (within 1 ulp of the exact GELU of the rounded
        output) where the launch streams or keeps the layer resident in LDS
        (HBM-bound, its VALU mostly idle) and on the tiled kernels.  ViT-B/16
        bs256, same box: bf16 15,510 -> 16,197 images/s fused; fp16 18,079 ->
        18,458 (fc1's launch grows by ~30%, less than torch's separate pass
        over the 3072-wide hidden state costs)."""
        if x.is_cuda and not self.training and self.use_packed and not self._records_grad(x):
            from . import _native as N
            from . import ops

            pw = self.packed(x.device)
            bias = None if self.bias is None else self.bias.detach()
            if self.act_quantizer is not None and not prequantized:
                if self._aq_fusable(pw, x):  # act quant, layer and GELU in one launch
                    return pw.act_quant_linear(x, self.act_quantizer.num_bits, bias, out_dtype=x.dtype, gelu=True)
                x = ops.act_quant(x, self.act_quantizer.num_bits)
            m = x.numel() // x.shape[-1]
            kern = pw.kernel_for(m, x.dtype, x.dtype, N.FLAG_GELU) if m else None
            if kern in N.STREAM_KERNELS or kern == N.KERNEL_RESIDENT or x.dtype == torch.bfloat16 or GELU_ON_TILED:
                return pw.linear(x, bias, out_dtype=x.dtype, gelu=True)
            return F.gelu(pw.linear(x, bias, out_dtype=x.dtype))
        return F.gelu(self.forward_prequantized(x) if prequantized else self.forward(x))

    def forward_layer_norm(self, x: torch.Tensor, ln_weight, ln_bias, eps: float, gelu: bool = False):
        """self(layer_norm(x)) (and its exact GELU if gelu) with the LayerNorm
        fused into the packed layer's launch (rpfq_layer_norm_wide_linear), or
        None where that launch does not apply (training, autograd, host
        tensors, activation quantization on, stage groups, a launch the fused
        kernel does not take: see PackedWide.ln_fusable).  With activation
        quantization the LayerNorm + act quant row kernel runs first instead:
        in the prologue of every one of qkv's 36 (fc1's 48) tiles it measured
        slower at one ViT-B/16 image (qkv 15.5 vs 5.2 + 9.5 us, fc1 19.3 vs
        5.2 + 12.0 us); the act quant alone pays in the prologue (proj 9.3 vs
        4.7 + 9.2 us), see _packed_forward / forward_residual.
        bf16 / float32 rows the DMA kernel takes (large M) instead go
        through the LayerNorm as prescaled fp16 operand rows
        (rpfq_layer_norm_prescaled): for bf16 bit-identical to the LayerNorm
        then the layer on the bf16 rows with their range-guard prescales,
        without the kernel's in-LDS bf16 conversion or the prescale pass
        (ViT-B/16 qkv at 50,432 rows: 303 -> 209 us); float32 rows leave the
        register-staged kernel with the same fp16 operands."""
        if not (x.is_cuda and not self.training and self.use_packed) or self.act_quantizer is not None \
                or self._records_grad(x):
            return None
        pw = self.packed(x.device)
        m = x.numel() // x.shape[-1]
        if not hasattr(pw, "ln_fusable") or m == 0:
            return None
        bias = None if self.bias is None else self.bias.detach()
        if pw.ln_fusable(m, x.dtype):
            return pw.layer_norm_linear(x, ln_weight, ln_bias, eps, bias, out_dtype=x.dtype, gelu=gelu)
        from . import _native as N
        from . import ops

        c = x.shape[-1]
        if (PRESCALED_LN and x.dtype in (torch.bfloat16, torch.float32) and c % 8 == 0 and c <= 4096
                and pw.kernel_for(m, torch.float16, x.dtype, N.FLAG_GELU if gelu else 0) == N.KERNEL_DMA):
            h, sc = ops.layer_norm_prescaled(x, ln_weight, ln_bias, eps)
            return pw.linear(h, bias, out_dtype=x.dtype, gelu=gelu, row_scale=sc)
        return None

    def forward_residual(self, x: torch.Tensor, residual: torch.Tensor, prequantized: bool = False) -> torch.Tensor:
        """residual + self(x); x already activation-quantized for this layer
        if prequantized.  On the packed HIP path the add is fused into the
        kernel's store (bit-identical to the unfused add in x's dtype);
        elsewhere it is the plain sum."""
        if x.is_cuda and not self.training and self.use_packed and not self._records_grad(x):
            from . import ops

            pw = self.packed(x.device)
            bias = None if self.bias is None else self.bias.detach()
            if self.act_quantizer is not None and not prequantized:
                if self._aq_fusable(pw, x):  # act quant, layer and residual add in one launch
                    return pw.act_quant_linear(x, self.act_quantizer.num_bits, bias, out_dtype=x.dtype,
                                               residual=residual)
                x = ops.act_quant(x, self.act_quantizer.num_bits)
            return pw.linear(x, bias, out_dtype=x.dtype, residual=residual)
        return residual + (self.forward_prequantized(x) if prequantized else self.forward(x))
