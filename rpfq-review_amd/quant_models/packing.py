"""Weight preparation: float32 master weights -> packed phase-code planes.

This is the offline step of the path (the reference's exporter role), run
once per layer when a model is packed, not per forward.  It follows the
reference arithmetic op for op in float32 torch so the codes and scales are
bit-identical to what the reference computes on the same device:

* training semantics  -- RPFQ-ViT-main/quant_models/quant_i.py:29-118, :425-435
  (per-tensor float32 scales, residual taken against the float32 stage);
* export semantics    -- RPFQ-ViTApple/scripts/export_rpfq_vit_to_mlx.py:121-289
  (gamma = fp16(1/scale), residual taken against the fp16-gamma stage).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _native as N

TRAIN_MIN_SCALE = 1e-5   # quant_i.py:29
EXPORT_MIN_SCALE = 1e-6  # export_rpfq_vit_to_mlx.py:121
SIGN_MIN_SCALE = 1e-6    # quant_i.py:26, :86-87


def split_blocks(weight: torch.Tensor):
    """[out, in] real weight -> U and W complex planes (quant_i.py:519-527).

    Returns (u_re, u_im, w_re, w_im), each [out/2, in/2]."""
    out_f, in_f = weight.shape
    if out_f % 2 or in_f % 2:
        raise ValueError("Complex-phase QAT requires even in/out features.")
    no, ni = out_f // 2, in_f // 2
    top, bot = weight[:no], weight[no:]
    a11, a12, a21, a22 = top[:, :ni], top[:, ni:], bot[:, :ni], bot[:, ni:]
    return 0.5 * (a11 + a22), 0.5 * (a21 - a12), 0.5 * (a11 - a22), 0.5 * (a12 + a21)


def join_blocks(u_re, u_im, w_re, w_im) -> torch.Tensor:
    """Quantized U/W -> fused real weight (quant_i.py:534-544)."""
    top = torch.cat((w_re + u_re, w_im - u_im), dim=1)
    bot = torch.cat((w_im + u_im, -w_re + u_re), dim=1)
    return torch.cat((top, bot), dim=0)


def dominant_axis(re: torch.Tensor, im: torch.Tensor):
    """(real_pos, real_neg, imag_pos, imag_neg) boolean masks with the
    quadrant tie rule of quant_i.py:36-62: |re| > |im| -> real axis,
    |im| > |re| -> imaginary axis; on |re| == |im| quadrants IV and II go to
    the real axis (+1 / -1), I and III to the imaginary axis (+i / -i), and
    (0, 0) to +1."""
    mag_re, mag_im = re.abs(), im.abs()
    on_re = mag_re > mag_im
    on_im = mag_im > mag_re
    even = ~(on_re | on_im)
    re_pos, re_neg = re > 0, re < 0
    im_pos, im_neg = im > 0, im < 0
    real_pos = (on_re & (re >= 0)) | (even & re_pos & im_neg) | (even & (re == 0) & (im == 0))
    real_neg = (on_re & (re < 0)) | (even & re_neg & im_pos)
    imag_pos = (on_im & (im >= 0)) | (even & re_pos & im_pos)
    imag_neg = (on_im & (im < 0)) | (even & re_neg & im_neg)
    return real_pos, real_neg, imag_pos, imag_neg


def masked_mean_abs(x: torch.Tensor, mask: torch.Tensor, floor: float) -> torch.Tensor:
    """Mean |x| over `mask`, floored (quant_i.py:29-33)."""
    m = mask.to(dtype=x.dtype)
    return ((x.abs() * m).sum() / m.sum().clamp_min(1.0)).clamp_min(floor)


@dataclass
class Stage:
    codes: torch.Tensor       # uint8 [N', K'] codes 0..3
    scale_re: torch.Tensor    # float32 0-dim multiplier
    scale_im: torch.Tensor
    value_re: torch.Tensor    # float32 [N', K'] quantized stage value
    value_im: torch.Tensor


def axis_stage(re: torch.Tensor, im: torch.Tensor, floor: float) -> Stage:
    """One axis stage (quant_i.py:65-81); codes as the exporter assigns them
    (real_pos=1, imag_neg=2, imag_pos=3, otherwise 0;
    export_rpfq_vit_to_mlx.py:214-218)."""
    rp, rn, ip, ineg = dominant_axis(re, im)
    s_re = masked_mean_abs(re, rp | rn, floor)
    s_im = masked_mean_abs(im, ip | ineg, floor)
    zero = torch.zeros_like(re)
    v_re = torch.where(rn, -s_re, torch.where(rp, s_re, zero))
    v_im = torch.where(ineg, -s_im, torch.where(ip, s_im, zero))
    codes = torch.zeros(re.shape, dtype=torch.uint8, device=re.device)
    codes[rp] = 1
    codes[ineg] = 2
    codes[ip] = 3
    return Stage(codes, s_re, s_im, v_re, v_im)


def sign_stage(re: torch.Tensor, im: torch.Tensor) -> Stage:
    """Quadrant-sign stage (quant_i.py:84-91): code bit0 = re >= 0,
    bit1 = im >= 0; scales are unmasked mean |.|."""
    s_re = re.abs().mean().clamp_min(SIGN_MIN_SCALE)
    s_im = im.abs().mean().clamp_min(SIGN_MIN_SCALE)
    pr, pi = re >= 0, im >= 0
    v_re = torch.where(pr, s_re, -s_re).to(re.dtype)
    v_im = torch.where(pi, s_im, -s_im).to(im.dtype)
    codes = pr.to(torch.uint8) | (pi.to(torch.uint8) << 1)
    return Stage(codes, s_re, s_im, v_re, v_im)


def residual_stages(re: torch.Tensor, im: torch.Tensor, steps: int, kind: str = "axis"):
    """Training-semantics residual quantization (quant_i.py:94-118):
    returns (stages, q_re, q_im) with q = sum of stage values."""
    q_re, q_im = torch.zeros_like(re), torch.zeros_like(im)
    r_re, r_im = re, im
    stages = []
    for _ in range(steps):
        st = axis_stage(r_re, r_im, TRAIN_MIN_SCALE) if kind == "axis" else sign_stage(r_re, r_im)
        q_re, q_im = q_re + st.value_re, q_im + st.value_im
        r_re, r_im = r_re - st.value_re, r_im - st.value_im
        stages.append(st)
    return stages, q_re, q_im


def export_stages(re: torch.Tensor, im: torch.Tensor, steps: int):
    """Export-semantics stages (export_rpfq_vit_to_mlx.py:189-289): per stage
    (codes, gamma_re, gamma_im) with fp16 gamma = 1/scale; each residual is
    taken against the codebook / gamma values."""
    r_re, r_im = re.clone(), im.clone()
    out = []
    for _ in range(steps):
        st = axis_stage(r_re, r_im, EXPORT_MIN_SCALE)
        g_re = torch.tensor(1.0 / float(st.scale_re), dtype=torch.float16)
        g_im = torch.tensor(1.0 / float(st.scale_im), dtype=torch.float16)
        d_re, d_im = decode_axis(st.codes, g_re.float(), g_im.float())
        r_re, r_im = r_re - d_re, r_im - d_im
        out.append((st.codes, g_re, g_im))
    return out


def decode_axis(codes: torch.Tensor, g_re: torch.Tensor, g_im: torch.Tensor):
    """codebook / gamma in float32 (export_rpfq_vit_to_mlx.py:236-253)."""
    one = torch.ones(codes.shape, dtype=torch.float32, device=codes.device)
    zero = torch.zeros_like(one)
    d_re = torch.where(codes == 0, -one, torch.where(codes == 1, one, zero)) / g_re
    d_im = torch.where(codes == 2, -one, torch.where(codes == 3, one, zero)) / g_im
    return d_re, d_im


def pack2(codes: torch.Tensor) -> torch.Tensor:
    """[rows, k] codes 0..3 -> [rows, k/4] uint8, first code in the low bits
    (export_rpfq_vit_to_mlx.py:148-159)."""
    rows, k = codes.shape
    if k % 4:
        raise ValueError("packed width must be divisible by 4")
    c = codes.to(torch.uint8).reshape(rows, k // 4, 4)
    return c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)


def pack4(codes: torch.Tensor) -> torch.Tensor:
    """[rows, k] codes 0..15 -> [rows, k/2] uint8, first code in the low nibble."""
    rows, k = codes.shape
    if k % 2:
        raise ValueError("4-bit packed width must be even")
    c = codes.to(torch.uint8).reshape(rows, k // 2, 2)
    return c[..., 0] | (c[..., 1] << 4)


def rotate_for_quant(re, im, cos_t, sin_t):
    """w * exp(-i theta) before quantization (quant_i.py:429-430)."""
    return re * cos_t + im * sin_t, im * cos_t - re * sin_t


def rotate_back(re, im, cos_t, sin_t):
    """q * exp(+i theta) after quantization (quant_i.py:433-434)."""
    return re * cos_t - im * sin_t, im * cos_t + re * sin_t


STAGES_OF = {
    "complex_phase_v1": ("axis", 1),
    "complex_phase_v2": ("axis", 2),
    "complex_phase_v3": ("axis", 3),
    "complex_phase_v4": ("axis", 4),
    "complex_phase_new_v2": ("sign", 2),
}


@dataclass
class LayerCodes:
    """Code planes and per-row scales of one layer, ready for PackedWide."""

    planes: list          # packed uint8 [N', K'/4] (or [N', K'/2] PSK16)
    scale_re: list        # float32 [N', nblk]
    scale_im: list
    n_complex: int
    k_complex: int
    codebook: int
    stages: int
    block: int = 0
    rotation: tuple | None = None


def quantize_layer(weight: torch.Tensor, method_u: str, method_w: str, rot_u=None, rot_w=None) -> LayerCodes:
    """Training-semantics codes of one QATLinearComplexPhase weight.

    rot_u / rot_w: float32 0-dim (cos, sin) tensors of the learned rotation or
    None.  The scales are the float32 per-tensor values, replicated per row."""
    if method_u not in STAGES_OF or method_w not in STAGES_OF:
        raise NotImplementedError(
            f"packed HIP path supports {sorted(STAGES_OF)}; got U={method_u}, W={method_w}")
    kind_u, steps_u = STAGES_OF[method_u]
    kind_w, steps_w = STAGES_OF[method_w]
    if kind_u != kind_w or steps_u != steps_w:
        raise NotImplementedError("packed HIP path needs the same method for U and W")
    w32 = weight.detach().float()
    u_re, u_im, w_re, w_im = split_blocks(w32)
    if (rot_u is None) != (rot_w is None):
        raise ValueError("rotation must be set for both U and W or neither")
    if rot_u is not None:
        u_re, u_im = rotate_for_quant(u_re, u_im, *rot_u)
        w_re, w_im = rotate_for_quant(w_re, w_im, *rot_w)
    n_c, k_c = u_re.shape
    planes, sre, sim = [], [], []
    for re, im in ((u_re, u_im), (w_re, w_im)):
        stages, _, _ = residual_stages(re, im, steps_u, kind_u)
        for st in stages:
            planes.append(pack2(st.codes))
            sre.append(st.scale_re.reshape(1, 1).expand(n_c, 1).contiguous())
            sim.append(st.scale_im.reshape(1, 1).expand(n_c, 1).contiguous())
    rotation = None
    if rot_u is not None:
        rotation = ((float(rot_u[0]), float(rot_u[1])), (float(rot_w[0]), float(rot_w[1])))
    cb = N.CB_AXIS if kind_u == "axis" else N.CB_SIGN
    return LayerCodes(planes, sre, sim, n_c, k_c, cb, steps_u, 0, rotation)


def quantize_layer_device(weight: torch.Tensor, method_u: str, method_w: str, rot_u=None, rot_w=None) -> LayerCodes:
    """quantize_layer on the GPU (rpfq_quantize_wide): the weight stays on
    its device and the planes and scales come back as device tensors.

    Codes follow from the scales bit-exactly; each scale is the float32
    rounding of the exact masked sum (float64 accumulation) where the host
    path reproduces torch's float32 CPU summation order, so the two agree to
    about 1 ulp per scale."""
    from . import ops

    if method_u not in STAGES_OF or method_w not in STAGES_OF:
        raise NotImplementedError(
            f"packed HIP path supports {sorted(STAGES_OF)}; got U={method_u}, W={method_w}")
    kind_u, steps_u = STAGES_OF[method_u]
    kind_w, steps_w = STAGES_OF[method_w]
    if kind_u != kind_w or steps_u != steps_w:
        raise NotImplementedError("packed HIP path needs the same method for U and W")
    if (rot_u is None) != (rot_w is None):
        raise ValueError("rotation must be set for both U and W or neither")
    dev = weight.device
    rot = None
    rotation = None
    if rot_u is not None:
        vals = [float(rot_u[0]), float(rot_u[1]), float(rot_w[0]), float(rot_w[1])]
        rot = torch.tensor(vals, dtype=torch.float32, device=dev)
        rotation = ((vals[0], vals[1]), (vals[2], vals[3]))
    _, scales, codes = ops.quantize_wide(weight.detach().float(), kind_u, steps_u, kind_w, steps_w, rot=rot,
                                         want_aq=False, want_codes=True)
    return quantizer_codes(scales, codes, weight.shape[0] // 2, weight.shape[1] // 2, kind_u, steps_u, rotation)


def quantizer_codes(scales: torch.Tensor, codes: torch.Tensor, n_c: int, k_c: int, kind: str, steps: int,
                    rotation=None) -> LayerCodes:
    """LayerCodes of rpfq_quantize_wide's outputs (scales [2, 4, 2] per
    U/W, stage, re/im; code planes [2 steps, N', K'/4]), device tensors
    kept on the device: per-tensor scales become per-row columns."""
    planes, sre, sim = [], [], []
    for p in range(2):
        for t in range(steps):
            planes.append(codes[p * steps + t])
            sre.append(scales[p, t, 0].reshape(1, 1).expand(n_c, 1).contiguous())
            sim.append(scales[p, t, 1].reshape(1, 1).expand(n_c, 1).contiguous())
    cb = N.CB_AXIS if kind == "axis" else N.CB_SIGN
    return LayerCodes(planes, sre, sim, n_c, k_c, cb, steps, 0, rotation)


def synthetic_layer(weight: torch.Tensor, generator: torch.Generator, lo: float = 0.01, hi: float = 0.1,
                    codebook: int = N.CB_AXIS) -> LayerCodes:
    """Benchmark weights: codes from the reference axis rule on a seeded
    float32 weight (two residual stages for U and W), per-(plane, row)
    magnitude scales ~U(lo, hi) shared by both axes; for PSK16 nearest of 16
    phases with per-(plane, row) magnitudes."""
    w32 = weight.detach().float().cpu()
    u_re, u_im, w_re, w_im = split_blocks(w32)
    n_c, k_c = u_re.shape
    planes, sre, sim = [], [], []
    if codebook == N.CB_PSK16:
        for re, im in ((u_re, u_im), (w_re, w_im)):
            ang = torch.atan2(im, re)
            codes = torch.remainder(torch.round(ang / (2 * math.pi / 16)), 16).to(torch.uint8)
            planes.append(pack4(codes))
            s = lo + (hi - lo) * torch.rand(n_c, 1, generator=generator)
            sre.append(s)
            sim.append(s)
        return LayerCodes(planes, sre, sim, n_c, k_c, N.CB_PSK16, 1)
    for re, im in ((u_re, u_im), (w_re, w_im)):
        stages, _, _ = residual_stages(re, im, 2, "axis")
        for st in stages:
            planes.append(pack2(st.codes))
            s = lo + (hi - lo) * torch.rand(n_c, 1, generator=generator)
            sre.append(s)
            sim.append(s.clone())
    return LayerCodes(planes, sre, sim, n_c, k_c, N.CB_AXIS, 2)
