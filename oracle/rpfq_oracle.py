"""CPU oracle for the packed complex-phase linear path (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  The HIP path under ``rpfq-review_amd/`` must not import or call it.

It restates, in numpy, the arithmetic of the reference's phase-quantized
Linear layer and of its packed deployment format.  Every function cites the
reference file:line it follows (paths relative to the reference checkout).

Parity status per function (how each one is pinned; see tests/test_oracle.py):

* ``axis_masks``            -- closed-form truth table (every tie case), and
                               golden vectors written by the reference itself.
* ``safe_mean_abs``         -- closed form; golden scales (to 1 ulp: numpy and
                               torch sum float32 in different orders).
* ``quantize_phase_axis`` / ``residual_quantize`` -- golden vectors
                               (stage-1 codes bit-exact; stage-2 codes and
                               scales to the ulp tolerance above).
* ``pack_codes`` / ``unpack_codes`` -- brute force over all 256 byte values;
                               golden packed planes.
* ``dequantize_axis``       -- golden dequantized planes (bit-exact).
* ``decompose`` / ``recompose`` -- algebraic round trip in float64; golden.
* ``act_quant``             -- closed form with half-to-even ties; golden.
* ``phase_linear``          -- compiled reference (oracle/_ref) and brute force.
* ``wide_linear``           -- compiled reference (oracle/_ref); equals
                               ``x @ A_q.T + b`` in float64 (golden A_q).
* ``wide_linear_grad_x``    -- the adjoint identity <gy, wide_linear(x)> =
                               <wide_linear_grad_x(gy), x> against the pinned
                               forward, and torch autograd of F.linear on the
                               same A_q (an independent library routine).
* ``fp16_add`` / ``recompose_fp16`` -- build-defined fp16 operand (no
                               reference counterpart): fp16_add pinned by exact
                               rational arithmetic (fractions) on every fp16
                               pair class incl. ties and subnormals;
                               recompose_fp16 by its error bound against the
                               reference A_q and by sign/permutation identities.
* ``recompose_split_fp16``  -- build-defined operand of the column-split
                               kernel: its fp16 rounding equals recompose_fp16
                               bit for bit; error bound against A_q; W = 0
                               case exact.
* ``linear_forward``        -- golden outputs of the reference layer.
* ``wide_parts(..., "table")`` -- the per-row value tables of the packed
                               next_v1 form: the golden next_v1 A_q of the
                               reference layer, bit-exact.
* ``quantize_sign_phase``, ``rotate_for_quant``, ``quantized_weight`` --
                               golden A_q of the reference layer for every
                               axis / sign method with rotation on and off
                               (to the scale-sum ulp tolerance above), and
                               closed-form sign cases.
* ``psk16_*``               -- PARITY UNPINNED by the reference (the 16-PSK
                               codebook does not exist there); pinned only by
                               its closed form (unit modulus, 16 distinct
                               phases in order) and float64 brute force.
"""
from __future__ import annotations

import math

import numpy as np

F32 = np.float32

# Codebook of the packed axis format: 00=-1, 01=+1, 10=-i, 11=+i
# (RPFQ-ViTApple/scripts/export_rpfq_vit_to_mlx.py:598-603,
#  RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:148-153).
AXIS_CODEBOOK = np.array([[-1.0, 0.0], [1.0, 0.0], [0.0, -1.0], [0.0, 1.0]], dtype=F32)

BLOCK_SIZE = 256  # export_rpfq_vit_to_mlx.py:28


# --------------------------------------------------------------------------
# widely-linear decomposition (quant_i.py:519-527, :534-544;
# export_rpfq_vit_to_mlx.py:317-333, :363-375)
# --------------------------------------------------------------------------
def decompose(weight: np.ndarray):
    """Split a real [out, in] weight into U and W complex planes.

    U = 0.5(A11+A22) + i 0.5(A21-A12),  W = 0.5(A11-A22) + i 0.5(A12+A21)
    (RPFQ-ViT-main/quant_models/quant_i.py:519-527).
    """
    weight = np.asarray(weight, dtype=F32)
    out_f, in_f = weight.shape
    if out_f % 2 or in_f % 2:
        raise ValueError("complex decomposition requires even dims")
    ho, hi = out_f // 2, in_f // 2
    a11, a12 = weight[:ho, :hi], weight[:ho, hi:]
    a21, a22 = weight[ho:, :hi], weight[ho:, hi:]
    half = F32(0.5)
    u_re = half * (a11 + a22)
    u_im = half * (a21 - a12)
    w_re = half * (a11 - a22)
    w_im = half * (a12 + a21)
    return u_re, u_im, w_re, w_im


def recompose(u_re, u_im, w_re, w_im):
    """Fused real weight from quantized U/W (quant_i.py:534-544)."""
    a11 = w_re + u_re
    a12 = w_im - u_im
    a21 = w_im + u_im
    a22 = -w_re + u_re
    return np.concatenate(
        [np.concatenate([a11, a12], axis=1), np.concatenate([a21, a22], axis=1)], axis=0
    ).astype(F32)


# --------------------------------------------------------------------------
# axis phase quantizer (quant_i.py:29-81; export_rpfq_vit_to_mlx.py:121-145,
# :189-224)
# --------------------------------------------------------------------------
def axis_masks(w_re: np.ndarray, w_im: np.ndarray):
    """Dominant-axis masks with quadrant tie rules (quant_i.py:36-62)."""
    ar, ai = np.abs(w_re), np.abs(w_im)
    real_dom = ar > ai
    imag_dom = ai > ar
    tie = ~(real_dom | imag_dom)
    zero_tie = tie & (w_re == 0) & (w_im == 0)
    tie_q1 = tie & (w_re > 0) & (w_im > 0)
    tie_q2 = tie & (w_re < 0) & (w_im > 0)
    tie_q3 = tie & (w_re < 0) & (w_im < 0)
    tie_q4 = tie & (w_re > 0) & (w_im < 0)
    real_pos = (real_dom & (w_re >= 0)) | tie_q4 | zero_tie
    real_neg = (real_dom & (w_re < 0)) | tie_q2
    imag_pos = (imag_dom & (w_im >= 0)) | tie_q1
    imag_neg = (imag_dom & (w_im < 0)) | tie_q3
    return real_pos, real_neg, imag_pos, imag_neg


def safe_mean_abs(x: np.ndarray, mask: np.ndarray, min_val: float) -> np.float32:
    """Masked mean |x|, clamped (quant_i.py:29-33 with 1e-5; export :121-124
    with 1e-6).  The sum is accumulated in float64 and rounded to float32; the
    reference sums float32 in torch's order, so results agree to ~1 ulp."""
    m = mask.astype(np.float64)
    num = F32(np.sum(np.abs(x.astype(np.float64)) * m))
    den = F32(max(np.sum(m), 1.0))
    mean = F32(num / den)
    return F32(max(mean, F32(min_val)))


def axis_codes(w_re: np.ndarray, w_im: np.ndarray) -> np.ndarray:
    """2-bit code per element: real_pos=1, imag_neg=2, imag_pos=3, else 0
    (export_rpfq_vit_to_mlx.py:214-218)."""
    real_pos, _real_neg, imag_pos, imag_neg = axis_masks(w_re, w_im)
    codes = np.zeros(w_re.shape, dtype=np.uint8)
    codes[real_pos] = 1
    codes[imag_neg] = 2
    codes[imag_pos] = 3
    return codes


def quantize_phase_axis(w_re, w_im, min_val: float = 1e-5):
    """One axis stage -> (codes, s_real, s_imag, q_re, q_im)
    (quant_i.py:65-81; export_rpfq_vit_to_mlx.py:207-218)."""
    w_re = np.asarray(w_re, dtype=F32)
    w_im = np.asarray(w_im, dtype=F32)
    real_pos, real_neg, imag_pos, imag_neg = axis_masks(w_re, w_im)
    s_re = safe_mean_abs(w_re, real_pos | real_neg, min_val)
    s_im = safe_mean_abs(w_im, imag_pos | imag_neg, min_val)
    q_re = np.zeros_like(w_re)
    q_im = np.zeros_like(w_im)
    q_re[real_pos] = s_re
    q_re[real_neg] = -s_re
    q_im[imag_pos] = s_im
    q_im[imag_neg] = -s_im
    codes = axis_codes(w_re, w_im)
    return codes, s_re, s_im, q_re, q_im


def quantize_sign_phase(w_re, w_im):
    """Quadrant-sign stage (quant_i.py:84-91) -> (codes, s_re, s_im, q_re,
    q_im): scale = mean |.| over the whole plane (float64 sum rounded to
    float32, then torch's CPU mean: float32 sum / numel), clamped at 1e-6;
    code bit0 = re >= 0, bit1 = im >= 0."""
    w_re = np.asarray(w_re, dtype=F32)
    w_im = np.asarray(w_im, dtype=F32)
    n = F32(w_re.size)
    s_re = max(F32(F32(np.sum(np.abs(w_re.astype(np.float64)))) / n), F32(1e-6))
    s_im = max(F32(F32(np.sum(np.abs(w_im.astype(np.float64)))) / n), F32(1e-6))
    pr, pi = w_re >= 0, w_im >= 0
    q_re = np.where(pr, s_re, -s_re).astype(F32)
    q_im = np.where(pi, s_im, -s_im).astype(F32)
    codes = pr.astype(np.uint8) | (pi.astype(np.uint8) << 1)
    return codes, F32(s_re), F32(s_im), q_re, q_im


def residual_quantize(w_re, w_im, steps: int, kind: str = "axis"):
    """Training-semantics residual stages (quant_i.py:94-118) of the axis
    (:65-81) or quadrant-sign (:84-91) quantizer: returns the summed
    quantized planes and the per-stage (codes, s_re, s_im)."""
    q_re = np.zeros_like(w_re, dtype=F32)
    q_im = np.zeros_like(w_im, dtype=F32)
    r_re = np.asarray(w_re, dtype=F32)
    r_im = np.asarray(w_im, dtype=F32)
    stages = []
    for _ in range(steps):
        if kind == "sign":
            codes, s_re, s_im, st_re, st_im = quantize_sign_phase(r_re, r_im)
        else:
            codes, s_re, s_im, st_re, st_im = quantize_phase_axis(r_re, r_im, 1e-5)
        q_re = q_re + st_re
        q_im = q_im + st_im
        r_re = r_re - st_re
        r_im = r_im - st_im
        stages.append((codes, s_re, s_im))
    return q_re, q_im, stages


def residual_quantize_export(w_re, w_im, steps: int):
    """Export-semantics stages: gamma = fp16(1/s) and each residual is taken
    against the fp16-gamma-dequantized stage (export_rpfq_vit_to_mlx.py:257-289,
    :221-223, :252-253).  Returns per-stage (codes, gamma_re_f16, gamma_im_f16)."""
    r_re = np.asarray(w_re, dtype=F32).copy()
    r_im = np.asarray(w_im, dtype=F32).copy()
    out = []
    for _ in range(steps):
        codes, s_re, s_im, _, _ = quantize_phase_axis(r_re, r_im, 1e-6)
        g_re = np.float16(1.0 / float(s_re))
        g_im = np.float16(1.0 / float(s_im))
        d_re, d_im = dequant_codes(codes, np.full(codes.shape[0], g_re), np.full(codes.shape[0], g_im))
        r_re = r_re - d_re
        r_im = r_im - d_im
        out.append((codes, g_re, g_im))
    return out


# --------------------------------------------------------------------------
# 2-bit packing (export_rpfq_vit_to_mlx.py:148-159, :234-240;
# phase_linear.cpp:15-19)
# --------------------------------------------------------------------------
def pack_codes(codes: np.ndarray) -> np.ndarray:
    """[rows, k] codes 0..3 -> [rows, k/4] uint8, low bits first."""
    codes = np.asarray(codes, dtype=np.uint8)
    rows, k = codes.shape
    if k % 4:
        raise ValueError("packed width must be divisible by 4")
    c = codes.reshape(rows, k // 4, 4)
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)


def unpack_codes(packed: np.ndarray, k: int | None = None) -> np.ndarray:
    """[rows, k/4] uint8 -> [rows, k] codes; code_k = (byte[k>>2] >> 2(k&3)) & 3."""
    packed = np.asarray(packed, dtype=np.uint8)
    rows, kb = packed.shape
    out = np.stack([(packed >> (2 * j)) & 3 for j in range(4)], axis=-1).reshape(rows, kb * 4)
    return out if k is None else out[:, :k]


def pack_codes4(codes: np.ndarray) -> np.ndarray:
    """4-bit codes (16-PSK), two per byte, low nibble first (build-defined)."""
    codes = np.asarray(codes, dtype=np.uint8)
    rows, k = codes.shape
    if k % 2:
        raise ValueError("4-bit packed width must be even")
    c = codes.reshape(rows, k // 2, 2)
    return (c[..., 0] | (c[..., 1] << 4)).astype(np.uint8)


def unpack_codes4(packed: np.ndarray) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    rows, kb = packed.shape
    return np.stack([packed & 15, packed >> 4], axis=-1).reshape(rows, kb * 2)


def dequant_codes(codes: np.ndarray, inv_or_gamma_re, inv_or_gamma_im, gamma: bool = True):
    """Decode unpacked 2-bit codes with per-row gamma (divide) or per-row
    inverse gamma (multiply).  Both give identical float32 values since
    +-1/g == +-(1/g) exactly (export :252-253 vs phase_linear.cpp:72-83)."""
    g_re = np.asarray(inv_or_gamma_re, dtype=F32)
    g_im = np.asarray(inv_or_gamma_im, dtype=F32)
    if g_re.shape != codes.shape:
        g_re = g_re.reshape(-1, 1)
    if g_im.shape != codes.shape:
        g_im = g_im.reshape(-1, 1)
    cb = AXIS_CODEBOOK[codes]
    if gamma:
        return (cb[..., 0] / g_re).astype(F32), (cb[..., 1] / g_im).astype(F32)
    return (cb[..., 0] * g_re).astype(F32), (cb[..., 1] * g_im).astype(F32)


def dequantize_axis(packed, gamma_re, gamma_im, rows: int, k: int, block: int = BLOCK_SIZE):
    """export_rpfq_vit_to_mlx.py:227-254: packed [rows, k/4] u8 and fp16 gammas
    [rows, ceil(k/block)] -> float32 (w_re, w_im) = codebook / gamma."""
    codes = unpack_codes(np.asarray(packed).reshape(rows, k // 4))
    g_re = np.repeat(np.asarray(gamma_re, dtype=np.float16).astype(F32), block, axis=1)[:, :k]
    g_im = np.repeat(np.asarray(gamma_im, dtype=np.float16).astype(F32), block, axis=1)[:, :k]
    cb = AXIS_CODEBOOK[codes]
    return (cb[..., 0] / g_re).astype(F32), (cb[..., 1] / g_im).astype(F32)


def inv_gamma(gamma_f16) -> np.ndarray:
    """1.0f / gamma in float32 (phase_linear.cpp:72-83)."""
    g = np.asarray(gamma_f16, dtype=np.float16).astype(F32)
    if np.any(g == 0):
        raise ValueError("zero gamma")
    return (F32(1.0) / g).astype(F32)


# --------------------------------------------------------------------------
# 16-PSK codebook (build-defined; no counterpart in the reference)
# --------------------------------------------------------------------------
def psk16_codebook() -> np.ndarray:
    """code c -> (cos 2 pi c/16, sin 2 pi c/16) in float32, built by exact
    octant symmetry from float32(cos pi/8), float32(sin pi/8) and
    float32(sqrt(2)/2) so the axes are exactly 0 and +-1.  Build-defined:
    PARITY UNPINNED by the reference (no 16-PSK codebook there)."""
    c1 = F32(math.cos(math.pi / 8))
    s1 = F32(math.sin(math.pi / 8))
    r2 = F32(math.sqrt(0.5))
    z, o = F32(0.0), F32(1.0)
    first = [(o, z), (c1, s1), (r2, r2), (s1, c1)]
    out = []
    for quarter in range(4):
        for (a, b) in first:
            for _ in range(quarter):  # multiply by i: (a, b) -> (-b, a)
                a, b = -b, a
            out.append((a, b))
    return np.array(out, dtype=F32) + F32(0.0)  # -0 -> +0


# --------------------------------------------------------------------------
# activation fake-quant (quant_i.py:438-455)
# --------------------------------------------------------------------------
def act_quant(x_re: np.ndarray, x_im: np.ndarray, num_bits: int):
    """Per-row symmetric fake quant of each half; np.rint is half-to-even like
    torch.round.  float32 throughout, same op order as the reference."""
    qmax = (1 << (num_bits - 1)) - 1
    qmin = -(1 << (num_bits - 1))
    out = []
    for x in (x_re, x_im):
        x = np.asarray(x, dtype=F32)
        amax = np.maximum(np.abs(x).max(axis=-1, keepdims=True), F32(1e-5)).astype(F32)
        # torch computes `float / tensor` as reciprocal(tensor) * float
        scale = ((F32(1.0) / amax).astype(F32) * F32(qmax)).astype(F32)
        q = np.clip(np.rint((x * scale).astype(F32)), qmin, qmax).astype(F32)
        out.append((q / scale).astype(F32))
    return out[0], out[1]


# --------------------------------------------------------------------------
# contractions (float64 accumulation = the exact value the GPU approximates)
# --------------------------------------------------------------------------
def phase_linear(xr, xi, codes, inv_re, inv_im, conj_input: bool = True):
    """Single packed plane, phaseLinearReference semantics
    (RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:119-164):
        Re = sum wRe*xr + wIm*xi ;  Im = sum wIm*xr - wRe*xi   (= W conj(x)).
    ``conj_input=False`` feeds (xr, -xi) as the U planes do (:189-192), giving
    the ordinary complex product W x.  codes: [N, K] unpacked; inv_re/inv_im:
    per-element or per-row float32 inverse gammas."""
    codes = np.asarray(codes)
    cb = AXIS_CODEBOOK[codes].astype(np.float64)
    inv_re = np.asarray(inv_re, dtype=np.float64)
    inv_im = np.asarray(inv_im, dtype=np.float64)
    if inv_re.ndim == 1:
        inv_re, inv_im = inv_re[:, None], inv_im[:, None]
    w_re = cb[..., 0] * inv_re
    w_im = cb[..., 1] * inv_im
    xr = np.asarray(xr, np.float64)
    xi = np.asarray(xi, np.float64)
    if not conj_input:
        xi = -xi
    y_re = xr @ w_re.T + xi @ w_im.T
    y_im = xr @ w_im.T - xi @ w_re.T
    return y_re, y_im


def sign_codes_values(codes, s_re, s_im):
    """Quadrant-sign code (bit0 = re >= 0, bit1 = im >= 0) -> float32 values
    (quant_i.py:84-91); s_re/s_im per row."""
    codes = np.asarray(codes)
    sr = np.asarray(s_re, F32)
    si = np.asarray(s_im, F32)
    sr = sr if sr.shape == codes.shape else sr.reshape(-1, 1)
    si = si if si.shape == codes.shape else si.reshape(-1, 1)
    v_re = np.where(codes & 1, sr, -sr).astype(F32)
    v_im = np.where(codes & 2, si, -si).astype(F32)
    return v_re, v_im


def derotate(re, im, c, s):
    """q * exp(+i theta) with float32 products rounded separately
    (quant_i.py:433-434)."""
    c, s = F32(c), F32(s)
    return (re * c - im * s).astype(F32), (im * c + re * s).astype(F32)


def wide_parts(planes, codebook: str = "axis", rotation=None):
    """Quantized U and W of the widely-linear layer as float32 (re, im) planes.

    planes: list of (codes [N,K] unpacked, s_re [N], s_im [N], kind) with kind
    'u' or 'w', stage order preserved; the per-stage float32 values are summed
    as the reference does (quant_i.py:111-118: q = 0 + step0 + step1), then
    optionally de-rotated (quant_i.py:433-434).  codebook 'axis' | 'sign' |
    'psk16' (for 'psk16' s_re is the magnitude and s_im is ignored) |
    'table' (codes index per-row [N, 16] value tables s_re / s_im: the
    packed form of complex_phase_next_v1's grouped quantizer,
    quant_i.py:193-351; one plane each for U and W)."""
    acc = {}
    for codes, s_re, s_im, kind in planes:
        if codebook == "psk16":
            cb = psk16_codebook()[np.asarray(codes)]
            mag = np.asarray(s_re, F32)
            mag = mag if mag.shape == np.shape(codes) else mag.reshape(-1, 1)
            v_re = (cb[..., 0] * mag).astype(F32)
            v_im = (cb[..., 1] * mag).astype(F32)
        elif codebook == "sign":
            v_re, v_im = sign_codes_values(codes, s_re, s_im)
        elif codebook == "table":  # s_re / s_im: per-row [N, 16] value tables, codes = indices
            v_re = np.take_along_axis(np.asarray(s_re, F32), np.asarray(codes, np.int64), axis=1)
            v_im = np.take_along_axis(np.asarray(s_im, F32), np.asarray(codes, np.int64), axis=1)
        else:
            v_re, v_im = dequant_codes(codes, s_re, s_im, gamma=False)
        q_re, q_im = acc.get(kind, (np.zeros_like(v_re), np.zeros_like(v_im)))
        acc[kind] = ((q_re + v_re).astype(F32), (q_im + v_im).astype(F32))
    u_re, u_im = acc["u"]
    w_re, w_im = acc["w"]
    if rotation is not None:
        (cu, su), (cw, sw) = rotation
        u_re, u_im = derotate(u_re, u_im, cu, su)
        w_re, w_im = derotate(w_re, w_im, cw, sw)
    return u_re, u_im, w_re, w_im


def fp16_add(a, b):
    """Correctly rounded fp16 sum of two fp16 arrays.  The exact sum of two
    fp16 numbers spans at most 40 bits, so it is exact in float64 and the one
    float64 -> fp16 conversion (round to nearest even) is the only rounding."""
    a = np.asarray(a, np.float16).astype(np.float64)
    b = np.asarray(b, np.float16).astype(np.float64)
    with np.errstate(over="ignore"):  # sums beyond 65504 round to +-inf, as in IEEE fp16
        return (a + b).astype(np.float16)


def recompose_fp16(u_re, u_im, w_re, w_im):
    """Fused weight as the MFMA operand of the HIP kernels: U and W rounded to
    fp16, then each coefficient one correctly rounded fp16 add in the
    reference's recombination order (quant_i.py:534-537).  Build-defined (the
    reference has no fp16 operand); returned as float32 holding fp16 values."""
    ur, ui, wr, wi = (np.asarray(v, F32).astype(np.float16) for v in (u_re, u_im, w_re, w_im))
    a11 = fp16_add(wr, ur)
    a12 = fp16_add(wi, -ui)
    a21 = fp16_add(wi, ui)
    a22 = fp16_add(-wr, ur)
    return np.concatenate(
        [np.concatenate([a11, a12], axis=1), np.concatenate([a21, a22], axis=1)], axis=0
    ).astype(F32)


def recompose_split_fp16(u_re, u_im, w_re, w_im):
    """Fused weight as the column-split streaming kernel (RPFQ_KERNEL_GEMV)
    contracts it: U and W rounded to fp16 and each coefficient their exact
    sum in the reference's recombination order (quant_i.py:534-537), float64
    (the kernel multiplies the fp16 parts separately and sums in float32
    accumulators).  Build-defined; its round-to-fp16 is recompose_fp16 bit
    for bit (both are the correctly rounded fp16 sum of the same operands)."""
    ur, ui, wr, wi = (np.asarray(v, F32).astype(np.float16).astype(np.float64) for v in (u_re, u_im, w_re, w_im))
    return np.concatenate(
        [np.concatenate([wr + ur, wi - ui], axis=1), np.concatenate([wi + ui, -wr + ur], axis=1)], axis=0)


def wide_weight(planes, codebook: str = "axis", rotation=None, fp16=False):
    """Fused real [2N, 2K] weight of the widely-linear layer: the reference's
    float32 A_q (quant_i.py:534-544), or with fp16=True the fp16 operand the
    MFMA sees (recompose_fp16), or with fp16="split" the exact sums of the
    fp16 parts the column-split kernel contracts (recompose_split_fp16)."""
    parts = wide_parts(planes, codebook, rotation)
    if fp16 == "split":
        return recompose_split_fp16(*parts)
    return recompose_fp16(*parts) if fp16 else recompose(*parts)


def wide_magnitude(planes, codebook: str = "axis", rotation=None):
    """|W part| + |U part| of every fused coefficient, [2N, 2K] float64: the
    scale of the fp16 fusing error, |recompose_fp16 - recompose| <=
    (2u + u^2) * magnitude with u = 2^-11 (normal fp16 range)."""
    u_re, u_im, w_re, w_im = (np.abs(np.asarray(v, np.float64)) for v in wide_parts(planes, codebook, rotation))
    m_re, m_im = w_re + u_re, w_im + u_im
    return np.concatenate(
        [np.concatenate([m_re, m_im], axis=1), np.concatenate([m_im, m_re], axis=1)], axis=0)


def wide_linear(x, planes, bias=None, codebook: str = "axis", rotation=None, fp16_weight: bool = False):
    """Widely-linear layer y = U x + W conj(x) on [re | im] features
    (phase_linear.cpp:166-207), evaluated as x @ A_q.T + b in float64.
    fp16_weight=True uses the fp16 operand the MFMA sees (recompose_fp16)."""
    a = wide_weight(planes, codebook, rotation, fp16=fp16_weight).astype(np.float64)
    y = np.asarray(x, np.float64) @ a.T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y


def wide_linear_grad_x(gy, planes, codebook: str = "axis", rotation=None, fp16_weight: bool = False):
    """Input gradient of wide_linear: gx = gy @ A_q in float64, the
    reference operator's backward grad_x = einsum('blo, oi -> bli',
    grad_output, w_quant) (kernel.py:585) with w_quant the fused A_q
    (quant_i.py:534-544); fp16_weight=True uses the MFMA operand."""
    a = wide_weight(planes, codebook, rotation, fp16=fp16_weight).astype(np.float64)
    return np.asarray(gy, np.float64) @ a


def rotate_for_quant(re, im, c, s):
    """w * exp(-i theta) with float32 products rounded separately
    (quant_i.py:429-430)."""
    c, s = F32(c), F32(s)
    return (re * c + im * s).astype(F32), (im * c - re * s).astype(F32)


def quantized_weight(weight, kind_u: str, steps_u: int, kind_w: str, steps_w: int, rotation=None):
    """A_q of QATLinearComplexPhase.forward (quant_i.py:513-544) for the
    axis / quadrant-sign residual methods, with the optional global rotation
    of ComplexWeightQuantizer.forward (:418-435).  rotation: None or
    ((cos_u, sin_u), (cos_w, sin_w)) float32.  Returns (a_q, stages_u,
    stages_w), stages as residual_quantize returns them."""
    u_re, u_im, w_re, w_im = decompose(weight)
    planes = []
    for i, (re, im, kind, steps) in enumerate(((u_re, u_im, kind_u, steps_u), (w_re, w_im, kind_w, steps_w))):
        if rotation is not None:
            re, im = rotate_for_quant(re, im, *rotation[i])
        q_re, q_im, st = residual_quantize(re, im, steps, kind)
        if rotation is not None:
            q_re, q_im = derotate(q_re, q_im, *rotation[i])
        planes.append((q_re, q_im, st))
    a_q = recompose(planes[0][0], planes[0][1], planes[1][0], planes[1][1])
    return a_q, planes[0][2], planes[1][2]


def linear_forward(x, weight, bias, steps_u: int, steps_w: int, act_bits: int | None):
    """QATLinearComplexPhase.forward (quant_i.py:513-554) for the axis
    residual methods, float64 contraction over the float32 A_q."""
    u_re, u_im, w_re, w_im = decompose(weight)
    uq_re, uq_im, _ = residual_quantize(u_re, u_im, steps_u)
    wq_re, wq_im, _ = residual_quantize(w_re, w_im, steps_w)
    a_q = recompose(uq_re, uq_im, wq_re, wq_im)
    x = np.asarray(x, F32)
    if act_bits is not None:
        half = x.shape[-1] // 2
        qr, qi = act_quant(x[..., :half], x[..., half:], act_bits)
        x = np.concatenate([qr, qi], axis=-1)
    y = x.astype(np.float64) @ a_q.astype(np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    return y, a_q
