"""Tensor-level entry points over the C ABI (include/rpfq.h).

Every function here runs the HIP kernels of librpfq.so on device tensors and
raises if the library is unavailable or a tensor is on the host.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field

import torch

from . import _native as N


def _aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """t itself when it is contiguous with a 16-byte aligned start (what the
    C ABI requires of row-major operands), else a fresh contiguous copy: a
    contiguous view at an odd offset is copied too, since contiguous() would
    return it unchanged."""
    if t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    return t.clone(memory_format=torch.contiguous_format)


# The forward's range guard: float32 / bf16 activations get per-row
# power-of-two prescales (rpfq_row_scales) so the kernels' fp16 operands keep
# the input's range (rpfq_wide_linear_scaled).  RPFQ_RANGE_GUARD=0 skips it
# (for measurement; rows outside fp16's range then overflow or underflow).
RANGE_GUARD = __import__("os").environ.get("RPFQ_RANGE_GUARD", "1") != "0"


def row_scales(x2: torch.Tensor) -> torch.Tensor:
    """Per-row power-of-two prescales of a [M, C] device tensor
    (rpfq_row_scales): 2^(14 - floor(log2 max|row|)), 1 for zero rows."""
    N.require_device(x2)
    m, c = x2.shape
    s = torch.empty(m, dtype=torch.float32, device=x2.device)
    if m:
        N.check("rpfq_row_scales", N.load().rpfq_row_scales(x2.data_ptr(), N.dtype_code(x2.dtype), m, c,
                                                          s.data_ptr(), N.stream_of(x2)))
    return s


# bf16 / float32 rows into a launch the DMA kernel takes for fp16 rows go
# there as prescaled fp16 rows (prescale_rows: for bf16 one pass instead of
# the row-scale pass plus the kernel's in-LDS conversion, same outputs bit
# for bit; float32 rows leave the register-staged kernel with the same
# operands); RPFQ_PRESCALE_ROWS=0 keeps the rows as they are.
PRESCALE_ROWS = __import__("os").environ.get("RPFQ_PRESCALE_ROWS", "1") != "0"


def prescale_rows(x2: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(y, row_scale) for a [M, C] bf16 / float32 device tensor
    (rpfq_row_prescale): row_scale = row_scales(x2) and y = x2 * row_scale
    rounded to fp16, the kernels' operand bits for those rows."""
    N.require_device(x2)
    if x2.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("prescale_rows takes bf16 or float32 rows")
    m, c = x2.shape
    y = torch.empty(m, c, dtype=torch.float16, device=x2.device)
    s = torch.empty(m, dtype=torch.float32, device=x2.device)
    if m:
        N.check("rpfq_row_prescale", N.load().rpfq_row_prescale(x2.data_ptr(), N.dtype_code(x2.dtype), m, c,
                                                              y.data_ptr(), s.data_ptr(), N.stream_of(x2)))
    return y, s


# Optional per-launch timing hook: when set, PackedWide.linear records HIP
# events around each wide-linear launch on the launch stream and hands
# (start_event, end_event, flops, algorithmic_bytes, shape) to the recorder.
_launch_recorder = None


def set_launch_recorder(recorder) -> None:
    global _launch_recorder
    _launch_recorder = recorder


def unpack(codes: torch.Tensor, bits: int, k: int, gamma_re: torch.Tensor | None = None,
           gamma_im: torch.Tensor | None = None, block: int = 0):
    """Decode a packed plane [rows, k*bits/8] -> float32 (re, im) [rows, k].

    With fp16 gammas the values are codebook / gamma, as
    export_rpfq_vit_to_mlx.py:227-254 computes them (bit-exact)."""
    N.require_device(codes, gamma_re, gamma_im)
    if codes.dtype != torch.uint8 or not codes.is_contiguous():
        raise TypeError("codes must be a contiguous uint8 tensor")
    for g in (gamma_re, gamma_im):
        if g is not None and (g.dtype != torch.float16 or not g.is_contiguous()):
            raise TypeError("gammas must be contiguous float16 tensors")
    rows = codes.shape[0]
    re = torch.empty(rows, k, dtype=torch.float32, device=codes.device)
    im = torch.empty_like(re)
    lib = N.load()
    N.check("rpfq_unpack", lib.rpfq_unpack(N.ptr(codes), bits, rows, k, N.ptr(gamma_re), N.ptr(gamma_im),
                                          block, N.ptr(re), N.ptr(im), N.stream_of(codes)))
    return re, im


def phase_linear(xr: torch.Tensor, xi: torch.Tensor, codes: torch.Tensor, gamma_re: torch.Tensor,
                 gamma_im: torch.Tensor, block: int = 0, conj_x: bool = True,
                 out_dtype: torch.dtype = torch.float32):
    """One packed plane, phaseLinearReference semantics
    (RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:119-164).
    conj_x=True computes W conj(x); False computes W x."""
    N.require_device(xr, xi, codes, gamma_re, gamma_im)
    if xr.shape != xi.shape or xr.dim() != 2:
        raise ValueError("xr and xi must be equal 2-D planes")
    if xr.dtype != xi.dtype:
        raise TypeError("xr and xi must share a dtype")
    xr, xi = xr.contiguous(), xi.contiguous()
    m, k = xr.shape
    n = codes.shape[0]
    yr = torch.empty(m, n, dtype=out_dtype, device=xr.device)
    yi = torch.empty_like(yr)
    lib = N.load()
    N.check("rpfq_phase_linear", lib.rpfq_phase_linear(
        N.ptr(xr), N.ptr(xi), N.dtype_code(xr.dtype), int(bool(conj_x)), m, k, N.ptr(codes.contiguous()),
        N.ptr(gamma_re.contiguous()), N.ptr(gamma_im.contiguous()), block, n, N.ptr(yr), N.ptr(yi),
        N.dtype_code(out_dtype), N.stream_of(xr)))
    return yr, yi


def act_quant(x: torch.Tensor, num_bits: int, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Per-row, per-half symmetric fake quantization of [..., 2K'] features
    (quant_i.py:438-455 applied at :546-551) on the device."""
    N.require_device(x)
    lead, f = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, f).contiguous()
    y = torch.empty(x2.shape, dtype=out_dtype or x.dtype, device=x.device)
    if x2.shape[0] == 0:
        return y.reshape(*lead, f)
    lib = N.load()
    N.check("rpfq_act_quant", lib.rpfq_act_quant(
        x2.data_ptr(), N.dtype_code(x2.dtype), x2.shape[0], f, int(num_bits), y.data_ptr(),
        N.dtype_code(y.dtype), N.stream_of(x2)))
    return y.reshape(*lead, f)


def gelu_act_quant(x: torch.Tensor, num_bits: int, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """act_quant(F.gelu(x)) with the exact GELU in float32 and no rounding to
    x's dtype in between (rpfq_gelu_act_quant: bit-identical to
    act_quant(F.gelu(x.float()), num_bits, out_dtype)); [..., C] rows, C %
    16 == 0, C <= 4096."""
    N.require_device(x)
    c = x.shape[-1]
    x2 = _aligned_rows(x.reshape(-1, c))
    y = torch.empty(x2.shape, dtype=out_dtype or x.dtype, device=x.device)
    if x2.shape[0] == 0:
        return y.reshape(x.shape)
    N.check("rpfq_gelu_act_quant", N.load().rpfq_gelu_act_quant(
        x2.data_ptr(), N.dtype_code(x2.dtype), x2.shape[0], c, int(num_bits), y.data_ptr(), N.dtype_code(y.dtype),
        N.stream_of(x2)))
    return y.reshape(x.shape)


def layer_norm(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None, eps: float,
               out_dtype: torch.dtype | None = None, act_bits: int = 0) -> torch.Tensor:
    """nn.LayerNorm over the last dimension on the device (rpfq_layer_norm):
    float32 statistics, output in out_dtype (default x.dtype).  weight/bias
    are taken as float32.  act_bits > 0: the float32 LayerNorm output is
    fake-quantized per row and half before the rounding to out_dtype
    (rpfq_layer_norm_act_quant, bit-identical to
    act_quant(layer_norm(x, out_dtype=float32), out_dtype=out_dtype))."""
    N.require_device(x, weight, bias)
    c = x.shape[-1]
    x2 = _aligned_rows(x.reshape(-1, c))
    y = torch.empty(x2.shape, dtype=out_dtype or x.dtype, device=x.device)
    if x2.shape[0] == 0:
        return y.reshape(x.shape)
    w = None if weight is None else weight.detach().float().contiguous()
    b = None if bias is None else bias.detach().float().contiguous()
    lib = N.load()
    if act_bits:
        N.check("rpfq_layer_norm_act_quant", lib.rpfq_layer_norm_act_quant(
            x2.data_ptr(), N.dtype_code(x2.dtype), x2.shape[0], c, N.ptr(w), N.ptr(b), float(eps), int(act_bits),
            y.data_ptr(), N.dtype_code(y.dtype), N.stream_of(x2)))
    else:
        N.check("rpfq_layer_norm", lib.rpfq_layer_norm(
            x2.data_ptr(), N.dtype_code(x2.dtype), x2.shape[0], c, N.ptr(w), N.ptr(b), float(eps), y.data_ptr(),
            N.dtype_code(y.dtype), N.stream_of(x2)))
    return y.reshape(x.shape)


def layer_norm_prescaled(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
                         eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(y, row_scale) for bf16 / float32 x (rpfq_layer_norm_prescaled): the
    rows of layer_norm(x) in x's dtype, times their power-of-two prescale
    row_scale (float32 [M], what row_scales() gives those rows), stored as
    fp16.  PackedWide.linear(y, ..., row_scale=row_scale) on a launch that
    takes the DMA kernel equals linear(layer_norm(x)) on bf16 rows bit for
    bit, without the kernel's in-LDS bf16 conversion or a row-scale pass,
    and gives float32 rows the register-staged kernel's operands."""
    N.require_device(x, weight, bias)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("layer_norm_prescaled takes bf16 or float32 rows")
    c = x.shape[-1]
    x2 = _aligned_rows(x.reshape(-1, c))
    m = x2.shape[0]
    y = torch.empty(x2.shape, dtype=torch.float16, device=x.device)
    sc = torch.empty(m, dtype=torch.float32, device=x.device)
    if m:
        w = None if weight is None else weight.detach().float().contiguous()
        b = None if bias is None else bias.detach().float().contiguous()
        N.check("rpfq_layer_norm_prescaled", N.load().rpfq_layer_norm_prescaled(
            x2.data_ptr(), N.dtype_code(x2.dtype), m, c, N.ptr(w), N.ptr(b), float(eps), y.data_ptr(), sc.data_ptr(),
            N.stream_of(x2)))
    return y.reshape(x.shape), sc


@dataclass
class PackedWide:
    """One widely-linear layer in the MI355X tiled layout (a device blob).

    n_complex / k_complex: N' = out/2, K' = in/2; codebook: _native.CB_*;
    stages: residual stages per U/W; rotation: ((cos_u, sin_u), (cos_w, sin_w))
    float32 values or None."""

    n_complex: int
    k_complex: int
    codebook: int
    stages: int
    block: int
    blob: torch.Tensor
    rotation: tuple | None = None
    desc: N.WideDesc = field(init=False, repr=False)
    _adjoint: torch.Tensor | None = field(default=None, init=False, repr=False, compare=False)

    def __post_init__(self):
        self.desc = make_desc(self.n_complex, self.k_complex, self.codebook, self.stages, self.block,
                              self.rotation)

    @property
    def in_features(self) -> int:
        return 2 * self.k_complex

    @property
    def out_features(self) -> int:
        return 2 * self.n_complex

    @classmethod
    def from_planes(cls, planes, scale_re, scale_im, n_complex: int, k_complex: int, codebook: int = N.CB_AXIS,
                    stages: int = 2, block: int = 0, rotation=None, sync: bool = True) -> "PackedWide":
        """planes: packed code planes (u_s0[, u_s1], w_s0[, w_s1] or u, w for
        PSK16) as uint8 device tensors; scale_re/scale_im: float32 [N', nblk]
        multipliers per plane.  sync=False skips the final stream
        synchronization: for sources produced and released on the current
        stream (the caching allocator reuses their memory in stream order)."""
        dev = planes[0].device
        N.require_device(*planes)
        desc = make_desc(n_complex, k_complex, codebook, stages, block, rotation)
        lib = N.load()
        nbytes = lib.rpfq_wide_packed_bytes(ctypes.byref(desc))
        if nbytes == 0:
            N.check("rpfq_wide_packed_bytes", 2)
        blob = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        planes = [p.contiguous() for p in planes]
        sre = [s.contiguous().float() for s in scale_re]
        sim = [s.contiguous().float() for s in (scale_im if scale_im is not None else scale_re)]
        arr = ctypes.c_void_p * len(planes)
        N.check("rpfq_wide_pack", lib.rpfq_wide_pack(
            ctypes.byref(desc), arr(*[p.data_ptr() for p in planes]), len(planes),
            arr(*[s.data_ptr() for s in sre]), arr(*[s.data_ptr() for s in sim]),
            blob.data_ptr(), nbytes, N.stream_of(blob)))
        # keep the sources alive until the pack kernels have consumed them
        if sync:
            torch.cuda.current_stream(dev).synchronize()
        return cls(n_complex, k_complex, codebook, stages, block, blob, rotation)

    def linear(self, x: torch.Tensor, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype | None = None, flags: int = 0,
               residual: torch.Tensor | None = None, gelu: bool = False,
               row_scale: torch.Tensor | None = None) -> torch.Tensor:
        """y = U x + W conj(x) + bias on [..., 2K'] -> [..., 2N'].
        flags: 0 (kernel chosen from the shape), _native.FLAG_TILE_M128,
        _native.FLAG_NO_STREAM or _native.FLAG_STREAM.  residual ([..., 2N'] of out_dtype): y =
        residual + layer(x), fused into the kernel's store and rounded as the
        unfused add would round it (rpfq_wide_linear_residual).  gelu: y =
        GELU(layer(x)) in the store (within 1 ulp of out_dtype of the exact
        GELU of the rounded output; not with a residual).  float32 / bf16 x:
        the rows are prescaled by powers of two (row_scale, float32 [M] as
        row_scales() computes it, or computed here) so any magnitude keeps
        its relative accuracy through the fp16 operands
        (rpfq_wide_linear_scaled)."""
        N.require_device(x, bias, residual, row_scale)
        if gelu:
            if residual is not None:
                raise ValueError("gelu and residual cannot be fused together")
            flags = int(flags) | N.FLAG_GELU
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected last dim {self.in_features}, got {x.shape[-1]}")
        lead = x.shape[:-1]
        x2 = _aligned_rows(x.reshape(-1, self.in_features))
        m = x2.shape[0]
        out_dtype = out_dtype or x.dtype
        y = torch.empty(m, self.out_features, dtype=out_dtype, device=x.device)
        r2 = None
        if residual is not None:
            if residual.shape[:-1] != lead or residual.shape[-1] != self.out_features:
                raise ValueError(f"residual must have shape {tuple(lead) + (self.out_features,)}")
            r2 = _aligned_rows(residual.to(out_dtype).reshape(-1, self.out_features))
        if row_scale is not None:
            if row_scale.shape != (m,) or row_scale.dtype != torch.float32:
                raise ValueError(f"row_scale must be a float32 tensor of shape ({m},)")
            row_scale = _aligned_rows(row_scale)
        if m == 0:
            return y.reshape(*lead, self.out_features)
        if bias is not None:
            bias = bias.contiguous().float()
        lib = N.load()
        # float32 / bf16 rows: the range guard's prescales (fp16 x is the
        # MFMA operand as it stands); supplied rows scales are used as given.
        # Rows the DMA kernel would take as fp16 arrive there as prescaled
        # fp16 rows instead (bf16: the same operand bits, no conversion in
        # the kernel; float32: the register-staged kernel's operands).
        if row_scale is None and RANGE_GUARD and x2.dtype != torch.float16:
            c = x2.shape[1]
            if (PRESCALE_ROWS and c % 8 == 0 and c <= 4096
                    and self.kernel_for(m, torch.float16, out_dtype, flags) == N.KERNEL_DMA):
                x2, row_scale = prescale_rows(x2)
            else:
                row_scale = row_scales(x2)
        rec = _launch_recorder
        if rec is not None:
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
        N.check("rpfq_wide_linear_scaled", lib.rpfq_wide_linear_scaled(
            ctypes.byref(self.desc), self.blob.data_ptr(), self.blob.numel(), x2.data_ptr(), N.dtype_code(x2.dtype),
            m, N.ptr(row_scale), N.ptr(bias), N.ptr(r2), y.data_ptr(), N.dtype_code(out_dtype), int(flags),
            N.stream_of(x2)))
        if rec is not None:
            ev1.record()
            nbytes = wide_bytes(m, self.n_complex, self.k_complex, x2.element_size(), y.element_size(),
                                self.code_bytes * 8 // max(1, self.n_complex * self.k_complex))
            if residual is not None:
                nbytes += m * self.out_features * y.element_size()
            # the device kernel (a fused GELU is a separate instantiation)
            kern = N.KERNEL_NAMES.get(self.kernel_for(m, x2.dtype, out_dtype, flags), "?")
            rec(ev0, ev1, wide_flops(m, self.n_complex, self.k_complex), nbytes,
                (m, self.n_complex, self.k_complex, kern + ("+gelu" if flags & N.FLAG_GELU else "")))
        return y.reshape(*lead, self.out_features)

    def ln_fusable(self, m: int, x_dtype: torch.dtype, y_dtype: torch.dtype | None = None) -> bool:
        """Whether layer_norm_linear() fuses the LayerNorm for m rows
        (rpfq_layer_norm_wide_linear_fusable, no GPU work)."""
        out = ctypes.c_int32(0)
        N.check("rpfq_layer_norm_wide_linear_fusable", N.load().rpfq_layer_norm_wide_linear_fusable(
            ctypes.byref(self.desc), int(m), N.dtype_code(x_dtype), N.dtype_code(y_dtype or x_dtype),
            ctypes.byref(out)))
        return bool(out.value)

    def layer_norm_linear(self, x: torch.Tensor, ln_weight: torch.Tensor | None, ln_bias: torch.Tensor | None,
                          eps: float, bias: torch.Tensor | None = None, out_dtype: torch.dtype | None = None,
                          gelu: bool = False) -> torch.Tensor:
        """self.linear(layer_norm(x, ln_weight, ln_bias, eps), bias) in one
        launch (rpfq_layer_norm_wide_linear): the LayerNorm over the 2K' input
        features runs in the streaming kernel's prologue, its output rounded
        to x's dtype as layer_norm() rounds it.  Only where ln_fusable();
        gelu as in linear()."""
        N.require_device(x, ln_weight, ln_bias, bias)
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected last dim {self.in_features}, got {x.shape[-1]}")
        lead = x.shape[:-1]
        x2 = _aligned_rows(x.reshape(-1, self.in_features))
        m = x2.shape[0]
        out_dtype = out_dtype or x.dtype
        y = torch.empty(m, self.out_features, dtype=out_dtype, device=x.device)
        if m == 0:
            return y.reshape(*lead, self.out_features)
        w = None if ln_weight is None else ln_weight.detach().float().contiguous()
        b = None if ln_bias is None else ln_bias.detach().float().contiguous()
        if bias is not None:
            bias = bias.contiguous().float()
        N.check("rpfq_layer_norm_wide_linear", N.load().rpfq_layer_norm_wide_linear(
            ctypes.byref(self.desc), self.blob.data_ptr(), self.blob.numel(), x2.data_ptr(), N.dtype_code(x2.dtype),
            m, N.ptr(w), N.ptr(b), float(eps), N.ptr(bias), y.data_ptr(), N.dtype_code(out_dtype),
            N.FLAG_GELU if gelu else 0, N.stream_of(x2)))
        return y.reshape(*lead, self.out_features)

    def act_quant_linear(self, x: torch.Tensor, bits: int, bias: torch.Tensor | None = None,
                         out_dtype: torch.dtype | None = None, gelu: bool = False,
                         residual: torch.Tensor | None = None, layer_norm=None) -> torch.Tensor:
        """self.linear(act_quant(x, bits), bias) -- or of act_quant(layer_norm(x))
        with layer_norm = (ln_weight, ln_bias, eps) -- in one launch
        (rpfq_act_quant_wide_linear): the streaming kernel's prologue quantizes
        the rows as act_quant() / layer_norm(act_bits=bits) does, bit for bit.
        residual ([..., 2N'] of out_dtype): added in the store.  Only where
        ln_fusable(); gelu as in linear() (not with a residual)."""
        N.require_device(x, bias, residual)
        if x.shape[-1] != self.in_features:
            raise ValueError(f"expected last dim {self.in_features}, got {x.shape[-1]}")
        lead = x.shape[:-1]
        x2 = _aligned_rows(x.reshape(-1, self.in_features))
        m = x2.shape[0]
        out_dtype = out_dtype or x.dtype
        y = torch.empty(m, self.out_features, dtype=out_dtype, device=x.device)
        r2 = None
        if residual is not None:
            if residual.shape[:-1] != lead or residual.shape[-1] != self.out_features:
                raise ValueError(f"residual must have shape {tuple(lead) + (self.out_features,)}")
            r2 = _aligned_rows(residual.to(out_dtype).reshape(-1, self.out_features))
        if m == 0:
            return y.reshape(*lead, self.out_features)
        w = b = None
        eps = 0.0
        if layer_norm is not None:
            ln_w, ln_b, eps = layer_norm
            N.require_device(ln_w, ln_b)
            w = None if ln_w is None else ln_w.detach().float().contiguous()
            b = None if ln_b is None else ln_b.detach().float().contiguous()
        if bias is not None:
            bias = bias.contiguous().float()
        N.check("rpfq_act_quant_wide_linear", N.load().rpfq_act_quant_wide_linear(
            ctypes.byref(self.desc), self.blob.data_ptr(), self.blob.numel(), x2.data_ptr(), N.dtype_code(x2.dtype),
            m, int(bits), int(layer_norm is not None), N.ptr(w), N.ptr(b), float(eps), N.ptr(bias), N.ptr(r2),
            y.data_ptr(), N.dtype_code(out_dtype), N.FLAG_GELU if gelu else 0, N.stream_of(x2)))
        return y.reshape(*lead, self.out_features)

    def kernel_for(self, m: int, x_dtype: torch.dtype, y_dtype: torch.dtype, flags: int = 0) -> int:
        """The kernel linear() runs for m rows (N.KERNEL_STREAM / _GEMV /
        _DMA / _TILED; rpfq_wide_linear_kernel, no GPU work)."""
        out = ctypes.c_int32(-1)
        N.check("rpfq_wide_linear_kernel", N.load().rpfq_wide_linear_kernel(
            ctypes.byref(self.desc), int(m), N.dtype_code(x_dtype), N.dtype_code(y_dtype), int(flags),
            ctypes.byref(out)))
        return out.value

    def linear_into(self, x: torch.Tensor, bias: torch.Tensor | None, y: torch.Tensor, flags: int = 0) -> None:
        """y[:] = U x + W conj(x) + bias for a contiguous [M, 2K'] x and a
        preallocated contiguous [M, 2N'] y; bias float32 [2N'] or None.
        Allocates nothing (usable under HIP graph capture)."""
        N.require_device(x, bias, y)
        m = x.shape[0]
        if x.dim() != 2 or x.shape[1] != self.in_features or not x.is_contiguous():
            raise ValueError(f"x must be a contiguous [M, {self.in_features}] tensor")
        if y.shape != (m, self.out_features) or not y.is_contiguous():
            raise ValueError(f"y must be a contiguous [{m}, {self.out_features}] tensor")
        if bias is not None and (bias.dtype != torch.float32 or not bias.is_contiguous()):
            raise TypeError("bias must be a contiguous float32 tensor")
        lib = N.load()
        N.check("rpfq_wide_linear", lib.rpfq_wide_linear(
            ctypes.byref(self.desc), self.blob.data_ptr(), self.blob.numel(), x.data_ptr(),
            N.dtype_code(x.dtype), m, N.ptr(bias), y.data_ptr(), N.dtype_code(y.dtype), int(flags),
            N.stream_of(x)))

    def adjoint(self) -> torch.Tensor:
        """The adjoint blob of this layer (rpfq_wide_pack_adjoint: transposed
        code tiles and U / W tables), built on first use and kept with the
        layer."""
        if self._adjoint is None:
            lib = N.load()
            nbytes = lib.rpfq_wide_adjoint_bytes(ctypes.byref(self.desc))
            if nbytes == 0:
                N.check("rpfq_wide_adjoint_bytes", 2)
            adj = torch.empty(nbytes, dtype=torch.uint8, device=self.blob.device)
            N.check("rpfq_wide_pack_adjoint", lib.rpfq_wide_pack_adjoint(
                ctypes.byref(self.desc), self.blob.data_ptr(), self.blob.numel(), adj.data_ptr(), nbytes,
                N.stream_of(self.blob)))
            self._adjoint = adj
        return self._adjoint

    def grad_x(self, grad_y: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """Input gradient of linear(): grad_y [..., 2N'] -> grad_y A
        [..., 2K'] with A the fused fp16 coefficients linear() contracts
        with (rpfq_wide_linear_grad_x; the backward of F.linear's input,
        RPFQ-ViT-main/quant_models/kernel.py:585)."""
        N.require_device(grad_y)
        if grad_y.shape[-1] != self.out_features:
            raise ValueError(f"expected last dim {self.out_features}, got {grad_y.shape[-1]}")
        lead = grad_y.shape[:-1]
        g2 = _aligned_rows(grad_y.reshape(-1, self.out_features))
        m = g2.shape[0]
        out_dtype = out_dtype or grad_y.dtype
        gx = torch.empty(m, self.in_features, dtype=out_dtype, device=grad_y.device)
        if m == 0:
            return gx.reshape(*lead, self.in_features)
        adj = self.adjoint()
        N.check("rpfq_wide_linear_grad_x", N.load().rpfq_wide_linear_grad_x(
            ctypes.byref(self.desc), adj.data_ptr(), adj.numel(), g2.data_ptr(), N.dtype_code(g2.dtype), m,
            gx.data_ptr(), N.dtype_code(out_dtype), N.stream_of(g2)))
        return gx.reshape(*lead, self.in_features)

    def decode(self, round_fp16: bool = False) -> torch.Tensor:
        """Fused float32 weight A_q [2N', 2K'] (quant_i.py:534-544 layout)."""
        a = torch.empty(self.out_features, self.in_features, dtype=torch.float32, device=self.blob.device)
        lib = N.load()
        N.check("rpfq_wide_decode", lib.rpfq_wide_decode(
            ctypes.byref(self.desc), self.blob.data_ptr(), self.blob.numel(), a.data_ptr(),
            int(bool(round_fp16)), N.stream_of(self.blob)))
        return a

    @property
    def code_bytes(self) -> int:
        """Algorithmic bytes of the packed codes: 2*stages planes of 2 bits
        (AXIS/SIGN) or 2 planes of 4 bits (PSK16, TABLE) per complex element."""
        bits = 8 if self.codebook in (N.CB_PSK16, N.CB_TABLE) else 4 * self.stages
        return self.n_complex * self.k_complex * bits // 8

    @property
    def device(self) -> torch.device:
        return self.blob.device


@dataclass
class PackedStages:
    """A layer whose U and W carry more than two residual stages
    (complex_phase_v3 / v4, quant_i.py:145-166), run as stage groups of at
    most two stages each: group 0 holds stages (0, 1) of U and W, group 1
    stages (2[, 3]).  The layer is linear in its stages, so

        y = G1 x + (G0 x + bias)

    with the inner sum added in group 1's store (rpfq_wide_linear_residual).
    Each group's fused fp16 coefficients satisfy the single-group bound
    against that group's float32 stage sum, and the intermediate G0 x + bias
    is rounded once to y's dtype."""

    groups: list

    @property
    def n_complex(self) -> int:
        return self.groups[0].n_complex

    @property
    def k_complex(self) -> int:
        return self.groups[0].k_complex

    @property
    def in_features(self) -> int:
        return self.groups[0].in_features

    @property
    def out_features(self) -> int:
        return self.groups[0].out_features

    @property
    def stages(self) -> int:
        return sum(g.stages for g in self.groups)

    @property
    def device(self) -> torch.device:
        return self.groups[0].device

    @property
    def code_bytes(self) -> int:
        return sum(g.code_bytes for g in self.groups)

    def linear(self, x: torch.Tensor, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype | None = None, flags: int = 0,
               residual: torch.Tensor | None = None) -> torch.Tensor:
        """PackedWide.linear over all stage groups (one launch per group)."""
        y = self.groups[0].linear(x, bias, out_dtype, flags, residual)
        for g in self.groups[1:]:
            y = g.linear(x, None, y.dtype, flags, residual=y)
        return y

    def grad_x(self, grad_y: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
        """Input gradient over all stage groups: the sum of the groups'
        grad_x, each in float32, rounded once to out_dtype."""
        gx = self.groups[0].grad_x(grad_y, torch.float32)
        for g in self.groups[1:]:
            gx += g.grad_x(grad_y, torch.float32)
        return gx.to(out_dtype or grad_y.dtype)

    def decode(self, round_fp16: bool = False) -> torch.Tensor:
        """Sum of the groups' fused weights (float32)."""
        a = self.groups[0].decode(round_fp16)
        for g in self.groups[1:]:
            a += g.decode(round_fp16)
        return a


def pack_layer(planes, scale_re, scale_im, n_complex: int, k_complex: int, codebook: int = N.CB_AXIS,
               stages: int = 2, block: int = 0, rotation=None, sync: bool = True):
    """PackedWide for stages <= 2, else PackedStages over groups of two
    stages.  planes / scales ordered u_s0..u_s{S-1}, w_s0..w_s{S-1} (AXIS,
    SIGN) as PackedWide.from_planes takes them."""
    if stages <= 2 or codebook in (N.CB_PSK16, N.CB_TABLE):
        return PackedWide.from_planes(planes, scale_re, scale_im, n_complex, k_complex, codebook, stages, block,
                                      rotation, sync)
    if len(planes) != 2 * stages:
        raise ValueError(f"expected {2 * stages} planes, got {len(planes)}")
    groups = []
    for lo in range(0, stages, 2):
        hi = min(lo + 2, stages)
        idx = list(range(lo, hi)) + list(range(stages + lo, stages + hi))
        groups.append(PackedWide.from_planes([planes[i] for i in idx], [scale_re[i] for i in idx],
                                             [scale_im[i] for i in idx], n_complex, k_complex, codebook,
                                             hi - lo, block, rotation, sync))
    return PackedStages(groups)


QUANT_KINDS = {"axis": N.QK_AXIS, "sign": N.QK_SIGN}


def quantize_wide(weight: torch.Tensor, kind_u: str, steps_u: int, kind_w: str, steps_w: int,
                  rot: torch.Tensor | None = None, want_aq: bool = True, want_codes: bool = False):
    """Training-semantics quantization of a float32 [2N', 2K'] master weight
    on the GPU (rpfq_quantize_wide; quant_i.py:513-544).

    rot: None or a float32 device tensor [cos_u, sin_u, cos_w, sin_w].
    Returns (a_q [2N', 2K'] float32 or None, scales [2, 4, 2] float32 (U/W,
    stage, re/im), codes [steps_u + steps_w, N', K'/4] uint8 or None)."""
    N.require_device(weight, rot)
    if weight.dtype != torch.float32 or weight.dim() != 2:
        raise TypeError("weight must be a 2-D float32 tensor")
    out_f, in_f = weight.shape
    if out_f % 2 or in_f % 2:
        raise ValueError("Complex-phase QAT requires even in/out features.")
    weight = weight.contiguous()
    d = N.QuantDesc()
    d.n_complex, d.k_complex = out_f // 2, in_f // 2
    d.kind[0], d.kind[1] = QUANT_KINDS[kind_u], QUANT_KINDS[kind_w]
    d.steps[0], d.steps[1] = int(steps_u), int(steps_w)
    if rot is not None:
        rot = rot.detach().reshape(4).float().contiguous()
    dev = weight.device
    lib = N.load()
    work = torch.empty(lib.rpfq_quantize_workspace_bytes(ctypes.byref(d)), dtype=torch.uint8, device=dev)
    scales = torch.empty(2, 4, 2, dtype=torch.float32, device=dev)
    a_q = torch.empty_like(weight) if want_aq else None
    codes = None
    if want_codes:
        codes = torch.empty(steps_u + steps_w, d.n_complex, d.k_complex // 4, dtype=torch.uint8, device=dev)
    N.check("rpfq_quantize_wide", lib.rpfq_quantize_wide(
        ctypes.byref(d), weight.data_ptr(), N.ptr(rot), N.ptr(a_q), scales.data_ptr(), N.ptr(codes),
        work.data_ptr(), work.numel(), N.stream_of(weight)))
    return a_q, scales, codes


def make_desc(n_complex, k_complex, codebook, stages, block, rotation) -> N.WideDesc:
    d = N.WideDesc()
    d.n_complex = int(n_complex)
    d.k_complex = int(k_complex)
    d.block = int(block)
    d.codebook = int(codebook)
    d.stages = int(stages)
    if rotation is not None:
        (cu, su), (cw, sw) = rotation
        d.rotate = 1
        d.rot_u[0], d.rot_u[1] = float(cu), float(su)
        d.rot_w[0], d.rot_w[1] = float(cw), float(sw)
    else:
        d.rotate = 0
    return d


def mlp_fusable(fc1, fc2, m: int, dtype: torch.dtype) -> bool:
    """Whether wide_mlp() takes fc1 -> GELU -> fc2 as one launch: single-group
    packed layers (PackedWide) with K' = 96, N1' a multiple of 96 up to
    1536, fc2 the inverse shape, per-row scales and one codebook, fp16
    activations, m >= 64 rows (the shapes rpfq_wide_mlp accepts)."""
    return (isinstance(fc1, PackedWide) and isinstance(fc2, PackedWide) and dtype == torch.float16 and m >= 64
            and fc1.k_complex == 96 and fc1.n_complex % 96 == 0 and fc1.n_complex <= 1536
            and fc2.k_complex == fc1.n_complex and fc2.n_complex == fc1.k_complex and fc1.block == 0
            and fc2.block == 0 and fc1.codebook == fc2.codebook)


def wide_mlp(fc1: "PackedWide", fc2: "PackedWide", x: torch.Tensor, bias1: torch.Tensor | None = None,
             bias2: torch.Tensor | None = None, residual: torch.Tensor | None = None) -> torch.Tensor:
    """residual + fc2(GELU(fc1(x) + bias1)) + bias2 on fp16 [..., 2K'] in one
    launch (rpfq_wide_mlp): the hidden activations stay in LDS, each the fp16
    rounding of fc1's output passed through the stores' GELU (within 1 ulp of
    the exact GELU), so y equals fc1.linear(x, bias1, gelu=True) followed by
    fc2.linear(h, bias2, residual=residual) on the large-M kernel bit for
    bit."""
    N.require_device(x, bias1, bias2, residual)
    if x.dtype != torch.float16:
        raise ValueError("wide_mlp takes fp16 activations")
    if x.shape[-1] != fc1.in_features:
        raise ValueError(f"expected last dim {fc1.in_features}, got {x.shape[-1]}")
    lead = x.shape[:-1]
    x2 = _aligned_rows(x.reshape(-1, fc1.in_features))
    m = x2.shape[0]
    if not mlp_fusable(fc1, fc2, m, x.dtype):
        raise ValueError("wide_mlp: unsupported layers or row count (see mlp_fusable)")
    y = torch.empty(m, fc2.out_features, dtype=torch.float16, device=x.device)
    r2 = None
    if residual is not None:
        if residual.shape[:-1] != lead or residual.shape[-1] != fc2.out_features:
            raise ValueError(f"residual must have shape {tuple(lead) + (fc2.out_features,)}")
        r2 = _aligned_rows(residual.to(torch.float16).reshape(-1, fc2.out_features))
    b1 = None if bias1 is None else bias1.contiguous().float()
    b2 = None if bias2 is None else bias2.contiguous().float()
    rec = _launch_recorder
    if rec is not None:
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
    N.check("rpfq_wide_mlp", N.load().rpfq_wide_mlp(
        ctypes.byref(fc1.desc), fc1.blob.data_ptr(), fc1.blob.numel(), ctypes.byref(fc2.desc), fc2.blob.data_ptr(),
        fc2.blob.numel(), x2.data_ptr(), m, N.ptr(b1), N.ptr(b2), N.ptr(r2), y.data_ptr(), N.stream_of(x2)))
    if rec is not None:
        ev1.record()
        n1, k = fc1.n_complex, fc1.k_complex
        nbytes = (wide_bytes(m, n1, k) + wide_bytes(m, k, n1) - 2 * m * 2 * n1 * 2
                  + (m * 2 * k * 2 if residual is not None else 0))
        rec(ev0, ev1, wide_flops(m, n1, k) + wide_flops(m, k, n1), nbytes, (m, n1, k, "rpfq::wide_mlp_kernel"))
    return y.reshape(*lead, fc2.out_features)


def layer_norm_wide_mlp(fc1: "PackedWide", fc2: "PackedWide", x: torch.Tensor, ln_weight: torch.Tensor | None,
                        ln_bias: torch.Tensor | None, eps: float, bias1: torch.Tensor | None = None,
                        bias2: torch.Tensor | None = None) -> torch.Tensor:
    """x + fc2(GELU(fc1(layer_norm(x)) + bias1)) + bias2 in one launch
    (rpfq_layer_norm_wide_mlp): the LayerNorm of the rows (float32 weight /
    bias over the last dim) in the MLP's prologue, equal to layer_norm()
    followed by wide_mlp(..., residual=x) bit for bit."""
    N.require_device(x, ln_weight, ln_bias, bias1, bias2)
    if x.dtype != torch.float16:
        raise ValueError("layer_norm_wide_mlp takes fp16 activations")
    if x.shape[-1] != fc1.in_features:
        raise ValueError(f"expected last dim {fc1.in_features}, got {x.shape[-1]}")
    lead = x.shape[:-1]
    x2 = _aligned_rows(x.reshape(-1, fc1.in_features))
    m = x2.shape[0]
    if not mlp_fusable(fc1, fc2, m, x.dtype):
        raise ValueError("layer_norm_wide_mlp: unsupported layers or row count (see mlp_fusable)")
    y = torch.empty(m, fc2.out_features, dtype=torch.float16, device=x.device)
    w = None if ln_weight is None else _aligned_rows(ln_weight.detach().float().contiguous())
    b = None if ln_bias is None else _aligned_rows(ln_bias.detach().float().contiguous())
    b1 = None if bias1 is None else bias1.contiguous().float()
    b2 = None if bias2 is None else bias2.contiguous().float()
    rec = _launch_recorder
    if rec is not None:
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record()
    N.check("rpfq_layer_norm_wide_mlp", N.load().rpfq_layer_norm_wide_mlp(
        ctypes.byref(fc1.desc), fc1.blob.data_ptr(), fc1.blob.numel(), ctypes.byref(fc2.desc), fc2.blob.data_ptr(),
        fc2.blob.numel(), x2.data_ptr(), m, N.ptr(w), N.ptr(b), float(eps), N.ptr(b1), N.ptr(b2), y.data_ptr(),
        N.stream_of(x2)))
    if rec is not None:
        ev1.record()
        n1, k = fc1.n_complex, fc1.k_complex
        nbytes = wide_bytes(m, n1, k) + wide_bytes(m, k, n1) - 2 * m * 2 * n1 * 2 + m * 2 * k * 2
        rec(ev0, ev1, wide_flops(m, n1, k) + wide_flops(m, k, n1), nbytes, (m, n1, k, "rpfq::wide_mlp_kernel+ln"))
    return y.reshape(*lead, fc2.out_features)


def wide_flops(m: int, n_complex: int, k_complex: int) -> int:
    """Algorithmic FLOPs of one widely-linear layer (one real GEMM)."""
    return 2 * m * (2 * k_complex) * (2 * n_complex)


def wide_bytes(m: int, n_complex: int, k_complex: int, act_bytes: int = 2, out_bytes: int = 2,
               code_bits: int = 8, nscale: int = 8) -> int:
    """Algorithmic HBM bytes: activations in/out, codes, per-row scales, bias."""
    return (m * 2 * k_complex * act_bytes + m * 2 * n_complex * out_bytes
            + math.ceil(n_complex * k_complex * code_bits / 8) + 4 * nscale * n_complex + 4 * 2 * n_complex)
