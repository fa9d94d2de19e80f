"""ctypes binding of the C ABI in include/rpfq.h (librpfq.so, built for gfx950).

Only plain pointers, sizes and a stream handle cross the boundary.  Tensor
helpers below translate torch tensors to those arguments; they raise when the
library is missing -- there is no host fallback for device tensors.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

# RPFQ_LIBRARY names another build of the library to load (e.g. an A/B build).
_LIB_PATH = os.environ.get("RPFQ_LIBRARY") or os.path.join(
    os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "librpfq.so")

RPFQ_OK = 0
ERRORS = {
    1: "RPFQ_ERR_NULL",
    2: "RPFQ_ERR_SHAPE",
    3: "RPFQ_ERR_ALIGN",
    4: "RPFQ_ERR_BITS",
    5: "RPFQ_ERR_DTYPE",
    6: "RPFQ_ERR_VALUE",
    7: "RPFQ_ERR_HIP",
}
F32, F16, BF16 = 0, 1, 2
CB_AXIS, CB_SIGN, CB_PSK16, CB_TABLE = 0, 1, 2, 3
QK_AXIS, QK_SIGN = 0, 1  # weight quantizer kinds of rpfq_quantize_wide
FLAG_TILE_M128 = 1  # force the register-staged 128-row kernel
FLAG_NO_STREAM = 2  # keep every M on the tiled kernels (no weight-streaming kernel)
FLAG_STREAM = 4  # force the weight-streaming kernel for any M (16-row chunks)
FLAG_GELU = 8  # exact GELU of the rounded output, fused into the store (no residual)
FLAG_RESIDENT = 16  # force the resident-weight kernel (small layers; fp16 / bf16 x and y)
KERNEL_STREAM, KERNEL_DMA, KERNEL_TILED, KERNEL_GEMV, KERNEL_RESIDENT = 0, 1, 2, 3, 4  # rpfq_wide_linear_kernel
STREAM_KERNELS = (KERNEL_STREAM, KERNEL_GEMV)  # the weight-streaming kernels (small M)
# device kernel behind each id (KERNEL_GEMV: wide_linear_gemv_persist_kernel
# where that form applies); launch records and reports name kernels by these
KERNEL_NAMES = {KERNEL_STREAM: "rpfq::wide_linear_skinny_kernel", KERNEL_DMA: "rpfq::wide_linear_dma_kernel",
                KERNEL_TILED: "rpfq::wide_linear_kernel", KERNEL_GEMV: "rpfq::wide_linear_gemv_kernel",
                KERNEL_RESIDENT: "rpfq::wide_linear_resident_kernel"}

_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# Every symbol include/rpfq.h declares (checked by tests/test_capi_cpu.py).
EXPORTED = (
    "rpfq_abi_version",
    "rpfq_last_error",
    "rpfq_unpack",
    "rpfq_phase_linear",
    "rpfq_wide_packed_bytes",
    "rpfq_wide_pack",
    "rpfq_wide_linear",
    "rpfq_wide_decode",
    "rpfq_act_quant",
    "rpfq_wide_linear_residual",
    "rpfq_wide_adjoint_bytes",
    "rpfq_wide_pack_adjoint",
    "rpfq_wide_linear_grad_x",
    "rpfq_layer_norm_wide_linear",
    "rpfq_layer_norm_wide_linear_fusable",
    "rpfq_act_quant_wide_linear",
    "rpfq_wide_linear_kernel",
    "rpfq_layer_norm",
    "rpfq_layer_norm_prescaled",
    "rpfq_row_prescale",
    "rpfq_layer_norm_act_quant",
    "rpfq_gelu_act_quant",
    "rpfq_quantize_workspace_bytes",
    "rpfq_quantize_wide",
    "rpfq_quantize_wide_noalloc",
    "rpfq_row_scales",
    "rpfq_wide_linear_scaled",
    "rpfq_wide_mlp",
    "rpfq_layer_norm_wide_mlp",
)


class WideDesc(ctypes.Structure):
    """Mirror of struct rpfq_wide_desc."""

    _fields_ = [
        ("n_complex", ctypes.c_int64),
        ("k_complex", ctypes.c_int64),
        ("block", ctypes.c_int64),
        ("codebook", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("rotate", ctypes.c_int32),
        ("rot_u", ctypes.c_float * 2),
        ("rot_w", ctypes.c_float * 2),
    ]


class QuantDesc(ctypes.Structure):
    """Mirror of struct rpfq_quant_desc."""

    _fields_ = [
        ("n_complex", ctypes.c_int64),
        ("k_complex", ctypes.c_int64),
        ("kind", ctypes.c_int32 * 2),
        ("steps", ctypes.c_int32 * 2),
    ]


class RPFQError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with {ERRORS.get(code, code)}: {msg}")
        self.code = code


_lib = None
_lock = threading.Lock()


def library_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load librpfq.so once; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"librpfq.so not found at {_LIB_PATH}; build it with "
                "`make -C rpfq-review_amd/csrc` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(_LIB_PATH)
        vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
        dp = ctypes.POINTER(WideDesc)
        lib.rpfq_abi_version.restype = i32
        lib.rpfq_last_error.restype = ctypes.c_char_p
        lib.rpfq_unpack.argtypes = [vp, i32, i64, i64, vp, vp, i64, vp, vp, vp]
        lib.rpfq_phase_linear.argtypes = [vp, vp, i32, i32, i64, i64, vp, vp, vp, i64, i64, vp, vp, i32, vp]
        lib.rpfq_wide_packed_bytes.argtypes = [dp]
        lib.rpfq_wide_packed_bytes.restype = sz
        lib.rpfq_wide_pack.argtypes = [dp, ctypes.POINTER(vp), i32, ctypes.POINTER(vp), ctypes.POINTER(vp), vp, sz, vp]
        lib.rpfq_wide_linear.argtypes = [dp, vp, sz, vp, i32, i64, vp, vp, i32, i32, vp]
        lib.rpfq_wide_decode.argtypes = [dp, vp, sz, vp, i32, vp]
        lib.rpfq_act_quant.argtypes = [vp, i32, i64, i64, i32, vp, i32, vp]
        lib.rpfq_wide_linear_residual.argtypes = [dp, vp, sz, vp, i32, i64, vp, vp, vp, i32, i32, vp]
        lib.rpfq_wide_linear_kernel.argtypes = [dp, i64, i32, i32, i32, ctypes.POINTER(i32)]
        lib.rpfq_wide_adjoint_bytes.argtypes = [dp]
        lib.rpfq_wide_adjoint_bytes.restype = sz
        lib.rpfq_wide_pack_adjoint.argtypes = [dp, vp, sz, vp, sz, vp]
        lib.rpfq_wide_linear_grad_x.argtypes = [dp, vp, sz, vp, i32, i64, vp, i32, vp]
        lib.rpfq_layer_norm_wide_linear.argtypes = [dp, vp, sz, vp, i32, i64, vp, vp, ctypes.c_float, vp, vp, i32,
                                                    i32, vp]
        lib.rpfq_layer_norm_wide_linear_fusable.argtypes = [dp, i64, i32, i32, ctypes.POINTER(i32)]
        lib.rpfq_act_quant_wide_linear.argtypes = [dp, vp, sz, vp, i32, i64, i32, i32, vp, vp, ctypes.c_float, vp,
                                                   vp, vp, i32, i32, vp]
        lib.rpfq_layer_norm.argtypes = [vp, i32, i64, i64, vp, vp, ctypes.c_float, vp, i32, vp]
        lib.rpfq_layer_norm_prescaled.argtypes = [vp, i32, i64, i64, vp, vp, ctypes.c_float, vp, vp, vp]
        lib.rpfq_row_prescale.argtypes = [vp, i32, i64, i64, vp, vp, vp]
        lib.rpfq_layer_norm_act_quant.argtypes = [vp, i32, i64, i64, vp, vp, ctypes.c_float, i32, vp, i32, vp]
        lib.rpfq_gelu_act_quant.argtypes = [vp, i32, i64, i64, i32, vp, i32, vp]
        qp = ctypes.POINTER(QuantDesc)
        lib.rpfq_quantize_workspace_bytes.argtypes = [qp]
        lib.rpfq_quantize_workspace_bytes.restype = sz
        lib.rpfq_quantize_wide.argtypes = [qp, vp, vp, vp, vp, vp, vp, sz, vp]
        lib.rpfq_quantize_wide_noalloc.argtypes = [qp, vp, vp, vp, vp, vp, vp]
        lib.rpfq_row_scales.argtypes = [vp, i32, i64, i64, vp, vp]
        lib.rpfq_wide_linear_scaled.argtypes = [dp, vp, sz, vp, i32, i64, vp, vp, vp, vp, i32, i32, vp]
        lib.rpfq_wide_mlp.argtypes = [dp, vp, sz, dp, vp, sz, vp, i64, vp, vp, vp, vp, vp]
        lib.rpfq_layer_norm_wide_mlp.argtypes = [dp, vp, sz, dp, vp, sz, vp, i64, vp, vp, ctypes.c_float, vp, vp, vp,
                                                 vp]
        for name in EXPORTED[2:]:
            if name not in ("rpfq_wide_packed_bytes", "rpfq_wide_adjoint_bytes", "rpfq_quantize_workspace_bytes"):
                getattr(lib, name).restype = i32
        _lib = lib
        return lib


def check(fn: str, rc: int) -> None:
    if rc != RPFQ_OK:
        msg = load().rpfq_last_error().decode(errors="replace")
        raise RPFQError(fn, rc, msg)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype not in _DTYPES:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16")
    return _DTYPES[dtype]


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int | None:
    """Raw hipStream_t of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream or None


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("rpfq HIP ops take device tensors only")
