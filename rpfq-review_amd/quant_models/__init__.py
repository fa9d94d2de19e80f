"""Complex phase-quantized ViT family on MI355X (gfx950).

Mirrors the reference package RPFQ-ViT-main/quant_models/__init__.py:
importing it registers every ``rpfq_*`` model name (ViT, distilled DeiT,
Swin) and the ``torch.ops.rpfq.*`` operators.  The quantized Linear layers run the hand-written HIP kernels of
librpfq.so through the C ABI in include/rpfq.h.
"""
from .quant_i import (  # noqa: F401
    SUPPORTED_QUANT_METHODS,
    ActivationQuantSTE,
    ComplexActivationQuantizer,
    ComplexWeightQuantizer,
    LearnableGroupedPhaseQuant,
    QATLinearComplexPhase,
)
from .quant_rpfq_deit import *  # noqa: F401,F403
from .quant_rpfq_swin import *  # noqa: F401,F403
from .quant_rpfq_vit import *  # noqa: F401,F403
from .registry import create_model, is_model, list_models, register_model  # noqa: F401
from . import torch_ops  # noqa: F401,E402  (registers torch.ops.rpfq.*)

__all__ = [
    "QATLinearComplexPhase",
    "ComplexWeightQuantizer",
    "ComplexActivationQuantizer",
    "SUPPORTED_QUANT_METHODS",
    "create_model",
    "is_model",
    "list_models",
    "register_model",
]
