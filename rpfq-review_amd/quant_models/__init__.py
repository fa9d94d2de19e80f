"""Complex phase-quantized ViT family on MI355X (gfx950).

Mirrors the reference package RPFQ-ViT-main/quant_models/__init__.py: importing
it registers every ``rpfq_*`` model name.  The quantized Linear layers run
the hand-written HIP kernels of librpfq.so (C ABI in include/rpfq.h).
"""
from .quant_i import (  # noqa: F401
    SUPPORTED_QUANT_METHODS,
    ActivationQuantSTE,
    ComplexActivationQuantizer,
    ComplexWeightQuantizer,
    LearnableGroupedPhaseQuant,
    QATLinearComplexPhase,
)
