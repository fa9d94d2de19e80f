"""Model-level helpers for the packed HIP path."""
from __future__ import annotations

from typing import Iterator, Tuple

import torch
import torch.nn as nn

from . import _native as N
from . import packing as P
from .quant_i import QATLinearComplexPhase


def quant_layers(model: nn.Module) -> Iterator[Tuple[str, QATLinearComplexPhase]]:
    for name, m in model.named_modules():
        if isinstance(m, QATLinearComplexPhase):
            yield name, m


def load_synthetic_codes(model: nn.Module, seed: int, codebook: int = N.CB_AXIS, lo: float = 0.01,
                         hi: float = 0.1) -> int:
    """Give every quantized layer benchmark codes: the reference axis rule on
    its (random-init) float32 weight, per-(plane, row) magnitudes ~U(lo, hi);
    PSK16 uses the nearest of 16 phases.  Returns the number of layers."""
    g = torch.Generator().manual_seed(seed)
    n = 0
    for _, layer in quant_layers(model):
        layer.load_packed(P.synthetic_layer(layer.weight, g, lo, hi, codebook))
        n += 1
    return n


def prepare_inference(model: nn.Module, device="cuda", dtype: torch.dtype = torch.float16) -> nn.Module:
    """eval(), move to `device`, pack every quantized layer once, and cast the
    remaining (non-quantized) parameters and buffers to `dtype`.  Quantized
    layers keep their float32 master weight and bias."""
    model.eval().to(device)
    for _, layer in quant_layers(model):
        layer.packed(torch.device(device))
    for m in model.modules():
        if isinstance(m, QATLinearComplexPhase):
            continue
        for name, p in list(m.named_parameters(recurse=False)):
            p.data = p.data.to(dtype)
        for name, b in list(m.named_buffers(recurse=False)):
            if b is not None and b.is_floating_point():
                setattr(m, name, b.to(dtype))
    return model


def packed_code_bytes(model: nn.Module) -> int:
    return sum(layer.packed(layer.weight.device).code_bytes for _, layer in quant_layers(model))
