"""Model registry with timm-compatible entry points.

The reference registers its models with timm's ``register_model`` and builds
them with ``timm.create_model`` (RPFQ-ViT-main/quant_models/quant_rpfq_vit.py:
10-13, :180-241; tests/test_models.py:24).  timm is not a dependency here, so
this module provides the same three calls over a local table.
"""
from __future__ import annotations

from typing import Callable, Dict, List

_MODELS: Dict[str, Callable] = {}


def register_model(fn: Callable) -> Callable:
    _MODELS[fn.__name__] = fn
    return fn


def is_model(name: str) -> bool:
    return name in _MODELS


def list_models(pattern: str = "") -> List[str]:
    return sorted(n for n in _MODELS if pattern in n)


def create_model(name: str, pretrained: bool = False, **kwargs):
    if name not in _MODELS:
        raise RuntimeError(f"Unknown model ({name})")
    return _MODELS[name](pretrained=pretrained, **kwargs)
