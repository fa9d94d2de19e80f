"""Complex-phase quantized distilled DeiT (RPFQ-ViT-main/quant_models/quant_rpfq_deit.py)."""
from __future__ import annotations

from typing import Dict

import torch.nn as nn

from ._swap import QuantSwapMixin
from .quant_i import SUPPORTED_QUANT_METHODS, QATLinearComplexPhase
from .registry import register_model
from .vision_transformer import VisionTransformerDistilled


def _validate_quant_method(method: str) -> None:
    if method not in SUPPORTED_QUANT_METHODS:
        raise ValueError(f"Unsupported DeiT complex quantization method: {method}. "
                         f"Allowed methods: {SUPPORTED_QUANT_METHODS}")


class ComplexDeiT(QuantSwapMixin, VisionTransformerDistilled):
    """Distilled DeiT with every Linear (incl. head and head_dist) quantized
    (quant_rpfq_deit.py:26-104)."""

    def __init__(self, *args, quant_method: str = "complex_phase_v1", quant_method_u: str | None = None,
                 quant_method_w: str | None = None, enable_act_quant: bool = True, act_num_bits: int = 4,
                 enable_rotation: bool = False, quant_group_size: int = 32, **kwargs):
        for key in ("pretrained_cfg", "pretrained_cfg_overlay", "cache_dir"):
            kwargs.pop(key, None)
        super().__init__(*args, **kwargs)
        self.quant_method_u = quant_method if quant_method_u is None else quant_method_u
        self.quant_method_w = quant_method if quant_method_w is None else quant_method_w
        _validate_quant_method(self.quant_method_u)
        _validate_quant_method(self.quant_method_w)
        self.enable_rotation = enable_rotation
        self.quant_group_size = quant_group_size
        self.enable_act_quant = enable_act_quant
        self.act_num_bits = act_num_bits
        self.target_linear = QATLinearComplexPhase
        self._announce()
        self._replace_quant_layers()


def _resolve_quant_kwargs(kwargs: dict) -> dict:
    """quant_rpfq_deit.py:107-123: rotation defaults to False."""
    return {
        "quant_method": kwargs.pop("quant_method", "complex_phase_v1"),
        "quant_method_u": kwargs.pop("quant_method_u", None),
        "quant_method_w": kwargs.pop("quant_method_w", None),
        "enable_act_quant": kwargs.pop("enable_act_quant", True),
        "act_num_bits": kwargs.pop("act_num_bits", 4),
        "enable_rotation": kwargs.pop("enable_rotation", False),
        "quant_group_size": kwargs.pop("quant_group_size", 32),
    }


def _build_rpfq_deit_model(*, model_cfg: Dict[str, int], pretrained: bool = False, **kwargs):
    quant_kwargs = _resolve_quant_kwargs(kwargs)
    return ComplexDeiT(qkv_bias=True, norm_layer=nn.LayerNorm, **model_cfg, **quant_kwargs, **kwargs)


def _deit(name, embed_dim, depth, num_heads):
    def fn(pretrained: bool = False, **kwargs):
        return _build_rpfq_deit_model(pretrained=pretrained, model_cfg={
            "patch_size": 16, "embed_dim": embed_dim, "depth": depth, "num_heads": num_heads, "mlp_ratio": 4},
            **kwargs)
    fn.__name__ = name
    fn.__doc__ = f"Complex-phase quantized {name} (quant_rpfq_deit.py:145-190)."
    return register_model(fn)


rpfq_deit_tiny_patch16_224_q = _deit("rpfq_deit_tiny_patch16_224_q", 192, 12, 3)
rpfq_deit_small_patch16_224_q = _deit("rpfq_deit_small_patch16_224_q", 384, 12, 6)
rpfq_deit_base_patch16_224_q = _deit("rpfq_deit_base_patch16_224_q", 768, 12, 12)
