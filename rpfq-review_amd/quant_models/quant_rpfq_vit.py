"""Complex-phase quantized ViT (RPFQ-ViT-main/quant_models/quant_rpfq_vit.py)."""
from __future__ import annotations

from typing import Dict

import torch.nn as nn

from ._swap import QuantSwapMixin
from .quant_i import SUPPORTED_QUANT_METHODS, QATLinearComplexPhase
from .registry import register_model
from .vision_transformer import VisionTransformer


class ComplexVisionTransformer(QuantSwapMixin, VisionTransformer):
    """ViT whose Linear layers (attention qkv/proj, MLP, head) are
    QATLinearComplexPhase (quant_rpfq_vit.py:21-128)."""

    attention_only_qkv_proj = True

    def __init__(self, *args, quant_method_u: str = "complex_phase_v1", quant_method_w: str = "complex_phase_v1",
                 enable_act_quant: bool = True, act_num_bits: int = 4, enable_rotation: bool = True,
                 quant_group_size: int = 32, **kwargs):
        for key in ("pretrained_cfg", "pretrained_cfg_overlay", "cache_dir"):
            kwargs.pop(key, None)
        super().__init__(*args, **kwargs)
        self.quant_method_u = quant_method_u
        self.quant_method_w = quant_method_w
        self.enable_act_quant = enable_act_quant
        self.act_num_bits = act_num_bits
        self.enable_rotation = enable_rotation
        self.quant_group_size = quant_group_size
        self.target_linear = QATLinearComplexPhase
        if quant_method_u not in SUPPORTED_QUANT_METHODS or quant_method_w not in SUPPORTED_QUANT_METHODS:
            print(f"Warning: non-standard quant methods: U={quant_method_u}, W={quant_method_w}. "
                  f"Supported: {SUPPORTED_QUANT_METHODS}")
        self._announce()
        self._replace_quant_layers()


def _build_rpfq_vit_model(*, model_cfg: Dict[str, int], pretrained: bool = False, **kwargs):
    """Builder with the reference's kwargs handling (quant_rpfq_vit.py:131-177):
    legacy quant_bits/quant_scheme are ignored, quant_method sets both U and W,
    rotation defaults to True, act quant to 4 bits."""
    kwargs.pop("quant_bits", None)
    kwargs.pop("quant_scheme", None)
    method_u = kwargs.pop("quant_method_u", "complex_phase_v1")
    method_w = kwargs.pop("quant_method_w", "complex_phase_v1")
    if "quant_method" in kwargs:
        method_u = method_w = kwargs.pop("quant_method")
    model = ComplexVisionTransformer(
        qkv_bias=True, norm_layer=nn.LayerNorm, quant_method_u=method_u, quant_method_w=method_w,
        enable_act_quant=kwargs.pop("enable_act_quant", True), act_num_bits=kwargs.pop("act_num_bits", 4),
        enable_rotation=kwargs.pop("enable_rotation", True), quant_group_size=kwargs.pop("quant_group_size", 32),
        **model_cfg, **kwargs)
    return model


def _vit(name, embed_dim, depth, num_heads):
    def fn(pretrained: bool = False, **kwargs):
        return _build_rpfq_vit_model(pretrained=pretrained, model_cfg={
            "patch_size": 16, "embed_dim": embed_dim, "depth": depth, "num_heads": num_heads, "mlp_ratio": 4},
            **kwargs)
    fn.__name__ = name
    fn.__doc__ = f"Complex-phase quantized {name} (quant_rpfq_vit.py:180-241)."
    return register_model(fn)


rpfq_vit_tiny_patch16_224_q = _vit("rpfq_vit_tiny_patch16_224_q", 192, 12, 3)
rpfq_vit_small_patch16_224_q = _vit("rpfq_vit_small_patch16_224_q", 384, 12, 6)
rpfq_vit_base_patch16_224_q = _vit("rpfq_vit_base_patch16_224_q", 768, 12, 12)
rpfq_vit_large_patch16_224_q = _vit("rpfq_vit_large_patch16_224_q", 1024, 24, 16)
