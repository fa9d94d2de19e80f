"""Complex-phase quantized Swin (RPFQ-ViT-main/quant_models/quant_rpfq_swin.py)."""
from __future__ import annotations

from typing import Dict

from ._swap import QuantSwapMixin
from .quant_i import SUPPORTED_QUANT_METHODS, QATLinearComplexPhase
from .quant_rpfq_deit import _resolve_quant_kwargs
from .registry import register_model
from .swin_transformer import SwinTransformer


def _validate_quant_method(method: str) -> None:
    if method not in SUPPORTED_QUANT_METHODS:
        raise ValueError(f"Unsupported Swin complex quantization method: {method}. "
                         f"Allowed methods: {SUPPORTED_QUANT_METHODS}")


class ComplexSwinTransformer(QuantSwapMixin, SwinTransformer):
    """Swin with every Linear quantized, PatchMerging.reduction included
    (quant_rpfq_swin.py:25-103)."""

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


def _build_rpfq_swin_model(*, model_cfg: Dict, pretrained: bool = False, **kwargs):
    quant_kwargs = _resolve_quant_kwargs(kwargs)
    return ComplexSwinTransformer(**model_cfg, **quant_kwargs, **kwargs)


def _swin(name, embed_dim, depths, num_heads):
    def fn(pretrained: bool = False, **kwargs):
        return _build_rpfq_swin_model(pretrained=pretrained, model_cfg={
            "patch_size": 4, "window_size": 7, "embed_dim": embed_dim, "depths": depths, "num_heads": num_heads},
            **kwargs)
    fn.__name__ = name
    fn.__doc__ = f"Complex-phase quantized {name} (quant_rpfq_swin.py:142-187)."
    return register_model(fn)


rpfq_swin_base_patch4_window7_224_q = _swin("rpfq_swin_base_patch4_window7_224_q", 128, (2, 2, 18, 2),
                                            (4, 8, 16, 32))
rpfq_swin_small_patch4_window7_224_q = _swin("rpfq_swin_small_patch4_window7_224_q", 96, (2, 2, 18, 2),
                                             (3, 6, 12, 24))
rpfq_swin_tiny_patch4_window7_224_q = _swin("rpfq_swin_tiny_patch4_window7_224_q", 96, (2, 2, 6, 2),
                                            (3, 6, 12, 24))
