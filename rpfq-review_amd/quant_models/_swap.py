"""The reference's plugin hook: replace nn.Linear children by `target_linear`.

Shared by the three adapters (quant_rpfq_vit.py:75-128, quant_rpfq_deit.py:
65-104, quant_rpfq_swin.py:64-103 of RPFQ-ViT-main/quant_models).
"""
from __future__ import annotations

import torch.nn as nn


class QuantSwapMixin:
    """Adds _create_quant_layer / _replace_quant_layers to a backbone that
    sets target_linear and the quantization attributes."""

    attention_only_qkv_proj = False

    def _create_quant_layer(self, original_layer: nn.Linear) -> nn.Module:
        if original_layer.in_features % 2 or original_layer.out_features % 2:
            print(f"Warning: keep FP layer ({original_layer.in_features}, {original_layer.out_features}) "
                  f"because complex-phase quant requires even dimensions.")
            return original_layer
        layer = self.target_linear(
            in_features=original_layer.in_features,
            out_features=original_layer.out_features,
            bias=original_layer.bias is not None,
            quant_method_u=self.quant_method_u,
            quant_method_w=self.quant_method_w,
            enable_act_quant=self.enable_act_quant,
            act_num_bits=self.act_num_bits,
            enable_rotation=self.enable_rotation,
            quant_group_size=self.quant_group_size,
        )
        layer.weight.data.copy_(original_layer.weight.data)
        if original_layer.bias is not None and layer.bias is not None:
            layer.bias.data.copy_(original_layer.bias.data)
        return layer

    def _replace_quant_layers(self) -> None:
        edges = []
        for parent in self.modules():
            for name, child in parent.named_children():
                if isinstance(child, nn.Linear) and not isinstance(child, self.target_linear):
                    edges.append((parent, name, child))
        for parent, name, child in edges:
            if self.attention_only_qkv_proj and "Attention" in type(parent).__name__ and name not in {"qkv", "proj"}:
                continue
            new = self._create_quant_layer(child)
            if new is not child:
                setattr(parent, name, new)

    def _announce(self) -> None:
        print(f"Using Quant Method - U: {self.quant_method_u}, W: {self.quant_method_w} | "
              f"Act Quant: {self.enable_act_quant} ({self.act_num_bits}-bit) | "
              f"LGPR Rotation: {self.enable_rotation}")
