"""Reader of the reference's exported model bundle (``model.safetensors`` +
``config.json``) into the MI355X packed layout.

The bundle is what RPFQ-ViTApple/scripts/export_rpfq_vit_to_mlx.py writes and
what the Android and Apple runtimes load
(RPFQ-ViTAndroid/app/src/main/cpp/bundle_loader.cpp:20-66,
ops/phase_linear.cpp:45-117):

* per quantized linear ``{prefix}.{u,w}_s{i}.codes`` -- uint8
  [out_complex_padded, in_complex_padded / 4], four 2-bit axis codes per byte,
  low bits first (export…py:148-159, :384-423); padding rows and columns hold
  code 0;
* ``{prefix}.{u,w}_s{i}.gamma_real`` / ``gamma_imag`` -- fp16
  [out_complex_padded, in_complex_padded / 256], value = code / gamma
  (export…py:189-254);
* ``{prefix}.bias`` -- fp16 [out_features];
* dense fp16 tensors for the patch embedding, tokens, norms and the head
  (whose weight is already the quantized forward weight, export…py:553);
* ``config.json``: dims, padded dims, ``residual_stages``, ``block_size``,
  ``layer_norm_eps`` (export…py:560-606).

Quantized linears go through rpfq_wide_pack into the tiled layout with the
exporter's 256-column gamma blocks and 1/gamma multipliers (+-1/g == +-(1/g)
exactly in float32, so the decoded weight equals the exporter's dequantized
weight bit for bit); the padding is dropped.  Files are read with
safetensors' loader and json only (nothing in a bundle is executed).
"""
from __future__ import annotations

import functools
import json
import os

import torch
import torch.nn as nn

from . import _native as N
from . import packing as P

BLOCK_SIZE = 256  # export_rpfq_vit_to_mlx.py:26
LINEARS = ("attn.qkv", "attn.proj", "mlp.fc1", "mlp.fc2")  # export…py:510-551


def read_config(bundle_dir: str) -> dict:
    with open(os.path.join(bundle_dir, "config.json"), encoding="utf-8") as f:
        return json.load(f)


def read_tensors(bundle_dir: str) -> dict:
    """Every tensor of the bundle's model.safetensors (host tensors)."""
    from safetensors.torch import load_file

    return load_file(os.path.join(bundle_dir, "model.safetensors"), device="cpu")


def layer_codes(tensors: dict, prefix: str, n_complex: int, k_complex: int, stages: int,
                block: int = BLOCK_SIZE) -> P.LayerCodes:
    """LayerCodes of one exported quantized linear: the stage planes of U and
    W cut to the valid [N', K'/4] bytes, and 1/gamma per (row, 256-column
    block) as the plane multipliers (phase_linear.cpp:45-83 reads the same
    keys and inverts the gammas the same way)."""
    if k_complex % 4:
        raise ValueError(f"in_complex={k_complex} must be a multiple of 4")
    nblk = -(-k_complex // block)
    planes, sre, sim = [], [], []
    for kind in ("u", "w"):
        for s in range(stages):
            key = f"{prefix}.{kind}_s{s}"
            codes = tensors[f"{key}.codes"]
            g_re, g_im = tensors[f"{key}.gamma_real"], tensors[f"{key}.gamma_imag"]
            if codes.dtype != torch.uint8 or g_re.dtype != torch.float16 or g_im.dtype != torch.float16:
                raise TypeError(f"{key}: expected uint8 codes and float16 gammas")
            if codes.shape[0] < n_complex or codes.shape[1] * 4 < k_complex:
                raise ValueError(f"{key}.codes {tuple(codes.shape)} does not cover [{n_complex}, {k_complex}/4]")
            if g_re.shape[0] < n_complex or g_re.shape[1] < nblk or g_im.shape != g_re.shape:
                raise ValueError(f"{key} gammas {tuple(g_re.shape)} do not cover [{n_complex}, {nblk}]")
            planes.append(codes[:n_complex, :k_complex // 4].contiguous())
            sre.append((1.0 / g_re[:n_complex, :nblk].float()).contiguous())
            sim.append((1.0 / g_im[:n_complex, :nblk].float()).contiguous())
    return P.LayerCodes(planes, sre, sim, n_complex, k_complex, N.CB_AXIS, stages,
                        block if nblk > 1 else 0, None)


def load_vit_bundle(bundle_dir: str, device="cuda", dtype: torch.dtype = torch.float16) -> nn.Module:
    """A ready-to-run ComplexVisionTransformer (eval, packed HIP layers,
    `dtype` activations) from an exported RPFQ-ViT bundle; the head is the
    bundle's dense quantized weight (export…py:553)."""
    from .inference import prepare_inference
    from .quant_rpfq_vit import ComplexVisionTransformer

    cfg = read_config(bundle_dir)
    t = read_tensors(bundle_dir)
    rv = cfg.get("rpfq_vit", {})
    stages = int(rv.get("residual_stages", 2))
    block = int(rv.get("block_size", BLOCK_SIZE))
    method = {1: "complex_phase_v1", 2: "complex_phase_v2"}.get(stages)
    if method is None:
        raise ValueError(f"unsupported residual_stages={stages}")
    hidden = int(cfg["hidden_size"])
    inter = int(cfg["intermediate_size"])
    patch = int(cfg.get("patch_size", 16))
    chans = int(cfg.get("num_channels", 3))
    classes = int(cfg["num_classes"])
    eps = float(cfg.get("layer_norm_eps", 1e-5))
    model = ComplexVisionTransformer(
        img_size=int(cfg.get("image_size", 224)), patch_size=patch, in_chans=chans, num_classes=classes,
        embed_dim=hidden, depth=int(cfg["num_hidden_layers"]), num_heads=int(cfg["num_attention_heads"]),
        mlp_ratio=inter / hidden, qkv_bias=True, norm_layer=functools.partial(nn.LayerNorm, eps=eps),
        quant_method_u=method, quant_method_w=method, enable_act_quant=False, enable_rotation=False)
    model.head = nn.Linear(hidden, classes)

    def put(param: torch.Tensor, key: str, shape=None):
        v = t[key].float()
        param.data.copy_(v.reshape(shape or param.shape))

    with torch.no_grad():
        put(model.patch_embed.proj.weight, "model.patch_embed.weight")
        put(model.patch_embed.proj.bias, "model.patch_embed.bias")
        put(model.cls_token, "model.cls_token")
        put(model.pos_embed, "model.pos_embed")
        for i, blk in enumerate(model.blocks):
            pre = f"model.layers.{i}"
            for n in ("norm1", "norm2"):
                put(getattr(blk, n).weight, f"{pre}.{n}.weight")
                put(getattr(blk, n).bias, f"{pre}.{n}.bias")
            for name in LINEARS:
                layer = blk.get_submodule(name)
                lc = layer_codes(t, f"{pre}.{name}", layer.out_features // 2, layer.in_features // 2, stages, block)
                layer.load_packed(lc)
                put(layer.bias, f"{pre}.{name}.bias")
        put(model.norm.weight, "model.norm.weight")
        put(model.norm.bias, "model.norm.bias")
        put(model.head.weight, "head.weight")
        put(model.head.bias, "head.bias")
    return prepare_inference(model, device, dtype)
