"""ViT and distilled-DeiT backbones with timm's module layout.

The reference builds on timm's VisionTransformer / VisionTransformerDistilled
(RPFQ-ViT-main/quant_models/quant_rpfq_vit.py:8, quant_rpfq_deit.py:8).  timm
is unavailable offline, so these backbones are written here with the same
submodule names (patch_embed.proj, cls_token, pos_embed, blocks.i.norm1,
attn.qkv, attn.proj, norm2, mlp.fc1, mlp.fc2, norm, head[, dist_token,
head_dist]) so the reference's checkpoints load by state-dict key, and with
the forward semantics the reference's parity audit spells out
(RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:518-558):
norm1 -> qkv -> SDPA -> proj -> +res -> norm2 -> fc1 -> GELU(erf) -> fc2 -> +res.
"""
from __future__ import annotations

import os

import torch
import torch.nn as nn
import torch.nn.functional as F

from .quant_i import records_grad

# Eval-mode device forward of a block uses the fused kernels: LayerNorm on the
# HIP kernel and the residual add after attn.proj / mlp.fc2 fused into the
# packed layer's store.  RPFQ_FUSED=0 keeps the module-by-module forward.
FUSED_BLOCKS = os.environ.get("RPFQ_FUSED", "1") != "0"
# Within the fused path, a LayerNorm feeding a packed layer with activation
# quantization also applies that quantization (rpfq_layer_norm_act_quant).
FUSE_ACT_QUANT = os.environ.get("RPFQ_FUSE_AQ", "1") != "0"
# Within the fused path, the MLP's exact GELU runs in fc1's store when fc1 is
# a packed phase-quantized Linear (rpfq_wide_linear with RPFQ_FLAG_GELU).
FUSE_GELU = os.environ.get("RPFQ_FUSE_GELU", "1") != "0"
# Within the fused path, fc1 -> GELU -> fc2 (+ the residual) as one launch
# with the hidden activations on chip (ops.wide_mlp) where both layers are
# packed and the shapes fit it (DeiT-Ti, Swin-T stage 1: K' = 96).
FUSE_MLP = os.environ.get("RPFQ_FUSE_MLP", "1") != "0"
# LayerNorm in the following packed layer's launch (norm1 -> qkv, norm2 ->
# fc1) where that layer streams: a block at batch 1-2.  RPFQ_FUSE_LN=0 keeps
# the LayerNorm kernel.
FUSE_LN = os.environ.get("RPFQ_FUSE_LN", "1") != "0"


def _fused(module: nn.Module, x: torch.Tensor) -> bool:
    """Whether the fused inference kernels run: eval-mode device tensors that
    autograd does not record (records_grad: grad mode on and x or a
    parameter of the module requiring a gradient).  Under autograd the blocks
    run module by module: torch's LayerNorm and GELU, and each packed layer
    either the reference formulation (weights requiring gradients) or the
    packed kernels with the input gradient on the device (frozen weights).
    Inference therefore runs under torch.no_grad() / torch.inference_mode(),
    as the reference's validation loop does, or on frozen parameters."""
    return FUSED_BLOCKS and x.is_cuda and not module.training and not records_grad(module, x)


def norm_fwd(norm: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """norm(x), on the device LayerNorm kernel for eval-mode device tensors
    (float32 copies of the affine parameters are cached on the module)."""
    if not (_fused(norm, x) and type(norm) is nn.LayerNorm and norm.normalized_shape[-1] % 8 == 0
            and len(norm.normalized_shape) == 1 and norm.normalized_shape[0] <= 4096):
        return norm(x)
    from . import ops

    w, b = _ln_params(norm)
    return ops.layer_norm(x, w, b, norm.eps)


def _ln_params(norm: nn.LayerNorm):
    """float32 copies of the affine parameters, cached on the module."""
    key = tuple((t.data_ptr(), t._version) if t is not None else None for t in (norm.weight, norm.bias))
    cache = getattr(norm, "_rpfq_f32", None)
    if cache is None or cache[0] != key:
        cache = (key, None if norm.weight is None else norm.weight.detach().float().contiguous(),
                 None if norm.bias is None else norm.bias.detach().float().contiguous())
        norm._rpfq_f32 = cache
    return cache[1], cache[2]


def norm_quant_fwd(norm: nn.Module, x: torch.Tensor, layer: nn.Module):
    """(h, prequantized): h = norm(x), with `layer`'s activation fake
    quantization applied in the same device kernel when layer is a packed
    phase-quantized Linear that quantizes its input; prequantized tells the
    caller to run layer.forward_prequantized(h) instead of layer(h)."""
    bits_of = getattr(layer, "packed_act_bits", None)
    bits = bits_of(x) if bits_of is not None else 0
    c = x.shape[-1]
    if not (bits and FUSE_ACT_QUANT and _fused(norm, x) and type(norm) is nn.LayerNorm and c % 16 == 0
            and c <= 4096 and len(norm.normalized_shape) == 1):
        return norm_fwd(norm, x), False
    from . import ops

    w, b = _ln_params(norm)
    return ops.layer_norm(x, w, b, norm.eps, act_bits=bits), True


def norm_layer_fwd(norm: nn.Module, x: torch.Tensor, layer: nn.Module, gelu: bool = False):
    """layer(norm(x)) (GELU'd if gelu) in one packed-layer launch with the
    LayerNorm in its prologue, or None where that does not apply (the
    caller then runs norm and layer separately)."""
    fwd = getattr(layer, "forward_layer_norm", None)
    if not (FUSE_LN and fwd is not None and _fused(norm, x) and type(norm) is nn.LayerNorm
            and len(norm.normalized_shape) == 1):
        return None
    w, b = _ln_params(norm)
    return fwd(x, w, b, norm.eps, gelu)


def call_layer(layer: nn.Module, h: torch.Tensor, prequantized: bool) -> torch.Tensor:
    return layer.forward_prequantized(h) if prequantized else layer(h)


def linear_residual(layer: nn.Module, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """residual + layer(x), with the add fused into the packed layer's store
    when the layer is a phase-quantized Linear on its HIP path."""
    fwd = getattr(layer, "forward_residual", None)
    if fwd is not None:
        return fwd(x, residual)
    return residual + layer(x)


def _trunc_normal_(t: torch.Tensor, std: float = 0.02) -> torch.Tensor:
    with torch.no_grad():
        return nn.init.trunc_normal_(t, std=std, a=-2 * std, b=2 * std)


class PatchEmbed(nn.Module):
    def __init__(self, img_size=224, patch_size=16, in_chans=3, embed_dim=768, norm_layer=None, flatten=True):
        super().__init__()
        self.img_size = (img_size, img_size)
        self.patch_size = (patch_size, patch_size)
        self.grid_size = (img_size // patch_size, img_size // patch_size)
        self.num_patches = self.grid_size[0] * self.grid_size[1]
        self.flatten = flatten
        self.proj = nn.Conv2d(in_chans, embed_dim, kernel_size=patch_size, stride=patch_size)
        self.norm = norm_layer(embed_dim) if norm_layer else nn.Identity()

    def forward(self, x):
        # stride == kernel: patchify is an exact reshape, then one GEMM with
        # the conv weight viewed as [C_out, C_in*p*p] (same result as the
        # Conv2d, without depending on the convolution library's kernel pick)
        b, c, h, w = x.shape
        p = self.patch_size[0]
        gh, gw = h // p, w // p
        patches = x.reshape(b, c, gh, p, gw, p).permute(0, 2, 4, 1, 3, 5).reshape(b, gh * gw, c * p * p)
        weight = self.proj.weight.reshape(self.proj.out_channels, -1)
        x = F.linear(patches, weight.to(patches.dtype),
                     None if self.proj.bias is None else self.proj.bias.to(patches.dtype))
        if not self.flatten:
            x = x.reshape(b, gh, gw, -1)  # B, H, W, C
        # Swin's patch norm (C = 96 over 401,408 rows at bs128) on the device
        # row kernel: torch's took 407 us a forward there
        return norm_fwd(self.norm, x)


class Mlp(nn.Module):
    def __init__(self, in_features, hidden_features, act_layer=nn.GELU, drop=0.0):
        super().__init__()
        self.fc1 = nn.Linear(in_features, hidden_features)
        self.act = act_layer()
        self.drop1 = nn.Dropout(drop)
        self.norm = nn.Identity()
        self.fc2 = nn.Linear(hidden_features, in_features)
        self.drop2 = nn.Dropout(drop)

    def forward(self, x):
        return self.drop2(self.fc2(self.norm(self.drop1(self.act(self.fc1(x))))))

    def forward_residual(self, x, residual, prequantized: bool = False):
        """residual + self(x) with the add fused into fc2 and an exact GELU
        into fc1's store when fc1 is a phase-quantized Linear (eval mode); x
        already activation-quantized for fc1 if prequantized.  When fc2
        quantizes its input, the GELU and that quantization run as one pass
        over fc1's output instead (rpfq_gelu_act_quant, float32 GELU
        quantized without rounding in between).  Where both layers are packed
        and fit rpfq_wide_mlp, the whole MLP and the add are one launch."""
        if not prequantized:
            y = self._wide_mlp(x, residual)
            if y is not None:
                return y
        gelu_exact = type(self.act) is nn.GELU and self.act.approximate == "none"
        bits = self._gelu_act_quant_bits(x)
        if bits:
            from . import ops

            h = ops.gelu_act_quant(call_layer(self.fc1, x, prequantized), bits)
            return self.fc2.forward_residual(h, residual, prequantized=True)
        fc1_gelu = getattr(self.fc1, "forward_gelu", None)
        if FUSE_GELU and fc1_gelu is not None and gelu_exact:
            h = fc1_gelu(x, prequantized)
        else:
            h = self.act(call_layer(self.fc1, x, prequantized))
        return self.forward_hidden_residual(h, residual)

    def _wide_mlp(self, x, residual, norm=None):
        """residual + fc2(GELU(fc1(x))) -- with norm: x + fc2(GELU(fc1(
        norm(x)))) -- as one packed launch (ops.wide_mlp /
        ops.layer_norm_wide_mlp: the LayerNorm in its prologue, the hidden
        activations on chip, the GELU as in the packed stores, within 1 ulp
        of the exact GELU), or None where that does not apply: fusion off,
        another activation or norm, no packed inference path on either layer
        (training, autograd, activation quantization), or shapes the kernel
        does not take."""
        if not (FUSE_MLP and FUSE_GELU and type(self.act) is nn.GELU and self.act.approximate == "none"
                and type(self.norm) is nn.Identity and x.dtype == torch.float16 and x.is_cuda):
            return None
        if norm is not None and not (FUSE_LN and type(norm) is nn.LayerNorm and len(norm.normalized_shape) == 1
                                     and norm.normalized_shape[0] == x.shape[-1] and residual is x):
            return None
        inf1 = getattr(self.fc1, "packed_inference", None)
        inf2 = getattr(self.fc2, "packed_inference", None)
        if inf1 is None or inf2 is None:
            return None
        p1, p2 = inf1(x), inf2(x)
        if p1 is None or p2 is None:
            return None
        from . import ops

        m = x.numel() // x.shape[-1]
        if not ops.mlp_fusable(p1, p2, m, x.dtype):
            return None
        if norm is not None and p1.ln_fusable(m, x.dtype):
            return None  # few rows: norm -> fc1 in fc1's streaming launch (forward_norm_residual) instead
        b1 = None if self.fc1.bias is None else self.fc1.bias.detach()
        b2 = None if self.fc2.bias is None else self.fc2.bias.detach()
        if norm is not None:
            w, b = _ln_params(norm)
            return ops.layer_norm_wide_mlp(p1, p2, x, w, b, norm.eps, b1, b2)
        return ops.wide_mlp(p1, p2, x, b1, b2, residual)

    def _gelu_act_quant_bits(self, x) -> int:
        """Bits of fc2's activation quantization when the exact GELU and that
        quantization run as one pass over fc1's output (rpfq_gelu_act_quant,
        bit-exact with torch's GELU followed by the act quant), else 0."""
        gelu_exact = type(self.act) is nn.GELU and self.act.approximate == "none"
        if not (FUSE_GELU and FUSE_ACT_QUANT and gelu_exact and type(self.norm) is nn.Identity):
            return 0
        bits_of = getattr(self.fc2, "packed_act_bits", None)
        bits = bits_of(x) if bits_of is not None else 0
        c = self.fc2.in_features
        return bits if bits and c % 16 == 0 and c <= 4096 else 0

    def forward_hidden_residual(self, h, residual):
        """residual + fc2(h) for h = act(fc1(x)) already computed."""
        return linear_residual(self.fc2, self.norm(self.drop1(h)), residual)

    def forward_norm_residual(self, norm, x):
        """x + self(norm(x)) with norm (and fc1's act quant) fused into fc1's
        launch and the GELU into its store -- or, when fc2 quantizes its
        input, the GELU and that act quant in one pass after fc1 -- or None
        where that does not apply.  Where both layers are packed and fit
        rpfq_layer_norm_wide_mlp, the norm, the whole MLP and the add are one
        launch."""
        y = self._wide_mlp(x, x, norm)
        if y is not None:
            return y
        bits = self._gelu_act_quant_bits(x)
        if bits:
            h = norm_layer_fwd(norm, x, self.fc1, False)
            if h is None:
                return None
            from . import ops

            return self.fc2.forward_residual(ops.gelu_act_quant(h, bits), x, prequantized=True)
        gelu = FUSE_GELU and type(self.act) is nn.GELU and self.act.approximate == "none"
        h = norm_layer_fwd(norm, x, self.fc1, gelu)
        if h is None:
            return None
        return self.forward_hidden_residual(h if gelu else self.act(h), x)


class Attention(nn.Module):
    def __init__(self, dim, num_heads=8, qkv_bias=False, attn_drop=0.0, proj_drop=0.0):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.q_norm = nn.Identity()
        self.k_norm = nn.Identity()
        self.attn_drop = nn.Dropout(attn_drop)
        self.proj = nn.Linear(dim, dim)
        self.proj_drop = nn.Dropout(proj_drop)

    def _mix(self, x, prequantized: bool = False):
        return self._attend(call_layer(self.qkv, x, prequantized))

    def _attend(self, qkv):
        b, n, c3 = qkv.shape
        c = c3 // 3
        qkv = qkv.reshape(b, n, 3, self.num_heads, self.head_dim)
        qkv = qkv.permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        x = F.scaled_dot_product_attention(q, k, v, dropout_p=self.attn_drop.p if self.training else 0.0)
        return x.transpose(1, 2).reshape(b, n, c)

    def forward(self, x):
        return self.proj_drop(self.proj(self._mix(x)))

    def forward_residual(self, x, residual, prequantized: bool = False):
        """residual + self(x) with the add fused into proj (eval mode); x
        already activation-quantized for qkv if prequantized."""
        return linear_residual(self.proj, self._mix(x, prequantized), residual)

    def forward_norm_residual(self, norm, x):
        """x + self(norm(x)) with norm fused into qkv's launch, or None where
        that does not apply."""
        qkv = norm_layer_fwd(norm, x, self.qkv)
        if qkv is None:
            return None
        return linear_residual(self.proj, self._attend(qkv), x)


class Block(nn.Module):
    def __init__(self, dim, num_heads, mlp_ratio=4.0, qkv_bias=False, norm_layer=nn.LayerNorm, drop=0.0,
                 attn_drop=0.0):
        super().__init__()
        self.norm1 = norm_layer(dim)
        self.attn = Attention(dim, num_heads=num_heads, qkv_bias=qkv_bias, attn_drop=attn_drop, proj_drop=drop)
        self.ls1 = nn.Identity()
        self.norm2 = norm_layer(dim)
        self.mlp = Mlp(dim, int(dim * mlp_ratio), drop=drop)
        self.ls2 = nn.Identity()

    def forward(self, x):
        if _fused(self, x) and isinstance(self.ls1, nn.Identity) and isinstance(self.ls2, nn.Identity):
            # audit_rpfq_vit_ios_parity.py:520-556 with the residual adds in
            # the proj / fc2 stores and LayerNorm on the device kernel
            y = self.attn.forward_norm_residual(self.norm1, x)
            if y is None:
                h, q = norm_quant_fwd(self.norm1, x, self.attn.qkv)
                y = self.attn.forward_residual(h, x, q)
            x = y
            y = self.mlp.forward_norm_residual(self.norm2, x)
            if y is None:
                h, q = norm_quant_fwd(self.norm2, x, self.mlp.fc1)
                y = self.mlp.forward_residual(h, x, q)
            return y
        x = x + self.ls1(self.attn(self.norm1(x)))
        x = x + self.ls2(self.mlp(self.norm2(x)))
        return x


class VisionTransformer(nn.Module):
    """Class-token ViT (timm VisionTransformer, global_pool='token')."""

    num_prefix_tokens = 1

    def __init__(self, img_size=224, patch_size=16, in_chans=3, num_classes=1000, embed_dim=768, depth=12,
                 num_heads=12, mlp_ratio=4.0, qkv_bias=True, norm_layer=None, drop_rate=0.0,
                 attn_drop_rate=0.0, drop_path_rate=0.0, **kwargs):
        super().__init__()
        norm_layer = norm_layer or (lambda d: nn.LayerNorm(d, eps=1e-6))
        self.num_classes = num_classes
        self.num_features = self.embed_dim = embed_dim
        self.patch_embed = PatchEmbed(img_size, patch_size, in_chans, embed_dim)
        num_patches = self.patch_embed.num_patches
        self.cls_token = nn.Parameter(torch.zeros(1, 1, embed_dim))
        self._init_extra_tokens(embed_dim)
        self.pos_embed = nn.Parameter(torch.zeros(1, num_patches + self.num_prefix_tokens, embed_dim))
        self.pos_drop = nn.Dropout(drop_rate)
        self.norm_pre = nn.Identity()
        self.blocks = nn.Sequential(*[
            Block(embed_dim, num_heads, mlp_ratio, qkv_bias, norm_layer, drop_rate, attn_drop_rate)
            for _ in range(depth)])
        self.norm = norm_layer(embed_dim)
        self.fc_norm = nn.Identity()
        self.head_drop = nn.Dropout(drop_rate)
        self.head = nn.Linear(embed_dim, num_classes) if num_classes > 0 else nn.Identity()
        self._init_extra_heads(embed_dim, num_classes)
        self._init_weights()

    def _init_extra_tokens(self, embed_dim):
        pass

    def _init_extra_heads(self, embed_dim, num_classes):
        pass

    def _init_weights(self):
        _trunc_normal_(self.pos_embed, 0.02)
        nn.init.normal_(self.cls_token, std=1e-6)
        for m in self.modules():
            if isinstance(m, nn.Linear):
                _trunc_normal_(m.weight, 0.02)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
            elif isinstance(m, nn.LayerNorm):
                nn.init.ones_(m.weight)
                nn.init.zeros_(m.bias)

    def _prefix_tokens(self, x):
        return self.cls_token.expand(x.shape[0], -1, -1).to(x.dtype)

    def forward_features(self, x):
        x = self.patch_embed(x)
        pre, pos = self._prefix_tokens(x), self.pos_embed.to(x.dtype)
        if torch.is_grad_enabled() and (x.requires_grad or pre.requires_grad or pos.requires_grad):
            x = torch.cat((pre, x), dim=1) + pos
        else:
            # prefix and patch tokens written with their position embedding
            # into one buffer: one pass instead of torch.cat and then the add
            # (the same elementwise sums)
            n = pre.shape[1]
            out = x.new_empty((x.shape[0], n + x.shape[1], x.shape[2]))
            torch.add(pre, pos[:, :n], out=out[:, :n])
            torch.add(x, pos[:, n:], out=out[:, n:])
            x = out
        x = self.norm_pre(self.pos_drop(x))
        x = self.blocks(x)
        return norm_fwd(self.norm, x)

    def forward_head(self, x, pre_logits: bool = False):
        x = self.head_drop(self.fc_norm(x[:, 0]))
        return x if pre_logits else self.head(x)

    def forward(self, x):
        return self.forward_head(self.forward_features(x))


class VisionTransformerDistilled(VisionTransformer):
    """DeiT with class and distillation tokens and two heads (timm
    VisionTransformerDistilled): eval output is the mean of both heads."""

    num_prefix_tokens = 2

    def _init_extra_tokens(self, embed_dim):
        self.dist_token = nn.Parameter(torch.zeros(1, 1, embed_dim))
        self.distilled_training = False

    def _init_extra_heads(self, embed_dim, num_classes):
        self.head_dist = nn.Linear(embed_dim, num_classes) if num_classes > 0 else nn.Identity()

    def _init_weights(self):
        super()._init_weights()
        _trunc_normal_(self.dist_token, 0.02)

    def _prefix_tokens(self, x):
        b = x.shape[0]
        return torch.cat((self.cls_token.expand(b, -1, -1), self.dist_token.expand(b, -1, -1)), dim=1).to(x.dtype)

    def forward_head(self, x, pre_logits: bool = False):
        x, x_dist = x[:, 0], x[:, 1]
        if pre_logits:
            return (x + x_dist) / 2
        x = self.head(x)
        x_dist = self.head_dist(x_dist)
        if self.distilled_training and self.training:
            return x, x_dist
        return (x + x_dist) / 2


def num_tokens(img_size: int, patch_size: int, prefix: int) -> int:
    return (img_size // patch_size) ** 2 + prefix


__all__ = ["VisionTransformer", "VisionTransformerDistilled", "PatchEmbed", "Attention", "Block", "Mlp",
           "num_tokens"]
