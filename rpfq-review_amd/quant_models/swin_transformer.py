"""Swin Transformer backbone with timm's module layout.

The reference quantizes timm's SwinTransformer
(RPFQ-ViT-main/quant_models/quant_rpfq_swin.py:8, :25-103): every Linear
(window-attention qkv/proj, MLP fc1/fc2, PatchMerging.reduction, head.fc)
becomes a QATLinearComplexPhase.  timm is unavailable offline; this backbone
keeps timm's submodule names (patch_embed.proj/norm, layers.i.downsample.
{norm,reduction}, layers.i.blocks.j.{norm1,attn.qkv,attn.proj,
attn.relative_position_bias_table,norm2,mlp.fc1,mlp.fc2}, norm, head.fc) and
its NHWC data layout.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .vision_transformer import Mlp, PatchEmbed, _fused, _trunc_normal_, call_layer, norm_fwd, norm_quant_fwd


def window_partition(x: torch.Tensor, ws: int) -> torch.Tensor:
    """(B, H, W, C) -> (B * nW, ws * ws, C)."""
    b, h, w, c = x.shape
    x = x.view(b, h // ws, ws, w // ws, ws, c).permute(0, 1, 3, 2, 4, 5)
    return x.reshape(-1, ws * ws, c)


def window_reverse(win: torch.Tensor, ws: int, h: int, w: int) -> torch.Tensor:
    c = win.shape[-1]
    x = win.view(-1, h // ws, w // ws, ws, ws, c).permute(0, 1, 3, 2, 4, 5)
    return x.reshape(-1, h, w, c)


def relative_position_index(ws: int) -> torch.Tensor:
    coords = torch.stack(torch.meshgrid(torch.arange(ws), torch.arange(ws), indexing="ij")).flatten(1)
    rel = (coords[:, :, None] - coords[:, None, :]).permute(1, 2, 0)
    rel[:, :, 0] += ws - 1
    rel[:, :, 1] += ws - 1
    rel[:, :, 0] *= 2 * ws - 1
    return rel.sum(-1)


class WindowAttention(nn.Module):
    def __init__(self, dim, num_heads, window_size=7, qkv_bias=True, attn_drop=0.0, proj_drop=0.0):
        super().__init__()
        self.dim = dim
        self.window_size = window_size
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.relative_position_bias_table = nn.Parameter(torch.zeros((2 * window_size - 1) ** 2, num_heads))
        self.register_buffer("relative_position_index", relative_position_index(window_size), persistent=False)
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.attn_drop = nn.Dropout(attn_drop)
        self.proj = nn.Linear(dim, dim)
        self.proj_drop = nn.Dropout(proj_drop)
        _trunc_normal_(self.relative_position_bias_table, 0.02)

    def _rel_bias(self) -> torch.Tensor:
        n = self.window_size * self.window_size
        bias = self.relative_position_bias_table[self.relative_position_index.view(-1)].view(n, n, -1)
        return bias.permute(2, 0, 1).contiguous().unsqueeze(0)  # 1, heads, N, N

    def forward(self, x, mask=None, prequantized: bool = False):
        bw, n, c = x.shape
        qkv = call_layer(self.qkv, x, prequantized).reshape(bw, n, 3, self.num_heads, self.head_dim)
        qkv = qkv.permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        bias = self._rel_bias().to(q.dtype)
        if mask is not None:
            nw = mask.shape[0]
            bias = (bias + mask.unsqueeze(1).to(q.dtype)).repeat(bw // nw, 1, 1, 1)
        x = F.scaled_dot_product_attention(q, k, v, attn_mask=bias,
                                           dropout_p=self.attn_drop.p if self.training else 0.0)
        x = x.transpose(1, 2).reshape(bw, n, c)
        return self.proj_drop(self.proj(x))


class SwinTransformerBlock(nn.Module):
    def __init__(self, dim, input_resolution, num_heads, window_size=7, shift_size=0, mlp_ratio=4.0,
                 qkv_bias=True, norm_layer=nn.LayerNorm):
        super().__init__()
        self.dim = dim
        self.input_resolution = input_resolution
        h, w = input_resolution
        if min(h, w) <= window_size:
            window_size, shift_size = min(h, w), 0
        self.window_size = window_size
        self.shift_size = shift_size
        self.norm1 = norm_layer(dim)
        self.attn = WindowAttention(dim, num_heads, window_size, qkv_bias)
        self.norm2 = norm_layer(dim)
        self.mlp = Mlp(dim, int(dim * mlp_ratio))
        ws = self.window_size
        self.padded = ((h + ws - 1) // ws * ws, (w + ws - 1) // ws * ws)
        self.register_buffer("attn_mask", self._mask(*self.padded), persistent=False)

    def _mask(self, h, w):
        if self.shift_size == 0:
            return None
        img = torch.zeros(1, h, w, 1)
        cnt = 0
        ws, ss = self.window_size, self.shift_size
        for hs in (slice(0, -ws), slice(-ws, -ss), slice(-ss, None)):
            for wsl in (slice(0, -ws), slice(-ws, -ss), slice(-ss, None)):
                img[:, hs, wsl, :] = cnt
                cnt += 1
        win = window_partition(img, ws).squeeze(-1)
        mask = win.unsqueeze(1) - win.unsqueeze(2)
        return mask.masked_fill(mask != 0, float(-100.0)).masked_fill(mask == 0, 0.0)

    def _attn(self, x, prequantized: bool = False):
        """Shifted-window attention of normalised tokens x; prequantized: x
        already carries qkv's activation quantization (per token row, so the
        padding, roll and window partition below commute with it: zero rows
        quantize to zero)."""
        b, h0, w0, c = x.shape
        h, w = self.padded
        if (h, w) != (h0, w0):  # pad to whole windows, cropped below
            x = F.pad(x, (0, 0, 0, w - w0, 0, h - h0))
        if self.shift_size:
            x = torch.roll(x, shifts=(-self.shift_size, -self.shift_size), dims=(1, 2))
        win = window_partition(x, self.window_size)
        win = self.attn(win, mask=self.attn_mask, prequantized=prequantized)
        x = window_reverse(win, self.window_size, h, w)
        if self.shift_size:
            x = torch.roll(x, shifts=(self.shift_size, self.shift_size), dims=(1, 2))
        return x[:, :h0, :w0, :]

    def forward(self, x):
        b, h, w, c = x.shape
        hn, q = norm_quant_fwd(self.norm1, x, self.attn.qkv)
        x = x + self._attn(hn, q)
        x = x.reshape(b, -1, c)
        if _fused(self, x):  # the MLP residual add fused into fc2's store (norm2 into fc1 where it streams)
            y = self.mlp.forward_norm_residual(self.norm2, x)
            if y is None:
                hn, q = norm_quant_fwd(self.norm2, x, self.mlp.fc1)
                y = self.mlp.forward_residual(hn, x, q)
            x = y
        else:
            x = x + self.mlp(self.norm2(x))
        return x.reshape(b, h, w, c)


class PatchMerging(nn.Module):
    """2x2 neighbourhood merge: (B, H, W, C) -> (B, H/2, W/2, 2C) through
    norm(4C) and a bias-free Linear(4C, 2C) (the quantized `reduction`)."""

    def __init__(self, dim, out_dim=None, norm_layer=nn.LayerNorm):
        super().__init__()
        self.dim = dim
        self.out_dim = out_dim or 2 * dim
        self.norm = norm_layer(4 * dim)
        self.reduction = nn.Linear(4 * dim, self.out_dim, bias=False)

    def forward(self, x):
        b, h, w, c = x.shape
        x = x.reshape(b, h // 2, 2, w // 2, 2, c).permute(0, 1, 3, 4, 2, 5).flatten(3)
        h, q = norm_quant_fwd(self.norm, x, self.reduction)
        return call_layer(self.reduction, h, q)


class SwinTransformerStage(nn.Module):
    def __init__(self, dim, out_dim, input_resolution, depth, downsample, num_heads, window_size, mlp_ratio,
                 qkv_bias, norm_layer):
        super().__init__()
        self.dim = dim
        if downsample:
            self.downsample = PatchMerging(dim, out_dim, norm_layer)
            input_resolution = (input_resolution[0] // 2, input_resolution[1] // 2)
        else:
            self.downsample = nn.Identity()
        self.output_resolution = input_resolution
        self.blocks = nn.Sequential(*[
            SwinTransformerBlock(out_dim, input_resolution, num_heads, window_size,
                                 0 if i % 2 == 0 else window_size // 2, mlp_ratio, qkv_bias, norm_layer)
            for i in range(depth)])

    def forward(self, x):
        return self.blocks(self.downsample(x))


class ClassifierHead(nn.Module):
    def __init__(self, in_features, num_classes):
        super().__init__()
        self.fc = nn.Linear(in_features, num_classes) if num_classes > 0 else nn.Identity()

    def forward(self, x):
        return self.fc(x.mean(dim=(1, 2)))


class SwinTransformer(nn.Module):
    def __init__(self, img_size=224, patch_size=4, in_chans=3, num_classes=1000, embed_dim=96,
                 depths=(2, 2, 6, 2), num_heads=(3, 6, 12, 24), window_size=7, mlp_ratio=4.0, qkv_bias=True,
                 norm_layer=nn.LayerNorm, **kwargs):
        super().__init__()
        self.num_classes = num_classes
        self.num_layers = len(depths)
        self.embed_dim = embed_dim
        self.num_features = int(embed_dim * 2 ** (self.num_layers - 1))
        self.patch_embed = PatchEmbed(img_size, patch_size, in_chans, embed_dim, norm_layer=norm_layer,
                                      flatten=False)
        res = self.patch_embed.grid_size
        layers = []
        dim = embed_dim
        for i in range(self.num_layers):
            out_dim = int(embed_dim * 2 ** i)
            stage = SwinTransformerStage(dim, out_dim, res, depths[i], i > 0, num_heads[i], window_size,
                                         mlp_ratio, qkv_bias, norm_layer)
            res = stage.output_resolution
            layers.append(stage)
            dim = out_dim
        self.layers = nn.Sequential(*layers)
        self.norm = norm_layer(self.num_features)
        self.head = ClassifierHead(self.num_features, num_classes)
        for m in self.modules():
            if isinstance(m, nn.Linear):
                _trunc_normal_(m.weight, 0.02)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)
            elif isinstance(m, nn.LayerNorm):
                nn.init.ones_(m.weight)
                nn.init.zeros_(m.bias)

    def forward_features(self, x):
        return norm_fwd(self.norm, self.layers(self.patch_embed(x)))

    def forward(self, x):
        return self.head(self.forward_features(x))
