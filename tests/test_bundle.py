"""Reader of the reference's exported bundle (model.safetensors +
config.json, export_rpfq_vit_to_mlx.py:384-606) into the packed layout.

* Layer: the reference exporter's own output for one linear (golden
  exp_L_*: codes padded to 256 complex rows / columns, fp16 gammas) read
  under the exporter's key names decodes to the exporter's quantized forward
  weight (golden exp_aq) bit for bit -- on the CPU through the oracle, on the
  GPU through rpfq_wide_pack + rpfq_wide_decode.
* Model: a two-block ViT bundle written in the exporter's layout (stages from
  packing.export_stages, pinned bit-exact against the exporter by
  tests/test_packing_cpu.py; padding as the exporter pads) loads into a
  packed fp16 model whose logits match a float32 CPU forward on the
  oracle-decoded weights: max-abs <= 2e-2 max|logit| + 2e-3.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import rpfq_oracle as O

DEV = "cuda"


def _golden_tensors(golden, tag="exp_L", prefix="L"):
    t = {}
    for kind in ("u", "w"):
        for s in range(2):
            for f in ("codes", "gamma_real", "gamma_imag"):
                t[f"{prefix}.{kind}_s{s}.{f}"] = torch.from_numpy(golden[f"{tag}_{kind}_s{s}_{f}"])
    t[f"{prefix}.bias"] = torch.from_numpy(golden[f"{tag}_bias"])
    return t


def _oracle_weight(lc):
    kinds = ["u"] * lc.stages + ["w"] * lc.stages
    planes = [(O.unpack_codes(p.cpu().numpy()), a.cpu().numpy(), b.cpu().numpy(), k)
              for p, a, b, k in zip(lc.planes, lc.scale_re, lc.scale_im, kinds)]
    if lc.block:  # per-(row, block) multipliers -> per element
        planes = [(c, np.repeat(a, lc.block, axis=1)[:, :c.shape[1]], np.repeat(b, lc.block, axis=1)[:, :c.shape[1]],
                   k) for c, a, b, k in planes]
    else:
        planes = [(c, a[:, 0], b[:, 0], k) for c, a, b, k in planes]
    return O.wide_weight(planes)


def test_layer_codes_reproduce_exporter_weight(golden):
    from quant_models import bundle

    lc = bundle.layer_codes(_golden_tensors(golden), "L", 32, 48, 2)
    assert [tuple(p.shape) for p in lc.planes] == [(32, 12)] * 4 and lc.block == 0
    assert np.array_equal(_oracle_weight(lc), golden["exp_aq"])
    # a block-aligned export (K' = 256, no padding): multipliers are 1/gamma
    lcb = bundle.layer_codes(_golden_tensors(golden, "expb_L"), "L", 24, 256, 2)
    g = golden["expb_L_u_s1_gamma_imag"].astype(np.float32)
    assert np.array_equal(lcb.scale_im[1].numpy(), (np.float32(1.0) / g))


def test_layer_codes_rejects_short_planes(golden):
    from quant_models import bundle

    t = _golden_tensors(golden)
    with pytest.raises(ValueError, match="does not cover"):
        bundle.layer_codes(t, "L", 300, 48, 2)
    with pytest.raises(KeyError):
        bundle.layer_codes(t, "L", 32, 48, 3)


def test_read_tensors_and_config_round_trip(golden, tmp_path):
    from safetensors.torch import save_file

    from quant_models import bundle

    t = _golden_tensors(golden, prefix="model.layers.0.attn.proj")
    save_file(t, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": 96}))
    back = bundle.read_tensors(str(tmp_path))
    assert set(back) == set(t) and all(torch.equal(back[k], t[k]) for k in t)
    assert bundle.read_config(str(tmp_path))["hidden_size"] == 96


@pytest.mark.gpu
def test_layer_codes_pack_and_decode_on_gpu(golden):
    from quant_models import bundle, ops

    lc = bundle.layer_codes(_golden_tensors(golden), "L", 32, 48, 2)
    pw = ops.pack_layer([p.to(DEV) for p in lc.planes], [s.to(DEV) for s in lc.scale_re],
                        [s.to(DEV) for s in lc.scale_im], 32, 48, lc.codebook, 2, lc.block, None)
    assert np.array_equal(pw.decode().cpu().numpy(), golden["exp_aq"])


# ---------------------------------------------------------------------------
# whole-model bundle
# ---------------------------------------------------------------------------
def _round_up(v, m):
    return -(-v // m) * m


def _export_linear(target, prefix, weight, bias, stages=2):
    """One linear in the exporter's layout (export…py:384-423), padded to
    256 complex rows / columns like the exporter pads qkv / fc1 / fc2."""
    from quant_models import packing as P

    u_re, u_im, w_re, w_im = P.split_blocks(weight.float())
    n_c, k_c = u_re.shape
    n_p, k_p = _round_up(n_c, 256), _round_up(k_c, 256)
    for kind, (re, im) in (("u", (u_re, u_im)), ("w", (w_re, w_im))):
        for s, (codes, g_re, g_im) in enumerate(P.export_stages(re, im, stages)):
            full = torch.zeros(n_p, k_p, dtype=torch.uint8)
            full[:n_c, :k_c] = codes
            target[f"{prefix}.{kind}_s{s}.codes"] = P.pack2(full)
            target[f"{prefix}.{kind}_s{s}.gamma_real"] = torch.full((n_p, k_p // 256), float(g_re),
                                                                    dtype=torch.float16)
            target[f"{prefix}.{kind}_s{s}.gamma_imag"] = torch.full((n_p, k_p // 256), float(g_im),
                                                                    dtype=torch.float16)
    target[f"{prefix}.bias"] = bias.to(torch.float16)


def _write_vit_bundle(path, hidden=64, depth=2, heads=2, inter=256, img=32, patch=16, classes=10, seed=0):
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(seed)
    rnd = lambda *s, std=0.05: torch.randn(*s, generator=g) * std  # noqa: E731
    t = {"model.patch_embed.weight": rnd(hidden, 3 * patch * patch).half(),
         "model.patch_embed.bias": rnd(hidden).half(),
         "model.cls_token": rnd(1, 1, hidden, std=0.5).half(),
         "model.pos_embed": rnd(1, (img // patch) ** 2 + 1, hidden, std=0.5).half()}
    dims = {"attn.qkv": (3 * hidden, hidden), "attn.proj": (hidden, hidden), "mlp.fc1": (inter, hidden),
            "mlp.fc2": (hidden, inter)}
    for i in range(depth):
        pre = f"model.layers.{i}"
        for n in ("norm1", "norm2"):
            t[f"{pre}.{n}.weight"] = (1.0 + rnd(hidden)).half()
            t[f"{pre}.{n}.bias"] = rnd(hidden).half()
        for name, (o, k) in dims.items():
            _export_linear(t, f"{pre}.{name}", rnd(o, k), rnd(o))
    t["model.norm.weight"] = (1.0 + rnd(hidden)).half()
    t["model.norm.bias"] = rnd(hidden).half()
    t["head.weight"] = rnd(classes, hidden).half()
    t["head.bias"] = rnd(classes).half()
    os.makedirs(path, exist_ok=True)
    save_file(t, os.path.join(path, "model.safetensors"))
    cfg = {"model_type": "rpfq_vit", "image_size": img, "patch_size": patch, "num_channels": 3,
           "hidden_size": hidden, "num_hidden_layers": depth, "num_attention_heads": heads,
           "intermediate_size": inter, "num_classes": classes, "layer_norm_eps": 1e-5,
           "rpfq_vit": {"residual_stages": 2, "block_size": 256, "quant_method": "complex_phase_v2"}}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)


def _reference_forward(bundle_dir, x):
    """float32 CPU forward of the same ViT with every quantized linear an
    nn.Linear on the oracle-decoded weight of the bundle's planes."""
    import functools

    import torch.nn as nn

    from quant_models import bundle
    from quant_models.quant_rpfq_vit import ComplexVisionTransformer

    cfg = bundle.read_config(bundle_dir)
    t = bundle.read_tensors(bundle_dir)
    hidden = cfg["hidden_size"]
    m = ComplexVisionTransformer(img_size=cfg["image_size"], patch_size=cfg["patch_size"],
                                 num_classes=cfg["num_classes"], embed_dim=hidden, depth=cfg["num_hidden_layers"],
                                 num_heads=cfg["num_attention_heads"], mlp_ratio=cfg["intermediate_size"] / hidden,
                                 qkv_bias=True, norm_layer=functools.partial(nn.LayerNorm, eps=1e-5),
                                 enable_act_quant=False, enable_rotation=False)
    with torch.no_grad():
        m.patch_embed.proj.weight.copy_(t["model.patch_embed.weight"].float().reshape(m.patch_embed.proj.weight.shape))
        m.patch_embed.proj.bias.copy_(t["model.patch_embed.bias"].float())
        m.cls_token.copy_(t["model.cls_token"].float())
        m.pos_embed.copy_(t["model.pos_embed"].float())
        for i, blk in enumerate(m.blocks):
            pre = f"model.layers.{i}"
            for n in ("norm1", "norm2"):
                getattr(blk, n).weight.copy_(t[f"{pre}.{n}.weight"].float())
                getattr(blk, n).bias.copy_(t[f"{pre}.{n}.bias"].float())
            for name in bundle.LINEARS:
                q = blk.get_submodule(name)
                lin = nn.Linear(q.in_features, q.out_features)
                lc = bundle.layer_codes(t, f"{pre}.{name}", q.out_features // 2, q.in_features // 2, 2)
                lin.weight.copy_(torch.from_numpy(_oracle_weight(lc)))
                lin.bias.copy_(t[f"{pre}.{name}.bias"].float())
                parent, attr = name.split(".")
                setattr(getattr(blk, parent), attr, lin)
        m.norm.weight.copy_(t["model.norm.weight"].float())
        m.norm.bias.copy_(t["model.norm.bias"].float())
        m.head = nn.Linear(hidden, cfg["num_classes"])
        m.head.weight.copy_(t["head.weight"].float())
        m.head.bias.copy_(t["head.bias"].float())
        return m.eval()(x)


@pytest.mark.gpu
def test_load_vit_bundle_matches_decoded_reference(tmp_path):
    from quant_models import bundle

    path = str(tmp_path / "bundle")
    _write_vit_bundle(path)
    model = bundle.load_vit_bundle(path, DEV, torch.float16)
    x = torch.randn(8, 3, 32, 32, generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        y = model(x.to(DEV).half()).float().cpu()
        y_ref = _reference_forward(path, x)
    err = float((y - y_ref).abs().max())
    assert err <= 2e-2 * float(y_ref.abs().max()) + 2e-3, err
