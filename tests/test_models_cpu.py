"""Model registration and creation, mirroring the reference's
RPFQ-ViT-main/tests/test_models.py (registration of the rpfq_* names; tiny
models at img_size 32 with act quant at 2 and 4 bits), plus the timm
state-dict layout the drop-in relies on."""
import pytest
import torch

NAMES = [
    "rpfq_vit_base_patch16_224_q", "rpfq_vit_large_patch16_224_q", "rpfq_vit_small_patch16_224_q",
    "rpfq_vit_tiny_patch16_224_q", "rpfq_deit_base_patch16_224_q", "rpfq_deit_small_patch16_224_q",
    "rpfq_deit_tiny_patch16_224_q", "rpfq_swin_base_patch4_window7_224_q", "rpfq_swin_small_patch4_window7_224_q",
    "rpfq_swin_tiny_patch4_window7_224_q",
]


def qm():
    import quant_models
    return quant_models


def test_registration():
    for n in NAMES:
        assert qm().is_model(n), n


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("name", ["rpfq_vit_tiny_patch16_224_q", "rpfq_deit_tiny_patch16_224_q",
                                  "rpfq_swin_tiny_patch4_window7_224_q"])
def test_tiny_model_creation(name, bits):
    m = qm().create_model(name, pretrained=False, num_classes=10, img_size=32, quant_method_u="complex_phase_v2",
                          quant_method_w="complex_phase_v2", enable_act_quant=True, enable_rotation=False,
                          act_num_bits=bits)
    m.eval()
    with torch.no_grad():
        out = m(torch.randn(1, 3, 32, 32))
    assert out.shape == (1, 10) and torch.isfinite(out).all()
    layers = [mod for mod in m.modules() if hasattr(mod, "act_quantizer")]
    assert layers and all(l.act_quantizer is not None and l.act_quantizer.num_bits == bits for l in layers)


def test_which_layers_are_quantized():
    from quant_models.quant_i import QATLinearComplexPhase

    vit = qm().create_model("rpfq_vit_tiny_patch16_224_q", img_size=32, num_classes=10)
    names = {n for n, mod in vit.named_modules() if isinstance(mod, QATLinearComplexPhase)}
    assert {"blocks.0.attn.qkv", "blocks.0.attn.proj", "blocks.0.mlp.fc1", "blocks.0.mlp.fc2", "head"} <= names
    assert len(names) == 12 * 4 + 1
    deit = qm().create_model("rpfq_deit_tiny_patch16_224_q", img_size=32, num_classes=10)
    assert isinstance(deit.head_dist, QATLinearComplexPhase)
    swin = qm().create_model("rpfq_swin_tiny_patch4_window7_224_q", img_size=32, num_classes=10)
    snames = {n for n, mod in swin.named_modules() if isinstance(mod, QATLinearComplexPhase)}
    assert {"layers.1.downsample.reduction", "layers.0.blocks.0.attn.qkv", "head.fc"} <= snames


def test_builder_defaults_follow_reference():
    vit = qm().create_model("rpfq_vit_tiny_patch16_224_q", img_size=32, num_classes=10)
    deit = qm().create_model("rpfq_deit_tiny_patch16_224_q", img_size=32, num_classes=10)
    assert vit.enable_rotation is True and deit.enable_rotation is False  # quant_rpfq_vit.py:156 vs deit :111
    assert vit.blocks[0].attn.qkv.quantizer_u.quant_method == "complex_phase_v1"
    legacy = qm().create_model("rpfq_vit_tiny_patch16_224_q", img_size=32, num_classes=10,
                               quant_method="complex_phase_v2", quant_bits=2)
    assert legacy.quant_method_u == legacy.quant_method_w == "complex_phase_v2"
    with pytest.raises(ValueError):
        qm().create_model("rpfq_deit_tiny_patch16_224_q", img_size=32, quant_method="bogus")


def test_timm_state_dict_keys():
    vit = qm().create_model("rpfq_vit_base_patch16_224_q", enable_rotation=False)
    keys = set(vit.state_dict())
    for k in ["cls_token", "pos_embed", "patch_embed.proj.weight", "blocks.11.attn.qkv.weight",
              "blocks.11.attn.qkv.bias", "blocks.0.mlp.fc2.bias", "norm.weight", "head.weight"]:
        assert k in keys
    assert vit.pos_embed.shape == (1, 197, 768)
    deit = qm().create_model("rpfq_deit_tiny_patch16_224_q")
    assert deit.pos_embed.shape == (1, 198, 192) and "dist_token" in deit.state_dict()


@pytest.mark.parametrize("name", ["rpfq_vit_tiny_patch16_224_q", "rpfq_deit_tiny_patch16_224_q"])
def test_token_write_matches_cat(name):
    """Outside autograd the prefix and patch tokens are written with their
    position embedding into one buffer; recorded for autograd the forward
    keeps torch.cat followed by the add. Both give the same bits (one class
    token for ViT, class + distillation tokens for DeiT)."""
    torch.manual_seed(0)
    m = qm().create_model(name, pretrained=False, num_classes=10, img_size=32, quant_method_u="complex_phase_v2",
                          quant_method_w="complex_phase_v2", enable_act_quant=False, enable_rotation=False)
    m.eval()
    with torch.no_grad():
        m.pos_embed.normal_()
        m.cls_token.normal_()
        if getattr(m, "dist_token", None) is not None:
            m.dist_token.normal_()
    m.blocks, m.norm = torch.nn.Identity(), torch.nn.Identity()
    x = torch.randn(3, 3, 32, 32)
    with torch.no_grad():
        fused = m.forward_features(x)
    xg = x.clone().requires_grad_(True)
    with torch.enable_grad():
        cat = m.forward_features(xg)
    assert cat.requires_grad and not fused.requires_grad
    assert torch.equal(fused, cat.detach())
