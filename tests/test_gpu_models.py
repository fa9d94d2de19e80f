"""GPU parity of the drop-in layer and models against the reference path.

* Layer: QATLinearComplexPhase in eval mode on the GPU (packed HIP path) vs
  the outputs the reference's own quant_i.QATLinearComplexPhase wrote
  (tests/golden), for the methods the packed path covers, with rotation and
  activation quantization on and off.  Bound: the kernel rounds the
  activations to fp16 (half ulp) and uses the fp16 fused operand
  (|A16 - A_q| <= (2u + u^2)(|W| + |U|), u = 2^-11), so
  |dy| <= u sum_k |x_k||A_k| + (2u + u^2) sum_k |x_k| (|W_k| + |U_k|) + 1e-5.
* Model: a DeiT-Tiny / ViT-Tiny forward in fp16 on the GPU vs the same model
  in float32 on the CPU with every quantized layer evaluated as
  x @ A_q.T + b on the oracle's decoded weight.  Stated tolerance: logits
  max-abs <= 2e-2 * max|logit| + 2e-3; top-1 agreement 100% on samples whose
  reference margin exceeds 4x the observed max logit error (margin-aware),
  raw top-1 agreement reported and required >= 99% over 64 images.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import rpfq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _layer(method, act, rot, golden):
    from quant_models.quant_i import QATLinearComplexPhase

    layer = QATLinearComplexPhase(quant_method_u=method, quant_method_w=method, enable_act_quant=bool(act),
                                  act_num_bits=4, enable_rotation=bool(rot), in_features=96, out_features=64)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(golden["w_weight"]))
        layer.bias.copy_(torch.from_numpy(golden["fwd_bias"]))
        if rot:
            layer.quantizer_u.rotation_angle.fill_(0.3)
            layer.quantizer_w.rotation_angle.fill_(-0.2)
    return layer


def _group_magnitude(golden, steps, rot):
    """|W_g| + |U_g| summed over the stage groups (0, 1), (2[, 3]) that the
    packed path runs as separate launches: the scale of the fp16 fusing
    error when U and W carry more than two stages."""
    u_re, u_im, w_re, w_im = O.decompose(golden["w_weight"])
    rotation = None
    if rot:
        cs = [(np.float32(np.cos(np.float32(t))), np.float32(np.sin(np.float32(t)))) for t in (0.3, -0.2)]
        rotation = tuple(cs)
        (cu, su), (cw, sw) = cs
        u_re, u_im = O.derotate(u_re, u_im, cu, -su)
        w_re, w_im = O.derotate(w_re, w_im, cw, -sw)
    _, _, su_st = O.residual_quantize(u_re, u_im, steps)
    _, _, sw_st = O.residual_quantize(w_re, w_im, steps)
    n = u_re.shape[0]
    mag = 0.0
    for lo in range(0, steps, 2):
        planes = [(c, np.full(n, a, np.float32), np.full(n, b, np.float32), "u") for c, a, b in su_st[lo:lo + 2]]
        planes += [(c, np.full(n, a, np.float32), np.full(n, b, np.float32), "w") for c, a, b in sw_st[lo:lo + 2]]
        mag = mag + O.wide_magnitude(planes, rotation=rotation)
    return mag


@pytest.mark.parametrize("method", ["complex_phase_v1", "complex_phase_v2", "complex_phase_v3", "complex_phase_v4",
                                    "complex_phase_new_v2", "complex_phase_next_v1"])
@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("rot", [0, 1])
def test_packed_layer_vs_reference_outputs(golden, method, act, rot):
    if method == "complex_phase_next_v1" and rot:
        pytest.skip("the reference recorded next_v1 without the global rotation (it has none)")
    layer = _layer(method, act, rot, golden).to(DEV).eval()
    x = torch.from_numpy(golden["fwd_x"])
    with torch.no_grad():
        y = layer(x.to(DEV)).cpu().numpy()
    tag = f"{method}_a{act}_r{rot}"
    y_ref = golden[f"fwd_y_{tag}"].astype(np.float64)
    a_ref = golden[f"fwd_aq_{tag}"].astype(np.float64)
    xs = golden["fwd_x"]
    if act:
        h = xs.shape[1] // 2
        xs = np.concatenate(O.act_quant(xs[:, :h], xs[:, h:], 4), axis=1)
    # x rounded to fp16 (half ulp) and the fp16 fused operand:
    # |A16 - A_q| <= (2u + u^2)(|W| + |U|), u = 2^-11, with U, W recovered from A_q
    ax = np.abs(xs.astype(np.float64))
    steps = {"complex_phase_v3": 3, "complex_phase_v4": 4}.get(method, 0)
    if steps:  # stage groups (0, 1) and (2[, 3]), each fused to fp16 on its own
        mag = _group_magnitude(golden, steps, rot)
    else:
        u_re, u_im, w_re, w_im = (np.abs(v) for v in O.decompose(a_ref))
        mag = np.block([[w_re + u_re, w_im + u_im], [w_im + u_im, w_re + u_re]])
    u = 2.0 ** -11
    bound = u * (ax @ np.abs(a_ref).T) + 1.001 * (2 * u + u * u) * (ax @ mag.T) + 1e-5
    assert np.all(np.abs(y - y_ref) <= bound), np.abs(y - y_ref).max()
    dec = layer.packed(torch.device(DEV)).decode().cpu().numpy()
    if steps:  # sum of the groups' float32 weights: the stage sum reassociated
        assert np.all(np.abs(dec - a_ref) <= 8 * 2.0 ** -24 * (mag + np.abs(a_ref)))
    else:  # the decoded float32 weight is the reference's A_q exactly
        assert np.array_equal(dec, golden[f"fwd_aq_{tag}"])


def test_packed_path_refuses_unsupported_method(golden):
    from quant_models.quant_i import QATLinearComplexPhase

    layer = QATLinearComplexPhase(quant_method_u="complex_phase_next_v1", quant_method_w="complex_phase_v2",
                                  enable_act_quant=False, in_features=96, out_features=64).to(DEV).eval()
    with pytest.raises(NotImplementedError):
        with torch.no_grad():
            layer(torch.randn(2, 96, device=DEV))


def test_packed_layer_repacks_after_weight_update(golden):
    layer = _layer("complex_phase_v2", 0, 0, golden).to(DEV).eval()
    x = torch.randn(3, 96, device=DEV)
    with torch.no_grad():
        y0 = layer(x)
        layer.weight.mul_(2.0)
        y1 = layer(x)
        ref = F.linear(x.cpu(), layer.cpu().quantized_weight(), layer.bias)
    assert not torch.allclose(y0.cpu(), y1.cpu())
    assert torch.allclose(y1.cpu(), ref, rtol=0, atol=2e-3)


def _reference_forward_cpu(model_gpu, name, x_cpu, state):
    """float32 CPU copy of the model whose quantized layers run x @ A_q.T + b
    on the oracle's decoding of exactly the codes the GPU model uses."""
    import copy

    import quant_models as qm
    from quant_models.inference import quant_layers

    ref = qm.create_model(name, img_size=224, quant_method_u="complex_phase_v2",
                          quant_method_w="complex_phase_v2", enable_act_quant=False, enable_rotation=False)
    ref.load_state_dict({k: v.float().cpu() for k, v in state.items()})
    ref.eval()
    for (n_g, l_g), (n_c, l_c) in zip(quant_layers(model_gpu), quant_layers(ref)):
        lc = l_g._override
        planes = [(O.unpack_codes(p.cpu().numpy()), a.cpu().numpy()[:, 0], b.cpu().numpy()[:, 0], k)
                  for p, a, b, k in zip(lc.planes, lc.scale_re, lc.scale_im, "uuww")]
        a_q = torch.from_numpy(O.wide_weight(planes))
        bias = None if l_c.bias is None else l_c.bias.detach().float()
        l_c.forward = (lambda xx, a_q=a_q, bias=bias: F.linear(xx, a_q, bias))
    with torch.no_grad():
        return ref(x_cpu)


@pytest.mark.parametrize("name", ["rpfq_deit_tiny_patch16_224_q", "rpfq_vit_tiny_patch16_224_q",
                                  "rpfq_swin_tiny_patch4_window7_224_q"])
def test_end_to_end_logits(name):
    import quant_models as qm
    from quant_models.inference import load_synthetic_codes, prepare_inference

    torch.manual_seed(1)
    model = qm.create_model(name, img_size=224, quant_method_u="complex_phase_v2",
                            quant_method_w="complex_phase_v2", enable_act_quant=False, enable_rotation=False)
    load_synthetic_codes(model, 1)
    # LayerNorm affine / embeddings get non-trivial values so logits spread
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, torch.nn.LayerNorm):
                m.weight.normal_(1.0, 0.1)
                m.bias.normal_(0.0, 0.1)
    ref_state = {k: v.clone() for k, v in model.state_dict().items()}
    prepare_inference(model, DEV, torch.float16)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(32 if "swin" in name else 64, 3, 224, 224, generator=g)
    with torch.no_grad():
        y = model(x.to(DEV, torch.float16)).float().cpu()
    # reference in float32 on the host with the same parameters and codes
    y_ref = _reference_forward_cpu(model, name, x, ref_state)
    err = (y - y_ref).abs()
    assert err.max() <= 2e-2 * y_ref.abs().max() + 2e-3, (err.max(), y_ref.abs().max())
    top = y_ref.topk(2, dim=1).values
    margin = top[:, 0] - top[:, 1]
    agree = (y.argmax(1) == y_ref.argmax(1)).float()
    confident = margin > 4 * err.max()
    assert bool(agree[confident].all())
    assert agree.mean() >= 0.99, f"top-1 agreement {agree.mean():.4f}"


@pytest.mark.parametrize("name", ["rpfq_vit_tiny_patch16_224_q", "rpfq_swin_tiny_patch4_window7_224_q"])
def test_fused_blocks_match_unfused(name):
    """Eval forward with the fused block path (device LayerNorm, residual adds
    in the proj / fc2 stores) vs the module-by-module forward on the same GPU
    model.  The residual adds are bit-identical by construction; LayerNorm
    statistics are ordered differently from torch's, so the stated bound is
    logits max-abs <= 1e-2 * max|logit| + 1e-3 with identical top-1 on
    margin-confident samples."""
    import quant_models as qm
    from quant_models import vision_transformer as vt
    from quant_models.inference import load_synthetic_codes, prepare_inference

    torch.manual_seed(3)
    model = qm.create_model(name, img_size=224, quant_method_u="complex_phase_v2",
                            quant_method_w="complex_phase_v2", enable_act_quant=False, enable_rotation=False)
    load_synthetic_codes(model, 3)
    prepare_inference(model, DEV, torch.float16)
    x = torch.randn(16, 3, 224, 224, generator=torch.Generator().manual_seed(5)).to(DEV, torch.float16)
    saved = vt.FUSED_BLOCKS
    try:
        with torch.no_grad():
            vt.FUSED_BLOCKS = True
            y_f = model(x).float().cpu()
            vt.FUSED_BLOCKS = False
            y_u = model(x).float().cpu()
    finally:
        vt.FUSED_BLOCKS = saved
    err = (y_f - y_u).abs().max()
    assert err <= 1e-2 * y_u.abs().max() + 1e-3, (err, y_u.abs().max())
    top = y_u.topk(2, dim=1).values
    confident = (top[:, 0] - top[:, 1]) > 4 * err
    assert bool((y_f.argmax(1) == y_u.argmax(1))[confident].all())


@pytest.mark.parametrize("name", ["rpfq_vit_tiny_patch16_224_q", "rpfq_swin_tiny_patch4_window7_224_q"])
def test_fused_act_quant_wiring(name):
    """With activation quantization on, the fused block path feeds qkv / fc1
    (and Swin's patch-merging reduction) from rpfq_layer_norm_act_quant and
    skips their own quantization pass.  That kernel is bit-identical to
    LayerNorm followed by act-quant, so the logits must equal those of the
    same fused path with the LN + act-quant fusion switched off: a layer
    quantized twice (or not at all) would change them."""
    import quant_models as qm
    from quant_models import vision_transformer as vt
    from quant_models.inference import load_synthetic_codes, prepare_inference

    torch.manual_seed(4)
    model = qm.create_model(name, img_size=224, quant_method_u="complex_phase_v2",
                            quant_method_w="complex_phase_v2", enable_act_quant=True, enable_rotation=False)
    load_synthetic_codes(model, 4)
    prepare_inference(model, DEV, torch.float16)
    x = torch.randn(8, 3, 224, 224, generator=torch.Generator().manual_seed(6)).to(DEV, torch.float16)
    saved = vt.FUSED_BLOCKS, vt.FUSE_ACT_QUANT
    try:
        with torch.no_grad():
            vt.FUSED_BLOCKS, vt.FUSE_ACT_QUANT = True, True
            y_f = model(x)
            vt.FUSE_ACT_QUANT = False
            y_u = model(x)
    finally:
        vt.FUSED_BLOCKS, vt.FUSE_ACT_QUANT = saved
    assert torch.isfinite(y_f).all()
    assert torch.equal(y_f, y_u)


@pytest.mark.parametrize("name", ["rpfq_vit_tiny_patch16_224_q", "rpfq_swin_tiny_patch4_window7_224_q"])
def test_fused_gelu_wiring(name):
    """The fused block path runs the MLP's exact GELU in fc1's store
    (RPFQ_FLAG_GELU), within 1 fp16 ulp of torch's GELU of the unfused fc1
    output (rarely off at all): the logits stay within 1e-2 * max|logit| +
    1e-3 of the same path with the GELU fusion off, with identical top-1 on
    margin-confident samples.  A GELU skipped or applied twice moves them by
    orders of magnitude more."""
    import quant_models as qm
    from quant_models import vision_transformer as vt
    from quant_models.inference import load_synthetic_codes, prepare_inference

    torch.manual_seed(5)
    model = qm.create_model(name, img_size=224, quant_method_u="complex_phase_v2",
                            quant_method_w="complex_phase_v2", enable_act_quant=False, enable_rotation=False)
    load_synthetic_codes(model, 5)
    prepare_inference(model, DEV, torch.float16)
    # one image: fc1 takes the streaming kernel, where the GELU is fused
    x = torch.randn(1, 3, 224, 224, generator=torch.Generator().manual_seed(7)).to(DEV, torch.float16)
    from quant_models import ops
    fused = []
    linear = ops.PackedWide.linear

    def counting(self, *args, **kw):
        fused.append(bool(kw.get("gelu", False)))
        return linear(self, *args, **kw)
    saved = vt.FUSED_BLOCKS, vt.FUSE_GELU
    try:
        ops.PackedWide.linear = counting
        with torch.no_grad():
            vt.FUSED_BLOCKS, vt.FUSE_GELU = True, True
            y_f = model(x)
            n_fused = sum(fused)
            vt.FUSE_GELU = False
            y_u = model(x)
    finally:
        ops.PackedWide.linear = linear
        vt.FUSED_BLOCKS, vt.FUSE_GELU = saved
    assert n_fused >= 2, n_fused
    assert torch.isfinite(y_f).all()
    y_f, y_u = y_f.float().cpu(), y_u.float().cpu()
    err = (y_f - y_u).abs().max()
    assert err <= 1e-2 * y_u.abs().max() + 1e-3, (err, y_u.abs().max())
    top = y_u.topk(2, dim=1).values
    confident = (top[:, 0] - top[:, 1]) > 4 * err
    assert bool((y_f.argmax(1) == y_u.argmax(1))[confident].all())
