"""The quantization-aware training path: the GPU weight quantizer
(rpfq_quantize_wide) against the CPU oracle, the device packer, and the HIP
training forward / backward of QATLinearComplexPhase against the reference
formulation in torch on the CPU.

Bars:
* quantizer: A_q, scales and code planes bit-exact with oracle.quantized_weight
  (the oracle accumulates each scale's sum in float64 and rounds once, as the
  kernel does; the oracle itself matches the reference's golden A_q to the
  scale-sum ulp tolerance, tests/test_oracle.py);
* device packer: the packed layer decodes to the quantizer's A_q bit-exactly;
* training layer: outputs within float32 GEMM rounding plus the scale ulps
  (rtol 1e-4 of max|y|), gradients likewise; the weight gradient is the A_q
  gradient (straight-through), the rotation gradient follows rotation_grad,
  which the CPU test pins against torch autograd of the reference formulation.
"""
import numpy as np
import pytest
import torch

from oracle import rpfq_oracle as O

DEV = "cuda"
KIND_OF = {"complex_phase_v1": ("axis", 1), "complex_phase_v2": ("axis", 2), "complex_phase_v3": ("axis", 3),
           "complex_phase_v4": ("axis", 4), "complex_phase_new_v2": ("sign", 2)}


def _rot_cos_sin(tu, tw):
    out = []
    for t in (tu, tw):
        th = torch.full((1,), t, dtype=torch.float32)
        out.append((np.float32(torch.cos(th).item()), np.float32(torch.sin(th).item())))
    return tuple(out)


# ---------------------------------------------------------------------------
# CPU: straight-through gradients of the rotation
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("method", ["complex_phase_v2", "complex_phase_new_v2", "complex_phase_v3"])
def test_rotation_grad_matches_autograd(method):
    from quant_models.quant_i import QATLinearComplexPhase, rotation_grad

    torch.manual_seed(0)
    layer = QATLinearComplexPhase(quant_method_u=method, quant_method_w=method, enable_act_quant=False,
                                  enable_rotation=True, in_features=64, out_features=48)
    with torch.no_grad():
        layer.quantizer_u.rotation_angle.fill_(0.3)
        layer.quantizer_w.rotation_angle.fill_(-0.7)
    a_q = layer.quantized_weight()
    g = torch.randn_like(a_q)
    (a_q * g).sum().backward()
    tu, tw = rotation_grad(g, layer.weight.detach(), a_q.detach())
    ref_u = layer.quantizer_u.rotation_angle.grad[0]
    ref_w = layer.quantizer_w.rotation_angle.grad[0]
    # every term of the gradient is g times a quantization error (weight - A_q)
    tol = 2e-6 * float((g.abs() * (layer.weight.detach() - a_q.detach()).abs()).sum())
    assert abs(float(tu - ref_u)) <= tol and abs(float(tw - ref_w)) <= tol
    # the gradients are far from 0 against the tolerance, so a dropped term or
    # a flipped sign (an error of the order of the gradient itself) fails
    assert abs(float(ref_u)) > 20 * tol and abs(float(ref_w)) > 20 * tol
    # straight-through: the weight receives the A_q gradient
    assert torch.allclose(layer.weight.grad, g, rtol=0, atol=1e-5)


# ---------------------------------------------------------------------------
# GPU: quantizer vs oracle
# ---------------------------------------------------------------------------
def _check_quantizer(weight, kind_u, steps_u, kind_w, steps_w, rotation=None, codes=True):
    from quant_models import ops

    rot = None
    if rotation is not None:
        rot = torch.tensor([rotation[0][0], rotation[0][1], rotation[1][0], rotation[1][1]], dtype=torch.float32,
                           device=DEV)
    a_q, scales, cp = ops.quantize_wide(torch.from_numpy(weight).to(DEV), kind_u, steps_u, kind_w, steps_w, rot=rot,
                                        want_codes=codes)
    ref, st_u, st_w = O.quantized_weight(weight, kind_u, steps_u, kind_w, steps_w, rotation)
    assert np.array_equal(a_q.cpu().numpy(), ref)
    sc = scales.cpu().numpy()
    for p, st in enumerate((st_u, st_w)):
        for t, (c, s_re, s_im) in enumerate(st):
            assert sc[p, t, 0] == s_re and sc[p, t, 1] == s_im, (p, t)
        assert np.all(sc[p, len(st):] == 0)
    if codes:
        planes = [c for c, _, _ in st_u] + [c for c, _, _ in st_w]
        got = cp.cpu().numpy()
        assert got.shape[0] == len(planes)
        for i, c in enumerate(planes):
            assert np.array_equal(got[i], O.pack_codes(c)), i


@pytest.mark.gpu
@pytest.mark.parametrize("method", sorted(KIND_OF))
@pytest.mark.parametrize("rot", [0, 1])
def test_quantize_wide_golden_weight(golden, method, rot):
    kind, steps = KIND_OF[method]
    _check_quantizer(golden["w_weight"], kind, steps, kind, steps, _rot_cos_sin(0.3, -0.2) if rot else None)


@pytest.mark.gpu
@pytest.mark.parametrize("n_c,k_c,ku,su,kw,sw,rot,codes", [
    (1536, 384, "axis", 2, "axis", 2, True, True),     # ViT-B fc1
    (384, 1536, "sign", 2, "sign", 2, False, True),    # ViT-B fc2, quadrant-sign
    (500, 384, "axis", 4, "sign", 1, True, True),      # ViT-B head, mixed kinds
    (100, 50, "axis", 3, "axis", 1, False, False),     # K' % 4 != 0: A_q only
    (1, 4, "axis", 1, "axis", 1, False, True),         # one complex row
])
def test_quantize_wide_random_shapes(n_c, k_c, ku, su, kw, sw, rot, codes):
    r = np.random.default_rng(n_c * 7 + k_c)
    weight = (r.standard_normal((2 * n_c, 2 * k_c)) * 0.02).astype(np.float32)
    _check_quantizer(weight, ku, su, kw, sw, _rot_cos_sin(0.41, -1.3) if rot else None, codes)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["axis", "sign"])
def test_quantize_wide_ties_and_zeros(kind):
    """U and W drawn from a small grid so |re| == |im| ties (every quadrant),
    exact zeros and signed zeros occur often; the 2x2 split recovers them
    exactly."""
    r = np.random.default_rng(5)
    n_c, k_c = 64, 96
    grid = np.array([-0.5, -0.25, -0.0, 0.0, 0.25, 0.5], np.float32)
    u_re, u_im, w_re, w_im = (grid[r.integers(0, 6, size=(n_c, k_c))] for _ in range(4))
    weight = O.recompose(u_re, u_im, w_re, w_im)
    assert all(np.array_equal(a, b) for a, b in zip(O.decompose(weight), (u_re, u_im, w_re, w_im)))
    _check_quantizer(weight, kind, 2, kind, 2)


@pytest.mark.gpu
def test_quantize_wide_unaligned_weight():
    """A weight that is not 16-byte aligned takes the one-column-per-thread
    path: the same A_q and scales; code planes are refused."""
    from quant_models import _native as N
    from quant_models import ops

    r = np.random.default_rng(9)
    w = (r.standard_normal((2 * 96, 2 * 64)) * 0.02).astype(np.float32)
    buf = torch.zeros(w.size + 1, dtype=torch.float32, device=DEV)
    wd = buf[1:].view(w.shape)
    wd.copy_(torch.from_numpy(w))
    assert wd.data_ptr() % 16 != 0
    a_q, scales, _ = ops.quantize_wide(wd, "axis", 2, "axis", 2)
    ref, st_u, _ = O.quantized_weight(w, "axis", 2, "axis", 2)
    assert np.array_equal(a_q.cpu().numpy(), ref)
    assert scales.cpu().numpy()[0, 1, 0] == st_u[1][1]
    with pytest.raises(N.RPFQError, match="aligned"):
        ops.quantize_wide(wd, "axis", 2, "axis", 2, want_codes=True)


@pytest.mark.gpu
def test_quantize_wide_argument_errors():
    from quant_models import _native as N
    from quant_models import ops

    w = torch.zeros(8, 10, device=DEV)
    with pytest.raises(N.RPFQError, match="k_complex % 4"):
        ops.quantize_wide(w, "axis", 1, "axis", 1, want_codes=True)
    with pytest.raises(N.RPFQError, match="steps=5"):
        ops.quantize_wide(torch.zeros(8, 8, device=DEV), "axis", 5, "axis", 1)


# ---------------------------------------------------------------------------
# GPU: device packer
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("method", sorted(KIND_OF))
@pytest.mark.parametrize("rot", [0, 1])
def test_device_pack_decodes_to_quantizer_weight(golden, method, rot):
    from quant_models import ops
    from quant_models.quant_i import QATLinearComplexPhase

    layer = QATLinearComplexPhase(quant_method_u=method, quant_method_w=method, enable_act_quant=False,
                                  enable_rotation=bool(rot), in_features=96, out_features=64).to(DEV).eval()
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(golden["w_weight"]))
        if rot:
            layer.quantizer_u.rotation_angle.fill_(0.3)
            layer.quantizer_w.rotation_angle.fill_(-0.2)
    layer.pack_on_device = True
    dec = layer.packed(torch.device(DEV)).decode().cpu().numpy()
    kind, steps = KIND_OF[method]
    rotation = _rot_cos_sin(0.3, -0.2) if rot else None
    ref, _, _ = O.quantized_weight(golden["w_weight"], kind, steps, kind, steps, rotation)
    if steps <= 2:
        assert np.array_equal(dec, ref)
    else:  # stage groups (0, 1) + (2[, 3]) summed: float32 reassociation of the stage sum
        assert np.allclose(dec, ref, rtol=0, atol=8 * 2.0 ** -24 * float(np.abs(ref).max()))
    rot_t = None
    if rot:
        rot_t = torch.tensor([v for cs in rotation for v in cs], dtype=torch.float32, device=DEV)
    a_q, _, _ = ops.quantize_wide(layer.weight.detach(), kind, steps, kind, steps, rot=rot_t)
    assert np.array_equal(a_q.cpu().numpy(), ref)


# ---------------------------------------------------------------------------
# GPU: training forward / backward
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("method,act,rot", [("complex_phase_v2", 1, 1), ("complex_phase_v2", 0, 0),
                                            ("complex_phase_new_v2", 1, 0), ("complex_phase_v4", 1, 1)])
def test_hip_training_step_matches_torch_formulation(method, act, rot):
    from quant_models.quant_i import QATLinearComplexPhase

    torch.manual_seed(3)
    cpu = QATLinearComplexPhase(quant_method_u=method, quant_method_w=method, enable_act_quant=bool(act),
                                act_num_bits=4, enable_rotation=bool(rot), in_features=192, out_features=128)
    with torch.no_grad():
        cpu.bias.normal_(0.0, 0.1)
        if rot:
            cpu.quantizer_u.rotation_angle.fill_(0.25)
            cpu.quantizer_w.rotation_angle.fill_(-0.6)
    gpu = QATLinearComplexPhase(quant_method_u=method, quant_method_w=method, enable_act_quant=bool(act),
                                act_num_bits=4, enable_rotation=bool(rot), in_features=192, out_features=128)
    gpu.load_state_dict(cpu.state_dict())
    gpu = gpu.to(DEV).train()
    assert gpu._hip_qat_spec(torch.zeros(1, device=DEV)) is not None
    x = torch.randn(3, 37, 192)
    gy = torch.randn(3, 37, 128)
    xc = x.clone().requires_grad_(True)
    y_c = cpu(xc)
    (y_c * gy).sum().backward()
    xg = x.to(DEV).requires_grad_(True)
    y_g = gpu(xg)
    (y_g * gy.to(DEV)).sum().backward()
    tol = 1e-4 * float(y_c.abs().max())
    assert float((y_g.detach().cpu() - y_c.detach()).abs().max()) <= tol
    for a, b in ((xg.grad, xc.grad), (gpu.weight.grad, cpu.weight.grad), (gpu.bias.grad, cpu.bias.grad)):
        assert torch.allclose(a.cpu(), b, rtol=1e-4, atol=1e-4 * float(b.abs().max()))
    if rot:
        for q in ("quantizer_u", "quantizer_w"):
            a = getattr(gpu, q).rotation_angle.grad.cpu()
            b = getattr(cpu, q).rotation_angle.grad
            assert torch.allclose(a, b, rtol=1e-3, atol=1e-4 * float(b.abs().max()))


@pytest.mark.gpu
@pytest.mark.parametrize("method,act,rot", [("complex_phase_v2", 1, 1), ("complex_phase_new_v2", 0, 0),
                                            ("complex_phase_v4", 1, 0)])
def test_hip_training_packed_grad_x(method, act, rot):
    """The training forward with the input gradient on the packed blob of
    the step's own codes (RPFQ_QAT_PACKED_GRAD): the output, weight, bias and
    rotation gradients equal the library path's (the same F.linear, STE and
    weight GEMM); x.grad is within the fp16 operand bound of grad_y A_q --
    grad_y rounded once to fp16 (u = 2^-11) and the fused fp16 coefficients,
    (2u + u^2)(|W| + |U|) -- of the library path's."""
    from quant_models import quant_i
    from quant_models.quant_i import QATLinearComplexPhase

    torch.manual_seed(5)
    layer = QATLinearComplexPhase(quant_method_u=method, quant_method_w=method, enable_act_quant=bool(act),
                                  act_num_bits=4, enable_rotation=bool(rot), in_features=192, out_features=128)
    with torch.no_grad():
        layer.bias.normal_(0.0, 0.1)
        if rot:
            layer.quantizer_u.rotation_angle.fill_(0.25)
            layer.quantizer_w.rotation_angle.fill_(-0.6)
    layer = layer.to(DEV).train()
    x = torch.randn(3, 37, 192, device=DEV)
    gy = torch.randn(3, 37, 128, device=DEV)
    res = {}
    saved = quant_i.QAT_PACKED_GRAD
    try:
        for mode in ("0", "1"):
            quant_i.QAT_PACKED_GRAD = mode
            layer.zero_grad(set_to_none=True)
            xg = x.clone().requires_grad_(True)
            y = layer(xg)
            y.backward(gy)
            grads = [xg.grad, layer.weight.grad, layer.bias.grad]
            if rot:
                grads += [layer.quantizer_u.rotation_angle.grad, layer.quantizer_w.rotation_angle.grad]
            res[mode] = (y.detach(), [g.detach().clone() for g in grads])
    finally:
        quant_i.QAT_PACKED_GRAD = saved
    (y0, g0), (y1, g1) = res["0"], res["1"]
    assert torch.equal(y0, y1)
    for a, b in zip(g1[1:], g0[1:]):
        assert torch.allclose(a, b, rtol=1e-5, atol=1e-6 * float(b.abs().max()))
    with torch.no_grad():
        a_q = layer.cpu().quantized_weight().double().numpy()
    u_re, u_im, w_re, w_im = (np.abs(v) for v in O.decompose(a_q))
    mag = np.block([[w_re + u_re, w_im + u_im], [w_im + u_im, w_re + u_re]])
    u = 2.0 ** -11
    ag = np.abs(gy.cpu().double().numpy().reshape(-1, 128))
    # v4 runs as two stage groups, each fused on its own: their magnitudes
    # add, up to twice the residual group's beyond |W| + |U| of the sum
    fuse = 3.0 if method == "complex_phase_v4" else 1.001
    bound = u * (ag @ np.abs(a_q)) + fuse * (2 * u + u * u) * (ag @ mag) + 1e-4
    diff = (g1[0] - g0[0]).cpu().double().numpy().reshape(-1, 192)
    assert np.all(np.abs(diff) <= bound), float(np.abs(diff).max())
    assert not torch.equal(g1[0], g0[0])  # the packed path ran


# ---------------------------------------------------------------------------
# torch.ops.rpfq.* (the reference's operator contract, kernel.py:599-605)
# ---------------------------------------------------------------------------
def test_rpfq_ops_registered_with_fake_shapes():
    import quant_models  # noqa: F401  (registers the operators)
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x, w, b = torch.empty(3, 5, 96), torch.empty(64, 96), torch.empty(64)
        assert torch.ops.rpfq.qat_linear(x, w, b, "complex_phase_v2", "complex_phase_v2", 4).shape == (3, 5, 64)
        # the reference operator's own (x, weight, bias) call (kernel.py:599-605)
        assert torch.ops.rpfq.qat_linear(x, w, b).shape == (3, 5, 64)
        blob = torch.empty(4096, dtype=torch.uint8)
        assert torch.ops.rpfq.wide_linear(x, blob, 32, 48, 0, 2, 0, None, b).shape == (3, 5, 64)
        assert torch.ops.rpfq.act_quant(x, 4).shape == (3, 5, 96)


@pytest.mark.gpu
@pytest.mark.parametrize("method,act", [("complex_phase_v2", 4), ("complex_phase_new_v2", 0), ("complex_phase_v3", 4)])
def test_rpfq_qat_linear_op_matches_layer(method, act):
    """torch.ops.rpfq.qat_linear == the HIP training forward of
    QATLinearComplexPhase (rotation off), and its registered backward gives
    the layer's autograd gradients."""
    import quant_models  # noqa: F401
    from quant_models.quant_i import QATLinearComplexPhase

    torch.manual_seed(4)
    layer = QATLinearComplexPhase(quant_method_u=method, quant_method_w=method, enable_act_quant=act > 0,
                                  act_num_bits=act or 4, enable_rotation=False, in_features=192,
                                  out_features=128).to(DEV).train()
    x = torch.randn(7, 192, device=DEV)
    gy = torch.randn(7, 128, device=DEV)
    x1 = x.clone().requires_grad_(True)
    y1 = layer(x1)
    (y1 * gy).sum().backward()
    w = layer.weight.detach().clone().requires_grad_(True)
    b = layer.bias.detach().clone().requires_grad_(True)
    x2 = x.clone().requires_grad_(True)
    y2 = torch.ops.rpfq.qat_linear(x2, w, b, method, method, act)
    assert torch.equal(y2, y1)
    (y2 * gy).sum().backward()
    for a, ref in ((x2.grad, x1.grad), (w.grad, layer.weight.grad), (b.grad, layer.bias.grad)):
        assert torch.allclose(a, ref, rtol=1e-5, atol=1e-6 * float(ref.abs().max()))


@pytest.mark.gpu
def test_rpfq_wide_linear_op_matches_packed(golden):
    import quant_models  # noqa: F401
    from quant_models import ops
    from quant_models import packing as P

    lc = P.quantize_layer(torch.from_numpy(golden["w_weight"]), "complex_phase_v2", "complex_phase_v2")
    pw = ops.pack_layer([p.to(DEV) for p in lc.planes], [s.to(DEV) for s in lc.scale_re],
                        [s.to(DEV) for s in lc.scale_im], lc.n_complex, lc.k_complex, lc.codebook, lc.stages)
    x = torch.randn(9, 96, device=DEV).half()
    bias = torch.randn(64, device=DEV)
    y_op = torch.ops.rpfq.wide_linear(x, pw.blob, pw.n_complex, pw.k_complex, pw.codebook, pw.stages, pw.block,
                                      None, bias)
    assert torch.equal(y_op, pw.linear(x, bias))
    assert torch.equal(torch.ops.rpfq.act_quant(x.float(), 4), ops.act_quant(x.float(), 4))


@pytest.mark.gpu
def test_rpfq_wide_linear_op_backward(golden):
    """The registered backward of torch.ops.rpfq.wide_linear: the input
    gradient is PackedWide.grad_x on the same blob (bit for bit) and the
    bias gradient the column sum of grad_y (kernel.py:585-588)."""
    import quant_models  # noqa: F401
    from quant_models import ops
    from quant_models import packing as P

    lc = P.quantize_layer(torch.from_numpy(golden["w_weight"]), "complex_phase_v2", "complex_phase_v2")
    pw = ops.pack_layer([p.to(DEV) for p in lc.planes], [s.to(DEV) for s in lc.scale_re],
                        [s.to(DEV) for s in lc.scale_im], lc.n_complex, lc.k_complex, lc.codebook, lc.stages)
    x = torch.randn(3, 9, 96, device=DEV).half().requires_grad_(True)
    bias = torch.randn(64, device=DEV).requires_grad_(True)
    y = torch.ops.rpfq.wide_linear(x, pw.blob, pw.n_complex, pw.k_complex, pw.codebook, pw.stages, pw.block,
                                   None, bias)
    gy = torch.randn(y.shape, device=DEV).half()
    y.backward(gy)
    assert x.grad.dtype == torch.float16 and bias.grad.dtype == torch.float32
    assert torch.equal(x.grad, pw.grad_x(gy, torch.float16))
    assert torch.allclose(bias.grad, gy.float().reshape(-1, 64).sum(0), rtol=1e-6, atol=1e-5)
