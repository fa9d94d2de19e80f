"""Pin the CPU oracle (oracle/rpfq_oracle.py) before trusting it.

Each function is checked against what the reference itself produced
(tests/golden/golden_v1.npz, written by tests/golden/gen_golden.py from
quant_i.py and the exporter), against closed forms chosen so a plausible
mistake (swapped tie quadrant, wrong sign, transposed block, wrong pack
order) fails, and against the compiled reference C++ when oracle/_ref exists.
"""
import math

import numpy as np
import pytest

from oracle import rpfq_oracle as O

F32 = np.float32


# -- axis masks ---------------------------------------------------------------
def test_axis_masks_golden(golden):
    got = np.stack(O.axis_masks(golden["masks_re"], golden["masks_im"])).astype(np.uint8)
    assert np.array_equal(got, golden["masks_out"])


@pytest.mark.parametrize("re,im,expect", [
    (1.0, 0.5, "real_pos"), (-1.0, 0.5, "real_neg"), (0.5, 1.0, "imag_pos"), (0.5, -1.0, "imag_neg"),
    (0.5, 0.5, "imag_pos"),    # tie in quadrant I -> +i
    (-0.5, 0.5, "real_neg"),   # tie in quadrant II -> -1
    (-0.5, -0.5, "imag_neg"),  # tie in quadrant III -> -i
    (0.5, -0.5, "real_pos"),   # tie in quadrant IV -> +1
    (0.0, 0.0, "real_pos"), (-0.0, 0.0, "real_pos"), (0.0, -0.0, "real_pos"),
    (0.0, 1.0, "imag_pos"), (-2.0, 0.0, "real_neg"),
])
def test_axis_masks_closed_form(re, im, expect):
    names = ["real_pos", "real_neg", "imag_pos", "imag_neg"]
    masks = O.axis_masks(np.array([re], F32), np.array([im], F32))
    assert [names[i] for i, m in enumerate(masks) if m[0]] == [expect]


# -- residual stages (training semantics) --------------------------------------
def _stage_codes(v_re, v_im):
    """Codes recovered from quantized stage values."""
    c = np.zeros(v_re.shape, np.uint8)
    c[v_re > 0] = 1
    c[(v_re == 0) & (v_im < 0)] = 2
    c[(v_re == 0) & (v_im > 0)] = 3
    return c


@pytest.mark.parametrize("plane", ["u", "w"])
@pytest.mark.parametrize("steps", [2, 4])
def test_residual_stages_golden(golden, plane, steps):
    u_re, u_im, w_re, w_im = O.decompose(golden["w_weight"])
    re, im = (u_re, u_im) if plane == "u" else (w_re, w_im)
    q_re, q_im, stages = O.residual_quantize(re, im, steps)
    for s, (codes, s_re, s_im) in enumerate(stages):
        g_re = golden[f"stage_{plane}_v{steps}_{s}_re"]
        g_im = golden[f"stage_{plane}_v{steps}_{s}_im"]
        assert np.array_equal(codes, _stage_codes(g_re, g_im)), f"stage {s} codes"
        # scales: float32 sums in a different order -> within 2 ulp
        ref_sr = np.abs(g_re[g_re != 0]).max() if np.any(g_re != 0) else 0
        ref_si = np.abs(g_im[g_im != 0]).max() if np.any(g_im != 0) else 0
        assert abs(float(s_re) - float(ref_sr)) <= 2 * np.spacing(F32(ref_sr))
        assert abs(float(s_im) - float(ref_si)) <= 2 * np.spacing(F32(ref_si))
    assert np.allclose(q_re, golden[f"resq_{plane}_v{steps}_re"], rtol=0, atol=1e-7)
    assert np.allclose(q_im, golden[f"resq_{plane}_v{steps}_im"], rtol=0, atol=1e-7)


def test_safe_mean_abs_closed_form():
    x = np.array([1.0, -2.0, 3.0, -4.0], F32)
    assert O.safe_mean_abs(x, np.array([1, 1, 0, 0], bool), 1e-5) == F32(1.5)
    assert O.safe_mean_abs(x, np.zeros(4, bool), 1e-5) == F32(1e-5)  # empty mask -> clamp
    assert O.safe_mean_abs(np.zeros(4, F32), np.ones(4, bool), 1e-6) == F32(1e-6)


# -- packing ------------------------------------------------------------------
def test_pack_unpack_all_bytes():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256)
    codes = O.unpack_codes(b)
    for v in range(256):
        assert list(codes[0, 4 * v:4 * v + 4]) == [(v >> (2 * j)) & 3 for j in range(4)]
    assert np.array_equal(O.pack_codes(codes), b)


def test_pack_low_bits_first():
    assert O.pack_codes(np.array([[1, 2, 3, 0]], np.uint8))[0, 0] == 1 | (2 << 2) | (3 << 4)
    assert np.array_equal(O.unpack_codes4(O.pack_codes4(np.array([[3, 12, 15, 0]], np.uint8))),
                          [[3, 12, 15, 0]])


def test_codebook_matches_reference_table():
    # export_rpfq_vit_to_mlx.py:598-603: 00=-1, 01=+1, 10=-i, 11=+i
    assert O.AXIS_CODEBOOK.tolist() == [[-1, 0], [1, 0], [0, -1], [0, 1]]


# -- exporter semantics ----------------------------------------------------------
@pytest.mark.parametrize("plane", ["u", "w"])
def test_export_stages_golden(golden, plane):
    u_re, u_im, w_re, w_im = O.decompose(golden["w_weight"])
    re, im = (u_re, u_im) if plane == "u" else (w_re, w_im)
    out = O.residual_quantize_export(re, im, 2)
    for s, (codes, g_re, g_im) in enumerate(out):
        gc = golden[f"exp_L_{plane}_s{s}_codes"]
        # golden planes are padded to 256 complex columns/rows with code 0
        assert np.array_equal(O.pack_codes(codes), gc[:codes.shape[0], :codes.shape[1] // 4])
        assert np.all(gc[codes.shape[0]:] == 0) and np.all(gc[:, codes.shape[1] // 4:] == 0)
        assert np.float16(g_re) == golden[f"exp_L_{plane}_s{s}_gamma_real"][0, 0]
        assert np.float16(g_im) == golden[f"exp_L_{plane}_s{s}_gamma_imag"][0, 0]


def test_dequantize_export_weight_golden(golden):
    """A_q of the exported planes (quantized_forward_weight) bit-exact."""
    n_c, k_c = 32, 48
    planes = []
    for plane in "uw":
        for s in range(2):
            codes = O.unpack_codes(golden[f"exp_L_{plane}_s{s}_codes"])[:n_c, :k_c]
            g_re = golden[f"exp_L_{plane}_s{s}_gamma_real"][:n_c, 0]
            g_im = golden[f"exp_L_{plane}_s{s}_gamma_imag"][:n_c, 0]
            planes.append((codes, O.inv_gamma(g_re), O.inv_gamma(g_im), plane))
    # dequantize_axis divides by gamma; +-1/g == +-(1/g) exactly
    d_re, d_im = O.dequantize_axis(golden["exp_L_u_s0_codes"], golden["exp_L_u_s0_gamma_real"],
                                   golden["exp_L_u_s0_gamma_imag"], 256, 256, 256)
    m_re, m_im = O.dequant_codes(planes[0][0], planes[0][1], planes[0][2], gamma=False)
    assert np.array_equal(d_re[:n_c, :k_c], m_re) and np.array_equal(d_im[:n_c, :k_c], m_im)
    assert np.array_equal(O.wide_weight(planes), golden["exp_aq"])


def test_export_block_aligned_golden(golden):
    """Unpadded export (K' = 256, one gamma block) on a second weight."""
    u_re, u_im, w_re, w_im = O.decompose(golden["expb_weight"])
    for plane, (re, im) in (("u", (u_re, u_im)), ("w", (w_re, w_im))):
        for s, (codes, g_re, g_im) in enumerate(O.residual_quantize_export(re, im, 2)):
            assert np.array_equal(O.pack_codes(codes), golden[f"expb_L_{plane}_s{s}_codes"])
            assert np.all(golden[f"expb_L_{plane}_s{s}_gamma_real"] == np.float16(g_re))


# -- widely-linear algebra ---------------------------------------------------------
def test_decompose_recompose_exact():
    rng = np.random.default_rng(0)
    a = (rng.integers(-64, 64, size=(12, 20)) * 2).astype(F32)  # even integers: halves exact
    assert np.array_equal(O.recompose(*O.decompose(a)), a)


def test_widely_linear_identity():
    """F.linear on [re|im] features == U x + W conj(x) (quant_i.py:519-554)."""
    rng = np.random.default_rng(1)
    a = rng.standard_normal((10, 14)).astype(np.float64)
    u_re, u_im, w_re, w_im = (p.astype(np.float64) for p in O.decompose(a.astype(F32)))
    a32 = a.astype(F32).astype(np.float64)
    x = rng.standard_normal(14)
    xc = x[:7] + 1j * x[7:]
    y = (u_re + 1j * u_im) @ xc + (w_re + 1j * w_im) @ np.conj(xc)
    assert np.allclose(np.concatenate([y.real, y.imag]), a32 @ x, atol=1e-5)


def test_phase_linear_brute_force():
    """phase_linear vs an explicit complex sum on a tiny case."""
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 4, size=(3, 8), dtype=np.uint8)
    inv = rng.uniform(1, 2, size=3).astype(F32)
    xr, xi = rng.standard_normal((2, 8)), rng.standard_normal((2, 8))
    y_re, y_im = O.phase_linear(xr, xi, codes, inv, inv, conj_input=True)
    unit = {0: -1, 1: 1, 2: -1j, 3: 1j}
    for t in range(2):
        for n in range(3):
            w = np.array([unit[c] for c in codes[n]]) * float(inv[n])
            ref = np.sum(w * np.conj(xr[t] + 1j * xi[t]))
            assert abs(ref.real - y_re[t, n]) < 1e-9 and abs(ref.imag - y_im[t, n]) < 1e-9
    y2_re, y2_im = O.phase_linear(xr, xi, codes, inv, inv, conj_input=False)
    w0 = np.array([unit[c] for c in codes[0]]) * float(inv[0])
    ref = np.sum(w0 * (xr[0] + 1j * xi[0]))
    assert abs(ref.real - y2_re[0, 0]) < 1e-9 and abs(ref.imag - y2_im[0, 0]) < 1e-9


# -- activation fake quant ---------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_act_quant_golden(golden, bits):
    qr, qi = O.act_quant(golden["act_xr"], golden["act_xi"], bits)
    assert np.array_equal(qr, golden[f"act{bits}_re"]) and np.array_equal(qi, golden[f"act{bits}_im"])


def test_act_quant_ties_half_even(golden):
    # row 0 has max 7.0 -> scale 1 for 4 bits: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2, -2.5 -> -2
    qr, _ = O.act_quant(golden["act_xr"], golden["act_xi"], 4)
    assert list(qr[0, :6]) == [7.0, 0.0, 2.0, 2.0, -0.0, -2.0]
    x = golden["actr_x"]
    q = np.concatenate(O.act_quant(x[:, :24], x[:, 24:], 4), axis=1)
    assert np.array_equal(q, golden["actr_q"])


# -- full layer ------------------------------------------------------------------
@pytest.mark.parametrize("method,steps", [("complex_phase_v1", 1), ("complex_phase_v2", 2),
                                          ("complex_phase_v3", 3), ("complex_phase_v4", 4)])
@pytest.mark.parametrize("act", [0, 1])
def test_linear_forward_golden(golden, method, steps, act):
    y, a_q = O.linear_forward(golden["fwd_x"], golden["w_weight"], golden["fwd_bias"], steps, steps,
                              4 if act else None)
    tag = f"{method}_a{act}_r0"
    # scale sums differ from torch's float32 order by <= 2 ulp of each scale
    # (~0.016 here, ulp 1.9e-9); A = W + U sums up to 2 stages of U and W
    assert np.allclose(a_q, golden[f"fwd_aq_{tag}"], rtol=0, atol=4 * steps * 2e-9)
    assert np.allclose(y, golden[f"fwd_y_{tag}"], rtol=1e-5, atol=1e-5)


def _rot_cos_sin():
    """float32 (cos, sin) of the golden layers' rotation angles (0.3 for U,
    -0.2 for W) evaluated by torch on the CPU, as the reference did."""
    import torch

    out = []
    for t in (0.3, -0.2):
        th = torch.full((1,), t, dtype=torch.float32)
        out.append((np.float32(torch.cos(th).item()), np.float32(torch.sin(th).item())))
    return tuple(out)


@pytest.mark.parametrize("method,kind,steps", [("complex_phase_v1", "axis", 1), ("complex_phase_v2", "axis", 2),
                                               ("complex_phase_v3", "axis", 3), ("complex_phase_v4", "axis", 4),
                                               ("complex_phase_new_v2", "sign", 2)])
@pytest.mark.parametrize("rot", [0, 1])
def test_quantized_weight_golden(golden, method, kind, steps, rot):
    a_q, st_u, st_w = O.quantized_weight(golden["w_weight"], kind, steps, kind, steps,
                                         _rot_cos_sin() if rot else None)
    assert len(st_u) == steps and len(st_w) == steps
    ref = golden[f"fwd_aq_{method}_a0_r{rot}"]
    # float64 scale sums vs torch's float32 order: <= 2 ulp per scale (ulp
    # ~1.9e-9 here), summed over the stages of U and W
    assert np.allclose(a_q, ref, rtol=0, atol=4 * steps * 2e-9)
    # a wrong sign, axis or rotation direction moves entries by a whole scale
    assert np.abs(a_q - ref).max() < 1e-6


def test_quantize_sign_phase_closed_form():
    re = np.array([[0.5, -0.25], [-0.0, 0.0]], np.float32)
    im = np.array([[-1.0, 0.75], [0.0, -0.5]], np.float32)
    codes, s_re, s_im, q_re, q_im = O.quantize_sign_phase(re, im)
    assert s_re == np.float32(0.75 / 4) and s_im == np.float32(2.25 / 4)
    # bit0 = re >= 0 (-0 counts as >= 0), bit1 = im >= 0
    assert codes.tolist() == [[1, 2], [3, 1]]
    assert q_re.tolist() == [[s_re, -s_re], [s_re, s_re]] and q_im.tolist() == [[-s_im, s_im], [s_im, -s_im]]
    # an all-zero plane takes the 1e-6 floor
    _, s0, _, _, _ = O.quantize_sign_phase(np.zeros((2, 2), np.float32), np.ones((2, 2), np.float32))
    assert s0 == np.float32(1e-6)


# -- 16-PSK (build-defined codebook: parity unpinned by the reference) -------------
def test_psk16_closed_form():
    cb = O.psk16_codebook().astype(np.float64)
    z = cb[:, 0] + 1j * cb[:, 1]
    assert np.all(np.abs(np.abs(z) - 1) < 1e-7)
    ang = np.mod(np.angle(z), 2 * math.pi)
    assert np.allclose(ang, 2 * math.pi * np.arange(16) / 16, atol=1e-6)
    assert cb[0].tolist() == [1, 0] and cb[4].tolist() == [0, 1] and cb[8].tolist() == [-1, 0] \
        and cb[12].tolist() == [0, -1]
    assert np.array_equal(cb[2], cb[2][::-1])  # exact diagonal symmetry


# -- compiled reference (oracle/_ref) -----------------------------------------------
def _ref():
    from oracle import ref_lib
    lib = ref_lib.load()
    if lib is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    return ref_lib


def test_oracle_phase_linear_vs_compiled_reference():
    ref = _ref()
    rng = np.random.default_rng(5)
    n, k = 40, 512
    codes = rng.integers(0, 4, size=(n, k), dtype=np.uint8)
    g_re = (1 / rng.uniform(0.01, 0.1, (n, 2))).astype(np.float16)
    g_im = (1 / rng.uniform(0.01, 0.1, (n, 2))).astype(np.float16)
    xr = rng.standard_normal((3, k)).astype(F32)
    xi = rng.standard_normal((3, k)).astype(F32)
    yr, yi = ref.phase_linear(xr, xi, codes, g_re, g_im, 256)
    inv_re = np.repeat(O.inv_gamma(g_re), 256, axis=1)
    inv_im = np.repeat(O.inv_gamma(g_im), 256, axis=1)
    orr, ori = O.phase_linear(xr, xi, codes, inv_re, inv_im, conj_input=True)
    assert np.allclose(yr, orr, rtol=1e-5, atol=1e-4) and np.allclose(yi, ori, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_oracle_wide_linear_vs_compiled_reference(mode):
    """mode 0: wideLinearReference (fp32); 1: the reference's fp16 fused
    coefficient cache; 2: its fused scalar path."""
    ref = _ref()
    rng = np.random.default_rng(6)
    n, k = 48, 256
    planes = [rng.integers(0, 4, size=(n, k), dtype=np.uint8) for _ in range(4)]
    g_re = [(1 / rng.uniform(0.01, 0.1, (n, 1))).astype(np.float16) for _ in range(4)]
    g_im = [(1 / rng.uniform(0.01, 0.1, (n, 1))).astype(np.float16) for _ in range(4)]
    bias = rng.standard_normal(2 * n).astype(F32)
    x = rng.standard_normal((7, 2 * k)).astype(F32)
    y = ref.wide_linear(x, planes, g_re, g_im, bias, k, mode, 2)
    op = [(p, O.inv_gamma(a)[:, 0], O.inv_gamma(b)[:, 0], kd) for p, a, b, kd in zip(planes, g_re, g_im, "uuww")]
    a = O.wide_weight(op)
    yo = O.wide_linear(x, op, bias)
    scale = np.abs(x.astype(np.float64)) @ np.abs(a.astype(np.float64)).T + np.abs(bias)
    tol = (2.0 ** -10 if mode == 1 else 1e-6) * scale + 1e-5
    assert np.all(np.abs(y - yo) <= tol)


# --------------------------------------------------------------------------
# fp16 operand of the HIP kernels (build-defined: pinned by exact arithmetic)
# --------------------------------------------------------------------------
def _fp16_round_exact(q):
    """Round a Fraction to the nearest fp16 (ties to even) by exhaustive
    neighbour search on the fp16 grid -- independent of numpy's rounding."""
    from fractions import Fraction
    if q == 0:
        return np.float16(0.0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = max(math.floor(math.log2(a)) if a > 0 else -24, -14)
    step = Fraction(2) ** (e - 10)  # fp16 spacing at this binade (subnormals: 2^-24)
    lo = (a // step) * step
    hi = lo + step
    if a - lo < hi - a:
        v = lo
    elif hi - a < a - lo:
        v = hi
    else:  # tie: even significand
        v = lo if (lo / step) % 2 == 0 else hi
    if v > Fraction(65504):
        return np.float16(sign * np.inf)
    return np.float16(sign * float(v))


def test_fp16_add_exact_rounding():
    from fractions import Fraction
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 0x7c00, size=(4000, 2), dtype=np.uint32).astype(np.uint16)  # finite magnitudes
    signs = rng.integers(0, 2, size=(4000, 2), dtype=np.uint16) << 15
    h = (bits | signs).view(np.float16)
    # add classes the random draw rarely hits: exact ties, cancellation, subnormals
    extra = np.array([[1.0, 2.0 ** -11], [1.0, 3 * 2.0 ** -12], [2.0 ** -24, 2.0 ** -24], [-6.1e-5, 6.1e-5],
                      [65504.0, 16.0], [0.1, -0.1], [1.0009765625, 2.0 ** -11]], np.float64).astype(np.float16)
    h = np.concatenate([h, extra])
    got = O.fp16_add(h[:, 0], h[:, 1])
    for (a, b), g in zip(h, got):
        want = _fp16_round_exact(Fraction(float(a)) + Fraction(float(b)))
        assert g.view(np.uint16) == want.view(np.uint16) or (g == 0 and want == 0), (a, b, g, want)


def _wide_case(seed, n=24, k=40, codebook="axis", rot=None):
    rng = np.random.default_rng(seed)
    ncode = 16 if codebook == "psk16" else 4
    planes = []
    for kind in "uuww" if codebook != "psk16" else "uw":
        planes.append((rng.integers(0, ncode, size=(n, k), dtype=np.uint8),
                       rng.uniform(0.01, 0.1, n).astype(F32), rng.uniform(0.01, 0.1, n).astype(F32), kind))
    return planes


@pytest.mark.parametrize("codebook,rot", [("axis", None), ("sign", None), ("psk16", None),
                                          ("axis", ((0.95533645, 0.29552022), (0.98006660, -0.19866933)))])
def test_recompose_fp16_bound_and_identities(codebook, rot):
    rotation = None if rot is None else tuple((F32(c), F32(s)) for c, s in rot)
    planes = _wide_case(12, codebook=codebook)
    a = O.wide_weight(planes, codebook, rotation).astype(np.float64)
    a16 = O.wide_weight(planes, codebook, rotation, fp16=True).astype(np.float64)
    mag = O.wide_magnitude(planes, codebook, rotation)
    u = 2.0 ** -11
    assert np.all(np.abs(a16 - a) <= (2 * u + u * u) * mag + 2.0 ** -25)
    # every value is an fp16 number
    assert np.array_equal(a16.astype(np.float16).astype(np.float64), a16)
    # block identities of the fused layout: A22 = -(W_re) + U_re and A11 = W_re + U_re
    # swap roles under W <-> conj-free negation: with U = 0, A11 = W_re = -A22
    u_re, u_im, w_re, w_im = O.wide_parts(planes, codebook, rotation)
    z = np.zeros_like(u_re)
    only_w = O.recompose_fp16(z, z, w_re, w_im).astype(np.float64)
    n, k = u_re.shape
    assert np.array_equal(only_w[:n, :k], -only_w[n:, k:])
    assert np.array_equal(only_w[:n, k:], only_w[n:, :k])
    only_u = O.recompose_fp16(u_re, u_im, z, z).astype(np.float64)
    assert np.array_equal(only_u[:n, :k], only_u[n:, k:])
    assert np.array_equal(only_u[:n, k:], -only_u[n:, :k])
    # exact where fp16 represents both terms and their sum (W = 0: coefficient = fp16(U))
    assert np.array_equal(only_u[:n, :k], u_re.astype(np.float16).astype(np.float64))


@pytest.mark.parametrize("codebook,rot", [("axis", None), ("sign", None), ("psk16", None),
                                          ("axis", ((0.95533645, 0.29552022), (0.98006660, -0.19866933)))])
def test_recompose_split_fp16(codebook, rot):
    """The column-split operand: its correctly rounded fp16 value is the
    fused operand bit for bit (fp16_add is pinned by exact rationals), it is
    within u (|U| + |W|) of the reference A_q (one fp16 rounding per part, no
    rounding of the sum), and with W = 0 it is fp16(U) exactly."""
    rotation = None if rot is None else tuple((F32(c), F32(s)) for c, s in rot)
    planes = _wide_case(13, codebook=codebook)
    a = O.wide_weight(planes, codebook, rotation).astype(np.float64)
    a16 = O.wide_weight(planes, codebook, rotation, fp16=True).astype(np.float64)
    asp = O.wide_weight(planes, codebook, rotation, fp16="split")
    assert asp.dtype == np.float64
    assert np.array_equal(asp.astype(np.float16).astype(np.float64), a16)
    mag = O.wide_magnitude(planes, codebook, rotation)
    u = 2.0 ** -11
    assert np.all(np.abs(asp - a) <= u * mag + 2.0 ** -25)
    assert not np.array_equal(asp, a16)  # the sums are not all fp16 numbers
    u_re, u_im, w_re, w_im = O.wide_parts(planes, codebook, rotation)
    z = np.zeros_like(u_re)
    n, k = u_re.shape
    only_u = O.recompose_split_fp16(u_re, u_im, z, z)
    assert np.array_equal(only_u[:n, :k], u_re.astype(np.float16).astype(np.float64))
    assert np.array_equal(only_u[:n, k:], -u_im.astype(np.float16).astype(np.float64))


@pytest.mark.parametrize("codebook,rot", [("axis", None), ("psk16", None),
                                          ("axis", ((0.95533645, 0.29552022), (0.98006660, -0.19866933)))])
@pytest.mark.parametrize("fp16", [False, True])
def test_wide_linear_grad_x_adjoint_and_autograd(codebook, rot, fp16):
    """wide_linear_grad_x is the adjoint of the pinned forward,
    <gy, wide_linear(x)> = <wide_linear_grad_x(gy), x>, and equals torch
    autograd of F.linear on the same A (N' != K', so a transposed operand
    cannot pass)."""
    import torch
    rotation = None if rot is None else tuple((F32(c), F32(s)) for c, s in rot)
    planes = _wide_case(14, n=24, k=40, codebook=codebook)
    rng = np.random.default_rng(15)
    x = rng.standard_normal((5, 80))
    gy = rng.standard_normal((5, 48))
    y = O.wide_linear(x, planes, None, codebook, rotation, fp16_weight=fp16)
    gx = O.wide_linear_grad_x(gy, planes, codebook, rotation, fp16_weight=fp16)
    assert gx.shape == x.shape
    lhs, rhs = float(np.sum(gy * y)), float(np.sum(gx * x))
    assert abs(lhs - rhs) <= 1e-12 * (np.abs(gy) @ np.abs(O.wide_weight(planes, codebook, rotation, fp16=fp16))
                                      .astype(np.float64) @ np.abs(x).T).sum()
    a = torch.from_numpy(O.wide_weight(planes, codebook, rotation, fp16=fp16).astype(np.float64))
    xt = torch.from_numpy(x).requires_grad_(True)
    torch.nn.functional.linear(xt, a).backward(torch.from_numpy(gy))
    assert np.allclose(xt.grad.numpy(), gx, rtol=1e-12, atol=1e-12)
