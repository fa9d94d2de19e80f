"""GPU parity of the HIP kernels against the CPU oracle (through the C ABI).

Bars: code unpacking, fused-weight decode and activation fake-quant are
bit-exact; contractions are checked (a) tightly against the float64 oracle fed
the very operands the MFMA consumes (fp16 inputs / fp16-rounded coefficients),
and (b) against the exact reference weight within the rigorous fp16-rounding
bound  |dy| <= 2^-11 * sum_k |x_k| |A_k| + 1e-5  written in each test.
"""
import numpy as np
import pytest
import torch

from oracle import rpfq_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def qm():
    from quant_models import _native, ops
    return ops, _native


def rng(seed):
    return np.random.default_rng(seed)


def ulp_distance(a, b):
    """Elementwise distance in units in the last place of a's dtype (fp16,
    bf16 or float32; +0 and -0 coincide)."""
    it = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}[a.dtype]
    sign = -(2 ** 15) if it == torch.int16 else -(2 ** 31)

    def key(t):
        k = t.contiguous().view(it).long()
        return torch.where(k < 0, -(k - sign), k)
    return (key(a) - key(b)).abs()


def rand_gamma(r, rows, nblk, lo=0.01, hi=0.1):
    """fp16 gammas = fp16(1/s), s ~ U(lo, hi) per (row, block)."""
    s = r.uniform(lo, hi, size=(rows, nblk))
    return (1.0 / s).astype(np.float16)


def tdev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


# ---------------------------------------------------------------------------
# unpack (export_rpfq_vit_to_mlx.py:227-254) -- bit-exact
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,k,block", [(7, 64, 32), (64, 768, 256), (3, 40, 0)])
def test_unpack_axis_bit_exact(rows, k, block):
    ops, _ = qm()
    r = rng(1)
    codes = r.integers(0, 4, size=(rows, k), dtype=np.uint8)
    packed = O.pack_codes(codes)
    nblk = 1 if block == 0 else -(-k // block)
    g_re, g_im = rand_gamma(r, rows, nblk), rand_gamma(r, rows, nblk)
    re, im = ops.unpack(tdev(packed), 2, k, tdev(g_re.view(np.float16)), tdev(g_im), block)
    ref_re, ref_im = O.dequantize_axis(packed, g_re, g_im, rows, k, block if block else k)
    assert np.array_equal(re.cpu().numpy(), ref_re)
    assert np.array_equal(im.cpu().numpy(), ref_im)
    # unit codebook
    ure, uim = ops.unpack(tdev(packed), 2, k)
    cb = O.AXIS_CODEBOOK[codes]
    assert np.array_equal(ure.cpu().numpy(), cb[..., 0]) and np.array_equal(uim.cpu().numpy(), cb[..., 1])


def test_unpack_all_byte_values():
    """Every byte value 0..255 decodes to its four codes (brute force)."""
    ops, _ = qm()
    packed = np.arange(256, dtype=np.uint8).reshape(256, 1)
    re, im = ops.unpack(tdev(packed), 2, 4)
    codes = O.unpack_codes(packed)
    cb = O.AXIS_CODEBOOK[codes]
    assert np.array_equal(re.cpu().numpy(), cb[..., 0]) and np.array_equal(im.cpu().numpy(), cb[..., 1])


def test_unpack_psk16_bit_exact():
    ops, _ = qm()
    r = rng(2)
    codes = r.integers(0, 16, size=(9, 32), dtype=np.uint8)
    packed = O.pack_codes4(codes)
    re, im = ops.unpack(tdev(packed), 4, 32)
    cb = O.psk16_codebook()[codes]
    assert np.array_equal(re.cpu().numpy(), cb[..., 0]) and np.array_equal(im.cpu().numpy(), cb[..., 1])


# ---------------------------------------------------------------------------
# activation fake-quant (quant_i.py:438-455) -- bit-exact in float32
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_act_quant_bit_exact(bits, golden):
    ops, _ = qm()
    x = np.concatenate([golden["act_xr"], golden["act_xi"]], axis=1)
    y = ops.act_quant(tdev(x), bits).cpu().numpy()
    assert np.array_equal(y[:, :8], golden[f"act{bits}_re"])
    assert np.array_equal(y[:, 8:], golden[f"act{bits}_im"])
    r = rng(3)
    xs = (r.standard_normal((37, 2 * 300)) * 3).astype(np.float32)
    ys = ops.act_quant(tdev(xs), bits).cpu().numpy()
    qr, qi = O.act_quant(xs[:, :300], xs[:, 300:], bits)
    assert np.array_equal(ys, np.concatenate([qr, qi], axis=1))


# ---------------------------------------------------------------------------
# single plane phase linear (phase_linear.cpp:119-164)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("m,k,n,block,conj", [(1576, 768, 3072, 0, False), (33, 64, 200, 32, True),
                                              (130, 256, 129, 64, False), (1, 512, 128, 256, True),
                                              (77, 160, 300, 0, True), (45, 224, 70, 96, False)])
def test_phase_linear_f32_split(m, k, n, block, conj):
    """Config 1 at full size and ragged shapes: M and N off the 64 x 128
    tile, an odd number of 32-column k-steps (the two-step pipeline's tail),
    per-block scales with a partial last block."""
    ops, _ = qm()
    r = rng(10 + m)
    xr = r.standard_normal((m, k)).astype(np.float32)
    xi = r.standard_normal((m, k)).astype(np.float32)
    codes = r.integers(0, 4, size=(n, k), dtype=np.uint8)
    nblk = 1 if block == 0 else -(-k // block)
    g_re, g_im = rand_gamma(r, n, nblk), rand_gamma(r, n, nblk)
    yr, yi = ops.phase_linear(tdev(xr), tdev(xi), tdev(O.pack_codes(codes)), tdev(g_re), tdev(g_im),
                              block, conj_x=conj)
    bs = block if block else k
    inv_re = np.repeat(O.inv_gamma(g_re), bs, axis=1)[:, :k]
    inv_im = np.repeat(O.inv_gamma(g_im), bs, axis=1)[:, :k]
    ref_re, ref_im = O.phase_linear(xr, xi, codes, inv_re, inv_im, conj_input=conj)
    scale = max(np.abs(ref_re).max(), np.abs(ref_im).max())
    # fp32 x split into two fp16 terms: relative error ~2^-22 per term
    assert np.abs(yr.cpu().numpy() - ref_re).max() <= 2e-6 * scale + 1e-6
    assert np.abs(yi.cpu().numpy() - ref_im).max() <= 2e-6 * scale + 1e-6


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_phase_linear_half_inputs(dt):
    ops, _ = qm()
    r = rng(20)
    m, k, n = 70, 96, 160
    xr = torch.from_numpy(r.standard_normal((m, k)).astype(np.float32)).to(dt)
    xi = torch.from_numpy(r.standard_normal((m, k)).astype(np.float32)).to(dt)
    codes = r.integers(0, 4, size=(n, k), dtype=np.uint8)
    g_re, g_im = rand_gamma(r, n, 1), rand_gamma(r, n, 1)
    yr, yi = ops.phase_linear(xr.to(DEV), xi.to(DEV), tdev(O.pack_codes(codes)), tdev(g_re), tdev(g_im), 0)
    ref_re, ref_im = O.phase_linear(xr.float().numpy(), xi.float().numpy(), codes, O.inv_gamma(g_re)[:, 0],
                                    O.inv_gamma(g_im)[:, 0], conj_input=True)
    scale = max(np.abs(ref_re).max(), np.abs(ref_im).max())
    assert np.abs(yr.cpu().numpy() - ref_re).max() <= 2e-6 * scale + 1e-6
    assert np.abs(yi.cpu().numpy() - ref_im).max() <= 2e-6 * scale + 1e-6


# ---------------------------------------------------------------------------
# widely-linear layer: pack -> decode (bit-exact) -> GEMM
# ---------------------------------------------------------------------------
def make_wide(r, n_c, k_c, codebook="axis", stages=2, per_row=True, block=0):
    """Random planes + per-(plane,row[,block]) scales in the oracle format."""
    _, N = qm()
    nplanes = 2 if codebook in ("psk16", "table") else 2 * stages
    nblk = 1 if block == 0 else -(-k_c // block)
    planes_np, sre, sim, packed = [], [], [], []
    for p in range(nplanes):
        if codebook == "table":  # 4-bit indices into per-row tables of 16 signed values
            c = r.integers(0, 16, size=(n_c, k_c), dtype=np.uint8)
            packed.append(O.pack_codes4(c))
            sgn = lambda: np.where(r.random((n_c, 16)) < 0.5, -1.0, 1.0)  # noqa: E731
            planes_np.append(c)
            sre.append((r.uniform(0.01, 0.2, size=(n_c, 16)) * sgn()).astype(np.float32))
            sim.append((r.uniform(0.01, 0.2, size=(n_c, 16)) * sgn()).astype(np.float32))
            continue
        if codebook == "psk16":
            c = r.integers(0, 16, size=(n_c, k_c), dtype=np.uint8)
            packed.append(O.pack_codes4(c))
        else:
            c = r.integers(0, 4, size=(n_c, k_c), dtype=np.uint8)
            packed.append(O.pack_codes(c))
        s1 = r.uniform(0.01, 0.1, size=(n_c, nblk)).astype(np.float32)
        s2 = r.uniform(0.01, 0.1, size=(n_c, nblk)).astype(np.float32)
        if not per_row:
            s1[:] = s1[0, 0]
            s2[:] = s2[0, 0]
        planes_np.append(c)
        sre.append(s1)
        sim.append(s2)
    kinds = (["u"] * (nplanes // 2)) + (["w"] * (nplanes // 2))
    cb = {"axis": N.CB_AXIS, "sign": N.CB_SIGN, "psk16": N.CB_PSK16, "table": N.CB_TABLE}[codebook]
    return planes_np, packed, sre, sim, kinds, cb, nblk


def oracle_planes(planes_np, sre, sim, kinds, k_c, block, codebook="axis"):
    """Expand per-block scales to per-element for the oracle (value tables
    of the 'table' codebook pass through)."""
    if codebook == "table":
        return list(zip(planes_np, sre, sim, kinds))
    out = []
    bs = block if block else k_c
    for c, a, b, kind in zip(planes_np, sre, sim, kinds):
        out.append((c, np.repeat(a, bs, axis=1)[:, :k_c], np.repeat(b, bs, axis=1)[:, :k_c], kind))
    return out


def expand_scales(planes):
    """oracle.wide_weight takes per-row or per-element scales."""
    return planes


CASES = [
    # n_c, k_c, codebook, stages, block, rotation
    (96, 64, "axis", 2, 0, None),
    (1536, 384, "axis", 2, 0, None),
    (50, 48, "axis", 2, 0, None),          # N' and K' not multiples of 32
    (64, 96, "axis", 1, 0, None),          # v1
    (130, 512, "axis", 2, 256, None),      # per-(row, block) scales
    (64, 64, "sign", 2, 0, None),          # new_v2
    (96, 128, "psk16", 1, 0, None),        # 16-PSK
    (128, 96, "axis", 2, 0, ((0.95533645, 0.29552022), (0.98006660, -0.19866933))),  # rotation
    (100, 96, "table", 1, 0, None),        # next_v1: per-row value tables
]


def build_packed(r, case):
    ops, N = qm()
    n_c, k_c, codebook, stages, block, rot = case
    planes_np, packed, sre, sim, kinds, cb, nblk = make_wide(r, n_c, k_c, codebook, stages, True, block)
    pw = ops.PackedWide.from_planes([tdev(p) for p in packed], [tdev(s) for s in sre], [tdev(s) for s in sim],
                                    n_c, k_c, cb, stages, block, rot)
    rotation = None
    if rot is not None:
        rotation = tuple((np.float32(c), np.float32(s)) for c, s in rot)
    oplanes = oracle_planes(planes_np, sre, sim, kinds, k_c, block, codebook)
    a_ref = O.wide_weight(oplanes, codebook, rotation)
    build_packed.last_oplanes, build_packed.last_rotation = oplanes, rotation
    return pw, oplanes, a_ref, codebook, rotation


def operand(pw, m, xdt=torch.float16, ydt=torch.float32, flags=0):
    """The MFMA operand of the launch: "split" on the column-split kernel
    (fp16 U and W products summed in float32, oracle.recompose_split_fp16),
    else True (fused fp16 coefficients, oracle.recompose_fp16)."""
    ops, N = qm()
    return "split" if pw.kernel_for(m, xdt, ydt, flags) == N.KERNEL_GEMV else True


def check_against_oracle(y, xf, bias, oplanes, codebook, rotation, out_ulp=0.0, fp16=True):
    """y from the HIP kernel vs the oracle on the same operands.
    (a) tight: the exact product with the operand the MFMA sees (fp16: see
        operand()), float32 accumulation error only;
    (b) against the reference's float32 A_q: the fp16 fusing bound
        |A16 - A_q| <= (2u + u^2) (|W| + |U|), u = 2^-11, per coefficient
        (the split operand is within u (|W| + |U|))."""
    bias = np.zeros(0) if bias is None else bias
    b = bias if bias.size else 0.0
    a16 = O.wide_weight(oplanes, codebook, rotation, fp16=fp16).astype(np.float64)
    a = O.wide_weight(oplanes, codebook, rotation).astype(np.float64)
    mag = O.wide_magnitude(oplanes, codebook, rotation)
    ax = np.abs(xf)
    y16 = xf @ a16.T + b
    scale = ax @ np.abs(a16).T + np.abs(b)
    assert np.all(np.abs(y - y16) <= 1e-5 * scale + out_ulp * np.abs(y16) + 1e-5)
    yex = xf @ a.T + b
    u = 2.0 ** -11
    assert np.all(np.abs(y - yex) <= (2 * u + u * u) * (ax @ mag.T) + 1e-5 * scale + out_ulp * np.abs(y16) + 1e-5)


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}-{c[2]}{c[3]}-b{c[4]}-r{int(c[5] is not None)}"
                                             for c in CASES])
def test_wide_decode_bit_exact(case):
    r = rng(100)
    pw, _, a_ref, _, _ = build_packed(r, case)
    a = pw.decode().cpu().numpy()
    assert a.shape == a_ref.shape
    assert np.array_equal(a, a_ref)
    a16 = pw.decode(round_fp16=True).cpu().numpy()
    assert np.array_equal(a16, O.wide_weight(build_packed.last_oplanes, case[2], build_packed.last_rotation, fp16=True))


@pytest.mark.parametrize("flags", [0, 2], ids=["auto", "tiled"])
@pytest.mark.parametrize("m", [1, 5, 31, 64, 65, 128, 129, 300])
@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}-{c[2]}{c[3]}-b{c[4]}-r{int(c[5] is not None)}"
                                             for c in CASES])
def test_wide_linear(case, m, flags):
    """flags 0: the kernel the shape selects (streaming for the small
    launches); 2 (RPFQ_FLAG_NO_STREAM): the tiled kernels at every M."""
    r = rng(200 + m)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    k_in = 2 * case[1]
    x = torch.from_numpy(r.standard_normal((m, k_in)).astype(np.float32)).to(torch.float16)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float32, flags=flags).cpu().numpy()
    xf = x.float().numpy().astype(np.float64)
    check_against_oracle(y, xf, bias, oplanes, codebook, rotation, fp16=operand(pw, m, flags=flags))


@pytest.mark.parametrize("m", [77, 300])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.float16, torch.float16), (torch.bfloat16, torch.float32),
                                     (torch.float16, torch.bfloat16)])
def test_wide_linear_dtypes(xdt, ydt, m):
    r = rng(300)
    case = (160, 128, "axis", 2, 0, None)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    x = torch.from_numpy(r.standard_normal((m, 256)).astype(np.float32)).to(xdt)
    y = pw.linear(x.to(DEV), None, out_dtype=ydt).float().cpu().numpy()
    # the kernel converts x to fp16 on load: reference on the same operands
    xf = x.float().to(torch.float16).float().numpy().astype(np.float64)
    out_ulp = {torch.float32: 1e-6, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[ydt]
    check_against_oracle(y, xf, None, oplanes, codebook, rotation, out_ulp)


# row magnitudes of the range-guard tests: far below fp16's normal range,
# inside it, at and beyond its overflow threshold, a zero row
# (the extremes first, so a launch of a few rows holds them too)
RANGE_MAGS = [1e30, 1e-30, 7e4, 0.0, 1e-3, 1e20, 3e-8, 6.5e4, 1.0, 1e10, 1e-20]


def _range_rows(r, m, k_in, xdt):
    mags = np.array([RANGE_MAGS[i % len(RANGE_MAGS)] for i in range(m)])
    x = r.standard_normal((m, k_in)) * mags[:, None]
    return torch.from_numpy(x.astype(np.float32)).to(xdt), mags


def _check_range(y, xf, a16, bias, mags, u_op):
    """Per row: |y - x A16^T - b| <= (u_op + 1e-5) sum |x||A16| + 2^-20 |b|,
    relative to the row's own magnitude (the guard keeps every row inside
    the fp16 operand's range); zero rows give exactly the bias."""
    ref = xf @ a16.T + bias
    scale = np.abs(xf) @ np.abs(a16).T
    assert np.all(np.isfinite(y)), "non-finite outputs"
    bound = (u_op + 1e-5) * scale + 2.0 ** -20 * np.abs(bias) + 1e-44
    bad = np.abs(y - ref) > bound
    assert not bad.any(), [(float(mags[i]), float((np.abs(y - ref)[i] / bound[i]).max()))
                           for i in sorted(set(np.nonzero(bad)[0].tolist()))[:5]]
    zero = mags == 0
    assert np.array_equal(y[zero], np.broadcast_to(bias.astype(np.float32), y[zero].shape))


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m,flags,kern", [(300, 2, "dma"), (300, 1, "tiled"), (45, 4, "stream"), (5, 0, "gemv"),
                                          (1, 0, "gemv")])
def test_wide_linear_range_guard(xdt, m, flags, kern):
    """The forward's range guard: float32 / bf16 rows at 1e-30 .. 1e30, at and
    past fp16's overflow threshold (6.5e4, 7e4) and a zero row, on the LDS-DMA
    (bf16), register-staged, row-chunked and column-split kernels.  Every row
    keeps the relative accuracy of an in-range row: bf16 operands exact
    (float32 accumulation only), float32 operands within one fp16 rounding
    (2^-11), both relative to the row's own sum |x||A16|; the zero row gives
    the bias exactly.  Without the prescales (rpfq_wide_linear) the 7e4 and
    larger rows overflow to inf."""
    ops, N = qm()
    r = rng(2500 + m + flags)
    case = (384, 384, "axis", 2, 0, None)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    want = {"dma": N.KERNEL_DMA, "tiled": N.KERNEL_TILED, "stream": N.KERNEL_STREAM, "gemv": N.KERNEL_GEMV}[kern]
    if kern == "dma" and xdt == torch.float32:
        want = N.KERNEL_TILED  # float32 x is staged through registers
    assert pw.kernel_for(m, xdt, torch.float32, flags) == want
    x, mags = _range_rows(r, m, 2 * case[1], xdt)
    # no bias: a row of 1e-30 would vanish in it
    y = pw.linear(x.to(DEV), None, out_dtype=torch.float32, flags=flags).cpu().numpy().astype(np.float64)
    xf = x.float().numpy().astype(np.float64)
    a16 = O.wide_weight(oplanes, codebook, rotation, fp16=operand(pw, m, xdt, torch.float32, flags)).astype(np.float64)
    _check_range(y, xf, a16, np.zeros(2 * case[0]), mags, 2.0 ** -11 if xdt == torch.float32 else 0.0)
    # the prescales are what keeps the large rows finite
    y0 = torch.empty(m, 2 * case[0], dtype=torch.float32, device=DEV)
    pw.linear_into(x.to(DEV), None, y0, flags)
    big = mags >= 7e4
    assert big.any() and not torch.isfinite(y0.cpu()[torch.from_numpy(big)]).all()


@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_row_scales(xdt):
    """rpfq_row_scales: 2^(14 - floor(log2 max|row|)) per row (the scaled
    maximum in [2^14, 2^15)), clamped to [2^-126, 2^126]; 1 for zero and
    non-finite rows; any C (element loads when C % 8 != 0)."""
    ops, _ = qm()
    r = rng(2600)
    for c in (768, 13):
        x, mags = _range_rows(r, 40, c, xdt)
        x[3] = float("inf")
        x[4, 2] = float("nan")
        s = ops.row_scales(x.to(DEV)).cpu().numpy().astype(np.float64)
        ax = x.float().abs()
        mx = torch.where(torch.isnan(ax), torch.zeros_like(ax), ax).amax(dim=1).numpy().astype(np.float64)
        for i in range(40):
            if mx[i] == 0 or not np.isfinite(mx[i]):
                assert s[i] == 1.0, (i, s[i])
                continue
            k = int(np.clip(14 - np.floor(np.log2(mx[i])), -126, 126))
            assert s[i] == 2.0 ** k, (i, mx[i], s[i])
            if -126 < k < 126:
                assert 2.0 ** 14 <= mx[i] * s[i] < 2.0 ** 15


def test_act_quant_prologue_range_guard():
    """The streaming kernel's act-quant row prologue on bf16 rows of every
    magnitude (1e-30 .. 1e30): the quantized rows take the prescale of their
    largest magnitude as rpfq_row_scales gives it to the row kernel's output,
    so the fused launch is bit-identical to act_quant followed by the
    guarded layer, and both meet the exact-operand bound."""
    ops, N = qm()
    r = rng(2700)
    case = (384, 384, "axis", 2, 0, None)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    m = 22
    assert pw.ln_fusable(m, torch.bfloat16)
    x, mags = _range_rows(r, m, 768, torch.bfloat16)
    bias = r.standard_normal(768).astype(np.float32)
    xd = x.to(DEV)
    y = pw.act_quant_linear(xd, 4, tdev(bias), out_dtype=torch.float32)
    h = ops.act_quant(xd, 4)
    y_sep = pw.linear(h, tdev(bias), out_dtype=torch.float32)
    assert torch.equal(y, y_sep)
    hf = h.float().cpu().numpy().astype(np.float64)
    a16 = O.wide_weight(oplanes, codebook, rotation, fp16=True).astype(np.float64)
    hm = np.abs(hf).max(axis=1)
    _check_range(y.cpu().numpy().astype(np.float64), hf, a16, bias.astype(np.float64), np.where(hm > 0, mags, 0.0),
                 0.0)


def test_wide_linear_matches_reference_android_runtime():
    """Same packed planes through the compiled reference (oracle/_ref,
    wideLinearReference) and through the HIP kernel."""
    ref = pytest.importorskip("oracle.ref_lib")
    lib = ref.load()
    if lib is None:
        pytest.skip("oracle/_ref not built")
    r = rng(400)
    n_c, k_c = 64, 256
    planes = [r.integers(0, 4, size=(n_c, k_c), dtype=np.uint8) for _ in range(4)]
    g_re = [rand_gamma(r, n_c, 1) for _ in range(4)]
    g_im = [rand_gamma(r, n_c, 1) for _ in range(4)]
    bias = r.standard_normal(2 * n_c).astype(np.float32)
    x = torch.from_numpy(r.standard_normal((9, 2 * k_c)).astype(np.float32)).to(torch.float16)
    xf = x.float().numpy()
    y_ref = ref.wide_linear(xf, planes, g_re, g_im, bias, block=k_c, mode=0)
    ops, N = qm()
    inv_re = [tdev(O.inv_gamma(g)) for g in g_re]
    inv_im = [tdev(O.inv_gamma(g)) for g in g_im]
    pw = ops.PackedWide.from_planes([tdev(O.pack_codes(p)) for p in planes], inv_re, inv_im, n_c, k_c,
                                    N.CB_AXIS, 2, 0, None)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float32).cpu().numpy()
    op = [(p, O.inv_gamma(gr)[:, 0], O.inv_gamma(gi)[:, 0], kd) for p, gr, gi, kd in zip(planes, g_re, g_im, "uuww")]
    a = O.wide_weight(op)
    mag = O.wide_magnitude(op)
    ax = np.abs(xf.astype(np.float64))
    scale = ax @ np.abs(a.astype(np.float64)).T + np.abs(bias)
    u = 2.0 ** -11
    assert np.all(np.abs(y - y_ref) <= (2 * u + u * u) * (ax @ mag.T) + 1e-5 * scale + 1e-4)


@pytest.mark.parametrize("flags", [2, 1])
@pytest.mark.parametrize("m", [33, 128, 300, 513])
@pytest.mark.parametrize("case", [CASES[1], CASES[2], CASES[4], CASES[7], CASES[8]],
                         ids=["1536x384", "50x48", "130x512-b256", "rot", "table"])
def test_wide_linear_kernels_agree(case, m, flags):
    """The LDS-DMA kernel (RPFQ_FLAG_NO_STREAM, fp16 x, K' % 32 == 0,
    M >= 128) and the register-staged kernel (RPFQ_FLAG_TILE_M128) meet the
    same bound, with fp16 outputs through the LDS-transposed epilogue."""
    r = rng(500 + m)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float16, flags=flags).float().cpu().numpy()
    xf = x.float().numpy().astype(np.float64)
    check_against_oracle(y, xf, bias, oplanes, codebook, rotation, out_ulp=2.0 ** -11)


# The packed layer shapes (N', K') the headline models run on the tiled
# kernels at batch >= 1: ViT-B/16 qkv, proj, fc1, fc2 and ViT-L/16 fc2 (axis
# codes, 2 stages) and ViT-L/16 qkv / fc2 in 16-PSK.
REAL_SHAPES = [
    (1152, 384, "axis", 2, 0, None),
    (384, 384, "axis", 2, 0, None),
    (1536, 384, "axis", 2, 0, None),
    (384, 1536, "axis", 2, 0, None),
    (512, 2048, "axis", 2, 0, None),
    (1536, 512, "psk16", 1, 0, None),
    (512, 2048, "psk16", 1, 0, None),
]


@pytest.mark.parametrize("flags", [0, 2], ids=["auto", "tiled"])
@pytest.mark.parametrize("m", [128, 300, 1000])
@pytest.mark.parametrize("case", REAL_SHAPES, ids=[f"{c[0]}x{c[1]}-{c[2]}" for c in REAL_SHAPES])
def test_wide_linear_model_shapes(case, m, flags):
    """The model layer shapes against the oracle at M = 128, 300, 1000 (the
    LDS-DMA kernel under RPFQ_FLAG_NO_STREAM and, by default, whichever
    kernel the shape selects), K' up to 2048 (64 k-steps), fp16 and float32
    outputs."""
    r = rng(1500 + m + case[0] + case[1])
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    xf = x.float().numpy().astype(np.float64)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float32, flags=flags).cpu().numpy()
    check_against_oracle(y, xf, bias, oplanes, codebook, rotation)
    y16 = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float16, flags=flags).float().cpu().numpy()
    check_against_oracle(y16, xf, bias, oplanes, codebook, rotation, out_ulp=2.0 ** -11)


@pytest.mark.parametrize("ydt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("case", [REAL_SHAPES[2], REAL_SHAPES[3], REAL_SHAPES[4], REAL_SHAPES[6]],
                         ids=["fc1", "fc2", "l-fc2", "l-fc2-psk16"])
def test_wide_linear_dma_bf16(case, ydt):
    """bf16 activations on the LDS-DMA kernel (converted to fp16 in LDS after
    each stage lands) at the model layer shapes, M = 300 (RPFQ_FLAG_NO_STREAM;
    the last m-tile shifted back), against the oracle on the fp16-converted
    activations."""
    ops, N = qm()
    r = rng(1700 + case[0] + case[1])
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    m = 300
    assert pw.kernel_for(m, torch.bfloat16, ydt, N.FLAG_NO_STREAM) == N.KERNEL_DMA
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.bfloat16)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=ydt, flags=N.FLAG_NO_STREAM).float().cpu().numpy()
    xf = x.float().to(torch.float16).float().numpy().astype(np.float64)
    out_ulp = {torch.float32: 1e-6, torch.bfloat16: 2.0 ** -7}[ydt]
    check_against_oracle(y, xf, bias, oplanes, codebook, rotation, out_ulp)


@pytest.mark.parametrize("case", [REAL_SHAPES[2], REAL_SHAPES[3], REAL_SHAPES[1], REAL_SHAPES[0]],
                         ids=["fc1", "fc2", "proj", "qkv"])
def test_wide_linear_full_batch_rows(case):
    """ViT-B/16 at batch 256 (M = 50,432 rows): the DMA kernel's output on
    sampled rows against the oracle -- the first m-tile, the last m-tile
    (shifted back to end at row M), 256 random rows -- with fp16 outputs as
    the model stores them.  proj and fc2 (N' = 384: 1,182 tiles, 2.31 rounds
    of the persistent grid) cover a partial last round."""
    r = rng(1600 + case[0] + case[1])
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    m = 50432
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16).to(DEV)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    ops, N = qm()
    assert pw.kernel_for(m, torch.float16, torch.float16) == N.KERNEL_DMA
    y = pw.linear(x, tdev(bias), out_dtype=torch.float16)
    rows = np.unique(np.concatenate([np.arange(128), np.arange(m - 128, m),
                                     r.choice(m, size=256, replace=False)]))
    idx = torch.from_numpy(rows).to(DEV)
    ys = y.index_select(0, idx).float().cpu().numpy()
    xf = x.index_select(0, idx).float().cpu().numpy().astype(np.float64)
    check_against_oracle(ys, xf, bias, oplanes, codebook, rotation, out_ulp=2.0 ** -11)


DMA_ROUND_CASES = [
    ((1152, 384, "axis", 2, 0, None), 20000, True),    # 1,413 tiles: 2.8 rounds, last m-tile shifted
    ((128, 96, "axis", 2, 0, None), 70001, False),     # K' = 96: 3 k-steps, no bias, shifted
    ((256, 512, "psk16", 1, 0, None), 65536, True),    # 16-PSK, 1,024 tiles: exactly 2 rounds
    ((128, 128, "sign", 2, 0, ((0.8, 0.6), (0.6, -0.8))), 30001, True),  # sign codes, rotation
]


@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case,m,with_bias", DMA_ROUND_CASES,
                         ids=[f"{c[0][0]}x{c[0][1]}-{c[0][2]}-m{c[1]}" for c in DMA_ROUND_CASES])
def test_wide_linear_dma_rounds(case, m, with_bias, ydt):
    """The DMA kernel over several rounds of its persistent grid (each
    workgroup's later tiles take their first loads from the previous tile's
    prefetch), with and without bias, 16-bit outputs, the shifted last m-tile,
    three codebooks: sampled rows (first and last m-tile, 256 random) against
    the oracle, and the whole output bit-identical to a second launch and to
    the same launch with a zero residual added in the store."""
    ops, N = qm()
    r = rng(1650 + case[0] + case[1] + m)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    assert pw.kernel_for(m, torch.float16, ydt) == N.KERNEL_DMA
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16).to(DEV)
    bias = r.standard_normal(2 * case[0]).astype(np.float32) if with_bias else None
    bd = tdev(bias) if with_bias else None
    y = pw.linear(x, bd, out_dtype=ydt)
    assert torch.equal(y, pw.linear(x, bd, out_dtype=ydt))
    zero = torch.zeros(m, 2 * case[0], dtype=ydt, device=DEV)
    assert torch.equal(y, pw.linear(x, bd, out_dtype=ydt, residual=zero))
    rows = np.unique(np.concatenate([np.arange(128), np.arange(m - 128, m), r.choice(m, size=256, replace=False)]))
    idx = torch.from_numpy(rows).to(DEV)
    ys = y.index_select(0, idx).float().cpu().numpy()
    xf = x.index_select(0, idx).float().cpu().numpy().astype(np.float64)
    out_ulp = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[ydt]
    check_against_oracle(ys, xf, bias, oplanes, codebook, rotation, out_ulp=out_ulp)


def test_wide_linear_kernels_consistent():
    """Both kernels contract the same fp16 operands (they differ only in the
    k order inside each MFMA), so float32 outputs agree to accumulation order."""
    r = rng(600)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, CASES[1])
    x = torch.from_numpy(r.standard_normal((1000, 768)).astype(np.float32)).to(torch.float16).to(DEV)
    y0 = pw.linear(x, None, out_dtype=torch.float32, flags=2).cpu().numpy().astype(np.float64)
    y1 = pw.linear(x, None, out_dtype=torch.float32, flags=1).cpu().numpy().astype(np.float64)
    scale = np.abs(x.float().cpu().numpy().astype(np.float64)) @ np.abs(
        O.wide_weight(oplanes, codebook, rotation, fp16=True).astype(np.float64)).T
    assert np.all(np.abs(y0 - y1) <= 2e-6 * scale + 1e-6)


def test_wide_linear_many_rounds():
    """M = 50,432 on a 1536 x 384 layer (4,728 tiles: 9.2 rounds of the
    persistent grid, the last m-tile shifted back): the DMA kernel agrees
    with the register-staged kernel to float32 accumulation order, and the
    fused residual stays bit-identical to the separate add."""
    r = rng(650)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, CASES[1])
    m = 50432
    x = torch.from_numpy(r.standard_normal((m, 768)).astype(np.float32)).to(torch.float16).to(DEV)
    bias = tdev(r.standard_normal(3072).astype(np.float32))
    y0 = pw.linear(x, bias, out_dtype=torch.float32, flags=0).double()
    y1 = pw.linear(x, bias, out_dtype=torch.float32, flags=1).double()
    a16 = torch.from_numpy(O.wide_weight(oplanes, codebook, rotation, fp16=True)).to(DEV).double()
    scale = x.double().abs() @ a16.abs().T + bias.double().abs()
    assert bool(((y0 - y1).abs() <= 2e-6 * scale + 1e-6).all())
    res = torch.from_numpy(r.standard_normal((m, 3072)).astype(np.float32)).to(torch.float16).to(DEV)
    want = res + pw.linear(x, bias, out_dtype=torch.float16)
    got = pw.linear(x, bias, out_dtype=torch.float16, residual=res)
    assert torch.equal(got, want)


# ---------------------------------------------------------------------------
# weight-streaming kernel (M <= 16): the same operands, 16x16x32 MFMAs
# ---------------------------------------------------------------------------
SKINNY_CASES = CASES + [
    (64, 1536, "axis", 2, 0, None),        # long K' (48 k-steps)
    (40, 2048, "axis", 2, 256, None),      # long K' + per-(row, block) scales
    (33, 1000, "psk16", 1, 0, None),       # K' % 32 != 0 (zeroed activation tail), 16-PSK
]


@pytest.mark.parametrize("m", [1, 2, 4, 7, 16])
@pytest.mark.parametrize("case", SKINNY_CASES, ids=[f"{c[0]}x{c[1]}-{c[2]}{c[3]}-b{c[4]}-r{int(c[5] is not None)}"
                                                    for c in SKINNY_CASES])
def test_wide_linear_streaming(case, m):
    r = rng(700 + m)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float32).cpu().numpy()
    xf = x.float().numpy().astype(np.float64)
    mode = operand(pw, m)
    check_against_oracle(y, xf, bias, oplanes, codebook, rotation, fp16=mode)
    # fp16 outputs through the 8-byte store path
    y16 = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float16).float().cpu().numpy()
    check_against_oracle(y16, xf, bias, oplanes, codebook, rotation, out_ulp=2.0 ** -11, fp16=mode)


@pytest.mark.parametrize("m", [17, 45, 197, 300])
@pytest.mark.parametrize("case", SKINNY_CASES, ids=[f"{c[0]}x{c[1]}-{c[2]}{c[3]}-b{c[4]}-r{int(c[5] is not None)}"
                                                    for c in SKINNY_CASES])
def test_wide_linear_stream_chunks(case, m):
    """RPFQ_FLAG_STREAM past 16 rows: one workgroup per (16-row chunk, tile),
    ragged last chunk, against the oracle; float32 and fp16 outputs."""
    ops, N = qm()
    r = rng(750 + m)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    xf = x.float().numpy().astype(np.float64)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float32, flags=N.FLAG_STREAM).cpu().numpy()
    check_against_oracle(y, xf, bias, oplanes, codebook, rotation)
    y16 = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.float16, flags=N.FLAG_STREAM).float().cpu().numpy()
    check_against_oracle(y16, xf, bias, oplanes, codebook, rotation, out_ulp=2.0 ** -11)


@pytest.mark.parametrize("m,k_c", [(3, 640), (12, 640), (3, 320), (8, 320)],
                         ids=["m3-fused", "m12-fused", "m3-gemv", "m8-gemv"])
@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.float16, torch.bfloat16), (torch.float32, torch.float16)])
def test_wide_linear_streaming_dtypes(xdt, ydt, m, k_c):
    """Both streaming kernels (K' = 640: the fused one, 20 k-steps on 5
    tiles; K' = 320 at M <= 8: the column-split one) with float32 and bf16
    activations (converted to fp16 on load) and every output dtype."""
    ops, N = qm()
    r = rng(800 + m + k_c)
    case = (160, k_c, "axis", 2, 0, None)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    mode = operand(pw, m, xdt, ydt)
    assert (mode == "split") == (k_c == 320)
    x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(xdt)
    y = pw.linear(x.to(DEV), None, out_dtype=ydt).float().cpu().numpy()
    xf = x.float().to(torch.float16).float().numpy().astype(np.float64)
    out_ulp = {torch.float32: 1e-6, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[ydt]
    check_against_oracle(y, xf, None, oplanes, codebook, rotation, out_ulp, fp16=mode)


@pytest.mark.parametrize("m,n_c,k_c", [(8, 66000, 96), (2, 70000, 64), (16, 16500, 640), (3, 16500, 200),
                                       (4, 3000, 2048), (2, 131104, 64), (12, 131072, 96), (1, 131200, 200),
                                       (2, 131104, 640), (5, 131072, 648), (1, 131072, 384), (6, 131104, 416),
                                       (3, 131072, 456)])
def test_wide_linear_streaming_persistent(m, n_c, k_c):
    """Large N' on the streaming kernels' forms: split K over 2 waves per
    tile for 400 .. 4095 workgroups (66000 x 96 at M = 8: 2063 tiles;
    70000 x 64: 2188; 16500 x 640: 516; 16500 x 200: 516 with a K' tail),
    over 4 waves below 400 (3000 x 2048: 94 tiles, 64 k-steps), one wave per
    tile from 4096 tiles (131,072+ rows at short K'), and the column-split
    kernel's 64-row workgroups from 4096 tiles: 2 waves at >= 16 k-steps
    (131104 x 640: an odd tile count, the last workgroup's second tile
    clamped; 131072 x 648: a K' tail), 1 wave at 12 .. 15 (131072 x 384;
    131104 x 416: odd tile count; 131072 x 456: a K' tail).  Each launch against the exact product
    of the operand it contracts (float32 outputs, float32 accumulation
    order), and the tiled kernel (RPFQ_FLAG_NO_STREAM) likewise."""
    ops, N = qm()
    r = rng(900 + m)
    planes_np, packed, sre, sim, kinds, cb, nblk = make_wide(r, n_c, k_c)
    pw = ops.PackedWide.from_planes([tdev(p) for p in packed], [tdev(s) for s in sre], [tdev(s) for s in sim],
                                    n_c, k_c, cb, 2, 0, None)
    x = torch.from_numpy(r.standard_normal((m, 2 * k_c)).astype(np.float32)).to(torch.float16).to(DEV)
    bias = tdev(r.standard_normal(2 * n_c).astype(np.float32))
    y0 = pw.linear(x, bias, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
    y1 = pw.linear(x, bias, out_dtype=torch.float32, flags=N.FLAG_NO_STREAM).cpu().numpy().astype(np.float64)
    xf = x.float().cpu().numpy().astype(np.float64)
    b = bias.cpu().numpy().astype(np.float64)
    a16 = pw.decode(round_fp16=True).cpu().numpy().astype(np.float64)
    scale = np.abs(xf) @ np.abs(a16).T + np.abs(b)
    assert np.all(np.abs(y1 - (xf @ a16.T + b)) <= 1e-5 * scale + 1e-5)
    if operand(pw, m) == "split":
        del a16
        oplanes = oracle_planes(planes_np, sre, sim, kinds, k_c, 0)
        a_op = O.wide_weight(oplanes, "axis", None, fp16="split")
    else:
        a_op = a16
    assert np.all(np.abs(y0 - (xf @ a_op.T + b)) <= 1e-5 * scale + 1e-5)


@pytest.mark.parametrize("xdt,ydt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.float32, torch.float16)])
def test_wide_linear_gemv_one_wave_dtypes(xdt, ydt):
    """The column-split kernel's one-wave many-tile form (>= 4096 tiles at
    12-15 k-steps: 131104 x 384, an odd tile count) with float32 and bf16
    activations (fp16 on load) and each output dtype, against the oracle on
    the split operand it contracts."""
    ops, N = qm()
    r = rng(1300)
    n_c, k_c, m = 131104, 384, 2
    planes_np, packed, sre, sim, kinds, cb, nblk = make_wide(r, n_c, k_c)
    pw = ops.PackedWide.from_planes([tdev(p) for p in packed], [tdev(s) for s in sre], [tdev(s) for s in sim],
                                    n_c, k_c, cb, 2, 0, None)
    assert pw.kernel_for(m, xdt, ydt) == N.KERNEL_GEMV
    x = torch.from_numpy(r.standard_normal((m, 2 * k_c)).astype(np.float32)).to(xdt)
    bias = r.standard_normal(2 * n_c).astype(np.float32)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=ydt).float().cpu().numpy()
    xf = x.float().to(torch.float16).float().numpy().astype(np.float64)
    out_ulp = {torch.float32: 1e-6, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[ydt]
    check_against_oracle(y, xf, bias, oracle_planes(planes_np, sre, sim, kinds, k_c, 0), "axis", None, out_ulp,
                         fp16="split")


def _device_axis_layer(n_c, k_c, seed):
    """A two-stage axis layer too large for the host-side generator: packed
    2-bit planes (4 codes per byte, oracle.pack_codes order) and per-row
    scales ~U(0.01, 0.1) drawn on the device."""
    ops, N = qm()
    g = torch.Generator(device=DEV).manual_seed(seed)
    packed = [torch.randint(0, 256, (n_c, k_c // 4), dtype=torch.uint8, device=DEV, generator=g) for _ in range(4)]
    sre = [torch.rand(n_c, 1, device=DEV, generator=g) * 0.09 + 0.01 for _ in range(4)]
    sim = [torch.rand(n_c, 1, device=DEV, generator=g) * 0.09 + 0.01 for _ in range(4)]
    pw = ops.PackedWide.from_planes(packed, sre, sim, n_c, k_c, N.CB_AXIS, 2, 0, None)
    return pw, packed, sre, sim


def _oracle_rows(packed, sre, sim, k_c, sel):
    """Oracle planes of the complex output rows `sel` only (the output's
    columns sel and N' + sel)."""
    idx = torch.from_numpy(sel).to(DEV)
    planes = [O.unpack_codes(p.index_select(0, idx).cpu().numpy(), k_c) for p in packed]
    s1 = [s.index_select(0, idx).cpu().numpy() for s in sre]
    s2 = [s.index_select(0, idx).cpu().numpy() for s in sim]
    return oracle_planes(planes, s1, s2, ["u", "u", "w", "w"], k_c, 0)


@pytest.mark.parametrize("m,n_c,k_c,xdt,ydt", [
    (1, 300032, 384, torch.float16, torch.float16),
    (4, 300032, 384, torch.bfloat16, torch.bfloat16),
    (8, 300032, 384, torch.float16, torch.bfloat16),
    (3, 300032, 384, torch.float32, torch.float16),
    (5, 300032, 384, torch.bfloat16, torch.float16),
    (7, 131072, 384, torch.float16, torch.float16),
], ids=["m1-f16", "m4-bf16", "m8-f16-bf16", "m3-f32-f16", "m5-bf16-f16", "m7-f16-n131072"])
def test_wide_linear_gemv_persistent(m, n_c, k_c, xdt, ydt):
    """The column-split kernel's persistent one-wave form (12 k-steps from
    4096 tiles, whole 64-row groups, per-row scales, 16-bit y): 4,688 groups
    at N' = 300,032, so the resident waves walk two or three each and the
    code ring runs across group boundaries, and 2,048 at N' = 131,072 (at
    most one per wave).  On 2,176 sampled rows (the first and last groups
    among them) against the oracle on the split operand it contracts, with
    bias and without (the LDS-staged bias is the only difference); a
    residual added in the store bit-identical to the unfused add (also in
    place, residual == y through the C ABI); the fused GELU within 1 ulp of
    the exact GELU of the unfused output."""
    import ctypes
    import math

    ops, N = qm()
    r = rng(1400 + m + k_c)
    pw, packed, sre, sim = _device_axis_layer(n_c, k_c, 1400 + m)
    assert pw.kernel_for(m, xdt, ydt) == N.KERNEL_GEMV
    g = torch.Generator(device=DEV).manual_seed(1401 + m)
    x = torch.randn(m, 2 * k_c, device=DEV, generator=g).to(xdt)
    bias = torch.randn(2 * n_c, device=DEV, generator=g)
    y = pw.linear(x, bias, out_dtype=ydt)
    sel = np.unique(np.concatenate([np.arange(64), np.arange(n_c - 64, n_c), r.choice(n_c, 2048, replace=False)]))
    oplanes = _oracle_rows(packed, sre, sim, k_c, sel)
    cols = np.concatenate([sel, n_c + sel])
    ys = y.float().cpu().numpy()[:, cols]
    xf = x.float().to(torch.float16).float().cpu().numpy().astype(np.float64)
    out_ulp = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[ydt]
    check_against_oracle(ys, xf, bias.cpu().numpy()[cols].astype(np.float64), oplanes, "axis", None, out_ulp,
                         fp16="split")
    y0 = pw.linear(x, None, out_dtype=ydt).float().cpu().numpy()[:, cols]
    check_against_oracle(y0, xf, None, oplanes, "axis", None, out_ulp, fp16="split")
    assert torch.equal(pw.linear(x, bias, out_dtype=ydt), y)  # deterministic
    if xdt != torch.float32:
        res = (torch.randn(m, 2 * n_c, device=DEV, generator=g) * 4).to(ydt)
        want = res + y
        assert torch.equal(pw.linear(x, bias, out_dtype=ydt, residual=res), want)
        if xdt == torch.float16:  # (bf16 x takes row prescales, which this entry point has no argument for)
            yi = res.clone()
            lib = N.load()
            N.check("rpfq_wide_linear_residual", lib.rpfq_wide_linear_residual(
                ctypes.byref(pw.desc), pw.blob.data_ptr(), pw.blob.numel(), x.data_ptr(), N.F16, m,
                bias.data_ptr(), yi.data_ptr(), yi.data_ptr(), N.dtype_code(ydt), 0, N.stream_of(x)))
            torch.cuda.synchronize()
            assert torch.equal(yi, want)
        yg = pw.linear(x, bias, out_dtype=ydt, gelu=True).cpu()
        yd = y.double().cpu()
        exact = yd * 0.5 * torch.special.erfc(-yd / math.sqrt(2.0))
        tiny = exact.abs() < 2.0 ** -126
        d = torch.where(tiny, torch.zeros_like(yg, dtype=torch.long), ulp_distance(yg, exact.to(ydt)))
        assert int(d.max()) <= 1 and float((d > 0).float().mean()) <= 1e-3


# ---------------------------------------------------------------------------
# resident-weight kernel (RPFQ_KERNEL_RESIDENT): the decoded layer stays in
# LDS while the waves stream 32-row subtiles of x (Swin-T stage 0)
# ---------------------------------------------------------------------------
RES_CASES = [
    (144, 48, "axis", 2, 0, None),                        # Swin-T stage 0 qkv: 16 staged rows of 576 B
    (48, 48, "axis", 2, 0, None),                         # stage 0 proj
    (192, 48, "psk16", 1, 0, None),                       # stage 0 fc1 in 16-PSK: staged in two 8-row halves
    (48, 192, "axis", 2, 64, None),                       # stage 0 fc2, 3 scale blocks per row (K' = 192)
    (96, 96, "sign", 2, 0, ((0.8, 0.6), (0.6, -0.8))),    # stage 1 proj, sign codes, rotation
    (96, 48, "table", 1, 0, None),                        # per-row tables
    (48, 96, "axis", 1, 0, None),                         # one stage (v1), K' = 96, N' = 48
]
RES_IDS = [f"{c[0]}x{c[1]}-{c[2]}-b{c[4]}" for c in RES_CASES]


def _res_input(r, m, k_in, xdt, seed):
    """x [m, k_in] on the device (standard normal, generated there for large
    m), and the sampled rows the oracle checks: the first and last 64 and
    192 random ones."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, k_in, device=DEV, generator=g).to(xdt)
    rows = np.unique(np.concatenate([np.arange(min(m, 64)), np.arange(max(0, m - 64), m),
                                     r.choice(m, size=min(m, 192), replace=False)]))
    return x, rows


@pytest.mark.parametrize("xdt,ydt", [(torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float16)], ids=["f16", "bf16", "bf16-f16"])
@pytest.mark.parametrize("m,flags", [(77, 16), (140001, 0)], ids=["m77-forced", "m140001-auto"])
@pytest.mark.parametrize("case", RES_CASES, ids=RES_IDS)
def test_wide_linear_resident(case, m, flags, xdt, ydt):
    """The resident-weight kernel against the oracle on sampled rows (the
    partial last subtile included) at M = 77 (RPFQ_FLAG_RESIDENT: three
    subtiles, the last of 13 rows) and M = 140,001 (chosen by default: 4,376
    subtiles, three rounds of the persistent waves), with bias, five
    codebook / scale / rotation variants, fp16 and bf16 activations (bf16
    through the range guard's row prescales) and 16-bit outputs; the launch
    is deterministic, and (N' <= 96, the layers it takes a residual for) a
    zero residual added in the store changes nothing."""
    ops, N = qm()
    r = rng(3100 + case[0] + case[1] + m)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    assert pw.kernel_for(m, xdt, ydt, flags) == N.KERNEL_RESIDENT
    x, rows = _res_input(r, m, 2 * case[1], xdt, 3100 + m)
    bias = r.standard_normal(2 * case[0]).astype(np.float32)
    y = pw.linear(x, tdev(bias), out_dtype=ydt, flags=flags)
    assert torch.equal(y, pw.linear(x, tdev(bias), out_dtype=ydt, flags=flags))
    if case[0] <= 96:
        zero = torch.zeros_like(y)
        assert torch.equal(y, pw.linear(x, tdev(bias), out_dtype=ydt, flags=flags, residual=zero))
    idx = torch.from_numpy(rows).to(DEV)
    ys = y.index_select(0, idx).float().cpu().numpy()
    # bf16 rows prescaled by a power of two are exact in fp16: the MFMA sees x itself
    xf = x.index_select(0, idx).float().cpu().numpy().astype(np.float64)
    out_ulp = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[ydt]
    check_against_oracle(ys, xf, bias, oplanes, codebook, rotation, out_ulp=out_ulp)


@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", [RES_CASES[1], RES_CASES[3], RES_CASES[4], RES_CASES[2]],
                         ids=["proj", "fc2", "proj-s1", "fc1"])
def test_wide_linear_resident_residual_gelu(case, ydt):
    """The resident kernel's fused store ops at M = 70,001 (default choice):
    on the layers that take a residual (N' <= 96) a residual add
    bit-identical to the unfused add in y's dtype, also in place (residual ==
    y through the C ABI); on all, the fused GELU within 1 ulp of the exact
    GELU of the unfused output (at most 0.1% of the elements off at all)."""
    import ctypes
    import math

    ops, N = qm()
    r = rng(3300 + case[0] + case[1])
    pw, *_ = build_packed(r, case)
    m = 70001
    assert pw.kernel_for(m, torch.float16, ydt) == N.KERNEL_RESIDENT
    x, _ = _res_input(r, m, 2 * case[1], torch.float16, 3300)
    bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
    g = torch.Generator(device=DEV).manual_seed(3301)
    res = (torch.randn(m, 2 * case[0], device=DEV, generator=g) * 4).to(ydt)
    y = pw.linear(x, bias, out_dtype=ydt)
    if case[0] <= 96:
        want = res + y
        assert torch.equal(pw.linear(x, bias, out_dtype=ydt, residual=res), want)
        yi = res.clone()
        lib = N.load()
        N.check("rpfq_wide_linear_residual", lib.rpfq_wide_linear_residual(
            ctypes.byref(pw.desc), pw.blob.data_ptr(), pw.blob.numel(), x.data_ptr(), N.F16, m, bias.data_ptr(),
            yi.data_ptr(), yi.data_ptr(), N.dtype_code(ydt), 0, N.stream_of(x)))
        torch.cuda.synchronize()
        assert torch.equal(yi, want)
    yg = pw.linear(x, bias, out_dtype=ydt, gelu=True).cpu()
    yd = y.double().cpu()
    exact = yd * 0.5 * torch.special.erfc(-yd / math.sqrt(2.0))
    tiny = exact.abs() < 2.0 ** -126
    d = torch.where(tiny, torch.zeros_like(yg, dtype=torch.long), ulp_distance(yg, exact.to(ydt)))
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) <= 1e-3


def test_wide_linear_resident_range_guard():
    """bf16 rows at 1e-30 .. 1e30, past fp16's overflow threshold and a zero
    row through the resident kernel (RPFQ_FLAG_RESIDENT, bf16 outputs): the
    row prescales keep each row's relative accuracy -- within the bf16
    output rounding of x A16^T (the operands exact, float32 accumulation) --
    and the zero row gives the bias rounded to bf16."""
    ops, N = qm()
    r = rng(3400)
    case = RES_CASES[0]
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    m = 300
    x, mags = _range_rows(r, m, 2 * case[1], torch.bfloat16)
    bias = np.zeros(2 * case[0], dtype=np.float32)
    y = pw.linear(x.to(DEV), tdev(bias), out_dtype=torch.bfloat16, flags=N.FLAG_RESIDENT).float().cpu().numpy()
    xf = x.float().numpy().astype(np.float64)
    a16 = O.wide_weight(oplanes, codebook, rotation, fp16=True).astype(np.float64)
    ref = xf @ a16.T
    scale = np.abs(xf) @ np.abs(a16).T
    assert np.all(np.isfinite(y))
    assert np.all(np.abs(y - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-5 * scale + 1e-44)
    assert np.all(y[mags == 0] == 0.0)



# ---------------------------------------------------------------------------
# fused MLP (rpfq_wide_mlp): fc1 -> GELU -> fc2 (+ residual) in one launch,
# equal bit for bit to the two large-M launches it replaces
# ---------------------------------------------------------------------------
MLP_CASES = [
    # (N1', codebook, stages, rotation): fc1 96 -> N1', fc2 N1' -> 96
    (384, "axis", 2, None),                                   # DeiT-Ti / Swin-T stage 1
    (768, "sign", 2, ((0.8, 0.6), (0.6, -0.8))),              # 8 chunks, sign codes, rotation
    (192, "psk16", 1, None),                                  # 16-PSK, 2 chunks
    (96, "table", 1, None),                                   # per-row tables, 1 chunk
    (1536, "axis", 1, None),                                  # the largest N1' (16 chunks)
]
MLP_IDS = [f"{c[0]}-{c[1]}{c[2]}-r{int(c[3] is not None)}" for c in MLP_CASES]


def _mlp_layers(r, case):
    n1, codebook, stages, rot = case
    p1, *_ = build_packed(r, (n1, 96, codebook, stages, 0, rot))
    p2, *_ = build_packed(r, (96, n1, codebook, stages, 0, rot))
    return p1, p2


def _two_launches(p1, p2, x, b1, b2, res):
    """fc1 with the fused GELU, then fc2 with the residual, both on the LDS-DMA
    kernel (RPFQ_FLAG_NO_STREAM at >= 128 rows); x padded to 128 rows (its
    first rows repeated) where it has fewer, the rows being independent."""
    _, N = qm()
    m = x.shape[0]
    xp, rp = x, res
    if m < 128:
        idx = torch.arange(128, device=x.device) % m
        xp = x[idx]
        rp = None if res is None else res[idx]
    assert p1.kernel_for(xp.shape[0], torch.float16, torch.float16, N.FLAG_NO_STREAM | N.FLAG_GELU) == N.KERNEL_DMA
    assert p2.kernel_for(xp.shape[0], torch.float16, torch.float16, N.FLAG_NO_STREAM) == N.KERNEL_DMA
    h = p1.linear(xp, b1, out_dtype=torch.float16, flags=N.FLAG_NO_STREAM, gelu=True)
    y = p2.linear(h, b2, out_dtype=torch.float16, flags=N.FLAG_NO_STREAM, residual=rp)
    return y[:m]


@pytest.mark.parametrize("m", [64, 100, 128, 300, 12672], ids=["m64", "m100", "m128", "m300", "m12672"])
@pytest.mark.parametrize("case", MLP_CASES, ids=MLP_IDS)
def test_wide_mlp_matches_two_launches(case, m):
    """rpfq_wide_mlp against fc1 (RPFQ_FLAG_GELU) and fc2 (with the residual)
    launched separately on the large-M kernel, bit for bit: five codebook /
    rotation / width cases (1-16 chunks of fc1 outputs), M = 64 (one tile),
    100 and 300 (the last tile shifted back over the previous one), 128 and
    12,672 (DeiT-Ti at batch 64), with biases and residual, without either,
    and in place (residual == y through the C ABI)."""
    import ctypes

    ops, N = qm()
    r = rng(3500 + case[0] + m)
    p1, p2 = _mlp_layers(r, case)
    g = torch.Generator(device=DEV).manual_seed(3501 + m)
    x = torch.randn(m, 192, device=DEV, generator=g).half()
    b1 = torch.randn(2 * case[0], device=DEV, generator=g)
    b2 = torch.randn(192, device=DEV, generator=g)
    res = (torch.randn(m, 192, device=DEV, generator=g) * 4).half()
    assert ops.mlp_fusable(p1, p2, m, torch.float16)
    want = _two_launches(p1, p2, x, b1, b2, res)
    got = ops.wide_mlp(p1, p2, x, b1, b2, res)
    assert torch.isfinite(got).all()
    assert torch.equal(got, want)
    assert torch.equal(ops.wide_mlp(p1, p2, x), _two_launches(p1, p2, x, None, None, None))
    yi = res.clone()
    N.check("rpfq_wide_mlp", N.load().rpfq_wide_mlp(
        ctypes.byref(p1.desc), p1.blob.data_ptr(), p1.blob.numel(), ctypes.byref(p2.desc), p2.blob.data_ptr(),
        p2.blob.numel(), x.data_ptr(), m, b1.data_ptr(), b2.data_ptr(), yi.data_ptr(), yi.data_ptr(),
        N.stream_of(x)))
    torch.cuda.synchronize()
    assert torch.equal(yi, want)


@pytest.mark.parametrize("m", [64, 300, 8191, 8192, 12672], ids=["m64", "m300", "m8191", "m8192", "m12672"])
@pytest.mark.parametrize("affine", [True, False], ids=["affine", "plain"])
def test_layer_norm_wide_mlp_matches(affine, m):
    """rpfq_layer_norm_wide_mlp against rpfq_layer_norm followed by
    rpfq_wide_mlp with x as the residual, bit for bit: the row kernel's 64
    lanes per row (M < 8,192) and 8 (M >= 8,192) reproduced in the prologue,
    with and without the affine parameters, rows of mixed scale and offset;
    and in place (y == x through the C ABI)."""
    import ctypes

    ops, N = qm()
    r = rng(3700 + m)
    p1, p2 = _mlp_layers(r, MLP_CASES[0])
    g = torch.Generator(device=DEV).manual_seed(3701 + m)
    x = (torch.randn(m, 192, device=DEV, generator=g) * (1 + 3 * torch.rand(m, 1, device=DEV, generator=g))
         + torch.randn(m, 1, device=DEV, generator=g)).half()
    w = torch.randn(192, device=DEV, generator=g) * 0.2 + 1 if affine else None
    b = torch.randn(192, device=DEV, generator=g) * 0.1 if affine else None
    b1 = torch.randn(768, device=DEV, generator=g)
    b2 = torch.randn(192, device=DEV, generator=g)
    eps = 1e-6
    want = ops.wide_mlp(p1, p2, ops.layer_norm(x, w, b, eps), b1, b2, residual=x)
    got = ops.layer_norm_wide_mlp(p1, p2, x, w, b, eps, b1, b2)
    assert torch.isfinite(got).all()
    assert torch.equal(got, want)
    xi = x.clone()
    N.check("rpfq_layer_norm_wide_mlp", N.load().rpfq_layer_norm_wide_mlp(
        ctypes.byref(p1.desc), p1.blob.data_ptr(), p1.blob.numel(), ctypes.byref(p2.desc), p2.blob.data_ptr(),
        p2.blob.numel(), xi.data_ptr(), m, N.ptr(w), N.ptr(b), eps, b1.data_ptr(), b2.data_ptr(), xi.data_ptr(),
        N.stream_of(x)))
    torch.cuda.synchronize()
    assert torch.equal(xi, want)


def test_wide_mlp_against_oracle():
    """The fused MLP against the oracle in float64 on the fp16 operands it
    contracts (DeiT-Ti's fc1 / fc2, axis codes, 300 rows): the hidden values
    GELU(fp16(x A1^T + b1)) within fc1's fp16 rounding and the GELU's 1 ulp,
    y within that propagated through fc2 plus fc2's own float32 accumulation
    and fp16 output rounding."""
    import math

    ops, N = qm()
    r = rng(3600)
    n1, m = 384, 300
    p1, o1, _, cb, rot = build_packed(r, (n1, 96, "axis", 2, 0, None))
    p2, o2, _, _, _ = build_packed(r, (96, n1, "axis", 2, 0, None))
    x = torch.from_numpy(r.standard_normal((m, 192)).astype(np.float32)).half()
    b1 = r.standard_normal(2 * n1).astype(np.float32)
    b2 = r.standard_normal(192).astype(np.float32)
    y = ops.wide_mlp(p1, p2, x.to(DEV), tdev(b1), tdev(b2)).double().cpu().numpy()
    a1 = O.wide_weight(o1, cb, rot, fp16=True).astype(np.float64)
    a2 = O.wide_weight(o2, cb, rot, fp16=True).astype(np.float64)
    xf = x.double().numpy()
    pre = xf @ a1.T + b1
    erf = np.vectorize(math.erf)
    h = pre * 0.5 * (1.0 + erf(pre / math.sqrt(2.0)))
    # |GELU'| <= 1.13: fc1's error (float32 sum + fp16 rounding) and the GELU's ulp carry into h
    hs = np.abs(xf) @ np.abs(a1).T + np.abs(b1)
    dh = 1.13 * (1e-5 * hs + 2.0 ** -11 * np.abs(pre)) + 2.0 ** -10 * np.abs(h) + 1e-7
    ref = h @ a2.T + b2
    tol = np.abs(dh) @ np.abs(a2).T + 1e-5 * (np.abs(h) @ np.abs(a2).T + np.abs(b2)) + 2.0 ** -10 * np.abs(ref)
    assert np.all(np.abs(y - ref) <= tol + 1e-4)

# ---------------------------------------------------------------------------
# fused residual add (rpfq_wide_linear_residual): bit-identical to the layer
# followed by the add in y's dtype, on every kernel path
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("m,flags", [(3, 0), (16, 0), (33, 2), (130, 2), (300, 1), (129, 2), (197, 4), (197, 0),
                                     (300, 4)],
                         ids=["stream3", "stream16", "reg33", "dma130", "reg128-300", "nostream129", "stream197",
                              "auto197", "stream300"])
@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16, torch.float32])
def test_wide_linear_residual_bit_exact(m, flags, ydt):
    r = rng(1000 + m)
    for case in (CASES[1], CASES[2]):  # N' % 8 == 0 (vector stores) and N' = 50 (element tail)
        pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
        x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16).to(DEV)
        bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
        res = torch.from_numpy(r.standard_normal((m, 2 * case[0])).astype(np.float32) * 4).to(ydt).to(DEV)
        y = pw.linear(x, bias, out_dtype=ydt, flags=flags)
        yf = pw.linear(x, bias, out_dtype=ydt, flags=flags, residual=res)
        assert torch.equal(yf, res + y), (case, m, flags, ydt)


def _bf16_rne_bits(v):
    """float32 -> bf16 bits, round to nearest even (NaN: any NaN pattern)."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


@pytest.mark.parametrize("m,flags", [(3, 0), (197, 0), (33, 2), (300, 2), (300, 1)],
                         ids=["stream3", "stream197", "reg33", "dma300", "reg128-300"])
def test_bf16_store_rounding(m, flags):
    """The stores' float32 -> bf16 conversion (the hardware's packed
    conversion) is round-to-nearest-even bit for bit: with x = 0 each output
    is 0 + bias exactly, so bias vectors of random float32 bit patterns plus
    ties (low half 0x8000, even and odd), subnormals, the largest finite
    value (rounds to inf), +-inf and NaN must come back as numpy's rounding of
    them -- on each kernel path, at whole-line (N' = 1536) and element-tail
    (N' = 50) stores; with a residual, res + bf16(bias) added in float32 and
    rounded again."""
    r = rng(1500 + m)
    special = np.array([0x3F808000, 0x3F818000, 0xBF808000, 0xBF818000, 0x00008000, 0x00018000, 0x00000001,
                        0x007FFFFF, 0x80000001, 0x807FFFFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7E8000,
                        0x7F800000, 0xFF800000, 0x7FC00001, 0xFFA12345, 0x3F80FFFF, 0x477FFFFF], np.uint32)
    for case in (CASES[1], CASES[2]):
        pw, *_ = build_packed(r, case)
        n = 2 * case[0]
        bits = r.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        bits[: len(special)] = special[:n]
        bits[(bits & 0x7FFFFFFF) == 0] = 0x3F800000  # no +-0: 0 + -0 is +0
        bias_np = bits.view(np.float32)
        x = torch.zeros((m, 2 * case[1]), dtype=torch.float16, device=DEV)
        y = pw.linear(x, tdev(bias_np), out_dtype=torch.bfloat16, flags=flags)
        got = y.view(torch.int16).cpu().numpy().view(np.uint16)
        want = _bf16_rne_bits(bias_np)
        nan = np.isnan(bias_np)
        got_nan = ((got & 0x7FFF) > 0x7F80)
        assert np.array_equal(got_nan, np.broadcast_to(nan, got.shape)), (case, m, flags)
        bad = (got != want) & ~nan
        assert not bad.any(), (case, m, flags, hex(int(bits[np.nonzero(bad)[1][0]])))
        # residual: res + bf16(bias) in float32, rounded again (finite biases)
        fin = np.isfinite(bias_np)
        res_np = (r.standard_normal((m, n)).astype(np.float32) * 4)
        res = torch.from_numpy(res_np).to(torch.bfloat16).to(DEV)
        yr = pw.linear(x, tdev(np.where(fin, bias_np, np.float32(1.0))), out_dtype=torch.bfloat16, flags=flags,
                       residual=res)
        rb = (res.view(torch.int16).cpu().numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        vb = (_bf16_rne_bits(np.where(fin, bias_np, np.float32(1.0))).astype(np.uint32) << 16).view(np.float32)
        want_r = _bf16_rne_bits((rb + vb[None, :]).astype(np.float32))
        got_r = yr.view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(got_r, want_r), (case, m, flags)


@pytest.mark.parametrize("m,flags", [(3, 0), (197, 0), (33, 2), (300, 2), (300, 1)],
                         ids=["stream3", "stream197", "reg33", "dma300", "reg128-300"])
@pytest.mark.parametrize("ydt", [torch.float16, torch.bfloat16, torch.float32])
def test_wide_linear_gelu(m, flags, ydt):
    """RPFQ_FLAG_GELU on every kernel path and dtype (N' = 1536: whole-line
    DMA epilogue; N' = 50: element tails).  The store evaluates GELU(y) =
    y Phi(y) of the output already rounded to y's dtype by the kernels' fast
    form (normal tail from exp and a fitted polynomial, ~1e-6 relative).
    Bars, on the unfused output of the same kernel:
      * against the exact GELU (float64 erfc) rounded to y's dtype: every
        element within 1 ulp, at most 0.1% off at all (float32 outputs:
        within 2e-6 relative);
      * against torch's F.gelu (x * 0.5 * (1 + erf(x / sqrt 2)) in float32,
        whose 1 + erf cancels for x < -3): within 1 ulp of y's dtype or
        within torch's own float32 error there, |y| * 6e-8 + 2e-6 |GELU|."""
    import math

    import torch.nn.functional as F

    ops, N = qm()
    r = rng(1200 + m)
    for case in (CASES[1], CASES[2]):
        pw, *_ = build_packed(r, case)
        x = torch.from_numpy(r.standard_normal((m, 2 * case[1])).astype(np.float32)).to(torch.float16).to(DEV)
        bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
        # (fp16 x: every output dtype keeps its kernel with the GELU)
        y = pw.linear(x, bias, out_dtype=ydt, flags=flags)
        yg = pw.linear(x, bias, out_dtype=ydt, flags=flags, gelu=True).cpu()
        yd = y.double().cpu()
        exact = yd * 0.5 * torch.special.erfc(-yd / math.sqrt(2.0))
        if ydt == torch.float32:
            rel = torch.where(yd > -5, 2e-6, 2e-5)  # the exponent's rounding grows with y^2 in the tail
            bad = (yg.double() - exact).abs() > rel * exact.abs() + 2.0 ** -125
            assert not bool(bad.any()), (case, m, flags, yd[bad][:4].tolist(), exact[bad][:4].tolist())
        else:
            # below float32's normal range (y < -13: bf16 subnormal GELU
            # values) the float32 evaluation may flush to zero
            tiny = exact.abs() < 2.0 ** -126
            d = torch.where(tiny, torch.zeros_like(yg, dtype=torch.long), ulp_distance(yg, exact.to(ydt)))
            assert bool((yg[tiny].double().abs() <= 2.0 ** -126).all()), (case, m, flags, ydt)
            assert int(d.max()) <= 1 and float((d > 0).float().mean()) <= 1e-3, (case, m, flags, ydt)
        tg = F.gelu(y).cpu()
        near = (yg.double() - tg.double()).abs() <= yd.abs() * 6e-8 + 2e-6 * exact.abs()
        if ydt != torch.float32:
            near |= ulp_distance(yg, tg) <= 1
        assert bool(near.all()), (case, m, flags, ydt)
    with pytest.raises(ValueError, match="gelu and residual"):
        pw.linear(x, bias, gelu=True, residual=torch.zeros_like(pw.linear(x, bias)))


def test_wide_linear_residual_in_place():
    """residual == y through the C ABI: every element is read before it is
    written by the same thread, and by one workgroup only -- on the
    streaming kernel (M = 4, 200 by default) and on the DMA kernel, also the
    rows of the last m-tile that it shifts back over the previous one
    (M % 128 != 0), over several rounds of the persistent grid (M = 40,037:
    3,756 tiles)."""
    ops, N = qm()
    import ctypes
    r = rng(1100)
    pw, *_ = build_packed(r, CASES[1])
    lib = N.load()
    for m, flags in ((4, 0), (200, 0), (200, N.FLAG_NO_STREAM), (40037, 0)):
        x = torch.from_numpy(r.standard_normal((m, 768)).astype(np.float32)).to(torch.float16).to(DEV)
        res = torch.from_numpy(r.standard_normal((m, 3072)).astype(np.float32)).to(torch.float16).to(DEV)
        want = res + pw.linear(x, None, out_dtype=torch.float16, flags=flags)
        y = res.clone()
        N.check("rpfq_wide_linear_residual", lib.rpfq_wide_linear_residual(
            ctypes.byref(pw.desc), pw.blob.data_ptr(), pw.blob.numel(), x.data_ptr(), N.F16, m, None,
            y.data_ptr(), y.data_ptr(), N.F16, flags, N.stream_of(x)))
        torch.cuda.synchronize()
        assert torch.equal(y, want), (m, flags)


def test_misaligned_views_are_copied():
    """Contiguous views that start off the C ABI's 16-byte row alignment (an
    odd element offset into a flat buffer) are copied before the call, for
    x, the residual and the LayerNorm input: results equal those of aligned
    copies of the same data."""
    ops, _ = qm()
    r = rng(1700)
    pw, *_ = build_packed(r, CASES[1])
    m = 5
    flat = tdev(r.standard_normal(m * 768 + 1).astype(np.float16))
    x = flat[1:].view(m, 768)
    assert x.is_contiguous() and x.data_ptr() % 16 != 0
    assert torch.equal(pw.linear(x, None, out_dtype=torch.float32), pw.linear(x.clone(), None, out_dtype=torch.float32))
    rflat = tdev(r.standard_normal(m * 3072 + 3).astype(np.float16))
    res = rflat[3:].view(m, 3072)
    assert res.data_ptr() % 16 != 0
    assert torch.equal(pw.linear(x, None, out_dtype=torch.float16, residual=res),
                       pw.linear(x.clone(), None, out_dtype=torch.float16, residual=res.clone()))
    g = tdev(r.standard_normal(768).astype(np.float32))
    b = tdev(r.standard_normal(768).astype(np.float32))
    assert torch.equal(ops.layer_norm(x, g, b, 1e-6), ops.layer_norm(x.clone(), g, b, 1e-6))


# ---------------------------------------------------------------------------
# LayerNorm (rpfq_layer_norm) against a float64 restatement of nn.LayerNorm
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("m,c", [(1, 8), (37, 96), (300, 768), (5, 1024), (9, 1536), (3, 4096)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)])
def test_layer_norm(m, c, xdt, ydt):
    ops, _ = qm()
    r = rng(1200 + c)
    x = torch.from_numpy((r.standard_normal((m, c)) * 3 + 1).astype(np.float32)).to(xdt)
    g = torch.from_numpy(r.standard_normal(c).astype(np.float32))
    b = torch.from_numpy(r.standard_normal(c).astype(np.float32))
    y = ops.layer_norm(x.to(DEV), g.to(DEV), b.to(DEV), 1e-6, out_dtype=ydt).float().cpu().numpy().astype(np.float64)
    xd = x.float().numpy().astype(np.float64)
    mu = xd.mean(axis=1, keepdims=True)
    var = ((xd - mu) ** 2).mean(axis=1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-6) * g.numpy() + b.numpy()
    # float32 statistics (relative ~1e-6 of the normalized value) plus one
    # rounding to y's dtype
    ulp = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[ydt]
    tol = ulp * np.abs(ref) + 2e-5 * (np.abs(g.numpy()) * np.abs((xd - mu) / np.sqrt(var + 1e-6)) + 1)
    assert np.all(np.abs(y - ref) <= tol)
    # no affine parameters
    y0 = ops.layer_norm(x.to(DEV), None, None, 1e-5, out_dtype=torch.float32).cpu().numpy()
    ref0 = (xd - mu) / np.sqrt(var + 1e-5)
    assert np.abs(y0 - ref0).max() <= 2e-5 * (np.abs(ref0).max() + 1)


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("gscale", [1.0, 1e6, 1e-9], ids=["g1", "g1e6", "g1e-9"])
@pytest.mark.parametrize("m,c", [(300, 768), (2047, 768), (2048, 768), (129, 3072), (64, 96)])
def test_layer_norm_prescaled(m, c, gscale, xdt):
    """rpfq_layer_norm_prescaled against the three steps it stands for:
    rpfq_layer_norm in x's dtype, rpfq_row_scales of those rows, and the fp16
    rounding of each row times its scale -- scales and fp16 bits equal,
    at both lane layouts of the row kernel (2,047 / 2,048 rows at C = 768),
    with affine parameters that put the rows beyond fp16's range (1e6) or
    below its normal range (1e-9), without them, and in place."""
    ops, _ = qm()
    r = rng(2100 + m + c)
    x = torch.from_numpy((r.standard_normal((m, c)) * 3 + 1).astype(np.float32)).to(xdt).to(DEV)
    g = tdev((r.standard_normal(c) * gscale).astype(np.float32))
    b = tdev((r.standard_normal(c) * gscale).astype(np.float32))
    for gg, bb in ((g, b), (None, None)):
        y, sc = ops.layer_norm_prescaled(x, gg, bb, 1e-6)
        h = ops.layer_norm(x, gg, bb, 1e-6)
        sc_ref = ops.row_scales(h)
        assert torch.equal(sc, sc_ref)
        y_ref = (h.float() * sc_ref[:, None]).half()
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    if xdt != torch.bfloat16:
        return
    # in place: the fp16 rows over the bf16 rows' storage
    N = qm()[1]
    x2 = x.clone()
    y2, sc2 = ops.layer_norm_prescaled(x2, g, b, 1e-6)
    N.check("rpfq_layer_norm_prescaled", N.load().rpfq_layer_norm_prescaled(
        x2.data_ptr(), N.dtype_code(x2.dtype), m, c, g.data_ptr(), b.data_ptr(), 1e-6, x2.data_ptr(),
        sc2.data_ptr(), N.stream_of(x2)))
    assert torch.equal(x2.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("m,c", [(300, 768), (129, 3072), (64, 4096), (37, 96)])
def test_row_prescale(m, c, xdt):
    """rpfq_row_prescale: the scales equal rpfq_row_scales and the fp16 rows
    equal the bf16 rows times them, rounded (the DMA kernel's operand bits),
    for rows of 1e30 .. 1e-30, 7e4, zero, maxima near 2e38, an infinite
    element (scale 1) and ordinary magnitudes, and in place."""
    ops, N = qm()
    r = rng(2300 + m + c)
    mags = np.array([1.0, 1e30, 1e-30, 7e4, 0.0, 3e-6, 1e-12, 5e37])
    xs = r.standard_normal((m, c)) * mags[np.arange(m) % len(mags)][:, None]
    xs[min(2, m - 1), 1] = np.inf
    x = torch.from_numpy(xs.astype(np.float32)).to(xdt).to(DEV)
    y, sc = ops.prescale_rows(x)
    sc_ref = ops.row_scales(x)
    assert torch.equal(sc, sc_ref)
    y_ref = (x.float() * sc_ref[:, None]).half()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    if xdt == torch.bfloat16:  # in place (same element size)
        x2 = x.clone()
        N.check("rpfq_row_prescale", N.load().rpfq_row_prescale(x2.data_ptr(), N.dtype_code(x2.dtype), m, c,
                                                              x2.data_ptr(), sc.data_ptr(), N.stream_of(x2)))
        assert torch.equal(x2.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("case", [REAL_SHAPES[0], REAL_SHAPES[3], CASES[7]], ids=["qkv", "fc2", "rot"])
def test_bf16_rows_prescaled_pass(case, monkeypatch):
    """bf16 rows into a DMA-kernel launch go through prescale_rows: outputs
    equal the bf16-row path (row scales, in-kernel conversion) bit for bit,
    with bias and residual, rows beyond fp16's range and below its normal
    range included; float32 rows through it onto the DMA kernel within
    float32 accumulation order of the register-staged kernel's result (and
    one fp16 rounding for fp16 outputs)."""
    ops, N = qm()
    r = rng(2400 + case[0] + case[1])
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    m = 12672
    c2 = 2 * case[1]
    mags = np.array([1.0, 1e6, 1e-9, 3.0])
    xs = (r.standard_normal((m, c2)) * mags[np.arange(m) % 4][:, None]).astype(np.float32)
    x = torch.from_numpy(xs).to(torch.bfloat16).to(DEV)
    bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
    res = torch.from_numpy(r.standard_normal((m, 2 * case[0])).astype(np.float32)).to(torch.bfloat16).to(DEV)
    calls = []
    pre = ops.prescale_rows

    def counting(*a, **k):
        calls.append(1)
        return pre(*a, **k)
    monkeypatch.setattr(ops, "prescale_rows", counting)
    y = pw.linear(x, bias, out_dtype=torch.bfloat16)
    yr = pw.linear(x, bias, out_dtype=torch.bfloat16, residual=res)
    assert len(calls) == 2
    monkeypatch.setattr(ops, "PRESCALE_ROWS", False)
    y_ref = pw.linear(x, bias, out_dtype=torch.bfloat16)
    yr_ref = pw.linear(x, bias, out_dtype=torch.bfloat16, residual=res)
    assert len(calls) == 2
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(yr.view(torch.int16), yr_ref.view(torch.int16))
    # float32 rows: the DMA kernel on the prescaled rows against the
    # register-staged kernel on the float32 rows -- the same fp16 operands, so
    # within float32 accumulation order of sum |x| |A16| (float32 outputs),
    # plus one fp16 rounding of the output (fp16 outputs)
    monkeypatch.setattr(ops, "PRESCALE_ROWS", True)
    x32 = torch.from_numpy(xs).to(DEV)
    assert pw.kernel_for(m, torch.float32, torch.float16) == N.KERNEL_TILED
    y16 = pw.linear(x32, bias, out_dtype=torch.float16).float()
    y32 = pw.linear(x32, bias, out_dtype=torch.float32)
    assert len(calls) == 4
    monkeypatch.setattr(ops, "PRESCALE_ROWS", False)
    y16_ref = pw.linear(x32, bias, out_dtype=torch.float16).float()
    y32_ref = pw.linear(x32, bias, out_dtype=torch.float32)
    a16 = tdev(np.abs(O.wide_weight(oplanes, codebook, rotation, fp16=True)).astype(np.float32))
    acc = 2.0 ** -24 * 4 * c2 * (x32.abs() @ a16.T + bias.abs())
    assert torch.all((y32 - y32_ref).abs() <= acc)
    near = (y16 - y16_ref).abs() <= 2.0 ** -10 * y16_ref.abs() + acc
    assert torch.all(near | (y16 == y16_ref))  # rows of 1e6: both overflow fp16 alike


PRESCALED_SHAPES = [REAL_SHAPES[0], REAL_SHAPES[2], REAL_SHAPES[3], REAL_SHAPES[5], CASES[7]]


@pytest.mark.parametrize("gscale", [1.0, 1e6], ids=["g1", "g1e6"])
@pytest.mark.parametrize("m,flags", [(128, 2), (300, 2), (12672, 0)])
@pytest.mark.parametrize("case", PRESCALED_SHAPES, ids=["qkv", "fc1", "fc2", "l-qkv-psk16", "rot"])
def test_wide_linear_prescaled_fp16_rows(case, m, flags, gscale):
    """A packed layer on the DMA kernel fed prescaled fp16 rows
    (rpfq_layer_norm_prescaled, then rpfq_wide_linear_scaled with fp16 x and
    the row scales) against the same layer on the bf16 LayerNorm output with
    its range-guard prescales: bf16 outputs bit-identical, with and without
    bias, with the residual add, and for rows beyond fp16's range; with the
    GELU in the store (the bf16 rows then take the register-staged kernel)
    within two bf16 roundings, the GELU's slope times one of them included,
    of the bf16-row path.  flags 2 (RPFQ_FLAG_NO_STREAM) puts the small
    launches on the DMA kernel; 12,672 rows take it by default."""
    ops, N = qm()
    r = rng(2200 + m + case[0] + case[1])
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    c2 = 2 * case[1]
    assert pw.kernel_for(m, torch.float16, torch.bfloat16, flags) == N.KERNEL_DMA
    assert pw.kernel_for(m, torch.float16, torch.bfloat16, flags | N.FLAG_GELU) == N.KERNEL_DMA
    x = torch.from_numpy((r.standard_normal((m, c2)) * 3 + 1).astype(np.float32)).to(torch.bfloat16).to(DEV)
    g = tdev((r.standard_normal(c2) * gscale).astype(np.float32))
    b = tdev((r.standard_normal(c2) * gscale).astype(np.float32))
    bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
    h16, sc = ops.layer_norm_prescaled(x, g, b, 1e-6)
    h = ops.layer_norm(x, g, b, 1e-6)
    for bb in (bias, None):
        y = pw.linear(h16, bb, out_dtype=torch.bfloat16, flags=flags, row_scale=sc)
        y_ref = pw.linear(h, bb, out_dtype=torch.bfloat16, flags=flags)
        assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16)), (case, m, bb is None)
    res = torch.from_numpy(r.standard_normal((m, 2 * case[0])).astype(np.float32)).to(torch.bfloat16).to(DEV)
    y = pw.linear(h16, bias, out_dtype=torch.bfloat16, flags=flags, residual=res, row_scale=sc)
    y_ref = pw.linear(h, bias, out_dtype=torch.bfloat16, flags=flags, residual=res)
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    if gscale == 1.0 and m <= 300:  # the oracle on the bf16 rows (exact prescales: the unscaled bound)
        hf = h.float().cpu().numpy().astype(np.float64)
        y32 = pw.linear(h16, bias, out_dtype=torch.float32, flags=flags, row_scale=sc).cpu().numpy()
        check_against_oracle(y32, hf, bias.cpu().numpy().astype(np.float64), oplanes, codebook, rotation)
    yg = pw.linear(h16, bias, out_dtype=torch.bfloat16, flags=flags, gelu=True, row_scale=sc).float()
    yg_ref = pw.linear(h, bias, out_dtype=torch.bfloat16, flags=flags, gelu=True).float()
    plain = pw.linear(h, bias, out_dtype=torch.float32, flags=flags).abs()
    # the two kernels accumulate in different orders: float32 rounding of
    # sum |h| |A| (2K' terms) on top of the bf16 roundings
    scale = h.float().abs() @ tdev(np.abs(a_ref).astype(np.float32)).T + bias.abs()
    bound = 2.0 ** -5 * torch.maximum(yg_ref.abs(), plain) + 2.0 ** -24 * 4 * c2 * scale
    assert torch.all((yg - yg_ref).abs() <= bound), float(((yg - yg_ref).abs() - bound).max())


# LayerNorm fused into the streaming kernel (rpfq_layer_norm_wide_linear):
# ViT-B/16 qkv / fc1 / proj (K' = 384, the largest fused K'), DeiT-Ti qkv
# with rotation, a 16-PSK layer, a sign-codebook layer
LN_CASES = [
    (1152, 384, "axis", 2, 0, None),
    (1536, 384, "axis", 2, 0, None),
    (384, 384, "axis", 2, 0, None),
    (288, 96, "axis", 2, 0, ((0.8, 0.6), (0.6, -0.8))),
    (1024, 384, "psk16", 1, 0, None),
    (200, 64, "sign", 2, 0, None),
]


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [9, 45, 197])
@pytest.mark.parametrize("case", LN_CASES, ids=[f"{c[0]}x{c[1]}-{c[2]}" for c in LN_CASES])
def test_layer_norm_wide_linear(case, m, xdt):
    """One launch of LayerNorm + packed layer against the two launches it
    replaces (rpfq_layer_norm with x's dtype, then rpfq_wide_linear on the
    same streaming kernel): the normalized rows differ only where the float32
    statistics, summed in another order, move a value across a rounding
    boundary of x's dtype, by one ulp u_x, so |y - y_sep| <= u_x |h| |A16| +
    float32 accumulation; the separate path itself against the oracle.  Also
    without the affine parameters and with the GELU in the store."""
    ops, N = qm()
    r = rng(1900 + m + case[0] + case[1])
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    assert pw.ln_fusable(m, xdt), (case, m)
    c2 = 2 * case[1]
    x = torch.from_numpy((r.standard_normal((m, c2)) * 3 + 1).astype(np.float32)).to(xdt).to(DEV)
    g = tdev(r.standard_normal(c2).astype(np.float32))
    b = tdev(r.standard_normal(c2).astype(np.float32))
    bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
    u_x = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[xdt]
    a16 = np.abs(O.wide_weight(oplanes, codebook, rotation, fp16=True).astype(np.float64))
    for gg, bb in ((g, b), (None, None)):
        y = pw.layer_norm_linear(x, gg, bb, 1e-6, bias, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
        h = ops.layer_norm(x, gg, bb, 1e-6)
        y_sep = pw.linear(h, bias, out_dtype=torch.float32).cpu().numpy().astype(np.float64)
        hf = h.float().cpu().numpy().astype(np.float64)
        scale = np.abs(hf) @ a16.T + np.abs(bias.cpu().numpy())
        assert np.all(np.abs(y - y_sep) <= u_x * (np.abs(hf) @ a16.T) + 2e-6 * scale + 1e-5), (case, m)
        check_against_oracle(y_sep, hf, bias.cpu().numpy().astype(np.float64), oplanes, codebook, rotation)
    yg = pw.layer_norm_linear(x, g, b, 1e-6, bias, out_dtype=torch.float16, gelu=True).float().cpu().numpy()
    h = ops.layer_norm(x, g, b, 1e-6)
    yg_sep = pw.linear(h, bias, out_dtype=torch.float16, gelu=True).float().cpu().numpy()
    hf = h.float().cpu().numpy().astype(np.float64)
    assert np.all(np.abs(yg - yg_sep) <= 1.2 * u_x * (np.abs(hf) @ a16.T) + 2.0 ** -9 * np.abs(yg_sep) + 1e-4)


AQ_CASES = [LN_CASES[0], LN_CASES[2], LN_CASES[3], LN_CASES[4], LN_CASES[5]]


@pytest.mark.parametrize("layer_norm", [False, True], ids=["aq", "ln-aq"])
@pytest.mark.parametrize("bits", [4, 8, 2, 16])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [9, 197])
@pytest.mark.parametrize("case", AQ_CASES, ids=[f"{c[0]}x{c[1]}-{c[2]}" for c in AQ_CASES])
def test_act_quant_wide_linear(case, m, xdt, bits, layer_norm):
    """The act quant (after the LayerNorm when layer_norm) in the streaming
    kernel's row prologue (rpfq_act_quant_wide_linear): the quantized rows are
    bit-identical to rpfq_act_quant / rpfq_layer_norm_act_quant's, so the
    output is the oracle's product on those rows within float32 accumulation
    only (a single element quantized differently moves its row by a whole
    quantization step and fails the bound); with a residual, the fp16 output
    within its two roundings of the oracle's sum."""
    ops, N = qm()
    r = rng(2100 + m + case[0] + case[1] + bits)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    assert pw.ln_fusable(m, xdt), (case, m)
    c2 = 2 * case[1]
    x = torch.from_numpy((r.standard_normal((m, c2)) * 3 + 1).astype(np.float32)).to(xdt).to(DEV)
    g = tdev(r.standard_normal(c2).astype(np.float32))
    b = tdev(r.standard_normal(c2).astype(np.float32))
    bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
    if layer_norm:
        h = ops.layer_norm(x, g, b, 1e-6, act_bits=bits)
        ln = (g, b, 1e-6)
    else:
        h = ops.act_quant(x, bits)
        ln = None
    hf = h.float().cpu().numpy().astype(np.float64)
    y = pw.act_quant_linear(x, bits, bias, out_dtype=torch.float32, layer_norm=ln).cpu().numpy()
    check_against_oracle(y, hf, bias.cpu().numpy().astype(np.float64), oplanes, codebook, rotation)
    res = torch.from_numpy(r.standard_normal((m, 2 * case[0])).astype(np.float32)).to(torch.float16).to(DEV)
    yr = pw.act_quant_linear(x, bits, bias, out_dtype=torch.float16, residual=res,
                             layer_norm=ln).float().cpu().numpy()
    a16 = O.wide_weight(oplanes, codebook, rotation, fp16=True).astype(np.float64)
    lay = hf @ a16.T + bias.cpu().numpy()
    ref = lay + res.float().cpu().numpy()
    scale = np.abs(hf) @ np.abs(a16).T + np.abs(bias.cpu().numpy())
    u = 2.0 ** -11
    assert np.all(np.abs(yr - ref) <= 1e-5 * scale + u * np.abs(lay) + 1.001 * u * np.abs(ref) + 1e-5)


def test_act_quant_wide_linear_refuses():
    """Launches outside the row prologue's forms and bad arguments raise."""
    ops, N = qm()
    r = rng(2190)
    pw, *_ = build_packed(r, LN_CASES[1])
    x = torch.zeros(300, 768, dtype=torch.float16, device=DEV)
    with pytest.raises(N.RPFQError, match="RPFQ_ERR_VALUE"):
        pw.act_quant_linear(torch.zeros(50432, 768, dtype=torch.float16, device=DEV), 4)
    with pytest.raises(N.RPFQError, match="RPFQ_ERR_BITS"):
        pw.act_quant_linear(x[:197], 1)
    with pytest.raises(N.RPFQError, match="RPFQ_ERR_VALUE"):
        pw.act_quant_linear(x[:197], 4, gelu=True, residual=torch.zeros(197, 3072, dtype=torch.float16,
                                                                      device=DEV))


def test_layer_norm_wide_linear_refuses_unfusable():
    """Launches outside the fused kernel's forms raise (the caller runs the
    LayerNorm and the layer separately)."""
    ops, N = qm()
    r = rng(1950)
    pw, *_ = build_packed(r, LN_CASES[1])
    x = torch.zeros(300, 768, dtype=torch.float16, device=DEV)
    assert not pw.ln_fusable(50432, torch.float16)
    assert not pw.ln_fusable(4, torch.float16)  # column-split kernel
    with pytest.raises(N.RPFQError, match="RPFQ_ERR_VALUE"):
        pw.layer_norm_linear(x.float(), None, None, 1e-6)


def test_ln_fusable_follows_row_kernel_lanes():
    """The fused prologue sums the LayerNorm statistics over 64 lanes per row;
    the row kernel takes 32 lanes for C = 768 from M = 2,048 rows (M x 32 >=
    65,536), so a narrow layer that still streams there (K' = 384, N' = 64)
    is fusable at M = 2,047 -- LayerNorm + act quant rows bit-identical to
    rpfq_layer_norm_act_quant, the output within float32 accumulation of the
    oracle on them -- and refused at M = 2,048."""
    ops, N = qm()
    case = (64, 384, "axis", 2, 0, None)
    r = rng(1960)
    pw, oplanes, a_ref, codebook, rotation = build_packed(r, case)
    assert not pw.ln_fusable(2048, torch.float16)
    assert pw.ln_fusable(2047, torch.float16)
    m, c2 = 2047, 768
    x = torch.from_numpy((r.standard_normal((m, c2)) * 3 + 1).astype(np.float32)).to(torch.float16).to(DEV)
    g = tdev(r.standard_normal(c2).astype(np.float32))
    b = tdev(r.standard_normal(c2).astype(np.float32))
    bias = tdev(r.standard_normal(2 * case[0]).astype(np.float32))
    h = ops.layer_norm(x, g, b, 1e-6, act_bits=4)
    hf = h.float().cpu().numpy().astype(np.float64)
    y = pw.act_quant_linear(x, 4, bias, out_dtype=torch.float32, layer_norm=(g, b, 1e-6)).cpu().numpy()
    check_against_oracle(y, hf, bias.cpu().numpy().astype(np.float64), oplanes, codebook, rotation)


@pytest.mark.parametrize("m,c", [(3, 96), (300, 768), (17, 1024), (5, 3072)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_layer_norm_act_quant_bit_exact(m, c, xdt, ydt, bits):
    """rpfq_layer_norm_act_quant == rpfq_act_quant(rpfq_layer_norm(x) in
    float32) rounded to y's dtype, bit for bit: the float32 LN output is
    quantized (as the reference quantizes its float32 LayerNorm output) and
    only the quantized value is rounded."""
    ops, _ = qm()
    r = rng(1300 + c + bits)
    x = torch.from_numpy((r.standard_normal((m, c)) * 2 + 0.5).astype(np.float32)).to(xdt).to(DEV)
    g = tdev(r.standard_normal(c).astype(np.float32))
    b = tdev(r.standard_normal(c).astype(np.float32))
    fused = ops.layer_norm(x, g, b, 1e-6, out_dtype=ydt, act_bits=bits)
    two = ops.act_quant(ops.layer_norm(x, g, b, 1e-6, out_dtype=torch.float32), bits, out_dtype=ydt)
    assert torch.equal(fused, two)
    # and the quantization itself is the oracle's on that float32 LN output
    ln = ops.layer_norm(x, g, b, 1e-6, out_dtype=torch.float32).cpu().numpy()
    qr, qi = O.act_quant(ln[:, :c // 2], ln[:, c // 2:], bits)
    ref = torch.from_numpy(np.concatenate([qr, qi], axis=1)).to(ydt)
    assert torch.equal(fused.cpu(), ref)


@pytest.mark.parametrize("m,c", [(3, 96), (300, 768), (17, 3072), (5, 4096), (1100, 3072), (1030, 768)])
@pytest.mark.parametrize("xdt,ydt", [(torch.float16, torch.float16), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_gelu_act_quant_bit_exact(m, c, xdt, ydt, bits):
    """rpfq_gelu_act_quant == rpfq_act_quant(torch's exact GELU in float32)
    rounded to y's dtype, bit for bit (the float32 GELU is quantized as the
    reference quantizes fc2's float32 input; only the quantized value is
    rounded), and that quantization is the oracle's; in place too."""
    import torch.nn.functional as F

    ops, _ = qm()
    r = rng(1400 + c + bits)
    x = torch.from_numpy((r.standard_normal((m, c)) * 2).astype(np.float32)).to(xdt).to(DEV)
    fused = ops.gelu_act_quant(x, bits, out_dtype=ydt)
    ge = F.gelu(x.float())
    assert torch.equal(fused, ops.act_quant(ge, bits, out_dtype=ydt))
    g = ge.cpu().numpy()
    qr, qi = O.act_quant(g[:, :c // 2], g[:, c // 2:], bits)
    assert torch.equal(fused.cpu(), torch.from_numpy(np.concatenate([qr, qi], axis=1)).to(ydt))
    if xdt == ydt:
        ops_, N = qm()
        y = x.clone()
        N.check("rpfq_gelu_act_quant", N.load().rpfq_gelu_act_quant(
            y.data_ptr(), N.dtype_code(xdt), m, c, bits, y.data_ptr(), N.dtype_code(ydt), N.stream_of(y)))
        torch.cuda.synchronize()
        assert torch.equal(y, fused)


def _gelu_boundary_rows(bits, c, r):
    """float32 rows whose GELU * scale crowds the act quant's rounding
    boundaries k + 1/2: one anchor element fixes the half's maximum (7.0,
    exactly its own GELU in float32; or 0.3, a maximum from the small
    positive range), the rest sits within +-3e-4 of the x whose exact GELU *
    scale is a boundary, on both sides.  Boundaries of the positive branch
    and, for the small anchor, of the negative one (x < -0.75)."""
    from scipy.optimize import brentq
    from scipy.special import ndtr

    def gelu(t):
        return t * ndtr(t)
    qmax = 2 ** (bits - 1) - 1
    rows = []
    half = c // 2
    for anchor in (7.0, 0.3):
        amax = gelu(anchor)
        sc = qmax / amax
        if anchor == 7.0:
            targets = [((k + 0.5) / sc, 0.0, 10.0) for k in range(0, min(qmax, 6))]
        else:
            targets = [(-(k + 0.5) / sc, -8.0, -0.7518) for k in range(0, 5) if (k + 0.5) / sc < 0.16]
        for tgt, lo, hi in targets:
            x0 = brentq(lambda t: gelu(t) - tgt, lo, hi, xtol=1e-15)
            xs = x0 + 2e-7 * max(1.0, abs(x0)) * np.arange(-(half // 2), half - half // 2)
            row_half = xs.astype(np.float32)
            row_half[r.integers(0, half)] = anchor
            other = r.standard_normal(half).astype(np.float32) * 0.05
            other[r.integers(0, half)] = anchor
            rows.append(np.concatenate([row_half, other]))
            rows.append(np.concatenate([other, row_half]))
    return np.stack(rows)


@pytest.mark.parametrize("c", [768, 3072])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("big", [False, True], ids=["block", "lanes64"])
def test_gelu_act_quant_near_boundaries(c, bits, big):
    """GELU + act quant against torch's GELU followed by the act quant, bit
    for bit, on rows built to crowd the rounding boundaries (any GELU that
    is not torch's float32 erf form, bit for bit, moves some of these
    elements a level); both kernel forms (a workgroup per row for few rows,
    64 lanes per row for many)."""
    import torch.nn.functional as F

    ops, _ = qm()
    r = rng(1500 + c + bits)
    rows = _gelu_boundary_rows(bits, c, r)
    if big:  # past the workgroup-per-row form's row limit
        rows = np.concatenate([rows] * (1100 // len(rows) + 1))
    x = torch.from_numpy(rows).to(DEV)
    fused = ops.gelu_act_quant(x, bits, out_dtype=torch.float32)
    ref = ops.act_quant(F.gelu(x), bits, out_dtype=torch.float32)
    assert torch.equal(fused, ref)
    g = F.gelu(x).cpu().numpy()
    qr, qi = O.act_quant(g[:, :c // 2], g[:, c // 2:], bits)
    assert torch.equal(fused.cpu(), torch.from_numpy(np.concatenate([qr, qi], axis=1)))


@pytest.mark.parametrize("bits", [4, 8])
def test_gelu_act_quant_maximum_candidates(bits):
    """The GELU + act-quant pass evaluates a fast GELU and torch's erf form
    only where they could quantize differently; the half's maximum must
    still be torch's: rows whose largest elements sit within a few ulps of
    each other (every one a candidate; ties included), rows whose maximum
    is below 0.25 (computed in torch's form throughout), a maximum from the
    negative branch, against torch's GELU + act quant bit for bit at 64
    lanes per row (M = 1,100)."""
    import torch.nn.functional as F

    ops, _ = qm()
    r = rng(1600 + bits)
    c, m = 3072, 1100
    x = (r.standard_normal((m, c)) * 0.5).astype(np.float32)
    for i in range(m):
        kind = i % 4
        top = np.float32(1.0 + 6.0 * r.random())
        idx = r.choice(c, size=24, replace=False)
        if kind == 0:    # near-ties below the maximum, both halves
            x[i, idx] = top - np.arange(24, dtype=np.float32) * np.spacing(top)
        elif kind == 1:  # exact ties
            x[i, idx] = top
        elif kind == 2:  # maxima below 0.25 (GELU of x < 0.4), negative branch included
            x[i] = (r.random(c).astype(np.float32) - 0.75) * 0.5
        else:            # the largest |GELU| from the negative branch (min GELU ~ -0.17 at x ~ -0.75)
            x[i] = (r.random(c).astype(np.float32) * 0.2 - 0.85)
    xd = tdev(x)
    fused = ops.gelu_act_quant(xd, bits, out_dtype=torch.float32)
    ref = ops.act_quant(F.gelu(xd), bits, out_dtype=torch.float32)
    assert torch.equal(fused, ref)


@pytest.mark.parametrize("c", [768, 3072])
@pytest.mark.parametrize("ydt", [torch.float16, torch.float32])
@pytest.mark.parametrize("bits", [2, 4])
def test_gelu_act_quant_fp16_every_input(c, ydt, bits):
    """fp16 rows past the workgroup-per-row limit read torch's float32 GELU
    from a per-device table (every fp16 x in (-16, 16)) and evaluate it per
    element beyond: every finite fp16 bit pattern, the table's edges and
    neighbours (16, -16) and magnitudes to 65504, M = 1,100. Bit for bit
    against the per-element kernel on the same rows (two 550-row launches,
    a workgroup per row), against torch's GELU followed by the act quant,
    and in place."""
    import torch.nn.functional as F

    ops, N = qm()
    r = rng(1700 + c + bits)
    m = 1100
    vals = (r.standard_normal((m, c)) * 3).astype(np.float16)
    flat = vals.reshape(-1)
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    allh = allh[np.isfinite(allh)]
    flat[: len(allh)] = allh
    edges = np.array([16.0, 15.99, 16.02, -16.0, -15.99, -16.02, 65504.0, -65504.0, 0.0, -0.0, 6e-8, -6e-8,
                      8.0, -10.0, 1000.0, -1000.0], np.float16)
    idx = r.choice(np.arange(len(allh), flat.size), size=len(edges) * 40, replace=False)
    flat[idx] = np.tile(edges, 40)
    x = torch.from_numpy(vals).to(DEV)
    fused = ops.gelu_act_quant(x, bits, out_dtype=ydt)
    per_elem = torch.cat([ops.gelu_act_quant(x[:550], bits, out_dtype=ydt),
                          ops.gelu_act_quant(x[550:], bits, out_dtype=ydt)])
    assert torch.equal(fused, per_elem)
    assert torch.equal(fused, ops.act_quant(F.gelu(x.float()), bits, out_dtype=ydt))
    if ydt == torch.float16:
        y = x.clone()
        N.check("rpfq_gelu_act_quant", N.load().rpfq_gelu_act_quant(
            y.data_ptr(), N.dtype_code(torch.float16), m, c, bits, y.data_ptr(), N.dtype_code(ydt),
            N.stream_of(y)))
        torch.cuda.synchronize()
        assert torch.equal(y, fused)


@pytest.mark.parametrize("k", [8, 384, 1536])
def test_act_quant_row_kernel_matches_oracle(k):
    """The register-resident act-quant kernel (K' % 8 == 0) is bit-exact with
    the oracle's restatement of quant_i.py:438-455 in float32."""
    ops, _ = qm()
    r = rng(1400 + k)
    xs = (r.standard_normal((41, 2 * k)) * 3).astype(np.float32)
    xs[0, :] = 0.0           # all-zero row: the 1e-5 clamp
    xs[1, :k] = 1.5          # ties at the half-scale points
    for bits in (2, 4, 8):
        ys = ops.act_quant(tdev(xs), bits).cpu().numpy()
        qr, qi = O.act_quant(xs[:, :k], xs[:, k:], bits)
        assert np.array_equal(ys, np.concatenate([qr, qi], axis=1))


# ---------------------------------------------------------------------------
# input gradient on the packed blob (rpfq_wide_linear_grad_x; the reference
# operator's backward grad_x = grad_output @ w_quant, kernel.py:585)
# ---------------------------------------------------------------------------
def check_grad_x(gx, gyf, oplanes, codebook, rotation, gy_rel=0.0, out_ulp=0.0):
    """gx from the HIP kernel vs the oracle's gy @ A16 on the forward's fp16
    operand: float32 accumulation within 1e-5 of sum |gy| |A16|, plus gy_rel
    of it for the fp16 rounding of a float32 grad_y (2^-11) and out_ulp of
    |gx| for the rounding of a 16-bit output."""
    a16 = O.wide_weight(oplanes, codebook, rotation, fp16=True).astype(np.float64)
    ref = O.wide_linear_grad_x(gyf, oplanes, codebook, rotation, fp16_weight=True)
    scale = np.abs(gyf) @ np.abs(a16)
    err = np.abs(gx.astype(np.float64) - ref)
    assert np.all(err <= (1e-5 + gy_rel) * scale + out_ulp * np.abs(ref) + 1e-35), \
        float((err / np.maximum(scale, 1e-300)).max())


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[4], CASES[6], CASES[7], CASES[8]],
                         ids=["96x64", "50x48", "130x512-b256", "psk16", "rot", "table"])
def test_wide_pack_adjoint_layout(case):
    """The adjoint blob: code byte (row n, column k) in tile (k // 32,
    n // 32), column k % 32, byte 16 g + 4 s + e where n % 32 = 8 s + 4 g + e
    -- the forward tiles' byte order with rows and columns exchanged -- bit
    for bit; and the U / W tables after the codes: entry (row n, block of k,
    index of (n, k)) is the fp16 rounding of the oracle's de-rotated U and W
    of element (n, k), for every element of the layer."""
    r = rng(400)
    pw, oplanes, _, codebook, rotation = build_packed(r, case)
    n_c, k_c, block = case[0], case[1], case[4]
    nt, ks = -(-n_c // 32), -(-k_c // 32)
    codes = pw.blob[: nt * ks * 1024].cpu().numpy().reshape(nt, ks, 32, 32)
    b = np.arange(32)
    perm = 8 * ((b >> 2) & 3) + 4 * (b >> 4) + (b & 3)  # index held by byte b of a tile row
    full = np.zeros((nt * 32, ks * 32), np.uint8)
    for t in range(nt):
        for s in range(ks):
            full[t * 32:(t + 1) * 32, s * 32 + perm] = codes[t, s]
    adj = pw.adjoint().cpu().numpy()
    assert adj.size == pw.adjoint().numel()
    tiles = adj[: nt * ks * 1024].reshape(ks, nt, 32, 32)
    want = np.zeros_like(tiles)
    for s in range(ks):
        for t in range(nt):
            want[s, t][:, b] = full[t * 32 + perm, s * 32:(s + 1) * 32].T
    assert np.array_equal(tiles, want)
    nblk = 1 if block == 0 else -(-k_c // block)
    lut = adj[nt * ks * 1024:].view(np.float16).reshape(nt * 32, nblk, 32, 2)
    u_re, u_im, w_re, w_im = (np.asarray(v, np.float32).astype(np.float16)
                              for v in O.wide_parts(oplanes, codebook, rotation))
    n_idx, k_idx = np.meshgrid(np.arange(n_c), np.arange(k_c), indexing="ij")
    blk = k_idx // block if block else np.zeros_like(k_idx)
    cb = full[:n_c, :k_c].astype(np.int64)
    got_u = lut[n_idx, blk, cb & 15]
    got_w = lut[n_idx, blk, 16 + (cb >> 4)]
    for got, re, im in ((got_u, u_re, u_im), (got_w, w_re, w_im)):
        assert np.array_equal(got[..., 0].view(np.uint16), re.view(np.uint16))
        assert np.array_equal(got[..., 1].view(np.uint16), im.view(np.uint16))


@pytest.mark.parametrize("m", [1, 64, 65, 300])
@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}-{c[2]}{c[3]}-b{c[4]}-r{int(c[5] is not None)}"
                                             for c in CASES])
def test_wide_linear_grad_x(case, m):
    """fp16 grad_y (exact operands) into float32 grad_x, every codebook,
    N' / K' tails, per-block scales, rotation, 64- and 128-row tiles."""
    r = rng(500 + m)
    pw, oplanes, _, codebook, rotation = build_packed(r, case)
    gy = torch.from_numpy(r.standard_normal((m, 2 * case[0])).astype(np.float32)).to(torch.float16)
    gx = pw.grad_x(gy.to(DEV), out_dtype=torch.float32).cpu().numpy()
    assert gx.shape == (m, 2 * case[1])
    check_grad_x(gx, gy.float().numpy().astype(np.float64), oplanes, codebook, rotation)


GRAD_DT = [(torch.float16, torch.float16), (torch.float16, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
           (torch.bfloat16, torch.float32), (torch.float32, torch.float32), (torch.float32, torch.float16)]
_ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8, torch.float32: 0.0}


@pytest.mark.parametrize("gdt,xdt", GRAD_DT, ids=[f"{str(a)[6:]}-{str(b)[6:]}" for a, b in GRAD_DT])
@pytest.mark.parametrize("case", [(160, 128, "axis", 2, 0, None), (100, 96, "sign", 2, 0, None)],
                         ids=["160x128", "100x96"])
@pytest.mark.parametrize("m", [77, 300])
def test_wide_linear_grad_x_dtypes(gdt, xdt, case, m):
    """grad_y fp16 / bf16 / float32 (bf16 values are exact fp16 operands
    after the per-row power-of-two scaling; float32 ones round once, 2^-11),
    16-bit outputs within their rounding; N' % 8 != 0 takes element loads."""
    r = rng(600 + m)
    pw, oplanes, _, codebook, rotation = build_packed(r, case)
    gy = torch.from_numpy(r.standard_normal((m, 2 * case[0])).astype(np.float32)).to(gdt)
    gx = pw.grad_x(gy.to(DEV), out_dtype=xdt).float().cpu().numpy()
    check_grad_x(gx, gy.float().numpy().astype(np.float64), oplanes, codebook, rotation,
                 gy_rel=2.0 ** -11 if gdt == torch.float32 else 0.0, out_ulp=_ULP[xdt])


@pytest.mark.parametrize("gdt", [torch.float32, torch.bfloat16])
def test_wide_linear_grad_x_row_scaling(gdt):
    """Rows far outside fp16's range (1e-9 flushes to zero in fp16, 1e30
    overflows) and a zero row keep each row's relative accuracy: the per-row
    power of two is applied before the fp16 rounding and undone exactly."""
    r = rng(700)
    case = (160, 128, "axis", 2, 0, None)
    pw, oplanes, _, codebook, rotation = build_packed(r, case)
    row_scale = np.array([1.0, 1e-9, 1e30, 1e-30, 0.0, 3e4, 7e-5])[:, None]
    gy = torch.from_numpy((r.standard_normal((7, 320)) * row_scale).astype(np.float32)).to(gdt)
    gx = pw.grad_x(gy.to(DEV), out_dtype=torch.float32).cpu().numpy()
    assert np.all(gx[4] == 0.0)
    check_grad_x(gx, gy.float().numpy().astype(np.float64), oplanes, codebook, rotation,
                 gy_rel=2.0 ** -11 if gdt == torch.float32 else 0.0)


@pytest.mark.parametrize("n_c,k_c", [(1152, 384), (384, 384), (1536, 384), (384, 1536), (512, 2048)],
                         ids=["qkv", "proj", "fc1", "fc2", "L-fc2"])
def test_wide_linear_grad_x_model_shapes(n_c, k_c):
    """The ViT-B/16 layer shapes (and ViT-L fc2) at M = 2000 and 128, fp16
    grad_y into fp16 grad_x, every row against the oracle."""
    r = rng(800)
    pw, oplanes, _, codebook, rotation = build_packed(r, (n_c, k_c, "axis", 2, 0, None))
    for m in (2000, 128):
        gy = torch.from_numpy(r.standard_normal((m, 2 * n_c)).astype(np.float32)).to(torch.float16)
        gx = pw.grad_x(gy.to(DEV), out_dtype=torch.float16).float().cpu().numpy()
        check_grad_x(gx, gy.float().numpy().astype(np.float64), oplanes, codebook, rotation,
                     out_ulp=2.0 ** -11)
