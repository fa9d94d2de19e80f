"""rpfq_quantize_wide_noalloc (the quantizer with its partials in a static
device array, for callers that cannot allocate) against rpfq_quantize_wide
with a caller workspace, through the C ABI: A_q, scales and code planes
bit-identical, on two calls in a row, the second with a smaller weight (so a
stale larger result in the shared array would show)."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(lib, N, fn, w, kind_u, steps_u, kind_w, steps_w, rot):
    d = N.QuantDesc()
    d.n_complex, d.k_complex = w.shape[0] // 2, w.shape[1] // 2
    d.kind[0], d.kind[1] = kind_u, kind_w
    d.steps[0], d.steps[1] = steps_u, steps_w
    a_q = torch.full_like(w, float("nan"))
    scales = torch.full((2, 4, 2), float("nan"), dtype=torch.float32, device=DEV)
    codes = torch.full((steps_u + steps_w, d.n_complex, d.k_complex // 4), 0xAB, dtype=torch.uint8, device=DEV)
    stream = N.stream_of(w)
    if fn == "workspace":
        work = torch.empty(lib.rpfq_quantize_workspace_bytes(ctypes.byref(d)), dtype=torch.uint8, device=DEV)
        rc = lib.rpfq_quantize_wide(ctypes.byref(d), w.data_ptr(), N.ptr(rot), a_q.data_ptr(), scales.data_ptr(),
                                    codes.data_ptr(), work.data_ptr(), work.numel(), stream)
        N.check("rpfq_quantize_wide", rc)
    else:
        rc = lib.rpfq_quantize_wide_noalloc(ctypes.byref(d), w.data_ptr(), N.ptr(rot), a_q.data_ptr(),
                                            scales.data_ptr(), codes.data_ptr(), stream)
        N.check("rpfq_quantize_wide_noalloc", rc)
    torch.cuda.synchronize()
    return a_q, scales, codes


def test_quantize_noalloc_matches_workspace_entry_point():
    from quant_models import _native as N

    lib = N.load()
    g = np.random.default_rng(2024)
    cases = [  # (out, in, kind_u, steps_u, kind_w, steps_w, rotated); the second is smaller
        (3072, 768, N.QK_AXIS, 2, N.QK_AXIS, 2, True),
        (192, 128, N.QK_SIGN, 2, N.QK_AXIS, 4, False),
    ]
    for out_f, in_f, ku, su, kw, sw, rotated in cases:
        w = torch.from_numpy((g.standard_normal((out_f, in_f)) * 0.02).astype(np.float32)).to(DEV)
        rot = None
        if rotated:
            th = np.array([0.3, -0.2], dtype=np.float32)
            rot = torch.tensor([np.cos(th[0]), np.sin(th[0]), np.cos(th[1]), np.sin(th[1])],
                               dtype=torch.float32, device=DEV)
        want = _run(lib, N, "workspace", w, ku, su, kw, sw, rot)
        got = _run(lib, N, "noalloc", w, ku, su, kw, sw, rot)
        for a, b, what in zip(got, want, ("a_q", "scales", "codes")):
            assert torch.equal(a, b), (out_f, in_f, what)
        assert not torch.isnan(got[0]).any()
