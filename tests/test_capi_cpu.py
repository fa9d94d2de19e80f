"""The C-ABI library loads, exports every symbol include/rpfq.h declares, and
rejects bad arguments with status codes -- all without a GPU (validation
runs before any HIP call)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rpfq.h")


def lib():
    from quant_models import _native
    if not os.path.exists(_native.library_path()):
        pytest.skip("librpfq.so not built")
    return _native.load(), _native


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(rpfq_\w+)\s*\(", text, re.M)))


def test_header_declares_the_binding_list():
    _, N = lib()
    assert declared() == sorted(N.EXPORTED)


def test_every_declared_symbol_exported():
    L, _ = lib()
    for name in declared():
        assert hasattr(L, name), name
    assert L.rpfq_abi_version() == 1


def _desc(N, n=64, k=64, block=0, cb=0, stages=2):
    d = N.WideDesc()
    d.n_complex, d.k_complex, d.block, d.codebook, d.stages, d.rotate = n, k, block, cb, stages, 0
    return d


def test_wide_packed_bytes_geometry():
    L, N = lib()
    d = _desc(N, n=50, k=48, block=0)
    nt, ks = 2, 2  # ceil(50/32), ceil(48/32)
    codes = nt * ks * 1024
    assert L.rpfq_wide_packed_bytes(ctypes.byref(d)) == ((codes + 255) // 256) * 256 + nt * 32 * 1 * 32
    d2 = _desc(N, n=64, k=512, block=256)
    assert L.rpfq_wide_packed_bytes(ctypes.byref(d2)) == 2 * 16 * 1024 + 2 * 32 * 2 * 32
    assert L.rpfq_wide_packed_bytes(ctypes.byref(_desc(N, k=12))) == 0  # invalid -> 0


@pytest.mark.parametrize("field,value,code", [
    ("k_complex", 12, 3), ("n_complex", 0, 2), ("block", 48, 6), ("codebook", 9, 4), ("stages", 3, 4),
    ("n_complex", 2 ** 30 + 1, 2), ("k_complex", 2 ** 24 + 8, 2)])
def test_wide_linear_rejects_bad_desc(field, value, code):
    L, N = lib()
    d = _desc(N)
    setattr(d, field, value)
    buf = ctypes.create_string_buffer(64)
    rc = L.rpfq_wide_linear(ctypes.byref(d), buf, 1 << 20, buf, 1, 4, None, buf, 1, 0, None)
    assert rc == code
    assert L.rpfq_last_error().decode()


def test_wide_linear_argument_errors():
    L, N = lib()
    d = _desc(N)
    p = ctypes.c_void_p(256)  # never dereferenced: validation fails first
    assert L.rpfq_wide_linear(None, p, 1 << 20, p, 1, 4, None, p, 1, 0, None) == 1
    assert L.rpfq_wide_linear(ctypes.byref(d), None, 1 << 20, p, 1, 4, None, p, 1, 0, None) == 1
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 1 << 20, p, 7, 4, None, p, 1, 0, None) == 5
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 1 << 20, p, 1, 0, None, p, 1, 0, None) == 2
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, p, 1, 32, None) == 6  # unknown flag bit
    # RPFQ_FLAG_RESIDENT on a layer it does not take (K' = 64); on a y that is not 16-byte aligned
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, p, 1, 16, None) == 2
    d48 = _desc(N, n=48, k=48)
    assert L.rpfq_wide_linear(ctypes.byref(d48), p, 1 << 20, p, 1, 4, None, ctypes.c_void_p(264), 1, 16,
                              None) == 3
    # RPFQ_FLAG_STREAM with a tiled-kernel flag; a streaming grid past 2^24 workgroups
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, p, 1, 4 | 1, None) == 6
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, p, 1, 4 | 2, None) == 6
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 1 << 20, p, 1, 1 << 30, None, p, 1, 4, None) == 2
    assert "2^24" in L.rpfq_last_error().decode()
    assert L.rpfq_wide_linear(ctypes.byref(d), p, 16, p, 1, 4, None, p, 1, 0, None) == 2
    assert L.rpfq_wide_linear(ctypes.byref(d), ctypes.c_void_p(258), 1 << 20, p, 1, 4, None, p, 1, 0, None) == 3
    assert "aligned" in L.rpfq_last_error().decode()


def test_unpack_phase_act_argument_errors():
    L, _ = lib()
    p = ctypes.c_void_p(256)
    assert L.rpfq_unpack(None, 2, 4, 8, None, None, 0, p, p, None) == 1
    assert L.rpfq_unpack(p, 3, 4, 8, None, None, 0, p, p, None) == 4
    assert L.rpfq_unpack(p, 2, 4, 6, None, None, 0, p, p, None) == 3
    assert L.rpfq_unpack(p, 2, 4, 8, p, None, 0, p, p, None) == 1
    assert L.rpfq_phase_linear(p, p, 0, 1, 4, 40, p, p, p, 0, 8, p, p, 0, None) == 3   # K % 32
    assert L.rpfq_phase_linear(p, p, 0, 1, 4, 64, p, p, p, 40, 8, p, p, 0, None) == 6  # block
    assert L.rpfq_phase_linear(p, p, 4, 1, 4, 64, p, p, p, 0, 8, p, p, 0, None) == 5   # dtype
    assert L.rpfq_act_quant(p, 0, 4, 7, 4, p, 0, None) == 2
    assert L.rpfq_act_quant(p, 0, 4, 8, 1, p, 0, None) == 4
    assert L.rpfq_act_quant(None, 0, 4, 8, 4, p, 0, None) == 1


def test_wide_pack_plane_count():
    L, N = lib()
    d = _desc(N)
    arr = (ctypes.c_void_p * 4)(256, 256, 256, 256)
    p = ctypes.c_void_p(256)
    assert L.rpfq_wide_pack(ctypes.byref(d), arr, 3, arr, arr, p, 1 << 20, None) == 4
    d.codebook, d.stages = 2, 1
    assert L.rpfq_wide_pack(ctypes.byref(d), arr, 4, arr, arr, p, 1 << 20, None) == 4


def test_residual_and_layer_norm_argument_errors():
    L, N = lib()
    d = _desc(N)
    p = ctypes.c_void_p(256)
    # NULL residual, bad dtype, bad flags, misaligned residual -- all before any HIP call
    assert L.rpfq_wide_linear_residual(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, None, p, 1, 0, None) == 1
    assert L.rpfq_wide_linear_residual(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, p, p, 9, 0, None) == 5
    assert L.rpfq_wide_linear_residual(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, p, p, 1, 32, None) == 6
    assert L.rpfq_wide_linear_residual(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, p, p, 1, 8, None) == 6  # GELU
    assert "GELU" in L.rpfq_last_error().decode()
    assert L.rpfq_wide_linear_residual(ctypes.byref(d), p, 1 << 20, p, 1, 4, None, ctypes.c_void_p(258), p, 1, 0,
                                       None) == 3
    assert L.rpfq_wide_linear_residual(ctypes.byref(d), p, 16, p, 1, 4, None, p, p, 1, 0, None) == 2
    assert L.rpfq_layer_norm(None, 1, 4, 64, None, None, 1e-6, p, 1, None) == 1
    assert L.rpfq_layer_norm(p, 1, 4, 60, None, None, 1e-6, p, 1, None) == 2     # C % 8
    assert L.rpfq_layer_norm(p, 1, 4, 8192, None, None, 1e-6, p, 1, None) == 2   # C > 4096
    assert L.rpfq_layer_norm(p, 1, 0, 64, None, None, 1e-6, p, 1, None) == 2
    assert L.rpfq_layer_norm(p, 5, 4, 64, None, None, 1e-6, p, 1, None) == 5
    assert L.rpfq_layer_norm(p, 1, 4, 64, None, None, -1.0, p, 1, None) == 6
    assert L.rpfq_layer_norm(ctypes.c_void_p(258), 1, 4, 64, None, None, 1e-6, p, 1, None) == 3
    assert L.rpfq_layer_norm(p, 1, 4, 64, ctypes.c_void_p(260), None, 1e-6, p, 1, None) == 3


def test_layer_norm_prescaled_argument_errors():
    """rpfq_layer_norm_prescaled and rpfq_row_prescale take bf16 / float32
    rows and a 16-byte aligned scale array; rpfq_wide_linear_scaled takes prescaled fp16
    rows only on a launch the DMA kernel runs."""
    L, N = lib()
    p = ctypes.c_void_p(256)
    assert L.rpfq_layer_norm_prescaled(None, 2, 4, 64, None, None, 1e-6, p, p, None) == 1
    assert L.rpfq_layer_norm_prescaled(p, 2, 4, 64, None, None, 1e-6, p, None, None) == 1
    assert L.rpfq_layer_norm_prescaled(p, 1, 4, 64, None, None, 1e-6, p, p, None) == 5  # fp16 x
    assert "bf16" in L.rpfq_last_error().decode()
    assert L.rpfq_layer_norm_prescaled(p, 2, 4, 60, None, None, 1e-6, p, p, None) == 2  # C % 8
    assert L.rpfq_layer_norm_prescaled(p, 2, 4, 64, None, None, -1.0, p, p, None) == 6
    assert L.rpfq_layer_norm_prescaled(p, 2, 4, 64, None, None, 1e-6, p, ctypes.c_void_p(260), None) == 3
    assert L.rpfq_row_prescale(None, 2, 4, 64, p, p, None) == 1
    assert L.rpfq_row_prescale(p, 2, 4, 64, p, None, None) == 1
    assert L.rpfq_row_prescale(p, 1, 4, 64, p, p, None) == 5  # fp16 x
    assert L.rpfq_row_prescale(p, 2, 4, 8192, p, p, None) == 2  # C > 4096
    assert L.rpfq_row_prescale(p, 2, 4, 64, ctypes.c_void_p(264), p, None) == 3
    assert L.rpfq_row_prescale(p, 2, 4, 64, p, ctypes.c_void_p(260), None) == 3
    d = _desc(N, n=1536, k=384)
    # fp16 x with row scales at 4 rows (a streaming launch) -> RPFQ_ERR_VALUE
    assert L.rpfq_wide_linear_scaled(ctypes.byref(d), p, 1 << 30, p, 1, 4, p, None, None, p, 2, 0, None) == 6
    assert "DMA" in L.rpfq_last_error().decode()


def test_layer_norm_act_quant_argument_errors():
    L, _ = lib()
    p = ctypes.c_void_p(256)
    assert L.rpfq_layer_norm_act_quant(None, 1, 4, 64, None, None, 1e-6, 4, p, 1, None) == 1
    assert L.rpfq_layer_norm_act_quant(p, 1, 4, 40, None, None, 1e-6, 4, p, 1, None) == 2   # C/2 % 8
    assert L.rpfq_layer_norm_act_quant(p, 1, 4, 64, None, None, 1e-6, 1, p, 1, None) == 4   # bits
    assert L.rpfq_layer_norm_act_quant(p, 1, 4, 64, None, None, 1e-6, 17, p, 1, None) == 4
    assert L.rpfq_layer_norm_act_quant(p, 3, 4, 64, None, None, 1e-6, 4, p, 1, None) == 5
    assert L.rpfq_layer_norm_act_quant(p, 1, 4, 64, None, None, -1.0, 4, p, 1, None) == 6


def test_gelu_act_quant_argument_errors():
    L, _ = lib()
    p = ctypes.c_void_p(256)
    assert L.rpfq_gelu_act_quant(None, 1, 4, 64, 4, p, 1, None) == 1
    assert L.rpfq_gelu_act_quant(p, 1, 4, 40, 4, p, 1, None) == 2      # C/2 % 8
    assert L.rpfq_gelu_act_quant(p, 1, 4, 8192, 4, p, 1, None) == 2    # C > 4096
    assert L.rpfq_gelu_act_quant(p, 1, 0, 64, 4, p, 1, None) == 2      # M
    assert L.rpfq_gelu_act_quant(p, 1, 4, 64, 1, p, 1, None) == 4      # bits
    assert L.rpfq_gelu_act_quant(p, 1, 4, 64, 17, p, 1, None) == 4
    assert L.rpfq_gelu_act_quant(p, 3, 4, 64, 4, p, 1, None) == 5
    assert L.rpfq_gelu_act_quant(ctypes.c_void_p(258), 1, 4, 64, 4, p, 1, None) == 3


def test_quantize_wide_argument_errors():
    L, N = lib()
    p = ctypes.c_void_p(256)
    d = N.QuantDesc()
    d.n_complex, d.k_complex = 32, 48
    d.kind[0], d.kind[1], d.steps[0], d.steps[1] = 0, 1, 2, 2
    ws = L.rpfq_quantize_workspace_bytes(ctypes.byref(d))
    assert ws == 1024 * 8 * 8
    assert L.rpfq_quantize_wide(None, p, None, p, p, None, p, ws, None) == 1
    assert L.rpfq_quantize_wide(ctypes.byref(d), None, None, p, p, None, p, ws, None) == 1   # weight
    assert L.rpfq_quantize_wide(ctypes.byref(d), p, None, p, None, None, p, ws, None) == 1   # scales
    assert L.rpfq_quantize_wide(ctypes.byref(d), p, None, p, p, None, p, ws - 8, None) == 2  # workspace
    for field, idx, value in (("kind", 0, 2), ("kind", 1, -1), ("steps", 0, 0), ("steps", 1, 5)):
        bad = N.QuantDesc()
        ctypes.pointer(bad)[0] = d
        getattr(bad, field)[idx] = value
        assert L.rpfq_quantize_wide(ctypes.byref(bad), p, None, p, p, None, p, ws, None) == 6, (field, idx)
    bad = N.QuantDesc()
    ctypes.pointer(bad)[0] = d
    bad.k_complex = 50
    assert L.rpfq_quantize_wide(ctypes.byref(bad), p, None, p, p, p, p, ws, None) == 3  # codes need K' % 4
    bad.k_complex = 0
    assert L.rpfq_quantize_wide(ctypes.byref(bad), p, None, p, p, None, p, ws, None) == 2


def test_quantize_wide_noalloc_argument_errors():
    """The no-allocation quantizer validates like rpfq_quantize_wide (no
    workspace argument), before any HIP call."""
    L, N = lib()
    p = ctypes.c_void_p(256)
    d = N.QuantDesc()
    d.n_complex, d.k_complex = 32, 48
    d.kind[0], d.kind[1], d.steps[0], d.steps[1] = 0, 1, 2, 2
    assert L.rpfq_quantize_wide_noalloc(None, p, None, p, p, None, None) == 1
    assert L.rpfq_quantize_wide_noalloc(ctypes.byref(d), None, None, p, p, None, None) == 1  # weight
    assert L.rpfq_quantize_wide_noalloc(ctypes.byref(d), p, None, p, None, None, None) == 1  # scales
    bad = N.QuantDesc()
    ctypes.pointer(bad)[0] = d
    bad.steps[1] = 5
    assert L.rpfq_quantize_wide_noalloc(ctypes.byref(bad), p, None, p, p, None, None) == 6
    bad.steps[1], bad.k_complex = 2, 50
    assert L.rpfq_quantize_wide_noalloc(ctypes.byref(bad), p, None, p, p, p, None) == 3  # codes need K' % 4
    assert "k_complex" in L.rpfq_last_error().decode()


def test_table_codebook_desc_rules():
    L, N = lib()
    d = _desc(N, n=64, k=64, cb=N.CB_TABLE, stages=1)
    # codes 2 x 2 tiles x 1 KB, then 64 rows x 32 (re, im) float32 pairs
    assert L.rpfq_wide_packed_bytes(ctypes.byref(d)) == 2 * 2 * 1024 + 64 * 64 * 4
    buf = ctypes.create_string_buffer(64)
    for field, value, code in (("stages", 2, 4), ("block", 256, 6), ("rotate", 1, 6)):
        bad = _desc(N, n=64, k=64, cb=N.CB_TABLE, stages=1)
        setattr(bad, field, value)
        assert L.rpfq_wide_linear(ctypes.byref(bad), buf, 1 << 20, buf, 1, 4, None, buf, 1, 0, None) == code, field
    p = ctypes.c_void_p(256)
    arr = (ctypes.c_void_p * 4)(p, p, p, p)
    assert L.rpfq_wide_pack(ctypes.byref(d), arr, 4, arr, arr, p, 1 << 20, None) == 4  # two planes (u, w)


def test_header_compiles_as_c99_and_links(tmp_path):
    """A native C caller (the Android runtime's role): include/rpfq.h is plain
    C99, the library links, and the validation paths answer from C."""
    import shutil
    import subprocess

    L, N = lib()
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "caller.c"
    src.write_text(r'''
#include <stdio.h>
#include "rpfq.h"
int main(void) {
    rpfq_wide_desc d = {0};
    d.n_complex = 64; d.k_complex = 64; d.block = 0; d.codebook = RPFQ_CB_AXIS; d.stages = 2; d.rotate = 0;
    if (rpfq_abi_version() != RPFQ_ABI_VERSION) return 1;
    if (rpfq_wide_packed_bytes(&d) == 0) return 2;
    d.k_complex = 12;                                  /* not a multiple of 8 */
    if (rpfq_wide_packed_bytes(&d) != 0) return 3;
    if (rpfq_wide_linear(&d, 0, 0, 0, RPFQ_F16, 4, 0, 0, RPFQ_F16, 0, 0) != RPFQ_ERR_ALIGN) return 4;
    if (rpfq_last_error()[0] == 0) return 5;
    rpfq_quant_desc q = {0};
    q.n_complex = 8; q.k_complex = 8; q.kind[0] = q.kind[1] = RPFQ_QK_AXIS; q.steps[0] = 5; q.steps[1] = 1;
    if (rpfq_quantize_wide(&q, 0, 0, 0, 0, 0, 0, 0, 0) == RPFQ_OK) return 6;
    printf("ok\n");
    return 0;
}
''')
    exe = tmp_path / "caller"
    libdir = os.path.dirname(N.library_path())
    cmd = [cc, "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe),
           "-L", libdir, "-lrpfq", f"-Wl,-rpath,{libdir}", "-Wl,-rpath,/opt/rocm/lib", "-L", "/opt/rocm/lib"]
    subprocess.run(cmd, check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and out.stdout.strip() == "ok", (out.returncode, out.stdout, out.stderr)


def test_layer_norm_wide_linear_fusable_and_errors():
    """rpfq_layer_norm_wide_linear_fusable (no GPU work): the LayerNorm fuses
    into the streaming kernel's split-K forms only -- ViT-B qkv / fc1 / proj
    at one image (197 rows), not at 50,432 rows (DMA kernel), not for M <= 8
    on the column-split kernel, not for K' > 384, float32 x, per-block scales
    or the TABLE codebook; rpfq_layer_norm_wide_linear validates its
    arguments on the host and refuses launches the query refuses."""
    L, N = lib()

    def fusable(d, m, xdt=1, ydt=1):
        out = ctypes.c_int32(-1)
        assert L.rpfq_layer_norm_wide_linear_fusable(ctypes.byref(d), m, xdt, ydt, ctypes.byref(out)) == 0
        return out.value
    for n, k in ((1152, 384), (1536, 384), (384, 384), (288, 96)):
        assert fusable(_desc(N, n=n, k=k), 197) == 1, (n, k)
        assert fusable(_desc(N, n=n, k=k), 197, xdt=2, ydt=2) == 1, (n, k)
    fc1 = _desc(N, n=1536, k=384)
    assert fusable(fc1, 50432) == 0
    assert fusable(fc1, 1) == 0          # column-split kernel
    assert fusable(fc1, 197, xdt=0) == 0  # float32 x
    assert fusable(_desc(N, n=1536, k=512), 197) == 0       # K' > 384 (ViT-L: measured slower fused)
    assert fusable(_desc(N, n=1536, k=384, block=128), 197) == 0
    assert fusable(_desc(N, n=1536, k=384, cb=N.CB_TABLE, stages=1), 197) == 0
    out = ctypes.c_int32(-1)
    assert L.rpfq_layer_norm_wide_linear_fusable(ctypes.byref(fc1), 197, 1, 1, None) == 1
    assert L.rpfq_layer_norm_wide_linear_fusable(ctypes.byref(fc1), 0, 1, 1, ctypes.byref(out)) == 2
    assert L.rpfq_layer_norm_wide_linear_fusable(ctypes.byref(fc1), 197, 7, 1, ctypes.byref(out)) == 5
    # launches: argument errors before any GPU work
    nbytes = L.rpfq_wide_packed_bytes(ctypes.byref(fc1))
    fake = 1 << 20  # an aligned non-NULL address; never dereferenced on these paths

    def call(d=fc1, packed=fake, nb=nbytes, x=fake, xdt=1, m=197, g=None, b=None, eps=1e-6, y=fake, ydt=1,
             flags=0):
        return L.rpfq_layer_norm_wide_linear(ctypes.byref(d), packed, nb, x, xdt, m, g, b, ctypes.c_float(eps),
                                             None, y, ydt, flags, None)
    assert call(packed=None) == 1 and call(x=None) == 1 and call(y=None) == 1
    assert call(xdt=9) == 5
    assert call(m=0) == 2
    assert call(flags=N.FLAG_NO_STREAM) == 6
    assert call(eps=-1.0) == 6
    assert call(nb=nbytes - 1) == 2
    assert call(x=fake + 8) == 3 and call(g=fake + 4) == 3
    assert call(m=50432) == 6  # not fusable: use rpfq_layer_norm + rpfq_wide_linear
    assert b"rpfq_layer_norm" in L.rpfq_last_error()


def test_wide_linear_kernel_choice():
    """rpfq_wide_linear_kernel (no GPU work): the streaming kernels for a few
    rows and for small one-tile-deep launches (the column-split one for
    M <= 8 on few tiles of short K' or many tiles of long K'), the DMA kernel
    for large fp16 launches, the register-staged kernel for float32 x, bf16
    x and output with GELU, or RPFQ_FLAG_TILE_M128; the flags force their
    kernels."""
    L, N = lib()
    d = _desc(N, n=1536, k=384)  # ViT-B fc1

    def kernel(m, xdt=1, ydt=1, flags=0):
        out = ctypes.c_int32(-1)
        assert L.rpfq_wide_linear_kernel(ctypes.byref(d), m, xdt, ydt, flags, ctypes.byref(out)) == 0
        return out.value
    assert kernel(1) == N.KERNEL_GEMV and kernel(8) == N.KERNEL_GEMV and kernel(9) == N.KERNEL_STREAM
    assert kernel(16) == N.KERNEL_STREAM
    assert kernel(197) == N.KERNEL_STREAM  # one image: 624 (chunk, tile) groups vs one 128-row tile deep
    assert kernel(50432) == N.KERNEL_DMA
    assert kernel(50432, flags=N.FLAG_GELU) == N.KERNEL_DMA
    assert kernel(50432, ydt=2, flags=N.FLAG_GELU) == N.KERNEL_DMA  # prescaled fp16 rows into a bf16 model's fc1
    assert kernel(50432, xdt=2, ydt=2, flags=N.FLAG_GELU) == N.KERNEL_TILED
    assert kernel(50432, xdt=0) == N.KERNEL_TILED
    assert kernel(300, flags=N.FLAG_TILE_M128) == N.KERNEL_TILED
    assert kernel(197, flags=N.FLAG_NO_STREAM) == N.KERNEL_DMA
    assert kernel(50432, flags=N.FLAG_STREAM) == N.KERNEL_STREAM
    assert kernel(8, flags=N.FLAG_STREAM) == N.KERNEL_GEMV
    d_long = _desc(N, n=384, k=1536)  # ViT-B fc2: 12 tiles of 48 k-steps
    d_many = _desc(N, n=131072, k=1536)  # 4096 tiles
    d_many_mid = _desc(N, n=131072, k=384)  # 12 k-steps: the one-wave column-split form
    d_many_short = _desc(N, n=131072, k=256)
    for dd, want in ((d_long, N.KERNEL_STREAM), (d_many, N.KERNEL_GEMV), (d_many_mid, N.KERNEL_GEMV),
                     (d_many_short, N.KERNEL_STREAM)):
        out = ctypes.c_int32(-1)
        assert L.rpfq_wide_linear_kernel(ctypes.byref(dd), 1, 1, 1, 0, ctypes.byref(out)) == 0
        assert out.value == want, (dd.n_complex, dd.k_complex, out.value)
    out = ctypes.c_int32(-1)
    assert L.rpfq_wide_linear_kernel(ctypes.byref(d), 4, 1, 1, 0, None) == 1
    assert L.rpfq_wide_linear_kernel(ctypes.byref(d), 0, 1, 1, 0, ctypes.byref(out)) == 2
    assert L.rpfq_wide_linear_kernel(ctypes.byref(d), 4, 1, 1, 32, ctypes.byref(out)) == 6


def test_wide_linear_resident_choice():
    """The resident-weight kernel: chosen by default for M >= 32768 on the
    layers it takes (Swin-T stage 0 and its stage-1 proj: K' = 48 with N' in
    {48, 96, 144, 192}, K' = 96 with N' in {48, 96}, K' = 192 with N' = 48;
    fp16 / bf16 x and y), never under
    the other kernel flags; RPFQ_FLAG_RESIDENT forces it at any M and is
    refused, before any GPU work, for a layer, dtype or flag set it does
    not take."""
    L, N = lib()

    def kernel(d, m, xdt=1, ydt=1, flags=0):
        out = ctypes.c_int32(-1)
        rc = L.rpfq_wide_linear_kernel(ctypes.byref(d), m, xdt, ydt, flags, ctypes.byref(out))
        return out.value if rc == 0 else -rc
    qkv, fc2, proj1 = _desc(N, n=144, k=48), _desc(N, n=48, k=192), _desc(N, n=96, k=96)
    for d in (qkv, fc2, proj1):
        assert kernel(d, 401408) == N.KERNEL_RESIDENT
        assert kernel(d, 32768, xdt=2, ydt=2) == N.KERNEL_RESIDENT
        assert kernel(d, 401408, flags=N.FLAG_GELU) == N.KERNEL_RESIDENT
        assert kernel(d, 32767) != N.KERNEL_RESIDENT
        assert kernel(d, 401408, xdt=0) != N.KERNEL_RESIDENT and kernel(d, 401408, ydt=0) != N.KERNEL_RESIDENT
        assert kernel(d, 401408, flags=N.FLAG_NO_STREAM) != N.KERNEL_RESIDENT
        assert kernel(d, 401408, flags=N.FLAG_TILE_M128) == N.KERNEL_TILED
        assert kernel(d, 5, flags=N.FLAG_RESIDENT) == N.KERNEL_RESIDENT
    assert kernel(fc2, 401408, flags=N.FLAG_NO_STREAM) == N.KERNEL_DMA
    # shapes it does not take
    for n, k in ((50, 48), (64, 48), (144, 64), (384, 384), (192, 192), (144, 96), (96, 192), (288, 48)):
        d = _desc(N, n=n, k=k)
        assert kernel(d, 401408) != N.KERNEL_RESIDENT
        assert kernel(d, 401408, flags=N.FLAG_RESIDENT) == -2
    assert kernel(qkv, 5, xdt=0, flags=N.FLAG_RESIDENT) == -5
    assert kernel(qkv, 5, ydt=0, flags=N.FLAG_RESIDENT) == -5
    for other in (N.FLAG_NO_STREAM, N.FLAG_STREAM, N.FLAG_TILE_M128):
        assert kernel(qkv, 5, flags=N.FLAG_RESIDENT | other) == -6
    # a residual only for N' <= 96 (its chunks are held through the MFMAs)
    p, y = ctypes.c_void_p(256), ctypes.c_void_p(512)
    assert L.rpfq_wide_linear_residual(ctypes.byref(qkv), p, 1 << 20, p, 1, 4, None, p, y, 1,
                                       N.FLAG_RESIDENT, None) == 2
    assert b"N' <= 96" in L.rpfq_last_error()


def test_wide_mlp_argument_errors():
    """rpfq_wide_mlp's host checks, all before any HIP call: NULL operands,
    fc2 not the inverse shape of fc1, the fused shapes (K' = 96, N1' a
    multiple of 96 up to 1536, block = 0, one codebook, M >= 64), short
    blobs and misaligned rows."""
    L, N = lib()
    p, y = ctypes.c_void_p(256), ctypes.c_void_p(512)
    fc1, fc2 = _desc(N, n=384, k=96), _desc(N, n=96, k=384)
    big = 1 << 24

    def mlp(d1, d2, m=12672, x=p, out=y, res=None, n1=big, n2=big, p1=p, p2=p):
        return L.rpfq_wide_mlp(ctypes.byref(d1), p1, n1, ctypes.byref(d2), p2, n2, x, m, None, None, res, out, None)

    assert mlp(fc1, fc2, x=None) == 1
    assert mlp(fc1, fc2, p2=None) == 1
    assert mlp(fc1, fc2, out=None) == 1
    assert mlp(fc1, _desc(N, n=96, k=288)) == 2 and b"invert" in L.rpfq_last_error()
    assert mlp(_desc(N, n=384, k=192), _desc(N, n=192, k=384)) == 2 and b"K'=96" in L.rpfq_last_error()
    assert mlp(_desc(N, n=400, k=96), _desc(N, n=96, k=400)) == 2      # N1' % 96
    assert mlp(_desc(N, n=1632, k=96), _desc(N, n=96, k=1632)) == 2    # N1' > 1536
    assert mlp(_desc(N, n=384, k=96, block=64), fc2) == 2                # per-block scales
    assert mlp(fc1, _desc(N, n=96, k=384, cb=N.CB_SIGN)) == 2           # two codebooks
    assert mlp(fc1, fc2, m=63) == 2
    assert mlp(fc1, fc2, m=0) == 2
    assert mlp(fc1, fc2, n1=1024) == 2                                   # short blob
    assert mlp(fc1, fc2, x=ctypes.c_void_p(264)) == 3
    assert mlp(fc1, fc2, res=ctypes.c_void_p(520)) == 3
    assert mlp(fc1, fc2, p1=ctypes.c_void_p(384)) == 3
    # the LayerNorm variant: the same checks, then eps and the affine rows' alignment
    ln = L.rpfq_layer_norm_wide_mlp
    assert ln(ctypes.byref(fc1), p, big, ctypes.byref(fc2), p, big, p, 12672, None, None, -1.0, None, None, y,
              None) == 6
    assert ln(ctypes.byref(fc1), p, big, ctypes.byref(fc2), p, big, p, 12672, ctypes.c_void_p(260), None, 1e-6,
              None, None, y, None) == 3
    assert ln(ctypes.byref(fc1), p, big, ctypes.byref(fc2), p, big, None, 12672, None, None, 1e-6, None, None, y,
              None) == 1
    assert ln(ctypes.byref(fc1), p, big, ctypes.byref(fc2), p, big, p, 32, None, None, 1e-6, None, None, y,
              None) == 2 and b"rpfq_layer_norm_wide_mlp" in L.rpfq_last_error()


def test_wide_grad_x_geometry_and_argument_errors():
    """rpfq_wide_adjoint_bytes is one 1 KiB code tile per (32-row tile,
    k-step) plus a 128-B U / W table per (row, scale block) of the padded
    rows; rpfq_wide_pack_adjoint and rpfq_wide_linear_grad_x validate every
    argument on the host before any GPU work."""
    L, N = lib()
    d = _desc(N, n=50, k=48)
    assert L.rpfq_wide_adjoint_bytes(ctypes.byref(d)) == 2 * 2 * 1024 + 64 * 128
    assert L.rpfq_wide_adjoint_bytes(ctypes.byref(_desc(N, n=1536, k=384))) == 48 * 12 * 1024 + 1536 * 128
    assert L.rpfq_wide_adjoint_bytes(ctypes.byref(_desc(N, n=64, k=512, block=256))) == 2 * 16 * 1024 + 64 * 2 * 128
    assert L.rpfq_wide_adjoint_bytes(ctypes.byref(_desc(N, k=12))) == 0  # invalid -> 0
    fc2 = _desc(N, n=384, k=1536)
    nbytes = L.rpfq_wide_packed_bytes(ctypes.byref(fc2))
    abytes = L.rpfq_wide_adjoint_bytes(ctypes.byref(fc2))
    fake = 1 << 20  # an aligned non-NULL address; never dereferenced on these paths

    def pack(packed=fake, nb=nbytes, adj=fake, ab=abytes):
        return L.rpfq_wide_pack_adjoint(ctypes.byref(fc2), packed, nb, adj, ab, None)
    assert pack(packed=None) == 1 and pack(adj=None) == 1
    assert pack(nb=nbytes - 1) == 2 and pack(ab=abytes - 1) == 2
    assert pack(adj=fake + 16) == 3

    def grad(adj=fake, ab=abytes, gy=fake, gdt=1, m=197, gx=fake, xdt=1):
        return L.rpfq_wide_linear_grad_x(ctypes.byref(fc2), adj, ab, gy, gdt, m, gx, xdt, None)
    assert grad(adj=None) == 1 and grad(gy=None) == 1 and grad(gx=None) == 1
    assert grad(gdt=7) == 5 and grad(xdt=9) == 5
    assert grad(m=0) == 2 and grad(m=(1 << 30) + 1) == 2
    assert grad(ab=abytes - 1) == 2
    assert grad(adj=fake + 128) == 3 and grad(gy=fake + 8) == 3  # N' % 8 == 0: 16-byte rows
    assert grad(gx=fake + 1) == 3
    assert L.rpfq_wide_linear_grad_x(ctypes.byref(_desc(N, k=12)), fake, abytes, fake, 1, 4, fake, 1, None) == 3


def test_act_quant_wide_linear_argument_errors():
    """rpfq_act_quant_wide_linear validates on the host before any GPU work:
    NULLs, dtypes, M, bits, flags (GELU not with a residual), eps, sizes,
    alignment, and launches outside the row prologue's forms."""
    L, N = lib()
    fc1 = _desc(N, n=1536, k=384)
    nbytes = L.rpfq_wide_packed_bytes(ctypes.byref(fc1))
    fake = 1 << 20  # an aligned non-NULL address; never dereferenced on these paths

    def call(packed=fake, nb=nbytes, x=fake, xdt=1, m=197, bits=4, ln=1, g=None, b=None, eps=1e-6, res=None,
             y=fake, ydt=1, flags=0):
        return L.rpfq_act_quant_wide_linear(ctypes.byref(fc1), packed, nb, x, xdt, m, bits, ln, g, b,
                                            ctypes.c_float(eps), None, res, y, ydt, flags, None)
    assert call(packed=None) == 1 and call(x=None) == 1 and call(y=None) == 1
    assert call(xdt=9) == 5
    assert call(m=0) == 2
    assert call(bits=1) == 4 and call(bits=17) == 4
    assert call(flags=N.FLAG_NO_STREAM) == 6
    assert call(flags=N.FLAG_GELU, res=fake) == 6
    assert call(eps=-1.0) == 6
    assert call(nb=nbytes - 1) == 2
    assert call(x=fake + 8) == 3 and call(res=fake + 4) == 3
    assert call(m=50432) == 6  # not on the streaming split-K kernel
    assert b"rpfq_act_quant" in L.rpfq_last_error()
    assert call(xdt=0) == 6  # float32 x
