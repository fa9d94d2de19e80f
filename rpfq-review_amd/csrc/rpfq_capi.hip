// C ABI entry points (include/rpfq.h): argument validation on the host, then
// dispatch to the launchers.  Every check runs before the first HIP call so
// the error paths are testable without a GPU.
#include <stdarg.h>
#include <stdio.h>

#include "rpfq_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int ok() {
    g_err[0] = 0;
    return RPFQ_OK;
}

int hip_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(RPFQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool dtype_ok(int dt) { return dt == RPFQ_F32 || dt == RPFQ_F16 || dt == RPFQ_BF16; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int check_desc(const rpfq_wide_desc* d) {
    if (!d) return fail(RPFQ_ERR_NULL, "desc is NULL");
    if (d->n_complex <= 0 || d->k_complex <= 0)
        return fail(RPFQ_ERR_SHAPE, "n_complex=%lld k_complex=%lld must be positive",
                    (long long)d->n_complex, (long long)d->k_complex);
    if (d->n_complex > (1LL << 30) || d->k_complex > (1LL << 24))
        return fail(RPFQ_ERR_SHAPE, "n_complex=%lld k_complex=%lld exceed 2^30 / 2^24",
                    (long long)d->n_complex, (long long)d->k_complex);
    if (d->k_complex % 8 != 0)
        return fail(RPFQ_ERR_ALIGN, "k_complex=%lld must be a multiple of 8", (long long)d->k_complex);
    if (d->block < 0 || (d->block > 0 && d->block % 32 != 0))
        return fail(RPFQ_ERR_VALUE, "block=%lld must be 0 or a multiple of 32", (long long)d->block);
    if (d->codebook != RPFQ_CB_AXIS && d->codebook != RPFQ_CB_SIGN && d->codebook != RPFQ_CB_PSK16 &&
        d->codebook != RPFQ_CB_TABLE)
        return fail(RPFQ_ERR_BITS, "unknown codebook %d", d->codebook);
    if ((d->codebook == RPFQ_CB_PSK16 || d->codebook == RPFQ_CB_TABLE) && d->stages != 1)
        return fail(RPFQ_ERR_BITS, "PSK16 / TABLE layers have one stage, got %d", d->stages);
    if (d->codebook == RPFQ_CB_TABLE && (d->block != 0 || d->rotate != 0))
        return fail(RPFQ_ERR_VALUE, "TABLE layers take block = 0 and rotate = 0 (the table holds final values)");
    if (d->stages != 1 && d->stages != 2)
        return fail(RPFQ_ERR_BITS, "stages=%d unsupported (1 or 2)", d->stages);
    if (d->rotate != 0 && d->rotate != 1) return fail(RPFQ_ERR_VALUE, "rotate must be 0 or 1");
    return RPFQ_OK;
}

int check_ln(const void* x, int x_dtype, int64_t M, int64_t C, const float* gamma, const float* beta, float eps,
             void* y, int y_dtype) {
    if (!x || !y) return fail(RPFQ_ERR_NULL, "x/y must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0 || C <= 0) return fail(RPFQ_ERR_SHAPE, "M=%lld C=%lld must be positive", (long long)M, (long long)C);
    if (C % 8 != 0 || C > 4096) return fail(RPFQ_ERR_SHAPE, "C=%lld must be a multiple of 8 and <= 4096", (long long)C);
    if (M > 0x7fffffffLL) return fail(RPFQ_ERR_SHAPE, "M=%lld too large", (long long)M);
    if (!(eps >= 0.0f)) return fail(RPFQ_ERR_VALUE, "eps must be non-negative");
    if (!aligned(x, 16) || !aligned(y, 16) || !aligned(gamma, 16) || !aligned(beta, 16))
        return fail(RPFQ_ERR_ALIGN, "x, y, gamma and beta must be 16-byte aligned");
    return RPFQ_OK;
}

}  // namespace

extern "C" {

int rpfq_abi_version(void) { return RPFQ_ABI_VERSION; }

const char* rpfq_last_error(void) { return g_err; }

int rpfq_unpack(const uint8_t* codes, int bits, int64_t rows, int64_t k, const uint16_t* gamma_re,
                const uint16_t* gamma_im, int64_t block, float* re, float* im, void* stream) {
    if (!codes || !re || !im) return fail(RPFQ_ERR_NULL, "codes/re/im must not be NULL");
    if ((gamma_re == nullptr) != (gamma_im == nullptr))
        return fail(RPFQ_ERR_NULL, "gamma_re and gamma_im must both be set or both NULL");
    if (bits != 2 && bits != 4) return fail(RPFQ_ERR_BITS, "bits=%d unsupported (2 or 4)", bits);
    if (rows <= 0 || k <= 0) return fail(RPFQ_ERR_SHAPE, "rows=%lld k=%lld must be positive", (long long)rows, (long long)k);
    if (k % (8 / bits) != 0) return fail(RPFQ_ERR_ALIGN, "k=%lld must fill whole bytes", (long long)k);
    if (block < 0) return fail(RPFQ_ERR_VALUE, "block must be >= 0");
    int64_t nblk = block > 0 ? (k + block - 1) / block : 1;
    return hip_status(rpfq::launch_unpack(codes, bits, rows, k, gamma_re, gamma_im, nblk, block, re, im,
                                          reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_unpack");
}

int rpfq_phase_linear(const void* xr, const void* xi, int x_dtype, int conj_x, int64_t M, int64_t K,
                      const uint8_t* codes, const uint16_t* gamma_re, const uint16_t* gamma_im, int64_t block,
                      int64_t N, void* yr, void* yi, int y_dtype, void* stream) {
    if (!xr || !xi || !codes || !gamma_re || !gamma_im || !yr || !yi)
        return fail(RPFQ_ERR_NULL, "rpfq_phase_linear: NULL pointer argument");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0 || K <= 0 || N <= 0)
        return fail(RPFQ_ERR_SHAPE, "M=%lld K=%lld N=%lld must be positive", (long long)M, (long long)K, (long long)N);
    if (K % 32 != 0) return fail(RPFQ_ERR_ALIGN, "K=%lld must be a multiple of 32", (long long)K);
    if (block < 0 || (block > 0 && block % 32 != 0))
        return fail(RPFQ_ERR_VALUE, "block=%lld must be 0 or a multiple of 32", (long long)block);
    if (!aligned(xr, 16) || !aligned(xi, 16) || !aligned(codes, 8))
        return fail(RPFQ_ERR_ALIGN, "x planes must be 16-byte and codes 8-byte aligned");
    int64_t nblk = block > 0 ? (K + block - 1) / block : 1;
    int64_t block_ks = block > 0 ? block / 32 : K / 32;
    return hip_status(rpfq::launch_phase_linear(xr, xi, x_dtype, conj_x, M, K, codes, gamma_re, gamma_im, nblk,
                                                block_ks, N, yr, yi, y_dtype, reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_phase_linear");
}

size_t rpfq_wide_packed_bytes(const rpfq_wide_desc* desc) {
    if (check_desc(desc) != RPFQ_OK) return 0;
    return rpfq::wide_geom(*desc).total_bytes;
}

int rpfq_wide_pack(const rpfq_wide_desc* desc, const uint8_t* const* planes, int nplanes,
                   const float* const* scale_re, const float* const* scale_im, void* packed, size_t packed_bytes,
                   void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!planes || !scale_re || !packed) return fail(RPFQ_ERR_NULL, "planes/scale_re/packed must not be NULL");
    int want = (desc->codebook == RPFQ_CB_PSK16 || desc->codebook == RPFQ_CB_TABLE) ? 2 : 2 * desc->stages;
    if (nplanes != want) return fail(RPFQ_ERR_BITS, "expected %d planes, got %d", want, nplanes);
    if (desc->codebook != RPFQ_CB_PSK16 && !scale_im) return fail(RPFQ_ERR_NULL, "scale_im must not be NULL");
    for (int p = 0; p < nplanes; ++p) {
        if (!planes[p] || !scale_re[p] || (desc->codebook != RPFQ_CB_PSK16 && !scale_im[p]))
            return fail(RPFQ_ERR_NULL, "plane %d has a NULL pointer", p);
    }
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (!aligned(packed, 256)) return fail(RPFQ_ERR_ALIGN, "packed buffer must be 256-byte aligned");
    return hip_status(rpfq::launch_wide_pack(*desc, g, planes, nplanes, scale_re, scale_im, packed,
                                             reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_wide_pack");
}

// Flags: known bits, no contradictory pair, GELU only without a residual,
// a streaming launch (one workgroup per 16-row chunk and 32-row tile)
// within the grid, and a forced resident-weight launch on a layer, dtypes
// and y it takes (y NULL: a kernel-choice query).
static int check_flags(int flags, const rpfq::WideGeom& g, int64_t M, bool residual, int x_dtype, int y_dtype,
                       const void* y) {
    if (flags & ~(RPFQ_FLAG_TILE_M128 | RPFQ_FLAG_NO_STREAM | RPFQ_FLAG_STREAM | RPFQ_FLAG_GELU | RPFQ_FLAG_RESIDENT))
        return fail(RPFQ_ERR_VALUE, "flags=%d: unknown flag bits", flags);
    if (residual && (flags & RPFQ_FLAG_GELU))
        return fail(RPFQ_ERR_VALUE, "RPFQ_FLAG_GELU is not defined with a residual");
    if ((flags & RPFQ_FLAG_STREAM) && (flags & (RPFQ_FLAG_TILE_M128 | RPFQ_FLAG_NO_STREAM)))
        return fail(RPFQ_ERR_VALUE, "flags=%d: RPFQ_FLAG_STREAM excludes the tiled-kernel flags", flags);
    if ((flags & RPFQ_FLAG_RESIDENT) && (flags & (RPFQ_FLAG_TILE_M128 | RPFQ_FLAG_NO_STREAM | RPFQ_FLAG_STREAM)))
        return fail(RPFQ_ERR_VALUE, "flags=%d: RPFQ_FLAG_RESIDENT excludes the other kernel flags", flags);
    if (flags & RPFQ_FLAG_RESIDENT) {
        if ((x_dtype != RPFQ_F16 && x_dtype != RPFQ_BF16) || (y_dtype != RPFQ_F16 && y_dtype != RPFQ_BF16))
            return fail(RPFQ_ERR_DTYPE, "RPFQ_FLAG_RESIDENT takes fp16 / bf16 x and y (x=%d y=%d)", x_dtype, y_dtype);
        if (!rpfq::wide_resident_eligible(g, x_dtype, y_dtype))
            return fail(RPFQ_ERR_SHAPE,
                        "RPFQ_FLAG_RESIDENT: N'=%lld K'=%lld (takes K' = 48 with N' in {48, 96, 144, 192}, "
                        "K' = 96 with N' in {48, 96}, K' = 192 with N' = 48)",
                        (long long)g.N, (long long)g.K);
        if (y && !aligned(y, 16)) return fail(RPFQ_ERR_ALIGN, "RPFQ_FLAG_RESIDENT needs y 16-byte aligned");
        if (residual && g.N > 96)
            return fail(RPFQ_ERR_SHAPE, "RPFQ_FLAG_RESIDENT with a residual needs N' <= 96 (N'=%lld)", (long long)g.N);
    }
    if ((flags & RPFQ_FLAG_STREAM) && (int64_t)g.NT * ((M + 15) / 16) > ((int64_t)1 << 24))
        return fail(RPFQ_ERR_SHAPE, "M=%lld: RPFQ_FLAG_STREAM allows at most 2^24 (chunk, tile) workgroups",
                    (long long)M);
    return 0;
}

int rpfq_wide_linear(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, const void* x,
                     int x_dtype, int64_t M, const float* bias, void* y, int y_dtype, int flags, void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!packed || !x || !y) return fail(RPFQ_ERR_NULL, "packed/x/y must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0) return fail(RPFQ_ERR_SHAPE, "M=%lld must be positive", (long long)M);
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if ((rc = check_flags(flags, g, M, false, x_dtype, y_dtype, y))) return rc;
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (!aligned(packed, 256) || !aligned(x, 16))
        return fail(RPFQ_ERR_ALIGN, "packed must be 256-byte and x 16-byte aligned");
    if (M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld too large", (long long)M);
    return hip_status(rpfq::launch_wide_linear(*desc, g, packed, x, x_dtype, M, nullptr, bias, nullptr, y, y_dtype, flags,
                                               reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_wide_linear");
}

int rpfq_wide_linear_kernel(const rpfq_wide_desc* desc, int64_t M, int x_dtype, int y_dtype, int flags,
                            int* kernel) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!kernel) return fail(RPFQ_ERR_NULL, "kernel must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0) return fail(RPFQ_ERR_SHAPE, "M=%lld must be positive", (long long)M);
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if ((rc = check_flags(flags, g, M, false, x_dtype, y_dtype, nullptr))) return rc;
    if (M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld too large", (long long)M);
    *kernel = rpfq::wide_linear_kernel_choice(g, x_dtype, M, y_dtype, flags);
    return RPFQ_OK;
}

int rpfq_layer_norm_wide_linear_fusable(const rpfq_wide_desc* desc, int64_t M, int x_dtype, int y_dtype,
                                        int* fusable) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!fusable) return fail(RPFQ_ERR_NULL, "fusable must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0 || M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld out of range", (long long)M);
    *fusable = rpfq::layer_norm_wide_fusable(rpfq::wide_geom(*desc), x_dtype, M, y_dtype, desc->codebook) ? 1 : 0;
    return RPFQ_OK;
}

int rpfq_layer_norm_wide_linear(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes,
                                const void* x, int x_dtype, int64_t M, const float* gamma, const float* beta,
                                float eps, const float* bias, void* y, int y_dtype, int flags, void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!packed || !x || !y) return fail(RPFQ_ERR_NULL, "packed/x/y must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0 || M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld out of range", (long long)M);
    if (flags & ~RPFQ_FLAG_GELU) return fail(RPFQ_ERR_VALUE, "flags=%d: only RPFQ_FLAG_GELU is allowed", flags);
    if (!(eps >= 0.0f)) return fail(RPFQ_ERR_VALUE, "eps must be >= 0");
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (!aligned(packed, 256) || !aligned(x, 16) || !aligned(gamma, 16) || !aligned(beta, 16))
        return fail(RPFQ_ERR_ALIGN, "packed must be 256-byte, x, gamma and beta 16-byte aligned");
    if (!rpfq::layer_norm_wide_fusable(g, x_dtype, M, y_dtype, desc->codebook))
        return fail(RPFQ_ERR_VALUE,
                    "M=%lld K'=%lld: the fused LayerNorm needs a streaming split-K launch, per-row scales, "
                    "K' %% 32 == 0, K' <= %d, fp16 / bf16 x and a non-table codebook "
                    "(use rpfq_layer_norm + rpfq_wide_linear)",
                    (long long)M, (long long)desc->k_complex, rpfq::kLnMaxK);
    return hip_status(rpfq::launch_layer_norm_wide_linear(*desc, g, packed, x, x_dtype, M, gamma, beta, eps, bias, y,
                                                          y_dtype, flags, reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_layer_norm_wide_linear");
}

int rpfq_act_quant_wide_linear(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, const void* x,
                               int x_dtype, int64_t M, int bits, int layer_norm, const float* gamma, const float* beta,
                               float eps, const float* bias, const void* residual, void* y, int y_dtype, int flags,
                               void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!packed || !x || !y) return fail(RPFQ_ERR_NULL, "packed/x/y must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0 || M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld out of range", (long long)M);
    if (bits < 2 || bits > 16) return fail(RPFQ_ERR_BITS, "bits=%d unsupported (2..16)", bits);
    if (flags & ~RPFQ_FLAG_GELU) return fail(RPFQ_ERR_VALUE, "flags=%d: only RPFQ_FLAG_GELU is allowed", flags);
    if ((flags & RPFQ_FLAG_GELU) && residual)
        return fail(RPFQ_ERR_VALUE, "the GELU and the residual add cannot be fused together");
    if (layer_norm && !(eps >= 0.0f)) return fail(RPFQ_ERR_VALUE, "eps must be >= 0");
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (!aligned(packed, 256) || !aligned(x, 16) || !aligned(gamma, 16) || !aligned(beta, 16) || !aligned(residual, 16))
        return fail(RPFQ_ERR_ALIGN, "packed must be 256-byte, x, gamma, beta and residual 16-byte aligned");
    if (!rpfq::layer_norm_wide_fusable(g, x_dtype, M, y_dtype, desc->codebook))
        return fail(RPFQ_ERR_VALUE,
                    "M=%lld K'=%lld: the act-quant prologue needs a streaming split-K launch, per-row scales, "
                    "K' %% 32 == 0, K' <= %d, fp16 / bf16 x and a non-table codebook "
                    "(use rpfq_layer_norm_act_quant / rpfq_act_quant + rpfq_wide_linear)",
                    (long long)M, (long long)desc->k_complex, rpfq::kLnMaxK);
    return hip_status(rpfq::launch_act_quant_wide_linear(*desc, g, packed, x, x_dtype, M, bits, layer_norm ? 1 : 0,
                                                         gamma, beta, eps, bias, residual, y, y_dtype, flags,
                                                         reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_act_quant_wide_linear");
}

int rpfq_wide_linear_residual(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, const void* x,
                              int x_dtype, int64_t M, const float* bias, const void* residual, void* y,
                              int y_dtype, int flags, void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!packed || !x || !y || !residual) return fail(RPFQ_ERR_NULL, "packed/x/residual/y must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0) return fail(RPFQ_ERR_SHAPE, "M=%lld must be positive", (long long)M);
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if ((rc = check_flags(flags, g, M, true, x_dtype, y_dtype, y))) return rc;
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (!aligned(packed, 256) || !aligned(x, 16) || !aligned(residual, 16))
        return fail(RPFQ_ERR_ALIGN, "packed must be 256-byte, x and residual 16-byte aligned");
    if (M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld too large", (long long)M);
    return hip_status(rpfq::launch_wide_linear(*desc, g, packed, x, x_dtype, M, nullptr, bias, residual, y, y_dtype, flags,
                                               reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_wide_linear_residual");
}


namespace {
int mlp_checked(const rpfq_wide_desc* desc1, const void* packed1, size_t packed1_bytes,
                const rpfq_wide_desc* desc2, const void* packed2, size_t packed2_bytes, const void* x, int64_t M,
                const float* bias1, const float* bias2, const void* residual, void* y, void* stream,
                const float* gamma, const float* beta, float eps, const char* fn) {
    int rc = check_desc(desc1);
    if (rc) return rc;
    if ((rc = check_desc(desc2))) return rc;
    if (!packed1 || !packed2 || !x || !y) return fail(RPFQ_ERR_NULL, "packed1/packed2/x/y must not be NULL");
    if (M <= 0 || M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld out of range", (long long)M);
    const rpfq::WideGeom g1 = rpfq::wide_geom(*desc1), g2 = rpfq::wide_geom(*desc2);
    if (g2.K != g1.N || g2.N != g1.K)
        return fail(RPFQ_ERR_SHAPE, "fc2 (%lld -> %lld) does not invert fc1 (%lld -> %lld)", (long long)g2.K,
                    (long long)g2.N, (long long)g1.K, (long long)g1.N);
    if (!rpfq::wide_mlp_shape(g1, g2, desc1->codebook, desc2->codebook, M))
        return fail(RPFQ_ERR_SHAPE,
                    "%s takes K'=96, N1' a multiple of 96 up to 1536, block=0 on both layers, one "
                    "codebook and M >= 64 (K'=%lld N1'=%lld M=%lld)",
                    fn, (long long)g1.K, (long long)g1.N, (long long)M);
    if (packed1_bytes < g1.total_bytes || packed2_bytes < g2.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffers hold %zu / %zu bytes, need %zu / %zu", packed1_bytes,
                    packed2_bytes, g1.total_bytes, g2.total_bytes);
    if (!aligned(packed1, 256) || !aligned(packed2, 256) || !aligned(x, 16) || !aligned(y, 16) ||
        (residual && !aligned(residual, 16)))
        return fail(RPFQ_ERR_ALIGN, "packed must be 256-byte, x, y and residual 16-byte aligned");
    return hip_status(rpfq::launch_wide_mlp_layers(*desc1, g1, packed1, *desc2, g2, packed2, x, M, bias1, bias2,
                                                   residual, y, reinterpret_cast<hipStream_t>(stream), gamma, beta,
                                                   eps),
                      fn);
}
}  // namespace

int rpfq_wide_mlp(const rpfq_wide_desc* desc1, const void* packed1, size_t packed1_bytes,
                  const rpfq_wide_desc* desc2, const void* packed2, size_t packed2_bytes, const void* x,
                  int64_t M, const float* bias1, const float* bias2, const void* residual, void* y,
                  void* stream) {
    return mlp_checked(desc1, packed1, packed1_bytes, desc2, packed2, packed2_bytes, x, M, bias1, bias2, residual, y,
                       stream, nullptr, nullptr, -1.0f, "rpfq_wide_mlp");
}

int rpfq_layer_norm_wide_mlp(const rpfq_wide_desc* desc1, const void* packed1, size_t packed1_bytes,
                             const rpfq_wide_desc* desc2, const void* packed2, size_t packed2_bytes, const void* x,
                             int64_t M, const float* gamma, const float* beta, float eps, const float* bias1,
                             const float* bias2, void* y, void* stream) {
    if (!(eps >= 0.0f)) return fail(RPFQ_ERR_VALUE, "eps=%g must be >= 0", (double)eps);
    if ((gamma && !aligned(gamma, 16)) || (beta && !aligned(beta, 16)))
        return fail(RPFQ_ERR_ALIGN, "gamma and beta must be 16-byte aligned");
    return mlp_checked(desc1, packed1, packed1_bytes, desc2, packed2, packed2_bytes, x, M, bias1, bias2, x, y, stream,
                       gamma, beta, eps, "rpfq_layer_norm_wide_mlp");
}

int rpfq_wide_linear_scaled(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, const void* x,
                            int x_dtype, int64_t M, const float* row_scale, const float* bias, const void* residual,
                            void* y, int y_dtype, int flags, void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!packed || !x || !y) return fail(RPFQ_ERR_NULL, "packed/x/y must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0) return fail(RPFQ_ERR_SHAPE, "M=%lld must be positive", (long long)M);
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if ((rc = check_flags(flags, g, M, residual != nullptr, x_dtype, y_dtype, y))) return rc;
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (!aligned(packed, 256) || !aligned(x, 16) || (residual && !aligned(residual, 16)))
        return fail(RPFQ_ERR_ALIGN, "packed must be 256-byte, x and residual 16-byte aligned");
    if (row_scale && !aligned(row_scale, 16)) return fail(RPFQ_ERR_ALIGN, "row_scale must be 16-byte aligned");
    if (M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld too large", (long long)M);
    if (row_scale && x_dtype == RPFQ_F16) {
        const int k = rpfq::wide_linear_kernel_choice(g, x_dtype, M, y_dtype, flags);
        if (k != RPFQ_KERNEL_DMA)
            return fail(RPFQ_ERR_VALUE, "prescaled fp16 rows (fp16 x with row_scale) run on the DMA kernel only; "
                                        "this launch takes kernel %d", k);
    }
    return hip_status(rpfq::launch_wide_linear(*desc, g, packed, x, x_dtype, M, row_scale, bias, residual, y, y_dtype,
                                               flags, reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_wide_linear_scaled");
}

int rpfq_row_scales(const void* x, int x_dtype, int64_t M, int64_t C, float* scale, void* stream) {
    if (!x || !scale) return fail(RPFQ_ERR_NULL, "x/scale must not be NULL");
    if (!dtype_ok(x_dtype)) return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d", x_dtype);
    if (M <= 0 || C <= 0 || M > (int64_t)1 << 31 || C > (int64_t)1 << 30)
        return fail(RPFQ_ERR_SHAPE, "M=%lld, C=%lld out of range", (long long)M, (long long)C);
    if (!aligned(x, x_dtype == RPFQ_F32 ? 4 : 2) || !aligned(scale, 4))
        return fail(RPFQ_ERR_ALIGN, "x and scale must be aligned to their element size");
    return hip_status(rpfq::launch_row_scales(x, x_dtype, M, C, scale, reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_row_scales");
}

size_t rpfq_wide_adjoint_bytes(const rpfq_wide_desc* desc) {
    if (check_desc(desc) != RPFQ_OK) return 0;
    return rpfq::wide_adjoint_bytes(rpfq::wide_geom(*desc));
}

int rpfq_wide_pack_adjoint(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, void* adjoint,
                           size_t adjoint_bytes, void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!packed || !adjoint) return fail(RPFQ_ERR_NULL, "packed/adjoint must not be NULL");
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (adjoint_bytes < rpfq::wide_adjoint_bytes(g))
        return fail(RPFQ_ERR_SHAPE, "adjoint buffer holds %zu bytes, need %zu", adjoint_bytes,
                    rpfq::wide_adjoint_bytes(g));
    if (!aligned(packed, 256) || !aligned(adjoint, 256))
        return fail(RPFQ_ERR_ALIGN, "packed and adjoint must be 256-byte aligned");
    if (g.NT * g.KS > 0x7fffffffLL) return fail(RPFQ_ERR_SHAPE, "layer too large for the adjoint relayout");
    return hip_status(rpfq::launch_wide_pack_adjoint(*desc, g, packed, adjoint, reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_wide_pack_adjoint");
}

int rpfq_wide_linear_grad_x(const rpfq_wide_desc* desc, const void* adjoint, size_t adjoint_bytes, const void* grad_y,
                            int grad_y_dtype, int64_t M, void* grad_x, int grad_x_dtype, void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!adjoint || !grad_y || !grad_x) return fail(RPFQ_ERR_NULL, "adjoint/grad_y/grad_x must not be NULL");
    if (!dtype_ok(grad_y_dtype) || !dtype_ok(grad_x_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype grad_y=%d grad_x=%d", grad_y_dtype, grad_x_dtype);
    if (M <= 0 || M > (int64_t)1 << 30) return fail(RPFQ_ERR_SHAPE, "M=%lld out of range", (long long)M);
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if (adjoint_bytes < rpfq::wide_adjoint_bytes(g))
        return fail(RPFQ_ERR_SHAPE, "adjoint buffer holds %zu bytes, need %zu", adjoint_bytes,
                    rpfq::wide_adjoint_bytes(g));
    if (!aligned(adjoint, 256)) return fail(RPFQ_ERR_ALIGN, "adjoint must be 256-byte aligned");
    const size_t esize = grad_y_dtype == RPFQ_F32 ? 4 : 2;
    if (g.N % 8 == 0 && !aligned(grad_y, 16))
        return fail(RPFQ_ERR_ALIGN, "grad_y must be 16-byte aligned");
    if (!aligned(grad_y, esize) || !aligned(grad_x, grad_x_dtype == RPFQ_F32 ? 4 : 2))
        return fail(RPFQ_ERR_ALIGN, "grad_y / grad_x must be aligned to their element size");
    // the launcher takes 64-row tiles for float32 grad_y and M <= 64, 128 otherwise:
    // count the smaller tile so the grid size fits an int either way
    const int64_t tiles = ((M + 63) / 64) * ((g.KS + 3) / 4);
    if (tiles > 0x7fffffffLL) return fail(RPFQ_ERR_SHAPE, "M=%lld: too many tiles", (long long)M);
    return hip_status(rpfq::launch_wide_linear_grad_x(*desc, g, adjoint, grad_y, grad_y_dtype, M, grad_x, grad_x_dtype,
                                                      reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_wide_linear_grad_x");
}

int rpfq_layer_norm(const void* x, int x_dtype, int64_t M, int64_t C, const float* gamma, const float* beta,
                    float eps, void* y, int y_dtype, void* stream) {
    int rc = check_ln(x, x_dtype, M, C, gamma, beta, eps, y, y_dtype);
    if (rc) return rc;
    return hip_status(rpfq::launch_layer_norm(x, x_dtype, M, C, gamma, beta, eps, 0, y, y_dtype,
                                              reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_layer_norm");
}

int rpfq_layer_norm_prescaled(const void* x, int x_dtype, int64_t M, int64_t C, const float* gamma,
                              const float* beta, float eps, void* y, float* row_scale, void* stream) {
    int rc = check_ln(x, x_dtype, M, C, gamma, beta, eps, y, RPFQ_F16);
    if (rc) return rc;
    if (x_dtype != RPFQ_BF16 && x_dtype != RPFQ_F32)
        return fail(RPFQ_ERR_DTYPE, "x must be bf16 or float32 (x_dtype=%d)", x_dtype);
    if (!row_scale) return fail(RPFQ_ERR_NULL, "row_scale must not be NULL");
    if (!aligned(row_scale, 16)) return fail(RPFQ_ERR_ALIGN, "row_scale must be 16-byte aligned");
    return hip_status(rpfq::launch_layer_norm_prescaled(x, x_dtype, M, C, gamma, beta, eps, y, row_scale,
                                                        reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_layer_norm_prescaled");
}

int rpfq_row_prescale(const void* x, int x_dtype, int64_t M, int64_t C, void* y, float* row_scale, void* stream) {
    int rc = check_ln(x, x_dtype, M, C, nullptr, nullptr, 0.0f, y, RPFQ_F16);
    if (rc) return rc;
    if (x_dtype != RPFQ_BF16 && x_dtype != RPFQ_F32)
        return fail(RPFQ_ERR_DTYPE, "x must be bf16 or float32 (x_dtype=%d)", x_dtype);
    if (!row_scale) return fail(RPFQ_ERR_NULL, "row_scale must not be NULL");
    if (!aligned(row_scale, 16)) return fail(RPFQ_ERR_ALIGN, "row_scale must be 16-byte aligned");
    return hip_status(rpfq::launch_row_prescale(x, x_dtype, M, C, y, row_scale,
                                                reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_row_prescale");
}

int rpfq_layer_norm_act_quant(const void* x, int x_dtype, int64_t M, int64_t C, const float* gamma,
                              const float* beta, float eps, int bits, void* y, int y_dtype, void* stream) {
    int rc = check_ln(x, x_dtype, M, C, gamma, beta, eps, y, y_dtype);
    if (rc) return rc;
    if (C % 16 != 0) return fail(RPFQ_ERR_SHAPE, "C=%lld: each half must be a multiple of 8", (long long)C);
    if (bits < 2 || bits > 16) return fail(RPFQ_ERR_BITS, "bits=%d unsupported (2..16)", bits);
    return hip_status(rpfq::launch_layer_norm(x, x_dtype, M, C, gamma, beta, eps, bits, y, y_dtype,
                                              reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_layer_norm_act_quant");
}

int rpfq_gelu_act_quant(const void* x, int x_dtype, int64_t M, int64_t C, int bits, void* y, int y_dtype,
                        void* stream) {
    int rc = check_ln(x, x_dtype, M, C, nullptr, nullptr, 0.0f, y, y_dtype);
    if (rc) return rc;
    if (C % 16 != 0) return fail(RPFQ_ERR_SHAPE, "C=%lld: each half must be a multiple of 8", (long long)C);
    if (bits < 2 || bits > 16) return fail(RPFQ_ERR_BITS, "bits=%d unsupported (2..16)", bits);
    return hip_status(rpfq::launch_gelu_act_quant(x, x_dtype, M, C, bits, y, y_dtype,
                                                  reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_gelu_act_quant");
}

int rpfq_act_quant(const void* x, int x_dtype, int64_t M, int64_t in_features, int bits, void* y, int y_dtype,
                   void* stream) {
    if (!x || !y) return fail(RPFQ_ERR_NULL, "x/y must not be NULL");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype))
        return fail(RPFQ_ERR_DTYPE, "unsupported dtype x=%d y=%d", x_dtype, y_dtype);
    if (M <= 0 || in_features <= 0 || in_features % 2 != 0)
        return fail(RPFQ_ERR_SHAPE, "M=%lld in_features=%lld: need M > 0 and even in_features > 0",
                    (long long)M, (long long)in_features);
    if (bits < 2 || bits > 16) return fail(RPFQ_ERR_BITS, "bits=%d unsupported (2..16)", bits);
    if (M > 0x7fffffffLL) return fail(RPFQ_ERR_SHAPE, "M=%lld too large", (long long)M);
    return hip_status(rpfq::launch_act_quant(x, x_dtype, M, in_features / 2, bits, y, y_dtype,
                                             reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_act_quant");
}

int rpfq_wide_decode(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, float* a, int round_fp16,
                     void* stream) {
    int rc = check_desc(desc);
    if (rc) return rc;
    if (!packed || !a) return fail(RPFQ_ERR_NULL, "packed/a must not be NULL");
    rpfq::WideGeom g = rpfq::wide_geom(*desc);
    if (packed_bytes < g.total_bytes)
        return fail(RPFQ_ERR_SHAPE, "packed buffer holds %zu bytes, need %zu", packed_bytes, g.total_bytes);
    if (!aligned(packed, 256)) return fail(RPFQ_ERR_ALIGN, "packed buffer must be 256-byte aligned");
    return hip_status(rpfq::launch_wide_decode(*desc, g, packed, a, round_fp16 ? 1 : 0,
                                               reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_wide_decode");
}

size_t rpfq_quantize_workspace_bytes(const rpfq_quant_desc* desc) {
    (void)desc;
    return (size_t)rpfq::kQuantMaxBlocks * 8 * sizeof(double);
}

// Shape, method and pointer checks shared by rpfq_quantize_wide and its
// no-allocation variant (everything but the workspace).
static int check_quantize(const rpfq_quant_desc* desc, const float* weight, const float* a_q, const float* scales,
                          const uint8_t* codes) {
    if (!desc) return fail(RPFQ_ERR_NULL, "desc is NULL");
    if (desc->n_complex <= 0 || desc->k_complex <= 0)
        return fail(RPFQ_ERR_SHAPE, "n_complex=%lld k_complex=%lld must be positive",
                    (long long)desc->n_complex, (long long)desc->k_complex);
    if (desc->n_complex > (1LL << 30) || desc->k_complex > (1LL << 24) ||
        desc->n_complex * desc->k_complex > (1LL << 40))
        return fail(RPFQ_ERR_SHAPE, "n_complex=%lld k_complex=%lld too large",
                    (long long)desc->n_complex, (long long)desc->k_complex);
    for (int p = 0; p < 2; ++p) {
        if (desc->kind[p] != RPFQ_QK_AXIS && desc->kind[p] != RPFQ_QK_SIGN)
            return fail(RPFQ_ERR_VALUE, "unknown quantizer kind %d", desc->kind[p]);
        if (desc->steps[p] < 1 || desc->steps[p] > 4)
            return fail(RPFQ_ERR_VALUE, "steps=%d unsupported (1..4)", desc->steps[p]);
    }
    if (!weight || !scales) return fail(RPFQ_ERR_NULL, "weight/scales must not be NULL");
    if (codes && desc->k_complex % 4 != 0)
        return fail(RPFQ_ERR_ALIGN, "code planes need k_complex %% 4 == 0, got %lld", (long long)desc->k_complex);
    if (codes && (!aligned(weight, 16) || (a_q && !aligned(a_q, 16))))
        return fail(RPFQ_ERR_ALIGN, "code planes need 16-byte aligned weight and a_q");
    return RPFQ_OK;
}

int rpfq_quantize_wide(const rpfq_quant_desc* desc, const float* weight, const float* rot, float* a_q,
                       float* scales, uint8_t* codes, void* work, size_t work_bytes, void* stream) {
    int rc = check_quantize(desc, weight, a_q, scales, codes);
    if (rc) return rc;
    if (!work) return fail(RPFQ_ERR_NULL, "work must not be NULL");
    if (work_bytes < rpfq_quantize_workspace_bytes(desc))
        return fail(RPFQ_ERR_SHAPE, "workspace holds %zu bytes, need %zu", work_bytes,
                    rpfq_quantize_workspace_bytes(desc));
    if (!aligned(work, 8)) return fail(RPFQ_ERR_ALIGN, "workspace must be 8-byte aligned");
    return hip_status(rpfq::launch_quantize_wide(*desc, weight, rot, a_q, scales, codes, work,
                                                 reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_quantize_wide");
}

int rpfq_quantize_wide_noalloc(const rpfq_quant_desc* desc, const float* weight, const float* rot, float* a_q,
                               float* scales, uint8_t* codes, void* stream) {
    int rc = check_quantize(desc, weight, a_q, scales, codes);
    if (rc) return rc;
    const size_t need = rpfq_quantize_workspace_bytes(desc), have = rpfq::quant_scratch_bytes();
    if (need > have)
        return fail(RPFQ_ERR_SHAPE, "rpfq_quantize_wide_noalloc: needs %zu bytes of scratch, the static device "
                    "array holds %zu", need, have);
    void* work = nullptr;
    rc = hip_status(rpfq::quant_scratch_ptr(&work), "rpfq_quantize_wide_noalloc (scratch address)");
    if (rc) return rc;
    return hip_status(rpfq::launch_quantize_wide(*desc, weight, rot, a_q, scales, codes, work,
                                                 reinterpret_cast<hipStream_t>(stream)),
                      "rpfq_quantize_wide_noalloc");
}

}  // extern "C"
