// Kernel choice and launch of the widely-linear layer (rpfq_wide_linear):
// the shape, dtypes and flags pick the streaming, LDS-DMA or register-staged
// kernel; each lives in its own translation unit per codebook.
#include <mutex>

#include "rpfq_internal.h"

namespace rpfq {

int device_cus() {
    static std::atomic<int> cached[64];  // zero-initialised (static storage)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
    int n = dev < 64 ? cached[dev].load(std::memory_order_relaxed) : 0;
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        if (dev < 64) cached[dev].store(n, std::memory_order_relaxed);
    }
    return n & ~3;  // keep the grid a multiple of 8 (XCD-local tile order)
}

hipError_t set_lds_attr_once(const void* kernel, int bytes, std::atomic<uint64_t>& done) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 64;
    const uint64_t bit = dev < 64 ? (uint64_t)1 << dev : 0;
    if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
    return e;
}

// Shape fields of the launch arguments (what the kernel choice reads).
static WideArgs wide_shape(const WideGeom& g, int64_t M, int flags) {
    WideArgs a = {};
    a.M = M;
    a.K = (int)g.K;
    a.N = (int)g.N;
    a.NT = (int)g.NT;
    a.KS = (int)g.KS;
    a.nblk = (int)g.nblk;
    a.block_ks = (int)g.block_ks;
    a.act = (flags & RPFQ_FLAG_GELU) ? 1 : 0;  // an epilogue op, not a kernel choice
    return a;
}

// Kernel choice for a small M.  A tiled kernel gives each workgroup one
// 128-row x 128-column output tile through all of K, so while the launch is
// at most one tile deep it costs about one tile's latency, ~5 + KS us on
// MI355X whatever M and N'.  The streaming kernel spreads its (16-row chunk,
// 32-row tile) groups over every SIMD: with split K ~4.5 us + groups x
// (7.7 + 0.49 KS) ns; with per-(row, block) scales (one wave per group
// through all of K) ~(2 + 0.55 KS) us while the groups fit ~900 at once,
// proportionally longer past that.  The fits are from fp16 ViT-B/L and
// DeiT-Ti layer shapes at M = 24 .. 1576; streaming is taken where it is
// predicted 10% faster, and always for M <= 16.
static bool stream_pays(const WideArgs& a) {
    if (a.M <= 16) return true;
    const int64_t tiles = ((a.M + 127) / 128) * ((a.NT + 3) / 4);
    if (tiles > 2 * (int64_t)device_cus()) return false;  // more than one round of the tiled grid
    const double groups = (double)sk_groups(a);
    const double t_stream = a.nblk > 1 ? (2.0 + 0.55 * a.KS) * (groups > 900.0 ? groups / 900.0 : 1.0)
                                       : 4.5 + groups * (0.0077 + 0.00049 * a.KS);
    const double t_tiled = 5.0 + a.KS;
    return t_stream < 0.9 * t_tiled;
}

#ifndef RPFQ_DMA_MIN_M
#define RPFQ_DMA_MIN_M 128
#endif
#ifndef RPFQ_RES_MIN_M
#define RPFQ_RES_MIN_M 32768
#endif
// Layers the resident-weight kernel takes (shape and dtypes; y 16-byte
// aligned, a NULL y counting as aligned for kernel-choice queries; a
// residual only with N' <= 96).
static bool resident_ok(const WideArgs& a, int xdt, int ydt) {
    return (xdt == RPFQ_F16 || xdt == RPFQ_BF16) && (ydt == RPFQ_F16 || ydt == RPFQ_BF16) && resident_shape(a) &&
           reinterpret_cast<uintptr_t>(a.y) % 16 == 0 && (a.res == nullptr || a.N <= 96);
}

bool wide_resident_eligible(const WideGeom& g, int xdt, int ydt) {
    return resident_ok(wide_shape(g, 1, 0), xdt, ydt);
}

// The kernel a launch runs (RPFQ_KERNEL_*), from the shape, dtypes and the
// kernel-choice flags (the GELU bit already moved into a.act).  The
// resident-weight kernel runs for large M where the layer fits, unless a
// flag asks for another kernel.
static int choose_kernel(const WideArgs& a, int xdt, int ydt, int flags) {
    if (flags & RPFQ_FLAG_RESIDENT) return RPFQ_KERNEL_RESIDENT;  // eligibility checked by the C API
    if ((flags & RPFQ_FLAG_STREAM) || (!(flags & (RPFQ_FLAG_TILE_M128 | RPFQ_FLAG_NO_STREAM)) && stream_pays(a)))
        return gemv_pays(a) ? RPFQ_KERNEL_GEMV : RPFQ_KERNEL_STREAM;
    if (flags == 0 && a.M >= RPFQ_RES_MIN_M && resident_ok(a, xdt, ydt)) return RPFQ_KERNEL_RESIDENT;
    flags &= ~RPFQ_FLAG_NO_STREAM;
    // (bf16 x and y with the fused GELU take the register-staged kernel,
    // measured as fast as the DMA kernel's in-LDS conversion plus the GELU)
    if ((xdt == RPFQ_F16 || xdt == RPFQ_BF16) && flags == 0 && a.K % 32 == 0 && a.M >= RPFQ_DMA_MIN_M &&
        !(a.act && ydt == RPFQ_BF16 && xdt == RPFQ_BF16))
        return RPFQ_KERNEL_DMA;
    return RPFQ_KERNEL_TILED;
}

template <int CB>
static hipError_t wide_cb(WideArgs& a, int xdt, int ydt, int flags, hipStream_t s) {
    const int k = choose_kernel(a, xdt, ydt, flags);
    if (k == RPFQ_KERNEL_STREAM || k == RPFQ_KERNEL_GEMV) return launch_wide_stream<CB>(a, xdt, ydt, s);
    if (k == RPFQ_KERNEL_DMA) return launch_wide_dma<CB>(a, xdt, ydt, s);
    if (k == RPFQ_KERNEL_RESIDENT) return launch_wide_resident<CB>(a, xdt, ydt, s);
    flags &= ~RPFQ_FLAG_NO_STREAM;
    const int bm = (flags & RPFQ_FLAG_TILE_M128) ? 128 : a.M <= 32 ? 32 : a.M <= 64 ? 64 : 128;
    return launch_wide_tiled<CB>(a, bm, xdt, ydt, s);
}

// The fused LayerNorm runs in the streaming kernel split over 4 waves (for
// launches of fewer than kSkSplitTiles workgroups: a layer at batch 1-2), per-row scales,
// K' % 32 == 0 and K' <= kLnMaxK, fp16 / bf16 x, not the TABLE codebook, and
// only where the row kernel would also sum the statistics over 64 lanes per
// row (ln_row_lanes), so the prepared rows stay bit-identical to it.
bool layer_norm_wide_fusable(const WideGeom& g, int xdt, int64_t M, int ydt, int codebook) {
    const WideArgs a = wide_shape(g, M, 0);
    return choose_kernel(a, xdt, ydt, 0) == RPFQ_KERNEL_STREAM && sk_groups(a) < kSkSplitTiles && a.nblk == 1 &&
           a.K % 32 == 0 && a.K <= kLnMaxK && (xdt == RPFQ_F16 || xdt == RPFQ_BF16) && codebook != RPFQ_CB_TABLE &&
           ln_row_lanes(M, 2 * a.K) == 64;
}

int wide_linear_kernel_choice(const WideGeom& g, int xdt, int64_t M, int ydt, int flags) {
    return choose_kernel(wide_shape(g, M, flags), xdt, ydt, flags & ~RPFQ_FLAG_GELU);
}

static hipError_t launch_wide(WideArgs& a, const rpfq_wide_desc& d, int xdt, int ydt, int flags, hipStream_t s) {
    switch (d.codebook) {
        case RPFQ_CB_SIGN: return wide_cb<RPFQ_CB_SIGN>(a, xdt, ydt, flags, s);
        case RPFQ_CB_PSK16: return wide_cb<RPFQ_CB_PSK16>(a, xdt, ydt, flags, s);
        case RPFQ_CB_TABLE: return wide_cb<RPFQ_CB_TABLE>(a, xdt, ydt, flags, s);
        default: return wide_cb<RPFQ_CB_AXIS>(a, xdt, ydt, flags, s);
    }
}

static void wide_operands(WideArgs& a, const rpfq_wide_desc& d, const WideGeom& g, const void* packed, const void* x,
                          const float* bias, const void* res, void* y) {
    a.x = x;
    a.codes = reinterpret_cast<const uint4*>(packed);
    a.params = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(packed) + g.codes_bytes);
    a.rot = rot_of(d);
    a.bias = bias;
    a.res = res;
    a.y = y;
    a.vec_store = (g.N % 8 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0);  // also covers 4-wide stores
    // whole 128-column tiles and >= 8 k-steps (ViT-B/L, not DeiT-Ti's K' = 96 / N' = 96 layers):
    // full-line stores pay for the two workgroup barriers per half tile
    a.wg_epi = (g.N % 128 == 0) && (g.KS >= 8);
}

hipError_t launch_layer_norm_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                                         const void* x, int xdt, int64_t M, const float* gamma, const float* beta,
                                         float eps, const float* bias, void* y, int ydt, int flags, hipStream_t s) {
    WideArgs a = wide_shape(g, M, flags);
    wide_operands(a, d, g, packed, x, bias, nullptr, y);
    a.ln = 1;
    a.ln_eps = eps;
    a.ln_gamma = gamma;
    a.ln_beta = beta;
    switch (d.codebook) {
        case RPFQ_CB_SIGN: return launch_wide_stream<RPFQ_CB_SIGN>(a, xdt, ydt, s);
        case RPFQ_CB_PSK16: return launch_wide_stream<RPFQ_CB_PSK16>(a, xdt, ydt, s);
        default: return launch_wide_stream<RPFQ_CB_AXIS>(a, xdt, ydt, s);
    }
}

hipError_t launch_act_quant_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                                        const void* x, int xdt, int64_t M, int bits, int layer_norm,
                                        const float* gamma, const float* beta, float eps, const float* bias,
                                        const void* res, void* y, int ydt, int flags, hipStream_t s) {
    WideArgs a = wide_shape(g, M, flags);
    wide_operands(a, d, g, packed, x, bias, res, y);
    a.ln = layer_norm ? 1 : 0;
    a.ln_eps = eps;
    a.ln_gamma = gamma;
    a.ln_beta = beta;
    a.aq_bits = bits;
    switch (d.codebook) {
        case RPFQ_CB_SIGN: return launch_wide_stream<RPFQ_CB_SIGN>(a, xdt, ydt, s);
        case RPFQ_CB_PSK16: return launch_wide_stream<RPFQ_CB_PSK16>(a, xdt, ydt, s);
        default: return launch_wide_stream<RPFQ_CB_AXIS>(a, xdt, ydt, s);
    }
}

hipError_t launch_wide_linear_grad_x(const rpfq_wide_desc& d, const WideGeom& g, const void* adjoint,
                                     const void* gy, int gdt, int64_t M, void* gx, int xdt, hipStream_t s) {
    AdjArgs a = {};
    a.gy = gy;
    a.M = M;
    a.K = (int)g.K;
    a.N = (int)g.N;
    a.NT = (int)g.NT;
    a.KS = (int)g.KS;
    a.nblk = (int)g.nblk;
    a.block_ks = (int)g.block_ks;
    a.codes_t = reinterpret_cast<const uint4*>(adjoint);
    a.lut_t = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(adjoint) + wide_adjoint_codes_bytes(g));
    a.gx = gx;
    a.vec_store = (g.K % 8 == 0) && (reinterpret_cast<uintptr_t>(gx) % 16 == 0);
    (void)d;
    return launch_wide_grad_x(a, gdt, xdt, s);
}

bool wide_mlp_shape(const WideGeom& g1, const WideGeom& g2, int cb1, int cb2, int64_t M) {
    return g1.K == 96 && g1.N % 96 == 0 && g1.N <= 1536 && g2.K == g1.N && g2.N == g1.K && g1.nblk == 1 &&
           g2.nblk == 1 && cb1 == cb2 && M >= 64;
}

hipError_t launch_wide_mlp_layers(const rpfq_wide_desc& d1, const WideGeom& g1, const void* packed1,
                                  const rpfq_wide_desc& d2, const WideGeom& g2, const void* packed2, const void* x,
                                  int64_t M, const float* bias1, const float* bias2, const void* res, void* y,
                                  hipStream_t s, const float* ln_gamma, const float* ln_beta, float ln_eps) {
    if (!wide_mlp_shape(g1, g2, d1.codebook, d2.codebook, M)) return hipErrorInvalidValue;
    MlpArgs a = {};
    a.x = x;
    a.M = M;
    a.K = (int)g1.K;
    a.N1 = (int)g1.N;
    a.codes1 = reinterpret_cast<const uint4*>(packed1);
    a.params1 = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(packed1) + g1.codes_bytes);
    a.rot1 = rot_of(d1);
    a.bias1 = bias1;
    a.codes2 = reinterpret_cast<const uint4*>(packed2);
    a.params2 = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(packed2) + g2.codes_bytes);
    a.rot2 = rot_of(d2);
    a.bias2 = bias2;
    a.res = res;
    a.y = y;
    if (ln_eps >= 0.0f) {  // as rpfq_layer_norm would normalize these M rows
        a.ln = ln_row_lanes(M, 2 * g1.K);
        a.ln_eps = ln_eps;
        a.ln_gamma = ln_gamma;
        a.ln_beta = ln_beta;
    }
    switch (d1.codebook) {
        case RPFQ_CB_SIGN: return launch_wide_mlp<RPFQ_CB_SIGN>(a, s);
        case RPFQ_CB_PSK16: return launch_wide_mlp<RPFQ_CB_PSK16>(a, s);
        case RPFQ_CB_TABLE: return launch_wide_mlp<RPFQ_CB_TABLE>(a, s);
        default: return launch_wide_mlp<RPFQ_CB_AXIS>(a, s);
    }
}

hipError_t launch_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed, const void* x,
                              int xdt, int64_t M, const float* xs, const float* bias, const void* res, void* y,
                              int ydt, int flags, hipStream_t s) {
    WideArgs a = wide_shape(g, M, flags);
    flags &= ~RPFQ_FLAG_GELU;
    wide_operands(a, d, g, packed, x, bias, res, y);
    // fp16 x is the MFMA operand as it stands; with xs its rows arrive
    // prescaled, which only the DMA kernel undoes (the C API checks)
    a.xs = xdt != RPFQ_F16 || choose_kernel(a, xdt, ydt, flags) == RPFQ_KERNEL_DMA ? xs : nullptr;
    return launch_wide(a, d, xdt, ydt, flags, s);
}

}  // namespace rpfq
