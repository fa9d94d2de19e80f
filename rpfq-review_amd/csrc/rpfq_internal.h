// Internal definitions shared by the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/rpfq.h"

namespace rpfq {

// ---------------------------------------------------------------------------
// Native tiled layout of a packed widely-linear layer (device blob).
//
//  codes : [NT][KS][32 rows][32 bytes]   NT = ceil(N'/32), KS = ceil(K'/32)
//          byte b of (row n, k-step ks) holds complex column
//          k' = 32 ks + 8 s + 4 g + e  with  g = b / 16, s = (b / 4) & 3,
//          e = b & 3, so MFMA lane group g streams its 16 bytes with one
//          128-bit load per k-step (and each 4-byte word holds 4
//          consecutive columns).  Each byte is one complex element:
//          low nibble = U index, high nibble = W index.  AXIS/SIGN:
//          index = c_s0 | c_s1 << 2; PSK16: index = 4-bit phase code.
//          Padding (n >= N' or k' >= K') is 0.
//  params: [NT*32 rows][nblk][8] float32 at an offset rounded up to 256 B:
//          AXIS/SIGN: u_s0 (re,im), u_s1 (re,im), w_s0 (re,im), w_s1 (re,im)
//          multipliers; PSK16: [s_u, 0, 0, 0, s_w, 0, 0, 0].  Padded rows 0.
//          TABLE: [NT*32 rows][32] (re, im) float32 pairs, entries 0..15 the
//          U values of indices 0..15, 16..31 the W values (nblk = 1).
// ---------------------------------------------------------------------------
struct WideGeom {
    int64_t N, K;        // complex dims
    int64_t NT, KS;      // 32-row tiles, 32-column k-steps
    int64_t nblk;        // scale blocks per row
    int64_t block_ks;    // k-steps per scale block
    size_t codes_bytes;  // offset of params
    size_t total_bytes;
};

inline WideGeom wide_geom(const rpfq_wide_desc& d) {
    WideGeom g;
    g.N = d.n_complex;
    g.K = d.k_complex;
    g.NT = (g.N + 31) / 32;
    g.KS = (g.K + 31) / 32;
    if (d.block == 0) {
        g.nblk = 1;
        g.block_ks = g.KS;
    } else {
        g.nblk = (g.K + d.block - 1) / d.block;
        g.block_ks = d.block / 32;
    }
    size_t codes = (size_t)g.NT * g.KS * 1024;
    g.codes_bytes = (codes + 255) & ~(size_t)255;
    const size_t row_floats = d.codebook == RPFQ_CB_TABLE ? 64 : (size_t)g.nblk * 8;
    g.total_bytes = g.codes_bytes + (size_t)g.NT * 32 * row_floats * sizeof(float);
    return g;
}

struct RotParams {
    int rotate;
    float cu, su, cw, sw;
};

inline RotParams rot_of(const rpfq_wide_desc& d) {
    RotParams r;
    r.rotate = d.rotate;
    r.cu = d.rot_u[0];
    r.su = d.rot_u[1];
    r.cw = d.rot_w[0];
    r.sw = d.rot_w[1];
    return r;
}

// Launch arguments of the widely-linear GEMM kernels.
struct WideArgs {
    const void* x;
    int64_t M;
    int K, N, NT, KS, nblk, block_ks;
    const uint4* codes;
    const float4* params;
    RotParams rot;
    const float* bias;
    const void* res;  // residual of y's dtype added to the output (NULL: none)
    void* y;
    int tiles_m, tiles_n;
    int vec_store;  // y rows allow 16-byte stores (N % 8 == 0, aligned y)
    int wg_epi;     // DMA epilogue: workgroup-wide full-line stores (else per wave)
    int act;        // 1: exact GELU of the rounded output (no residual), 0: none
    // LayerNorm of x fused into the streaming kernel's prologue (ln = 1):
    // the layer contracts LN(x) = (x - mean) / sqrt(var + eps) * gamma + beta
    // over the 2K' features of each row, rounded to x's dtype.
    int ln;
    float ln_eps;
    const float* ln_gamma;  // [2K'] or NULL (ones)
    const float* ln_beta;   // [2K'] or NULL (zeros)
    // Activation fake quantization of x (after the LayerNorm when ln = 1) in
    // the same prologue: bits 2 .. 16, 0 = none (rpfq_act_quant's arithmetic
    // per row and half, rounded to x's dtype).
    int aq_bits;
    // Per-row prescale of float32 / bf16 x ([M] powers of two, row_prescale
    // of the row's largest magnitude; NULL: none; unused for fp16 x): row m
    // is multiplied by xs[m] before its fp16 rounding and its outputs by
    // 1 / xs[m] before the bias.
    const float* xs;
};

// ---------------------------------------------------------------------------
// Adjoint blob (rpfq_wide_pack_adjoint), the packed layer arranged for
// contractions over N' (grad_x):
//  codesT: [KS][NT][32 columns][32 bytes]: byte b of (complex column k,
//          row step t) holds the code byte of row n' = 32 t + 8 s + 4 g + e
//          (g = b / 16, s = (b / 4) & 3, e = b & 3) and column k, so MFMA
//          lane group g of the lane owning column k streams its 16 rows of
//          a row step with one 128-bit load.
//  lutT:   at wide_adjoint_codes_bytes: [NT*32 rows][nblk][32] fp16 (re, im)
//          pairs, entries 0..15 U(index), 16..31 W(index) of the row (and
//          scale block), de-rotated and rounded to fp16 -- the tables the
//          forward kernels build in LDS.  Padded rows 0.
// ---------------------------------------------------------------------------
inline size_t wide_adjoint_codes_bytes(const WideGeom& g) { return (size_t)g.NT * g.KS * 1024; }
inline size_t wide_adjoint_bytes(const WideGeom& g) {
    return wide_adjoint_codes_bytes(g) + (size_t)g.NT * 32 * g.nblk * 128;
}

// Launch arguments of the grad_x kernel: gx [M, 2K'] = gy [M, 2N'] A.
struct AdjArgs {
    const void* gy;
    int64_t M;
    int K, N, NT, KS, nblk, block_ks;
    const uint4* codes_t;  // adjoint code tiles
    const uint4* lut_t;    // adjoint U / W tables, 8 uint4 per (row, block)
    RotParams rot;
    void* gx;
    int tiles_m, tiles_k;
    int vec_store;  // gx rows allow 16-byte stores (K' % 8 == 0, aligned gx)
};

// Compute units of the current device (cached per device, thread-safe;
// 256 on MI355X), rounded down to a multiple of 4 so a persistent grid of
// 2 workgroups per CU stays a multiple of 8 (XCD-local tile order).
int device_cus();

// hipFuncSetAttribute(kernel, MaxDynamicSharedMemorySize, bytes) once per
// device: `done` holds one bit per device index (< 64; devices past that
// set the attribute on every call).  Concurrent first calls may both set
// it, which is harmless (the call is idempotent).
hipError_t set_lds_attr_once(const void* kernel, int bytes, std::atomic<uint64_t>& done);

// Widely-linear GEMM launchers, one translation unit per codebook (CB):
// wide_dma.hip (fp16 / bf16 x, LDS DMA, M >= 128), wide_stream.hip (weight
// streaming, row-chunked and column-split), wide_tiled.hip (register-staged tiles, bm = 32, 64 or 128).
template <int CB> hipError_t launch_wide_dma(WideArgs& a, int xdt, int ydt, hipStream_t s);
template <int CB> hipError_t launch_wide_stream(WideArgs& a, int xdt, int ydt, hipStream_t s);
template <int CB> hipError_t launch_wide_tiled(WideArgs& a, int bm, int xdt, int ydt, hipStream_t s);
template <int CB> hipError_t launch_wide_resident(WideArgs& a, int xdt, int ydt, hipStream_t s);

// Fused MLP (wide_mlp.hip): y = residual + fc2(GELU(fc1(x))) for fp16 x / y,
// fc1 K' -> N1', fc2 N1' -> K', one 64-row tile of x per workgroup of
// K' / 32 waves, the hidden activations in LDS.
struct MlpArgs {
    const void* x;  // [M, 2 K'] fp16
    int64_t M;
    int K, N1;  // fc1: K' inputs, N1' outputs; fc2: N1' inputs, K' outputs
    const uint4* codes1;
    const float4* params1;
    RotParams rot1;
    const float* bias1;  // [2 N1'] or NULL
    const uint4* codes2;
    const float4* params2;
    RotParams rot2;
    const float* bias2;  // [2 K'] or NULL
    const void* res;     // [M, 2 K'] fp16 or NULL (may be y)
    void* y;             // [M, 2 K'] fp16
    int tiles;           // row tiles (set by the launcher)
    // LayerNorm of x's rows before fc1 (ln = the row kernel's lanes per row
    // for this M, ln_row_lanes: 8 or 64; 0 = none), in that kernel's order
    int ln;
    float ln_eps;
    const float* ln_gamma;  // [2 K'] or NULL (ones)
    const float* ln_beta;   // [2 K'] or NULL (zeros)
};
template <int CB> hipError_t launch_wide_mlp(const MlpArgs& a, hipStream_t s);
// The fused MLP's shapes: K' = 96 (three waves), N1' a multiple of 96 up
// to 1536, per-row scales on both layers, one codebook, M >= 64.
bool wide_mlp_shape(const WideGeom& g1, const WideGeom& g2, int cb1, int cb2, int64_t M);
hipError_t launch_wide_mlp_layers(const rpfq_wide_desc& d1, const WideGeom& g1, const void* packed1,
                                  const rpfq_wide_desc& d2, const WideGeom& g2, const void* packed2, const void* x,
                                  int64_t M, const float* bias1, const float* bias2, const void* res, void* y,
                                  hipStream_t s, const float* ln_gamma = nullptr, const float* ln_beta = nullptr,
                                  float ln_eps = -1.0f);

// Resident-weight kernel (wide_resident.hip): one workgroup of kResWaves
// waves per CU holds the whole decoded layer in LDS (2N' x 2K' fp16 as MFMA
// A operands, plus the float32 bias) and streams 16-row subtiles of x, each
// wave holding whole output rows.  Shapes: K' = 48 with N' in {48, 96, 144,
// 192}, K' = 96 with N' in {48, 96}, K' = 192 with N' = 48 (Swin-T stage 0
// and its stage-1 proj); fp16 / bf16 x and y.
constexpr int kResWaves = 8;
constexpr int kResLdsMax = 160 * 1024;
// LDS of the decoded layer (kc = 2K' / 32 k-chunks, nb = 2N' / 16 blocks)
// and the bias
constexpr int res_lds_layer(int kc, int nb) { return nb * kc * 1024 + 64 * nb; }
// Rows of output each wave stages in LDS before its full-line stores: 16
// (a whole subtile), 8 (half of it) or 0 (no room left beside the layer:
// direct 16-B stores).  An output row is 4N' = 32 nb bytes, staged at a
// pitch 16 B longer (res_stage_pitch) so the 16 rows of one staging write
// fall on distinct banks.
constexpr int res_stage_pitch(int nb) { return 32 * nb + 16; }
constexpr int res_stage_rows(int kc, int nb) {
    return res_lds_layer(kc, nb) + kResWaves * 16 * res_stage_pitch(nb) <= kResLdsMax               ? 16
           : res_lds_layer(kc, nb) + kResWaves * (8 * res_stage_pitch(nb) + 512) <= kResLdsMax ? 8
                                                                                                  : 0;
}
// (staging 8 rows at a time, the lanes of the other 8 rows write a 512-B
// scratch area per wave instead)
constexpr int res_lds(int kc, int nb) {
    return res_lds_layer(kc, nb) + kResWaves * res_stage_rows(kc, nb) * res_stage_pitch(nb) +
           (res_stage_rows(kc, nb) == 8 ? kResWaves * 512 : 0);
}
inline int resident_lds(const WideArgs& a) { return res_lds(a.K / 16, a.N / 8); }
// shape and dtypes of a layer the kernel takes (wide_dispatch.hip)
bool wide_resident_eligible(const WideGeom& g, int xdt, int ydt);
inline bool resident_shape(const WideArgs& a) {
    if (a.K == 48) return a.N == 48 || a.N == 96 || a.N == 144 || a.N == 192;
    if (a.K == 96) return a.N == 48 || a.N == 96;
    return a.K == 192 && a.N == 48;
}

// workgroups of the streaming kernel: one per (16-row chunk, 32-row tile)
inline int64_t sk_groups(const WideArgs& a) { return a.NT * ((a.M + 15) / 16); }

// Streaming launches (M <= 8) that take the column-split kernel: for many
// tiles (>= 4096, one workgroup per 64 rows) when K' spans >= 12 k-steps,
// and for few tiles (split K) when it spans fewer than 20.  Measured per
// launch at M = 1 / 8 on MI355X: N' stacked to 1 GiB of codes, K' = 1536:
// 317 / 396 us vs 355 / 460 us (fused kernel); K' = 2048: 303 / 386 vs
// 360 / 456; K' = 512: 363 / 456 vs 388 / 510; K' = 384: 460 / 570 vs
// 446 / 554.  Single ViT layers: K' = 384, N' = 1536: 4.98 / 5.81 vs
// 5.46 / 5.86 us; K' = 1536, N' = 384: 9.21 / 10.39 vs 8.88 / 9.26 us.
// (A persistent single-wave form that streams codes across row groups
// measured 10-40% slower than both.)  Below 16 k-steps the many-tile form
// runs one wave per 64 rows instead of two (each wave then walks all of
// K'): K' = 384 at M = 1 / 4, 1 GiB stacked, 431 / 409 us against 455 / 510
// (two waves) and 440 / 473 (fused kernel); K' = 512 352 / 386 against
// 343 / 385; K' = 1536 325 / 348 against 299 / 342, so longer K' keeps two.
// Streaming workgroups: split K over 4 waves below kSkNw2Groups, over 2 up
// to kSkSplitTiles, one wave per tile (the column-split kernel: 1 or 2
// waves per 64 rows, above) from there.
constexpr int64_t kSkNw2Groups = 400, kSkSplitTiles = 4096;
constexpr int kGemvMaxM = 8;
inline bool gemv_pays(const WideArgs& a) {
    if (a.M > kGemvMaxM || a.nblk > 1) return false;
    return a.NT >= kSkSplitTiles ? a.KS >= 12 : a.KS < 20;
}
inline bool gemv_single_wave(const WideArgs& a) { return a.NT >= kSkSplitTiles && a.KS < 16; }

// launchers (rpfq_kernels.hip); return hipError_t
hipError_t launch_unpack(const uint8_t* codes, int bits, int64_t rows, int64_t k,
                         const uint16_t* gre, const uint16_t* gim, int64_t nblk, int64_t block,
                         float* re, float* im, hipStream_t s);
hipError_t launch_phase_linear(const void* xr, const void* xi, int xdt, int conj_x, int64_t M,
                               int64_t K, const uint8_t* codes, const uint16_t* gre,
                               const uint16_t* gim, int64_t nblk, int64_t block_ks, int64_t N,
                               void* yr, void* yi, int ydt, hipStream_t s);
hipError_t launch_wide_pack(const rpfq_wide_desc& d, const WideGeom& g, const uint8_t* const* planes,
                            int nplanes, const float* const* sre, const float* const* sim,
                            void* packed, hipStream_t s);
// dispatch (wide_dispatch.hip)
hipError_t launch_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                              const void* x, int xdt, int64_t M, const float* xs, const float* bias,
                              const void* res, void* y, int ydt, int flags, hipStream_t s);
// per-row prescales of x [M, C] (rpfq_row_scales; rpfq_kernels.hip)
hipError_t launch_row_scales(const void* x, int xdt, int64_t M, int64_t C, float* scale, hipStream_t s);
int wide_linear_kernel_choice(const WideGeom& g, int xdt, int64_t M, int ydt, int flags);  // RPFQ_KERNEL_*
// LayerNorm fused into the streaming kernel: whether the launch qualifies, and the launch.
// K' <= 384: the normalized 16-row tile (<= 25 KB) stays in LDS.  ViT-B,
// DeiT-Ti and Swin-T layers at batch 1 gain (0.775 -> 0.712, 0.598 -> 0.502,
// 1.024 -> 0.985 ms per forward); ViT-L's K' = 512 lost (1.75 -> 1.96 ms).
constexpr int kLnMaxK = 384;
// Lanes per row of the LayerNorm row kernel (layer_norm_kernel, modes 1-4)
// for M rows of C features: the smallest of 8, 16, 32, 64 that keeps every
// lane at <= 4 chunks of 8 (C <= 2048), and 64 whenever that choice would
// launch fewer than 256 workgroups (M * lanes < 65,536) or C > 1024.  The
// fused row prologue of the streaming kernel sums the LayerNorm statistics
// in the 64-lane order, so it is bit-identical to the row kernel only where
// this returns 64.
inline int ln_row_lanes(int64_t M, int64_t C) {
    const int64_t nch = C / 8;
    const int tpr = nch <= 32 ? 8 : nch <= 64 ? 16 : nch <= 128 ? 32 : 64;
    return (nch <= 256 && tpr < 64 && M * tpr < 256 * 256) ? 64 : tpr;
}
bool layer_norm_wide_fusable(const WideGeom& g, int xdt, int64_t M, int ydt, int codebook);
hipError_t launch_layer_norm_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                                         const void* x, int xdt, int64_t M, const float* gamma, const float* beta,
                                         float eps, const float* bias, void* y, int ydt, int flags, hipStream_t s);
// The same row prologue with the act quant (layer_norm = 0: act quant of x
// alone) and an optional residual added in the store.
hipError_t launch_act_quant_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                                        const void* x, int xdt, int64_t M, int bits, int layer_norm,
                                        const float* gamma, const float* beta, float eps, const float* bias,
                                        const void* res, void* y, int ydt, int flags, hipStream_t s);
hipError_t launch_layer_norm(const void* x, int xdt, int64_t M, int64_t C, const float* gamma,
                             const float* beta, float eps, int bits, void* y, int ydt, hipStream_t s);
hipError_t launch_gelu_act_quant(const void* x, int xdt, int64_t M, int64_t C, int bits, void* y, int ydt,
                                 hipStream_t s);
hipError_t launch_layer_norm_prescaled(const void* x, int xdt, int64_t M, int64_t C, const float* gamma,
                                       const float* beta, float eps, void* y, float* scale, hipStream_t s);
hipError_t launch_row_prescale(const void* x, int xdt, int64_t M, int64_t C, void* y, float* scale, hipStream_t s);
hipError_t launch_act_quant(const void* x, int xdt, int64_t M, int64_t K, int bits, void* y, int ydt,
                            hipStream_t s);
// weight quantizer (rpfq_quant.hip): reduction blocks per stage, and so the
// workspace of rpfq_quantize_wide (kQuantMaxBlocks x 8 float64 partials)
constexpr int kQuantMaxBlocks = 1024;
hipError_t launch_quantize_wide(const rpfq_quant_desc& d, const float* weight, const float* rot, float* aq,
                                float* scales, uint8_t* codes, void* work, hipStream_t s);
// the static device scratch of rpfq_quantize_wide_noalloc: its size, and its
// device address on the current device (resolved once per device)
size_t quant_scratch_bytes();
hipError_t quant_scratch_ptr(void** out);
hipError_t launch_wide_decode(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                              float* a, int round_fp16, hipStream_t s);
// adjoint blob (rpfq_kernels.hip) and the grad_x kernel (wide_adjoint.hip)
hipError_t launch_wide_pack_adjoint(const rpfq_wide_desc& d, const WideGeom& g, const void* packed, void* adjoint,
                                    hipStream_t s);
hipError_t launch_wide_grad_x(AdjArgs& a, int gdt, int xdt, hipStream_t s);
hipError_t launch_wide_linear_grad_x(const rpfq_wide_desc& d, const WideGeom& g, const void* adjoint,
                                     const void* gy, int gdt, int64_t M, void* gx, int xdt, hipStream_t s);

}  // namespace rpfq
