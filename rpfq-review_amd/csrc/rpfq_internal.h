// Internal definitions shared by the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
hipError_t launch_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                              const void* x, int xdt, int64_t M, const float* bias, const void* res,
                              void* y, int ydt, int flags, hipStream_t s);
int wide_linear_kernel_choice(const WideGeom& g, int xdt, int64_t M, int ydt, int flags);  // RPFQ_KERNEL_*
hipError_t launch_layer_norm(const void* x, int xdt, int64_t M, int64_t C, const float* gamma,
                             const float* beta, float eps, int bits, void* y, int ydt, hipStream_t s);
hipError_t launch_act_quant(const void* x, int xdt, int64_t M, int64_t K, int bits, void* y, int ydt,
                            hipStream_t s);
// weight quantizer (rpfq_quant.hip): reduction blocks per stage, and so the
// workspace of rpfq_quantize_wide (kQuantMaxBlocks x 8 float64 partials)
constexpr int kQuantMaxBlocks = 1024;
hipError_t launch_quantize_wide(const rpfq_quant_desc& d, const float* weight, const float* rot, float* aq,
                                float* scales, uint8_t* codes, void* work, hipStream_t s);
hipError_t launch_wide_decode(const rpfq_wide_desc& d, const WideGeom& g, const void* packed,
                              float* a, int round_fp16, hipStream_t s);

}  // namespace rpfq
