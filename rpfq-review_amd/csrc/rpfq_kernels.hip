// HIP kernels for gfx950 (MI355X) besides the widely-linear GEMMs:
//
//   unpack_kernel        bit-exact decode of one packed plane
//   phase_linear_kernel  single plane, ternary MFMA operands, scales in epilogue
//   wide_pack_*_kernel   reference planes -> native tiled blob
//   wide_decode_kernel   fused float32 weight, same decode as the GEMM
//   act_quant_kernel     per-row activation fake quantization
//   layer_norm_kernel    LayerNorm / act quant / both, rows in registers
//
// The widely-linear GEMM kernels are in wide_dma.hip, wide_stream.hip and
// wide_tiled.hip, their dispatch in wide_dispatch.hip.
#include <cstdlib>
#include <mutex>

#include "rpfq_device.h"

namespace rpfq {

// ---------------------------------------------------------------------------
// unpack / dequantize one plane (export_rpfq_vit_to_mlx.py:227-254)
// ---------------------------------------------------------------------------
__global__ void unpack_kernel(const uint8_t* __restrict__ codes, int bits, int64_t rows, int64_t k,
                              const uint16_t* __restrict__ gre, const uint16_t* __restrict__ gim,
                              int64_t nblk, int64_t block, float* __restrict__ re,
                              float* __restrict__ im) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * k) return;
    int64_t row = i / k, col = i - row * k;
    float vr, vi;
    if (bits == 2) {
        uint32_t byte = codes[row * (k >> 2) + (col >> 2)];
        uint32_t c = (byte >> (2 * (col & 3))) & 3u;
        float2 v = axis_val(c, 1.0f, 1.0f);
        vr = v.x;
        vi = v.y;
    } else {
        uint32_t byte = codes[row * (k >> 1) + (col >> 1)];
        uint32_t c = (byte >> (4 * (col & 1))) & 15u;
        vr = kPskCos[c];
        vi = kPskSin[c];
    }
    if (gre != nullptr) {
        int64_t b = block > 0 ? col / block : 0;
        float g_re = (float)__builtin_bit_cast(_Float16, gre[row * nblk + b]);
        float g_im = (float)__builtin_bit_cast(_Float16, gim[row * nblk + b]);
        vr = vr / g_re;
        vi = vi / g_im;
    }
    re[i] = vr;
    im[i] = vi;
}

// ---------------------------------------------------------------------------
// single-plane phase linear (phase_linear.cpp:119-164 semantics)
// ---------------------------------------------------------------------------
struct PhaseArgs {
    const void* xr;
    const void* xi;
    int64_t M, K, N;
    const uint8_t* codes;   // [N, K/4]
    const uint16_t* gre;    // [N, nblk] fp16 bits
    const uint16_t* gim;
    int64_t nblk, block_ks;
    float xsign;            // +1: W conj(x), -1: W x
    void* yr;
    void* yi;
    int tiles_m, tiles_n;
};

// Ternary operand table: nibble (c0 | c1 << 2) -> fp16 pairs (tr0, tr1), (ti0, ti1)
// with tr = Re(code), ti = Im(code) in {-1, 0, +1}.
__device__ __forceinline__ uint2 tern_entry(uint32_t nib) {
    const uint16_t h[4][2] = {{0xBC00u, 0x0000u}, {0x3C00u, 0x0000u}, {0x0000u, 0xBC00u}, {0x0000u, 0x3C00u}};
    uint32_t c0 = nib & 3u, c1 = nib >> 2;
    uint2 e;
    e.x = (uint32_t)h[c0][0] | ((uint32_t)h[c1][0] << 16);
    e.y = (uint32_t)h[c0][1] | ((uint32_t)h[c1][1] << 16);
    return e;
}

// Workgroup = 4 waves, tile = BM rows of x times 128 output columns; wave w
// owns columns 32w..32w+31 for all BM rows.  BM = 32 (the launcher's
// choice): four workgroups per CU with per-row scales, so config 1's 1,200
// tiles fill more of the 1,024 slots per round than 600 tiles of 64 rows on
// 512 (measured 8% faster).  Per k-step of 32 columns the
// x tile goes global -> registers -> (fp16, or fp16 hi + lo for float32 x)
// -> LDS; the raw loads of k-step ks + 2 are issued before the MFMAs of ks
// and converted only when k-step ks + 1 is written to LDS, so every load has
// two k-steps of MFMAs to land (two register sets, two LDS stages).  Loads
// are unconditional (rows past M read row M - 1, k-steps past the end read
// the last one) so the loop body is straight-line and the wait counts exact;
// rows and columns past the edges are never stored.
template <int BM, int XDT, int YDT, bool PERBLOCK>
__global__ void __launch_bounds__(256, PERBLOCK ? 2 : 4) phase_linear_kernel(PhaseArgs a) {
    constexpr bool SPLIT = (XDT == RPFQ_F32);
    constexpr int MB = BM / 32;
    constexpr int XROW = SPLIT ? 272 : 144;  // bytes per LDS row (+16 pad)
    constexpr int XSTAGE = BM * XROW;
    constexpr int CPT = BM / 32;             // 16-byte chunks per thread per plane pair
    constexpr int RAW = SPLIT ? 8 : 4;       // dwords of one raw chunk (8 floats or 8 halves)
    __shared__ __align__(16) char smem[2 * XSTAGE];
    __shared__ uint2 codes_lds[2][128];  // per stage: the k-step's 8 code bytes of each output column
    __shared__ uint2 tern[16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, g = lane >> 5;
    const int tile = xcd_tile(blockIdx.x, a.tiles_m * a.tiles_n);
    const int mt = tile / a.tiles_n, ntl = tile - mt * a.tiles_n;
    const int64_t m0 = (int64_t)mt * BM;
    const int64_t n = (int64_t)ntl * 128 + wave * 32 + r;
    const bool n_ok = n < a.N;
    const int64_t n_ld = n_ok ? n : a.N - 1;
    const int KS = (int)(a.K / 32);
    const int64_t kb = a.K / 4;

    if (tid < 16) tern[tid] = tern_entry(tid);

    // chunk j of this thread: row, plane and 8-column group of a k-step
    constexpr int ESZ = SPLIT ? 4 : 2;  // bytes per element of x
    const char* src[CPT];
    int soff[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tid + 256 * j;
        const int row = c >> 3, part = (c >> 2) & 1, sub = c & 3;
        const int64_t m = m0 + row < a.M ? m0 + row : a.M - 1;
        src[j] = reinterpret_cast<const char*>(part ? a.xi : a.xr) + (m * a.K + sub * 8) * ESZ;
        soff[j] = row * XROW + part * 64 + sub * 16;
    }

    // one k-step in flight: the raw x chunks and the column's 8 code bytes
    struct Raw {
        uint32_t x[CPT][RAW];
        uint2 c;
    };
    Raw raw0, raw1;
    auto load = [&](int ks, Raw& raw) __attribute__((always_inline)) {
        ks = ks < KS ? ks : KS - 1;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const uint4* p = reinterpret_cast<const uint4*>(src[j] + ks * 32 * ESZ);
            const uint4 u = p[0];
            raw.x[j][0] = u.x; raw.x[j][1] = u.y; raw.x[j][2] = u.z; raw.x[j][3] = u.w;
            if (SPLIT) {
                const uint4 v = p[1];
                raw.x[j][4] = v.x; raw.x[j][5] = v.y; raw.x[j][6] = v.z; raw.x[j][7] = v.w;
            }
        }
        raw.c = *reinterpret_cast<const uint2*>(a.codes + n_ld * kb + ks * 8);
    };
    auto store = [&](int stage, const Raw& raw) __attribute__((always_inline)) {
        char* xs = smem + stage * XSTAGE;
        if (g == 0) codes_lds[stage][wave * 32 + r] = raw.c;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            uint4 h, l;
            if (SPLIT) {
                split2(__uint_as_float(raw.x[j][0]), __uint_as_float(raw.x[j][1]), h.x, l.x);
                split2(__uint_as_float(raw.x[j][2]), __uint_as_float(raw.x[j][3]), h.y, l.y);
                split2(__uint_as_float(raw.x[j][4]), __uint_as_float(raw.x[j][5]), h.z, l.z);
                split2(__uint_as_float(raw.x[j][6]), __uint_as_float(raw.x[j][7]), h.w, l.w);
            } else if (XDT == RPFQ_BF16) {
                h.x = pack_h2(bf16_to_f32(raw.x[j][0] & 0xffffu), bf16_to_f32(raw.x[j][0] >> 16));
                h.y = pack_h2(bf16_to_f32(raw.x[j][1] & 0xffffu), bf16_to_f32(raw.x[j][1] >> 16));
                h.z = pack_h2(bf16_to_f32(raw.x[j][2] & 0xffffu), bf16_to_f32(raw.x[j][2] >> 16));
                h.w = pack_h2(bf16_to_f32(raw.x[j][3] & 0xffffu), bf16_to_f32(raw.x[j][3] >> 16));
            } else {
                h = make_uint4(raw.x[j][0], raw.x[j][1], raw.x[j][2], raw.x[j][3]);
            }
            *reinterpret_cast<uint4*>(xs + soff[j]) = h;
            if (SPLIT) *reinterpret_cast<uint4*>(xs + soff[j] + 128) = l;
        }
    };

    floatx16 c1[MB], c2[MB], c3[MB], c4[MB];
    floatx16 tre[PERBLOCK ? MB : 1], tim[PERBLOCK ? MB : 1];
#pragma unroll
    for (int i = 0; i < MB; ++i) c1[i] = c2[i] = c3[i] = c4[i] = floatx16{0};
#pragma unroll
    for (int i = 0; i < (PERBLOCK ? MB : 1); ++i) tre[i] = tim[i] = floatx16{0};

    // per-(row, block) scales applied to the four partial sums
    auto flush = [&](int blk) __attribute__((always_inline)) {
        float sr = 0.0f, si = 0.0f;
        if (n_ok) {
            sr = 1.0f / (float)__builtin_bit_cast(_Float16, a.gre[n * a.nblk + blk]);
            si = 1.0f / (float)__builtin_bit_cast(_Float16, a.gim[n * a.nblk + blk]);
        }
        const float xs = a.xsign;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                tre[i][v] += sr * c1[i][v] + xs * (si * c2[i][v]);
                tim[i][v] += si * c3[i][v] - xs * (sr * c4[i][v]);
            }
            c1[i] = c2[i] = c3[i] = c4[i] = floatx16{0};
        }
    };

    auto mfmas = [&](int ks) __attribute__((always_inline)) {
        const char* xs = smem + (ks & 1) * XSTAGE;
        const uint2 cw = codes_lds[ks & 1][wave * 32 + r];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint32_t c16 = ((s ? cw.y : cw.x) >> (16 * g)) & 0xffffu;
            const uint2 t0 = tern[c16 & 15u], t1 = tern[(c16 >> 4) & 15u];
            const uint2 t2 = tern[(c16 >> 8) & 15u], t3 = tern[c16 >> 12];
            const half8 btr = as_half8(make_uint4(t0.x, t1.x, t2.x, t3.x));
            const half8 bti = as_half8(make_uint4(t0.y, t1.y, t2.y, t3.y));
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const char* rp = xs + (i * 32 + r) * XROW + (16 * s + 8 * g) * 2;
                const half8 axr = *reinterpret_cast<const half8*>(rp);
                const half8 axi = *reinterpret_cast<const half8*>(rp + 64);
                c1[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axr, btr, c1[i], 0, 0, 0);
                c2[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axi, bti, c2[i], 0, 0, 0);
                c3[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axr, bti, c3[i], 0, 0, 0);
                c4[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axi, btr, c4[i], 0, 0, 0);
                if (SPLIT) {
                    const half8 lxr = *reinterpret_cast<const half8*>(rp + 128);
                    const half8 lxi = *reinterpret_cast<const half8*>(rp + 192);
                    c1[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxr, btr, c1[i], 0, 0, 0);
                    c2[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxi, bti, c2[i], 0, 0, 0);
                    c3[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxr, bti, c3[i], 0, 0, 0);
                    c4[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxi, btr, c4[i], 0, 0, 0);
                }
            }
        }
        if (PERBLOCK && (ks + 1) % a.block_ks == 0) flush((int)(ks / a.block_ks));
    };

    // k-step ks: loads of ks + 2 into the free register set, MFMAs of ks,
    // k-step ks + 1 (loaded one k-step earlier) converted into the other stage
    auto step = [&](int ks, Raw& rfree, const Raw& rnext) __attribute__((always_inline)) {
        load(ks + 2, rfree);
        __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
        mfmas(ks);
        __builtin_amdgcn_sched_barrier(0);  // and the conversion behind them
        store((ks + 1) & 1, rnext);
        __syncthreads();
    };

    load(0, raw0);
    load(1, raw1);
    store(0, raw0);
    __syncthreads();
    int ks = 0;
    for (; ks + 1 < KS; ks += 2) {
        step(ks, raw0, raw1);
        step(ks + 1, raw1, raw0);
    }
    if (ks < KS) step(ks, raw0, raw1);

    if (!n_ok) return;
    float sr = 0.0f, si = 0.0f;
    if (PERBLOCK) {
        if (KS % a.block_ks != 0) flush(KS / a.block_ks);
    } else {
        sr = 1.0f / (float)__builtin_bit_cast(_Float16, a.gre[n]);
        si = 1.0f / (float)__builtin_bit_cast(_Float16, a.gim[n]);
    }
    const float xs = a.xsign;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t m = m0 + i * 32 + acc_row(v, g);
            float vr, vi;
            if (PERBLOCK) {
                vr = tre[i][v];
                vi = tim[i][v];
            } else {
                vr = sr * c1[i][v] + xs * (si * c2[i][v]);
                vi = si * c3[i][v] - xs * (sr * c4[i][v]);
            }
            if (m < a.M) {
                store1<YDT>(a.yr, m * a.N + n, vr);
                store1<YDT>(a.yi, m * a.N + n, vi);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// native packing (loadWideParams analogue, phase_linear.cpp:90-117)
// ---------------------------------------------------------------------------
struct PackArgs {
    const uint8_t* planes[4];
    const float* sre[4];
    const float* sim[4];
    int nplanes, stages, codebook;
    int64_t N, K, NT, KS, nblk;
    uint8_t* codes;
    float* params;
};

__global__ void wide_pack_codes_kernel(PackArgs a) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t total = a.NT * a.KS * 1024;
    if (idx >= total) return;
    int b = (int)(idx & 31), rr = (int)((idx >> 5) & 31);
    int64_t t = idx >> 10;
    int64_t ks = t % a.KS, nt = t / a.KS;
    int64_t n = nt * 32 + rr;
    int gg = b >> 4, s = (b >> 2) & 3, e = b & 3;
    int64_t k = ks * 32 + 8 * s + 4 * gg + e;
    uint32_t out = 0;
    if (n < a.N && k < a.K) {
        if (a.codebook == RPFQ_CB_PSK16 || a.codebook == RPFQ_CB_TABLE) {
            int64_t kb = a.K >> 1;
            uint32_t cu = (a.planes[0][n * kb + (k >> 1)] >> (4 * (k & 1))) & 15u;
            uint32_t cw = (a.planes[1][n * kb + (k >> 1)] >> (4 * (k & 1))) & 15u;
            out = cu | (cw << 4);
        } else {
            int64_t kb = a.K >> 2;
            int sh = 2 * (int)(k & 3);
            uint32_t c[4] = {0, 0, 0, 0};
            for (int p = 0; p < a.nplanes; ++p) c[p] = (a.planes[p][n * kb + (k >> 2)] >> sh) & 3u;
            uint32_t iu, iw;
            if (a.stages == 2) {
                iu = c[0] | (c[1] << 2);
                iw = c[2] | (c[3] << 2);
            } else {
                iu = c[0];
                iw = c[1];
            }
            out = iu | (iw << 4);
        }
    }
    a.codes[idx] = (uint8_t)out;
}

// TABLE: row n's 16 U then 16 W (re, im) values; padded rows 0.
__global__ void wide_pack_table_kernel(PackArgs a) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t total = a.NT * 32 * 32;
    if (idx >= total) return;
    int64_t n = idx >> 5;
    int e = (int)(idx & 31), p = e >> 4, i = e & 15;
    float re = 0.0f, im = 0.0f;
    if (n < a.N) {
        re = a.sre[p][n * 16 + i];
        im = a.sim[p][n * 16 + i];
    }
    reinterpret_cast<float2*>(a.params)[idx] = make_float2(re, im);
}

__global__ void wide_pack_params_kernel(PackArgs a) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t total = a.NT * 32 * a.nblk;
    if (idx >= total) return;
    int64_t n = idx / a.nblk;
    float p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (n < a.N) {
        if (a.codebook == RPFQ_CB_PSK16) {
            p[0] = a.sre[0][idx];
            p[4] = a.sre[1][idx];
        } else if (a.stages == 2) {
            for (int q = 0; q < 4; ++q) {
                p[2 * q] = a.sre[q][idx];
                p[2 * q + 1] = a.sim[q][idx];
            }
        } else {
            p[0] = a.sre[0][idx];
            p[1] = a.sim[0][idx];
            p[4] = a.sre[1][idx];
            p[5] = a.sim[1][idx];
        }
    }
    float4* dst = reinterpret_cast<float4*>(a.params + idx * 8);
    dst[0] = make_float4(p[0], p[1], p[2], p[3]);
    dst[1] = make_float4(p[4], p[5], p[6], p[7]);
}
// Adjoint code tiles: one workgroup per 32 x 32 block of codes.  The block
// of (row tile t, k-step ks) is staged in LDS as it lies ([row][byte]), and
// thread i writes dword i & 7 of column i >> 3 of the transposed block
// (ks, t): its byte e of that dword is code (row 8 s + 4 g + e, column
// k = i >> 3) with s = (i & 7) & 3, g = (i & 7) >> 2, taken from byte
// 16 g' + 4 s' + e' of the row (k = 8 s' + 4 g' + e').
__global__ void __launch_bounds__(256) wide_pack_adjoint_kernel(const uint32_t* __restrict__ codes,
                                                                uint32_t* __restrict__ codes_t, int64_t NT,
                                                                int64_t KS) {
    __shared__ uint32_t blk[256];
    const int64_t b = blockIdx.x;  // source block index t * KS + ks
    const int64_t t = b / KS, ks = b - t * KS;
    const int i = threadIdx.x;
    blk[i] = codes[b * 256 + i];
    __syncthreads();
    const int k = i >> 3, d = i & 7;
    const int src_b = 16 * ((k >> 2) & 1) + 4 * (k >> 3) + (k & 3);  // byte of column k in a row
    const int row0 = 8 * (d & 3) + 4 * (d >> 2);
    const uint8_t* bytes = reinterpret_cast<const uint8_t*>(blk);
    uint32_t out = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) out |= (uint32_t)bytes[(row0 + e) * 32 + src_b] << (8 * e);
    codes_t[(ks * NT + t) * 256 + i] = out;
}

// Adjoint U / W tables: thread (row, block, index) writes entry `index` of U
// and of W as the GEMM kernels' LUT builders compute it (same entry
// function, de-rotation and fp16 rounding).
template <int CB>
__global__ void wide_adjoint_lut_kernel(const float4* __restrict__ params, int64_t rows, int64_t nblk, RotParams rot,
                                        uint32_t* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nblk * 16) return;
    const uint32_t idx = (uint32_t)(i & 15);
    const int64_t rb = i >> 4;  // row * nblk + block
    float2 u, w;
    if constexpr (CB == RPFQ_CB_TABLE) {
        const float2* t = reinterpret_cast<const float2*>(params) + rb * 32;  // nblk = 1
        u = t[idx];
        w = t[16 + idx];
    } else {
        const float4* p = params + rb * 2;
        u = lut_entry<CB>(idx, p[0]);
        w = lut_entry<CB>(idx, p[1]);
    }
    if (rot.rotate) {
        u = derotate(u, rot.cu, rot.su);
        w = derotate(w, rot.cw, rot.sw);
    }
    out[rb * 32 + idx] = cvt_pk(u.x, u.y);
    out[rb * 32 + 16 + idx] = cvt_pk(w.x, w.y);
}

// Fused weight A_q [2N, 2K] from the native blob (same decode as the GEMM).
template <int CB>
__global__ void wide_decode_kernel(const uint8_t* __restrict__ codes, const float4* __restrict__ params,
                                   int64_t N, int64_t K, int64_t KS, int64_t nblk, int64_t block_ks,
                                   RotParams rot, float* __restrict__ out, int round_fp16) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N * K) return;
    int64_t n = i / K, k = i - n * K;
    int64_t nt = n >> 5, rr = n & 31, ks = k >> 5, kk = k & 31;
    int s = (int)(kk >> 3), gg = (int)((kk >> 2) & 1), e = (int)(kk & 3);
    int b = gg * 16 + s * 4 + e;
    uint32_t byte = codes[((nt * KS + ks) * 32 + rr) * 32 + b];
    float2 U, W;
    if constexpr (CB == RPFQ_CB_TABLE) {
        const float2* t = reinterpret_cast<const float2*>(params) + n * 32;
        U = t[byte & 15u];
        W = t[16 + (byte >> 4)];
    } else {
        int64_t blk = ks / block_ks;
        const float4* p = params + (n * nblk + blk) * 2;
        U = lut_entry<CB>(byte & 15u, p[0]);
        W = lut_entry<CB>(byte >> 4, p[1]);
    }
    if (rot.rotate) {
        U = derotate(U, rot.cu, rot.su);
        W = derotate(W, rot.cw, rot.sw);
    }
    float a11 = W.x + U.x, a12 = W.y - U.y, a21 = W.y + U.y, a22 = -W.x + U.x;
    if (round_fp16) {  // the MFMA operand: fp16 U, W and one fp16 add each (fuse_h)
        uint32_t p1, p2;
        fuse_h(cvt_pk(U.x, U.y), cvt_pk(W.x, W.y), p1, p2);
        const half2v h1 = __builtin_bit_cast(half2v, p1), h2 = __builtin_bit_cast(half2v, p2);
        a11 = (float)h1.x;
        a12 = (float)h1.y;
        a21 = (float)h2.x;
        a22 = (float)h2.y;
    }
    int64_t ld = 2 * K;
    out[n * ld + k] = a11;
    out[n * ld + K + k] = a12;
    out[(N + n) * ld + k] = a21;
    out[(N + n) * ld + K + k] = a22;
}

// ---------------------------------------------------------------------------
// activation fake quantization (quant_i.py:438-455, applied at :546-551)
// ---------------------------------------------------------------------------
template <int XDT>
__device__ __forceinline__ float load1(const void* base, int64_t off) {
    if (XDT == RPFQ_F32) return reinterpret_cast<const float*>(base)[off];
    if (XDT == RPFQ_F16) return (float)reinterpret_cast<const _Float16*>(base)[off];
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[off]);
}

// One 256-thread workgroup per row; each half [0, K) and [K, 2K) gets its own
// scale = qmax * (1 / max(max|x|, 1e-5)) and x_hat = clamp(rint(x scale)) / scale,
// all in float32 (rint = round half to even, as torch.round).
// x and y may be the same buffer (in-place act quant): neither is __restrict__.
template <int XDT, int YDT>
__global__ void __launch_bounds__(256) act_quant_kernel(const void* x, int64_t K, int bits, void* y) {
    __shared__ float red[2][4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t base = row * 2 * K;
    float mx[2] = {0.0f, 0.0f};
    for (int h = 0; h < 2; ++h)
        for (int64_t k = tid; k < K; k += 256) mx[h] = fmaxf(mx[h], fabsf(load1<XDT>(x, base + h * K + k)));
    for (int h = 0; h < 2; ++h) {
        float v = mx[h];
        for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
        if (lane == 0) red[h][wave] = v;
    }
    __syncthreads();
    const float qmax = (float)((1 << (bits - 1)) - 1);
    const float qmin = -(float)(1 << (bits - 1));
    for (int h = 0; h < 2; ++h) {
        float amax = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
        // torch evaluates `float(qmax) / tensor` as reciprocal(tensor) * qmax
        float scale = (1.0f / fmaxf(amax, 1e-5f)) * qmax;
        for (int64_t k = tid; k < K; k += 256) {
            float q = rintf(load1<XDT>(x, base + h * K + k) * scale);
            q = fminf(fmaxf(q, qmin), qmax);
            store1<YDT>(y, base + h * K + k, q / scale);
        }
    }
}

// ---------------------------------------------------------------------------
// LayerNorm (nn.LayerNorm over the last dimension, biased variance)
// ---------------------------------------------------------------------------
// TPR lanes per row (8 .. 64, so that no lane holds more than NC 8-element
// chunks): lane l of a row holds chunks l, l + TPR, ... in registers, so the
// row is read once; mean, then the variance of the held values about it
// (two passes over registers, float32), then the affine map with gamma and
// beta read as float4.
template <int XDT>
__device__ __forceinline__ void load8_ln(const void* base, int64_t off, float* v) {
    if (XDT == RPFQ_F16) {
        const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const half2v h = __builtin_bit_cast(half2v, w[i]);
            v[2 * i] = (float)h.x;
            v[2 * i + 1] = (float)h.y;
        }
    } else {
        load8_f32<XDT>(base, off, v);
    }
}

template <int YDT>
__device__ __forceinline__ void store8_ln(void* base, int64_t off, const float* v) {
    if (YDT == RPFQ_F32) {
        float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + off);
        p[0] = make_float4(v[0], v[1], v[2], v[3]);
        p[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else if (YDT == RPFQ_F16) {
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + off) =
            make_uint4(cvt_pk(v[0], v[1]), cvt_pk(v[2], v[3]), cvt_pk(v[4], v[5]), cvt_pk(v[6], v[7]));
    } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = pack_bf2(v[2 * i], v[2 * i + 1]);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + off) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}


// Row kernel for LayerNorm and / or activation fake quantization.
// LN: y = (x - mean) / sqrt(var + eps) * gamma + beta (nn.LayerNorm);
// AQ: per row and per half [0, C/2), [C/2, C): scale = qmax * (1 / max(max|v|,
// 1e-5)), v = clamp(rint(v * scale), qmin, qmax) / scale in float32
// (quant_i.py:438-455).  LN + AQ quantizes the float32 LN output, as the
// reference quantizes its float32 LayerNorm output, and rounds only the
// quantized value to y's dtype: bit-identical to LN with float32 output
// followed by AQ with y's dtype as output.
// GE + AQ: the exact GELU of each element in float32 (gelu_f, torch's
// formula), quantized without rounding to y's dtype in between -- as the
// reference quantizes fc2's float32 input -- then rounded to y's dtype:
// bit-identical to GELU with float32 output followed by AQ.
// Requires C % 8 == 0 and (AQ) C/2 % 8 == 0, so no 8-element chunk straddles
// the two halves.
// PS (bf16 / float32 x, fp16 y; after the LayerNorm or alone): the row in
// x's dtype (bf16: the LayerNorm's output rounded as rpfq_layer_norm would
// store it), then multiplied by its power-of-two prescale
// (row_prescale of its largest magnitude, written to scale[row]) and stored
// as fp16 -- the bits the DMA kernel's stage makes of the bf16 row with the
// prescale rpfq_row_scales gives it, so a layer on the fp16 rows undoes the
// prescale and matches the bf16 path bit for bit.
template <int XDT, int YDT, int TPR, int NC, bool LN, bool AQ, bool GE = false, bool PS = false>
__global__ void __launch_bounds__(256) layer_norm_kernel(const void* x, int64_t M, int C,  // y may equal x
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float eps, int bits,
                                                         void* y, float* scale) {
    const int sub = threadIdx.x % TPR;
    const int64_t row = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
    if (row >= M) return;  // whole groups leave together: TPR divides the wave
    const int nch = C >> 3;
    const int64_t base = row * C;
    float v[NC][8];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = sub + TPR * j;
        if (c < nch) {
            load8_ln<XDT>(x, base + 8 * c, v[j]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] = 0.0f;
        }
    }
    if (LN) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j)
            if (sub + TPR * j < nch) {
#pragma unroll
                for (int e = 0; e < 8; ++e) s += v[j][e];
            }
        const float mean = group_sum<TPR>(s) / (float)C;
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (sub + TPR * j < nch) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float d = v[j][e] - mean;
                    s2 += d * d;
                }
            }
        }
        const float rstd = 1.0f / sqrtf(group_sum<TPR>(s2) / (float)C + eps);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = sub + TPR * j;
            if (c < nch) {
                float gk[8], bk[8];
                if (gamma) {
                    const float4* gp = reinterpret_cast<const float4*>(gamma + 8 * c);
                    const float4 g0 = gp[0], g1 = gp[1];
                    gk[0] = g0.x; gk[1] = g0.y; gk[2] = g0.z; gk[3] = g0.w;
                    gk[4] = g1.x; gk[5] = g1.y; gk[6] = g1.z; gk[7] = g1.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) gk[e] = 1.0f;
                }
                if (beta) {
                    const float4* bp = reinterpret_cast<const float4*>(beta + 8 * c);
                    const float4 b0 = bp[0], b1 = bp[1];
                    bk[0] = b0.x; bk[1] = b0.y; bk[2] = b0.z; bk[3] = b0.w;
                    bk[4] = b1.x; bk[5] = b1.y; bk[6] = b1.z; bk[7] = b1.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) bk[e] = 0.0f;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v[j][e] = (v[j][e] - mean) * rstd * gk[e] + bk[e];
                }
            }
        }
    }
    if (GE) {
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            if (sub + TPR * j < nch) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[j][e] = gelu_f(v[j][e]);
            }
        }
    }
    if (AQ) {
        const int half_ch = nch >> 1;  // chunks of the real half
        float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = sub + TPR * j;
            if (c < nch) {
                float mx = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[j][e]));
                if (c < half_ch) m0 = fmaxf(m0, mx); else m1 = fmaxf(m1, mx);
            }
        }
        m0 = group_max<TPR>(m0);
        m1 = group_max<TPR>(m1);
        const float qmax = (float)((1 << (bits - 1)) - 1);
        const float qmin = -(float)(1 << (bits - 1));
        // torch evaluates `float(qmax) / tensor` as reciprocal(tensor) * qmax
        const float sc0 = (1.0f / fmaxf(m0, 1e-5f)) * qmax, sc1 = (1.0f / fmaxf(m1, 1e-5f)) * qmax;
        if (TPR >= 32 && NC <= 6 && bits <= 4) {
            // q / scale for the <= 16 integer levels q: lane sub < 32 of the
            // row divides level (sub & 15) - 8 by the scale of half sub >> 4
            // once, and every element fetches its quotient from that lane
            // (ds_bpermute) instead of dividing; the sign is q's, so -0
            // levels stay -0 as the division leaves them.  M = 50,432 rows,
            // 4 bits: act quant C = 3072 120 vs 136 us, LayerNorm + act quant
            // 188 vs 220 us, GELU + act quant 223 vs 236 us; with 8 chunks
            // per lane (C = 4096) the extra registers cost more than the
            // divisions save.
            // (every lane of the row takes part in each ds_bpermute, which
            // reads only active lanes' values: no guard around them; lanes
            // past the row's chunks hold zeros and store nothing)
            const int row_lane0 = (int)(threadIdx.x & 63) - sub;
            const float tv = (float)((sub & 15) - 8) / ((sub & 16) ? sc1 : sc0);
            const int tvb = __float_as_int(tv);
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int c = sub + TPR * j;
                const bool hi = c >= half_ch;
                const float sc = hi ? sc1 : sc0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float qv = rintf(v[j][e] * sc);
                    qv = fminf(fmaxf(qv, qmin), qmax);
                    const int src = row_lane0 + (hi ? 16 : 0) + (int)qv + 8;
                    const float d = __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, tvb));
                    v[j][e] = copysignf(d, qv);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int c = sub + TPR * j;
                if (c < nch) {
                    const float sc = c < half_ch ? sc0 : sc1;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        float qv = rintf(v[j][e] * sc);
                        qv = fminf(fmaxf(qv, qmin), qmax);
                        v[j][e] = qv / sc;
                    }
                }
            }
        }
    }
    if constexpr (PS) {
        float mx = 0.0f;  // chunks past the row hold zeros
#pragma unroll
        for (int j = 0; j < NC; ++j) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if constexpr (XDT == RPFQ_BF16) v[j][e] = bf16_to_f32(f32_to_bf16(v[j][e]));
                mx = fmaxf(mx, fabsf(v[j][e]));
            }
        }
        const float sc = row_prescale(group_max<TPR>(mx));
        if (sub == 0) scale[row] = sc;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] *= sc;  // exact (a power of two)
        }
    }
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = sub + TPR * j;
        if (c < nch) store8_ln<YDT>(y, base + 8 * c, v[j]);
    }
}
// ---------------------------------------------------------------------------
// per-row prescales (rpfq_row_scales): one wave per row, the row's largest
// magnitude (exact: max is order-free) through row_prescale
// ---------------------------------------------------------------------------
template <int XDT>
__global__ void __launch_bounds__(256) row_scale_kernel(const void* x, int64_t M, int64_t C, int vec,
                                                        float* scale) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;  // whole waves leave together
    const int64_t base = row * C;
    float mx = 0.0f;
    if (vec) {  // C % 8 == 0, 16-byte aligned rows: 8 elements per load
        for (int64_t c = lane; c < C / 8; c += 64) {
            float v[8];
            load8_ln<XDT>(x, base + 8 * c, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
        }
    } else {
        for (int64_t c = lane; c < C; c += 64) mx = fmaxf(mx, fabsf(load1<XDT>(x, base + c)));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) scale[row] = row_prescale(mx);
}

template <int XDT>
static hipError_t row_scales_go(const void* x, int64_t M, int64_t C, float* scale, hipStream_t s) {
    const int vec = C % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    hipLaunchKernelGGL((row_scale_kernel<XDT>), dim3((unsigned)((M + 3) / 4)), dim3(256), 0, s, x, M, C, vec, scale);
    return hipGetLastError();
}

hipError_t launch_row_scales(const void* x, int xdt, int64_t M, int64_t C, float* scale, hipStream_t s) {
    switch (xdt) {
        case RPFQ_F32: return row_scales_go<RPFQ_F32>(x, M, C, scale, s);
        case RPFQ_F16: return row_scales_go<RPFQ_F16>(x, M, C, scale, s);
        default: return row_scales_go<RPFQ_BF16>(x, M, C, scale, s);
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
// The act-quant and GELU + act-quant row passes (modes 2 and 4 of
// layer_norm_kernel) with a whole workgroup per row, for launches of few
// rows (a layer at batch 1-4), where 64 lanes per row leave each lane up to
// 48 elements of float32 GELU on the critical path: 256 lanes per row, 8 or
// 16 elements each.  Every output is computed per element and the per-half
// maxima are exact, so the result is bit-identical to the 64-lane form.
template <int XDT, int YDT, bool GE>
__global__ void __launch_bounds__(256) row_aq_block_kernel(const void* x, int C, int bits, void* y) {  // y may equal x
    __shared__ float red[2][4];
    constexpr int NC = 2;  // C <= 4096: 512 chunks of 8 over 256 lanes
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nch = C >> 3, half_ch = nch >> 1;
    const int64_t base = (int64_t)blockIdx.x * C;
    float v[NC][8];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = tid + 256 * j;
        if (c < nch) {
            load8_ln<XDT>(x, base + 8 * c, v[j]);
            if (GE) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[j][e] = gelu_f(v[j][e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] = 0.0f;
        }
    }
    float m[2] = {0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = tid + 256 * j;
        float mx = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[j][e]));
        if (c < half_ch) m[0] = fmaxf(m[0], mx); else m[1] = fmaxf(m[1], mx);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m[h] = fmaxf(m[h], __shfl_xor(m[h], o, 64));
        if (lane == 0) red[h][wave] = m[h];
    }
    __syncthreads();
    const float m0 = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
    const float m1 = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    const float qmax = (float)((1 << (bits - 1)) - 1);
    const float qmin = -(float)(1 << (bits - 1));
    // torch evaluates `float(qmax) / tensor` as reciprocal(tensor) * qmax
    const float sc0 = (1.0f / fmaxf(m0, 1e-5f)) * qmax, sc1 = (1.0f / fmaxf(m1, 1e-5f)) * qmax;
    // <= 4 bits: each wave divides the 16 levels of both halves once (lane
    // l < 32: level (l & 15) - 8 of half l >> 4) and fetches every quotient
    // with ds_bpermute, every lane taking part (lanes past the row hold zeros
    // and store nothing)
    const int tvb = __float_as_int((float)((lane & 15) - 8) / ((lane & 16) ? sc1 : sc0));
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = tid + 256 * j;
        const bool hi = c >= half_ch;
        const float sc = hi ? sc1 : sc0;
        float qv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[e] = fminf(fmaxf(rintf(v[j][e] * sc), qmin), qmax);
        if (bits <= 4) {
            int d[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) d[e] = __builtin_amdgcn_ds_bpermute(((hi ? 16 : 0) + (int)qv[e] + 8) << 2, tvb);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] = copysignf(__int_as_float(d[e]), qv[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] = qv[e] / sc;
        }
        if (c < nch) store8_ln<YDT>(y, base + 8 * c, v[j]);
    }
}

static inline unsigned grid1d(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

hipError_t launch_unpack(const uint8_t* codes, int bits, int64_t rows, int64_t k, const uint16_t* gre,
                         const uint16_t* gim, int64_t nblk, int64_t block, float* re, float* im,
                         hipStream_t s) {
    int64_t total = rows * k;
    hipLaunchKernelGGL(unpack_kernel, dim3(grid1d(total, 256)), dim3(256), 0, s, codes, bits, rows, k, gre,
                       gim, nblk, block, re, im);
    return hipGetLastError();
}

template <int BM, int XDT, int YDT, bool PB>
static hipError_t phase_go(PhaseArgs& a, hipStream_t s) {
    a.tiles_m = (int)((a.M + BM - 1) / BM);
    a.tiles_n = (int)((a.N + 127) / 128);
    hipLaunchKernelGGL((phase_linear_kernel<BM, XDT, YDT, PB>), dim3(a.tiles_m * a.tiles_n), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int XDT, int YDT>
static hipError_t phase_pb(PhaseArgs& a, hipStream_t s) {
    if (a.nblk > 1) return phase_go<32, XDT, YDT, true>(a, s);
    return phase_go<32, XDT, YDT, false>(a, s);
}

template <int XDT>
static hipError_t phase_y(PhaseArgs& a, int ydt, hipStream_t s) {
    switch (ydt) {
        case RPFQ_F32: return phase_pb<XDT, RPFQ_F32>(a, s);
        case RPFQ_F16: return phase_pb<XDT, RPFQ_F16>(a, s);
        default: return phase_pb<XDT, RPFQ_BF16>(a, s);
    }
}

hipError_t launch_phase_linear(const void* xr, const void* xi, int xdt, int conj_x, int64_t M, int64_t K,
                               const uint8_t* codes, const uint16_t* gre, const uint16_t* gim, int64_t nblk,
                               int64_t block_ks, int64_t N, void* yr, void* yi, int ydt, hipStream_t s) {
    PhaseArgs a;
    a.xr = xr;
    a.xi = xi;
    a.M = M;
    a.K = K;
    a.N = N;
    a.codes = codes;
    a.gre = gre;
    a.gim = gim;
    a.nblk = nblk;
    a.block_ks = block_ks;
    a.xsign = conj_x ? 1.0f : -1.0f;
    a.yr = yr;
    a.yi = yi;
    switch (xdt) {
        case RPFQ_F32: return phase_y<RPFQ_F32>(a, ydt, s);
        case RPFQ_F16: return phase_y<RPFQ_F16>(a, ydt, s);
        default: return phase_y<RPFQ_BF16>(a, ydt, s);
    }
}

hipError_t launch_wide_pack(const rpfq_wide_desc& d, const WideGeom& g, const uint8_t* const* planes, int nplanes,
                            const float* const* sre, const float* const* sim, void* packed, hipStream_t s) {
    PackArgs a;
    for (int p = 0; p < 4; ++p) {
        a.planes[p] = p < nplanes ? planes[p] : nullptr;
        a.sre[p] = p < nplanes ? sre[p] : nullptr;
        a.sim[p] = (p < nplanes && sim) ? sim[p] : nullptr;
    }
    a.nplanes = nplanes;
    a.stages = d.stages;
    a.codebook = d.codebook;
    a.N = g.N;
    a.K = g.K;
    a.NT = g.NT;
    a.KS = g.KS;
    a.nblk = g.nblk;
    a.codes = reinterpret_cast<uint8_t*>(packed);
    a.params = reinterpret_cast<float*>(reinterpret_cast<char*>(packed) + g.codes_bytes);
    int64_t nc = g.NT * g.KS * 1024;
    hipLaunchKernelGGL(wide_pack_codes_kernel, dim3(grid1d(nc, 256)), dim3(256), 0, s, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (d.codebook == RPFQ_CB_TABLE) {
        int64_t nt = g.NT * 32 * 32;
        hipLaunchKernelGGL(wide_pack_table_kernel, dim3(grid1d(nt, 256)), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    int64_t np = g.NT * 32 * g.nblk;
    hipLaunchKernelGGL(wide_pack_params_kernel, dim3(grid1d(np, 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int XDT>
static hipError_t act_y(const void* x, int64_t M, int64_t K, int bits, void* y, int ydt, hipStream_t s) {
    switch (ydt) {
        case RPFQ_F32: hipLaunchKernelGGL((act_quant_kernel<XDT, RPFQ_F32>), dim3(M), dim3(256), 0, s, x, K, bits, y); break;
        case RPFQ_F16: hipLaunchKernelGGL((act_quant_kernel<XDT, RPFQ_F16>), dim3(M), dim3(256), 0, s, x, K, bits, y); break;
        default: hipLaunchKernelGGL((act_quant_kernel<XDT, RPFQ_BF16>), dim3(M), dim3(256), 0, s, x, K, bits, y); break;
    }
    return hipGetLastError();
}

static hipError_t row_op(const void* x, int xdt, int64_t M, int64_t C, const float* gamma, const float* beta,
                         float eps, int mode, int bits, void* y, int ydt, hipStream_t s, float* scale = nullptr);

hipError_t launch_act_quant(const void* x, int xdt, int64_t M, int64_t K, int bits, void* y, int ydt, hipStream_t s) {
    // rows held in registers when no 8-element chunk straddles the halves
    const bool vec = K % 8 == 0 && 2 * K <= 4096 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(y) % 16 == 0;
    if (vec) return row_op(x, xdt, M, 2 * K, nullptr, nullptr, 0.0f, 2, bits, y, ydt, s);
    switch (xdt) {
        case RPFQ_F32: return act_y<RPFQ_F32>(x, M, K, bits, y, ydt, s);
        case RPFQ_F16: return act_y<RPFQ_F16>(x, M, K, bits, y, ydt, s);
        default: return act_y<RPFQ_BF16>(x, M, K, bits, y, ydt, s);
    }
}

template <int XDT, int YDT, int TPR, int NC>
static hipError_t ln_launch(const void* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                            int mode, int bits, void* y, float* scale, hipStream_t s) {
    const dim3 grid((unsigned)((M + 256 / TPR - 1) / (256 / TPR)));
    if (mode == 1)
        hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, true, false>), grid, dim3(256), 0, s, x, M, C, gamma,
                           beta, eps, bits, y, scale);
    else if (mode == 2)
        hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, false, true>), grid, dim3(256), 0, s, x, M, C, gamma,
                           beta, eps, bits, y, scale);
    else if (mode == 4)
        hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, false, true, true>), grid, dim3(256), 0, s, x, M, C,
                           gamma, beta, eps, bits, y, scale);
    else if (mode == 5 || mode == 6) {
        if constexpr ((XDT == RPFQ_BF16 || XDT == RPFQ_F32) && YDT == RPFQ_F16) {
            if (mode == 5)
                hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, true, false, false, true>), grid, dim3(256),
                                   0, s, x, M, C, gamma, beta, eps, bits, y, scale);
            else
                hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, false, false, false, true>), grid,
                                   dim3(256), 0, s, x, M, C, gamma, beta, eps, bits, y, scale);
        } else {
            return hipErrorInvalidValue;
        }
    } else
        hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, true, true>), grid, dim3(256), 0, s, x, M, C, gamma,
                           beta, eps, bits, y, scale);
    return hipGetLastError();
}

// Lanes per row: the smallest of 8, 16, 32, 64 that keeps every lane at <= 4
// chunks (C <= 2048), else 64 lanes with up to 6 (C <= 3072) or 8 chunks
// (C <= 4096); 64
// lanes whenever that smallest choice would launch fewer than 256
// workgroups (a batch-1 forward: 197 rows), so the launch spreads over the
// CUs and each lane's chain of loads and reductions is shorter.
// mode: 1 LayerNorm, 2 activation quantization, 3 both, 4 GELU + activation
// quantization, 5 LayerNorm into prescaled fp16 rows, 6 prescaled fp16 rows.
template <int XDT, int YDT>
static hipError_t ln_go(const void* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                        int mode, int bits, void* y, float* scale, hipStream_t s) {
    const int nch = C / 8;
    if (nch <= 256 && ln_row_lanes(M, C) == 64)
        return ln_launch<XDT, YDT, 64, 4>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
    if (nch <= 32) return ln_launch<XDT, YDT, 8, 4>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
    if (nch <= 64) return ln_launch<XDT, YDT, 16, 4>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
    if (nch <= 128) return ln_launch<XDT, YDT, 32, 4>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
    if (nch <= 256) return ln_launch<XDT, YDT, 64, 4>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
    if (nch <= 384) return ln_launch<XDT, YDT, 64, 6>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
    return ln_launch<XDT, YDT, 64, 8>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
}

// Rows at or below which the act-quant passes (modes 2, 4) take a workgroup
// per row.  GELU + act quant of fc1's output (C = 3072) at one image (197
// rows): 12.1 us with 64 lanes per row.
constexpr int64_t kRowBlockMaxM = 1024;

template <int XDT, int YDT>
static hipError_t row_block_go(const void* x, int64_t M, int C, int mode, int bits, void* y, hipStream_t s) {
    if (mode == 4)
        hipLaunchKernelGGL((row_aq_block_kernel<XDT, YDT, true>), dim3((unsigned)M), dim3(256), 0, s, x, C, bits, y);
    else
        hipLaunchKernelGGL((row_aq_block_kernel<XDT, YDT, false>), dim3((unsigned)M), dim3(256), 0, s, x, C, bits, y);
    return hipGetLastError();
}

// GELU + act quant of fp16 rows (mode 4) with torch's float32 GELU taken from
// a table: the GELU of an fp16 input depends on its 16 bits only, so gelu_f
// of every fp16 x in (-16, 16) is computed once per device (gelu_tab_kernel,
// the function layer_norm_kernel evaluates per element) and each element
// reads its entry from the workgroup's LDS copy; inputs outside the table
// (larger magnitudes, inf, NaN) evaluate gelu_f.  Everything after the GELU
// is layer_norm_kernel's 64-lane act quant (exact per-half maxima, the
// quotient table of the <= 16 levels by ds_bpermute), so the output equals
// that kernel's bit for bit without its ~45 VALU of erff per element.
// Table index: the fp16 bits for x in [+0, 16) (bits < 0x4C00), kGeluTabPos +
// (bits & 0x7fff) for x in [-0, -16) (bits in [0x8000, 0xCC00)): at the
// spread of ViT-B's fc1 outputs (sigma ~3) almost no row holds an input
// outside, which would re-read the row for gelu_f.
constexpr int kGeluTabPos = 0x4C00, kGeluTabNeg = 0x4C00;
constexpr int kGeluTab = kGeluTabPos + kGeluTabNeg;  // 38,912 floats = 155,648 B of LDS (of 160 KB)
static_assert(kGeluTab % 4 == 0, "the table is copied as float4");
__device__ __align__(16) float g_gelu_tab[kGeluTab];

__global__ void __launch_bounds__(256) gelu_tab_kernel() {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= kGeluTab) return;
    const uint16_t h = (uint16_t)(i < kGeluTabPos ? i : 0x8000 + (i - kGeluTabPos));
    g_gelu_tab[i] = gelu_f((float)__builtin_bit_cast(_Float16, h));
}

// One workgroup of 16 waves per CU (the table fills most of the LDS); each
// wave walks rows, a row at a time over its 64 lanes (lane l: 8-element
// chunks l, l + 64, ...; NC chunks at most).  y may equal x: a row is read
// whole before it is stored, by one wave.
template <int YDT, int NC>
__global__ void __launch_bounds__(1024) gelu_aq_tab_kernel(const void* x, int64_t M, int C, int bits, void* y) {
    extern __shared__ __align__(16) float tab[];
    for (int i = 4 * (int)threadIdx.x; i < kGeluTab; i += 4 * 1024)
        *reinterpret_cast<float4*>(tab + i) = *reinterpret_cast<const float4*>(g_gelu_tab + i);
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nch = C >> 3, half_ch = nch >> 1;
    const float qmax = (float)((1 << (bits - 1)) - 1);
    const float qmin = -(float)(1 << (bits - 1));
    for (int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 6); row < M; row += (int64_t)gridDim.x * 16) {
        const int64_t base = row * C;
        // the row's fp16 words (chunks past the row read as +0, whose entry is +0)
        uint4 raw[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = lane + 64 * j;
            raw[j] = c < nch ? *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + base + 8 * c)
                             : make_uint4(0u, 0u, 0u, 0u);
        }
        // every element reads an entry (entry 0 where the table has none), so
        // the reads issue back to back; the rare others evaluate gelu_f after
        float v[NC][8];
        bool outside = false;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const uint32_t w[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t hb = (e & 1) ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu;
                const uint32_t mag = hb & 0x7fffu;
                const bool neg = hb >= 0x8000u;
                const bool in = neg ? mag < (uint32_t)kGeluTabNeg : mag < (uint32_t)kGeluTabPos;
                v[j][e] = tab[in ? (neg ? (uint32_t)kGeluTabPos + mag : mag) : 0u];
                outside |= !in;
            }
        }
        if (outside) {  // re-read (the row is stored only below, so x still holds it in place)
#pragma unroll
            for (int j = 0; j < NC; ++j) {
                const int c = lane + 64 * j;
                if (c >= nch) continue;
                const uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + base + 8 * c);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t hb = (e & 1) ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu;
                    const uint32_t mag = hb & 0x7fffu;
                    const bool in = hb >= 0x8000u ? mag < (uint32_t)kGeluTabNeg : mag < (uint32_t)kGeluTabPos;
                    if (!in) v[j][e] = gelu_f((float)__builtin_bit_cast(_Float16, (uint16_t)hb));
                }
            }
        }
        float m0 = 0.0f, m1 = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = lane + 64 * j;
            if (c < nch) {
                float mx = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[j][e]));
                if (c < half_ch) m0 = fmaxf(m0, mx); else m1 = fmaxf(m1, mx);
            }
        }
        m0 = group_max<64>(m0);
        m1 = group_max<64>(m1);
        // torch evaluates `float(qmax) / tensor` as reciprocal(tensor) * qmax
        const float sc0 = (1.0f / fmaxf(m0, 1e-5f)) * qmax, sc1 = (1.0f / fmaxf(m1, 1e-5f)) * qmax;
        // lane l < 32 divides level (l & 15) - 8 by the scale of half l >> 4
        // once; each element fetches its quotient from that lane (every lane
        // takes part; lanes past the row hold zeros and store nothing)
        const float tv = (float)((lane & 15) - 8) / ((lane & 16) ? sc1 : sc0);
        const int tvb = __float_as_int(tv);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const bool hi = lane + 64 * j >= half_ch;
            const float sc = hi ? sc1 : sc0;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float qv = rintf(v[j][e] * sc);
                qv = fminf(fmaxf(qv, qmin), qmax);
                const int src = (hi ? 16 : 0) + (int)qv + 8;
                const float d = __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, tvb));
                v[j][e] = copysignf(d, qv);
            }
        }
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = lane + 64 * j;
            if (c < nch) store8_ln<YDT>(y, base + 8 * c, v[j]);
        }
    }
}

static std::atomic<uint64_t> g_gelu_tab_ready{0};
static std::mutex g_gelu_tab_mu;

// The table path is on unless RPFQ_GELU_TABLE=0.  The current device's table
// is filled on the first call outside graph capture (on that call's stream,
// synchronized once, so every later launch on any stream sees it); calls
// under capture before that take the per-element kernel.
static bool gelu_table_ready(hipStream_t s) {
    static const bool enabled = [] {
        const char* e = std::getenv("RPFQ_GELU_TABLE");
        return !(e && e[0] == '0');
    }();
    if (!enabled) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    const uint64_t bit = (uint64_t)1 << dev;
    if (g_gelu_tab_ready.load(std::memory_order_acquire) & bit) return true;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return false;
    std::lock_guard<std::mutex> lock(g_gelu_tab_mu);
    if (g_gelu_tab_ready.load(std::memory_order_acquire) & bit) return true;
    hipLaunchKernelGGL(gelu_tab_kernel, dim3((kGeluTab + 255) / 256), dim3(256), 0, s);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) return false;
    g_gelu_tab_ready.fetch_or(bit, std::memory_order_release);
    return true;
}

template <int YDT, int NC>
static hipError_t gelu_aq_tab_launch(const void* x, int64_t M, int C, int bits, void* y, hipStream_t s) {
    static std::atomic<uint64_t> attr_done{0};
    constexpr int lds = kGeluTab * 4;
    const hipError_t e =
        set_lds_attr_once(reinterpret_cast<const void*>(&gelu_aq_tab_kernel<YDT, NC>), lds, attr_done);
    if (e != hipSuccess) return e;
    const int64_t groups = (M + 15) / 16;
    const int grid = (int)(groups < device_cus() ? groups : device_cus());
    hipLaunchKernelGGL((gelu_aq_tab_kernel<YDT, NC>), dim3(grid), dim3(1024), lds, s, x, M, C, bits, y);
    return hipGetLastError();
}

template <int YDT>
static hipError_t gelu_aq_tab_go(const void* x, int64_t M, int C, int bits, void* y, hipStream_t s) {
    const int nch = C / 8;
    if (nch <= 128) return gelu_aq_tab_launch<YDT, 2>(x, M, C, bits, y, s);
    if (nch <= 256) return gelu_aq_tab_launch<YDT, 4>(x, M, C, bits, y, s);
    return gelu_aq_tab_launch<YDT, 6>(x, M, C, bits, y, s);
}

template <int XDT>
static hipError_t ln_y(const void* x, int64_t M, int C, const float* gamma, const float* beta, float eps, int mode,
                       int bits, void* y, int ydt, float* scale, hipStream_t s) {
    if constexpr (XDT == RPFQ_F16) {
        if (mode == 4 && M > kRowBlockMaxM && C % 16 == 0 && C / 8 <= 384 && bits >= 1 && bits <= 4 &&
            reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0 &&
            gelu_table_ready(s)) {
            switch (ydt) {
                case RPFQ_F32: return gelu_aq_tab_go<RPFQ_F32>(x, M, C, bits, y, s);
                case RPFQ_F16: return gelu_aq_tab_go<RPFQ_F16>(x, M, C, bits, y, s);
                default: return gelu_aq_tab_go<RPFQ_BF16>(x, M, C, bits, y, s);
            }
        }
    }
    if ((mode == 2 || mode == 4) && M <= kRowBlockMaxM && C % 16 == 0) {
        switch (ydt) {
            case RPFQ_F32: return row_block_go<XDT, RPFQ_F32>(x, M, C, mode, bits, y, s);
            case RPFQ_F16: return row_block_go<XDT, RPFQ_F16>(x, M, C, mode, bits, y, s);
            default: return row_block_go<XDT, RPFQ_BF16>(x, M, C, mode, bits, y, s);
        }
    }
    switch (ydt) {
        case RPFQ_F32: return ln_go<XDT, RPFQ_F32>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
        case RPFQ_F16: return ln_go<XDT, RPFQ_F16>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
        default: return ln_go<XDT, RPFQ_BF16>(x, M, C, gamma, beta, eps, mode, bits, y, scale, s);
    }
}

static hipError_t row_op(const void* x, int xdt, int64_t M, int64_t C, const float* gamma, const float* beta,
                         float eps, int mode, int bits, void* y, int ydt, hipStream_t s, float* scale) {
    switch (xdt) {
        case RPFQ_F32: return ln_y<RPFQ_F32>(x, M, (int)C, gamma, beta, eps, mode, bits, y, ydt, scale, s);
        case RPFQ_F16: return ln_y<RPFQ_F16>(x, M, (int)C, gamma, beta, eps, mode, bits, y, ydt, scale, s);
        default: return ln_y<RPFQ_BF16>(x, M, (int)C, gamma, beta, eps, mode, bits, y, ydt, scale, s);
    }
}

hipError_t launch_layer_norm(const void* x, int xdt, int64_t M, int64_t C, const float* gamma, const float* beta,
                             float eps, int bits, void* y, int ydt, hipStream_t s) {
    return row_op(x, xdt, M, C, gamma, beta, eps, bits > 0 ? 3 : 1, bits, y, ydt, s);
}

hipError_t launch_gelu_act_quant(const void* x, int xdt, int64_t M, int64_t C, int bits, void* y, int ydt,
                                 hipStream_t s) {
    return row_op(x, xdt, M, C, nullptr, nullptr, 0.0f, 4, bits, y, ydt, s);
}

hipError_t launch_layer_norm_prescaled(const void* x, int xdt, int64_t M, int64_t C, const float* gamma,
                                       const float* beta, float eps, void* y, float* scale, hipStream_t s) {
    return row_op(x, xdt, M, C, gamma, beta, eps, 5, 0, y, RPFQ_F16, s, scale);
}

hipError_t launch_row_prescale(const void* x, int xdt, int64_t M, int64_t C, void* y, float* scale, hipStream_t s) {
    return row_op(x, xdt, M, C, nullptr, nullptr, 0.0f, 6, 0, y, RPFQ_F16, s, scale);
}

template <int CB>
static void launch_adjoint_lut(const WideGeom& g, const float4* params, const RotParams& rot, uint32_t* out,
                               hipStream_t s) {
    const int64_t total = g.NT * 32 * g.nblk * 16;
    hipLaunchKernelGGL(wide_adjoint_lut_kernel<CB>, dim3(grid1d(total, 256)), dim3(256), 0, s, params,
                       g.NT * 32, g.nblk, rot, out);
}

hipError_t launch_wide_pack_adjoint(const rpfq_wide_desc& d, const WideGeom& g, const void* packed, void* adjoint,
                                    hipStream_t s) {
    const int64_t blocks = g.NT * g.KS;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(wide_pack_adjoint_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       reinterpret_cast<const uint32_t*>(packed), reinterpret_cast<uint32_t*>(adjoint), g.NT, g.KS);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const float4* params = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(packed) + g.codes_bytes);
    uint32_t* lut = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(adjoint) + wide_adjoint_codes_bytes(g));
    const RotParams rot = rot_of(d);
    switch (d.codebook) {
        case RPFQ_CB_SIGN: launch_adjoint_lut<RPFQ_CB_SIGN>(g, params, rot, lut, s); break;
        case RPFQ_CB_PSK16: launch_adjoint_lut<RPFQ_CB_PSK16>(g, params, rot, lut, s); break;
        case RPFQ_CB_TABLE: launch_adjoint_lut<RPFQ_CB_TABLE>(g, params, rot, lut, s); break;
        default: launch_adjoint_lut<RPFQ_CB_AXIS>(g, params, rot, lut, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_wide_decode(const rpfq_wide_desc& d, const WideGeom& g, const void* packed, float* out,
                              int round_fp16, hipStream_t s) {
    const uint8_t* codes = reinterpret_cast<const uint8_t*>(packed);
    const float4* params = reinterpret_cast<const float4*>(reinterpret_cast<const char*>(packed) + g.codes_bytes);
    int64_t total = g.N * g.K;
    RotParams rot = rot_of(d);
    dim3 grid(grid1d(total, 256));
    switch (d.codebook) {
        case RPFQ_CB_SIGN:
            hipLaunchKernelGGL(wide_decode_kernel<RPFQ_CB_SIGN>, grid, dim3(256), 0, s, codes, params, g.N, g.K,
                               g.KS, g.nblk, g.block_ks, rot, out, round_fp16);
            break;
        case RPFQ_CB_PSK16:
            hipLaunchKernelGGL(wide_decode_kernel<RPFQ_CB_PSK16>, grid, dim3(256), 0, s, codes, params, g.N, g.K,
                               g.KS, g.nblk, g.block_ks, rot, out, round_fp16);
            break;
        case RPFQ_CB_TABLE:
            hipLaunchKernelGGL(wide_decode_kernel<RPFQ_CB_TABLE>, grid, dim3(256), 0, s, codes, params, g.N, g.K,
                               g.KS, g.nblk, g.block_ks, rot, out, round_fp16);
            break;
        default:
            hipLaunchKernelGGL(wide_decode_kernel<RPFQ_CB_AXIS>, grid, dim3(256), 0, s, codes, params, g.N, g.K,
                               g.KS, g.nblk, g.block_ks, rot, out, round_fp16);
            break;
    }
    return hipGetLastError();
}

}  // namespace rpfq
