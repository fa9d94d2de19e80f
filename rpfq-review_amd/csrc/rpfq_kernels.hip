// HIP kernels for gfx950 (MI355X): packed complex-phase linear layers.
//
//   unpack_kernel        bit-exact decode of one packed plane
//   phase_linear_kernel  single plane, ternary MFMA operands, scales in epilogue
//   wide_pack_kernel     reference planes -> native tiled blob
//   wide_linear_kernel   widely-linear layer: per-row LUT decode in LDS ->
//                        fp16 fused coefficients -> 32x32x16 f16 MFMA
//   wide_decode_kernel   fused float32 weight, same decode as the GEMM
//
// Arithmetic order of the decoded coefficients follows the reference exactly
// (RPFQ-ViT-main/quant_models/quant_i.py:111-118 stage sums, :534-544
// recombination) so the float32 coefficient is bit-identical to A_q; it is
// rounded once to fp16 for the MFMA.
#include <mutex>

#include "rpfq_internal.h"

namespace rpfq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// codebooks
// ---------------------------------------------------------------------------
// 16-PSK: exact octant symmetry from three float32 constants
// (cos pi/8, sin pi/8, sqrt(2)/2 rounded to nearest float32).
#define PSK_C1 0x1.d906bcp-1f  /* float32(cos pi/8) */
#define PSK_S1 0x1.87de2ap-2f  /* float32(sin pi/8) */
#define PSK_R2 0x1.6a09e6p-1f  /* float32(sqrt(2)/2) */
__constant__ float kPskCos[16] = {1.0f,    PSK_C1,  PSK_R2,  PSK_S1,  0.0f,    -PSK_S1, -PSK_R2, -PSK_C1,
                                  -1.0f,   -PSK_C1, -PSK_R2, -PSK_S1, 0.0f,    PSK_S1,  PSK_R2,  PSK_C1};
__constant__ float kPskSin[16] = {0.0f,    PSK_S1,  PSK_R2,  PSK_C1,  1.0f,    PSK_C1,  PSK_R2,  PSK_S1,
                                  0.0f,    -PSK_S1, -PSK_R2, -PSK_C1, -1.0f,   -PSK_C1, -PSK_R2, -PSK_S1};

// 2-bit axis code -> value, codes 00=-1, 01=+1, 10=-i, 11=+i
// (export_rpfq_vit_to_mlx.py:598-603; phase_linear.cpp:143-154).
__device__ __forceinline__ float2 axis_val(uint32_t c, float sr, float si) {
    float2 v;
    v.x = (c & 2u) ? 0.0f : ((c & 1u) ? sr : -sr);
    v.y = (c & 2u) ? ((c & 1u) ? si : -si) : 0.0f;
    return v;
}

// 2-bit quadrant-sign code: bit0 = re >= 0, bit1 = im >= 0 (quant_i.py:84-91).
__device__ __forceinline__ float2 sign_val(uint32_t c, float sr, float si) {
    float2 v;
    v.x = (c & 1u) ? sr : -sr;
    v.y = (c & 2u) ? si : -si;
    return v;
}

// Quantized complex value of one U (or W) index under the per-row
// parameters p = (s0 re, s0 im, s1 re, s1 im).  Stages are summed in the
// reference's order q = step0 + step1 (quant_i.py:111-118).
template <int CB>
__device__ __forceinline__ float2 lut_entry(uint32_t idx, float4 p) {
    if (CB == RPFQ_CB_PSK16) {
        return make_float2(p.x * kPskCos[idx], p.x * kPskSin[idx]);
    }
    float2 v0, v1;
    if (CB == RPFQ_CB_SIGN) {
        v0 = sign_val(idx & 3u, p.x, p.y);
        v1 = sign_val(idx >> 2, p.z, p.w);
    } else {
        v0 = axis_val(idx & 3u, p.x, p.y);
        v1 = axis_val(idx >> 2, p.z, p.w);
    }
    return make_float2(v0.x + v1.x, v0.y + v1.y);
}

// De-rotation after quantization (quant_i.py:433-434); built without
// contraction (-ffp-contract=off) so each product rounds as in torch.
__device__ __forceinline__ float2 derotate(float2 q, float c, float s) {
    float a = q.x * c;
    float b = q.y * s;
    float d = q.y * c;
    float e = q.x * s;
    return make_float2(a - b, d + e);
}

// ---------------------------------------------------------------------------
// element I/O
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// 8 consecutive elements at element offset `off` -> 8 fp16 in a uint4.
template <int XDT>
__device__ __forceinline__ uint4 load8_f16(const void* base, int64_t off) {
    if (XDT == RPFQ_F16) {
        return *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
    } else if (XDT == RPFQ_BF16) {
        uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
        uint4 o;
        o.x = pack_h2(bf16_to_f32(v.x & 0xffffu), bf16_to_f32(v.x >> 16));
        o.y = pack_h2(bf16_to_f32(v.y & 0xffffu), bf16_to_f32(v.y >> 16));
        o.z = pack_h2(bf16_to_f32(v.z & 0xffffu), bf16_to_f32(v.z >> 16));
        o.w = pack_h2(bf16_to_f32(v.w & 0xffffu), bf16_to_f32(v.w >> 16));
        return o;
    } else {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
        float4 a = p[0], b = p[1];
        uint4 o;
        o.x = pack_h2(a.x, a.y);
        o.y = pack_h2(a.z, a.w);
        o.z = pack_h2(b.x, b.y);
        o.w = pack_h2(b.z, b.w);
        return o;
    }
}

// float32 -> (hi, lo) fp16 pair with x ~= hi + lo (relative error ~2^-22).
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
    _Float16 ha = (_Float16)a, hb = (_Float16)b;
    _Float16 la = (_Float16)(a - (float)ha), lb = (_Float16)(b - (float)hb);
    hi = (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
    lo = (uint32_t)__builtin_bit_cast(uint16_t, la) | ((uint32_t)__builtin_bit_cast(uint16_t, lb) << 16);
}

template <int YDT>
__device__ __forceinline__ void store1(void* base, int64_t off, float v) {
    if (YDT == RPFQ_F32) {
        reinterpret_cast<float*>(base)[off] = v;
    } else if (YDT == RPFQ_F16) {
        reinterpret_cast<_Float16*>(base)[off] = (_Float16)v;
    } else {
        reinterpret_cast<uint16_t*>(base)[off] = f32_to_bf16(v);
    }
}

__device__ __forceinline__ half8 as_half8(uint4 v) { return __builtin_bit_cast(half8, v); }

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// One element of y's dtype as float32.
template <int YDT>
__device__ __forceinline__ float load_y1(const void* base, int64_t off) {
    if (YDT == RPFQ_F32) return reinterpret_cast<const float*>(base)[off];
    if (YDT == RPFQ_F16) return (float)reinterpret_cast<const _Float16*>(base)[off];
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[off]);
}

// Fused residual add, rounded as the unfused sequence rounds it: the layer
// output v is first rounded to y's dtype, then res + that is rounded again by
// the store (the sum of two fp16 values is exact in float32, so the store's
// rounding equals an fp16 add; bf16 and float32 add in float32 as torch does).
template <int YDT>
__device__ __forceinline__ float with_res(float v, const void* res, int64_t off) {
    if (!res) return v;
    float r = v;
    if (YDT == RPFQ_F16) r = (float)(_Float16)v;
    if (YDT == RPFQ_BF16) r = bf16_to_f32(f32_to_bf16(v));
    return load_y1<YDT>(res, off) + r;
}

// 8 (uint4) or 4 (uint2) packed 16-bit outputs plus the residual at `off`.
__device__ __forceinline__ uint32_t add2_y(uint32_t v, uint32_t r, bool f16) {
    if (f16) return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, r) + __builtin_bit_cast(half2v, v));
    const float lo = bf16_to_f32(r & 0xffffu) + bf16_to_f32(v & 0xffffu);
    const float hi = bf16_to_f32(r >> 16) + bf16_to_f32(v >> 16);
    return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}
template <int YDT>
__device__ __forceinline__ uint4 add_res8(uint4 v, const void* res, int64_t off) {
    const uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(res) + off);
    const bool f16 = YDT == RPFQ_F16;
    return make_uint4(add2_y(v.x, r.x, f16), add2_y(v.y, r.y, f16), add2_y(v.z, r.z, f16), add2_y(v.w, r.w, f16));
}
template <int YDT>
__device__ __forceinline__ uint2 add_res4(uint2 v, const void* res, int64_t off) {
    const uint2 r = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(res) + off);
    const bool f16 = YDT == RPFQ_F16;
    return make_uint2(add2_y(v.x, r.x, f16), add2_y(v.y, r.y, f16));
}

// Fused activation of the stored output (WideArgs::act = 1): exact GELU
// (approximate = 'none') of the value already rounded to y's dtype, computed
// in float32 by the formula of torch's GELU kernel for 16-bit and float32
// tensors, x * 0.5 * (1 + erf(x * sqrt(1/2))), and rounded to y's dtype by
// the store.  The empty asm keeps that float32 rounding: without it the
// backend may fold the last multiply and the fp16 conversion into one
// v_fma_mixlo_f16 (a single rounding), which changes the result where the
// exact value lies near an fp16 rounding tie, and differently per kernel.
__device__ __forceinline__ float gelu_f(float x) {
    float g = x * 0.5f * (1.0f + erff(x * 0.707106781186547524f));
    asm volatile("" : "+v"(g));
    return g;
}

template <int YDT>
__device__ __forceinline__ float act_y(float v, int act) {
    if (!act) return v;
    if (YDT == RPFQ_F16) v = (float)(_Float16)v;
    if (YDT == RPFQ_BF16) v = bf16_to_f32(f32_to_bf16(v));
    return gelu_f(v);
}
// two packed 16-bit outputs of y's dtype
__device__ __forceinline__ uint32_t gelu2_y(uint32_t v, bool f16) {
    if (f16) {
        const half2v h = __builtin_bit_cast(half2v, v);
        const half2v o = {(_Float16)gelu_f((float)h.x), (_Float16)gelu_f((float)h.y)};
        return __builtin_bit_cast(uint32_t, o);
    }
    return (uint32_t)f32_to_bf16(gelu_f(bf16_to_f32(v & 0xffffu))) |
           ((uint32_t)f32_to_bf16(gelu_f(bf16_to_f32(v >> 16))) << 16);
}
__device__ __forceinline__ uint4 gelu8_y(uint4 v, bool f16) {
    return make_uint4(gelu2_y(v.x, f16), gelu2_y(v.y, f16), gelu2_y(v.z, f16), gelu2_y(v.w, f16));
}
__device__ __forceinline__ uint16_t gelu1_y(uint16_t e, bool f16) {
    if (f16) return __builtin_bit_cast(uint16_t, (_Float16)gelu_f((float)__builtin_bit_cast(_Float16, e)));
    return f32_to_bf16(gelu_f(bf16_to_f32(e)));
}
// The same 8 outputs one at a time in a rolled loop (the 16-bit values shift
// through the four words), so only one erf body is live: unrolled, the DMA
// kernel's allocator pays for the epilogue's GELU with spills in its k-loop.
__device__ __forceinline__ uint4 gelu8_rolled(uint4 v, bool f16) {
    uint32_t w0 = v.x, w1 = v.y, w2 = v.z, w3 = v.w;
#pragma unroll 1
    for (int k = 0; k < 8; ++k) {
        const uint32_t o = gelu1_y((uint16_t)(w0 & 0xffffu), f16);
        w0 = (w0 >> 16) | (w1 << 16);
        w1 = (w1 >> 16) | (w2 << 16);
        w2 = (w2 >> 16) | (w3 << 16);
        w3 = (w3 >> 16) | (o << 16);
    }
    return make_uint4(w0, w1, w2, w3);
}

__device__ __forceinline__ half8 to_half8(const float* v) {
    uint4 u;
    u.x = pack_h2(v[0], v[1]);
    u.y = pack_h2(v[2], v[3]);
    u.z = pack_h2(v[4], v[5]);
    u.w = pack_h2(v[6], v[7]);
    return as_half8(u);
}

// Workgroup id -> tile id so that each XCD (ids are dealt round-robin over 8
// XCDs) owns one contiguous run of tiles; consecutive tiles share an M-tile
// and hit the same L2.
__device__ __forceinline__ int xcd_tile(int bid, int total) {
    int xcd = bid & 7, local = bid >> 3;
    int q = total >> 3, r = total & 7;
    return (xcd < r) ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// Row i of the 32x32 MFMA accumulator element v held by lane group g (lane/32).
__device__ __forceinline__ int acc_row(int v, int g) { return 8 * (v >> 2) + 4 * g + (v & 3); }

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

template <int BM, int XDT, int YDT, bool PERBLOCK>
__global__ void __launch_bounds__(256) phase_linear_kernel(PhaseArgs a) {
    constexpr bool SPLIT = (XDT == RPFQ_F32);
    constexpr int MB = BM / 32;
    constexpr int XROW = SPLIT ? 272 : 144;  // bytes per LDS row (+16 pad)
    constexpr int XSTAGE = BM * XROW;
    constexpr int CPT = BM / 32;             // 16-byte chunks per thread per plane pair
    __shared__ __align__(16) char smem[2 * XSTAGE];
    __shared__ uint2 tern[16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, g = lane >> 5;
    const int tile = xcd_tile(blockIdx.x, a.tiles_m * a.tiles_n);
    const int mt = tile / a.tiles_n, ntl = tile - mt * a.tiles_n;
    const int64_t m0 = (int64_t)mt * BM;
    const int64_t n = (int64_t)ntl * 128 + wave * 32 + r;
    const bool n_ok = n < a.N;
    const int64_t KS = a.K / 32;
    const int64_t kb = a.K / 4;

    if (tid < 16) tern[tid] = tern_entry(tid);

    uint4 xh[CPT], xl[CPT];
    uint2 creg = make_uint2(0, 0);

    auto load_x = [&](int64_t ks) {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            int c = tid + 256 * j;
            int row = c >> 3, part = (c >> 2) & 1, sub = c & 3;
            int64_t m = m0 + row;
            const void* plane = part ? a.xi : a.xr;
            int64_t off = m * a.K + ks * 32 + sub * 8;
            if (m < a.M) {
                if (SPLIT) {
                    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(plane) + off);
                    float4 u = p[0], v = p[1];
                    split2(u.x, u.y, xh[j].x, xl[j].x);
                    split2(u.z, u.w, xh[j].y, xl[j].y);
                    split2(v.x, v.y, xh[j].z, xl[j].z);
                    split2(v.z, v.w, xh[j].w, xl[j].w);
                } else {
                    xh[j] = load8_f16<XDT>(plane, off);
                }
            } else {
                xh[j] = make_uint4(0, 0, 0, 0);
                xl[j] = make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto store_x = [&](int stage) {
        char* xs = smem + stage * XSTAGE;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            int c = tid + 256 * j;
            int row = c >> 3, part = (c >> 2) & 1, sub = c & 3;
            *reinterpret_cast<uint4*>(xs + row * XROW + part * 64 + sub * 16) = xh[j];
            if (SPLIT) *reinterpret_cast<uint4*>(xs + row * XROW + 128 + part * 64 + sub * 16) = xl[j];
        }
    };
    auto load_codes = [&](int64_t ks) {
        creg = n_ok ? *reinterpret_cast<const uint2*>(a.codes + n * kb + ks * 8) : make_uint2(0, 0);
    };

    floatx16 c1[MB], c2[MB], c3[MB], c4[MB], tre[MB], tim[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        c1[i] = c2[i] = c3[i] = c4[i] = floatx16{0};
        tre[i] = tim[i] = floatx16{0};
    }

    auto flush = [&](int64_t blk) {
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

    load_x(0);
    load_codes(0);
    store_x(0);
    __syncthreads();

    for (int64_t ks = 0; ks < KS; ++ks) {
        const uint2 cw = creg;
        const bool more = ks + 1 < KS;
        if (more) {
            load_x(ks + 1);
            load_codes(ks + 1);
        }
        const char* xs = smem + (ks & 1) * XSTAGE;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            uint32_t c16 = ((s ? cw.y : cw.x) >> (16 * g)) & 0xffffu;
            uint2 t0 = tern[c16 & 15u], t1 = tern[(c16 >> 4) & 15u];
            uint2 t2 = tern[(c16 >> 8) & 15u], t3 = tern[c16 >> 12];
            half8 btr = as_half8(make_uint4(t0.x, t1.x, t2.x, t3.x));
            half8 bti = as_half8(make_uint4(t0.y, t1.y, t2.y, t3.y));
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const char* rp = xs + (i * 32 + r) * XROW + (16 * s + 8 * g) * 2;
                half8 axr = *reinterpret_cast<const half8*>(rp);
                half8 axi = *reinterpret_cast<const half8*>(rp + 64);
                c1[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axr, btr, c1[i], 0, 0, 0);
                c2[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axi, bti, c2[i], 0, 0, 0);
                c3[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axr, bti, c3[i], 0, 0, 0);
                c4[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(axi, btr, c4[i], 0, 0, 0);
                if (SPLIT) {
                    half8 lxr = *reinterpret_cast<const half8*>(rp + 128);
                    half8 lxi = *reinterpret_cast<const half8*>(rp + 192);
                    c1[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxr, btr, c1[i], 0, 0, 0);
                    c2[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxi, bti, c2[i], 0, 0, 0);
                    c3[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxr, bti, c3[i], 0, 0, 0);
                    c4[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(lxi, btr, c4[i], 0, 0, 0);
                }
            }
        }
        if (PERBLOCK && (ks + 1) % a.block_ks == 0) flush(ks / a.block_ks);
        if (more) store_x((ks + 1) & 1);
        __syncthreads();
    }
    if (!PERBLOCK) flush(0);
    else if (KS % a.block_ks != 0) flush(KS / a.block_ks);

    if (!n_ok) return;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            int64_t m = m0 + i * 32 + acc_row(v, g);
            if (m < a.M) {
                store1<YDT>(a.yr, m * a.N + n, tre[i][v]);
                store1<YDT>(a.yi, m * a.N + n, tim[i][v]);
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

// ---------------------------------------------------------------------------
// widely-linear GEMM
// ---------------------------------------------------------------------------
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
};

// LDS activation row: 32 complex columns as (re, im) fp16 pairs = 128 B,
// padded to 144 B so the 8 lanes of a 128-bit read hit distinct banks.
constexpr int kXRow = 144;
constexpr int kLutWave = 32 * 32 * 4;  // 32 entries x 32 rows x fp16 pair

constexpr int kTRow = 64 * 2 + 16;     // epilogue tile row: 64 fp16 outputs (+16 pad)

template <int BM>
constexpr int wide_lds_bytes() {
    return (2 * BM * kXRow + 4 * kLutWave) > (4 * BM * kTRow) ? (2 * BM * kXRow + 4 * kLutWave)
                                                               : (4 * BM * kTRow);
}

// Two floats -> packed fp16 pair (one v_cvt_pk_f16_f32, round to nearest even).
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
    half2v h = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, h);
}

// Fused fp16 coefficient pairs of one code byte from its U and W entries
// (fp16 (re, im) pairs): p1 = (A11, A12) = (Wre + Ure, Wim - Uim),
// p2 = (A21, A22) = (Wim + Uim, -Wre + Ure), each one correctly rounded fp16
// add in the reference's recombination order (quant_i.py:534-537); one
// v_pk_add_f16 per pair.
__device__ __forceinline__ void fuse_h(uint32_t U, uint32_t W, uint32_t& p1, uint32_t& p2) {
    const half2v u = __builtin_bit_cast(half2v, U), w = __builtin_bit_cast(half2v, W);
    p1 = __builtin_bit_cast(uint32_t, w + (half2v){u.x, -u.y});
    p2 = __builtin_bit_cast(uint32_t, (half2v){w.y, -w.x} + (half2v){u.y, u.x});
}

// Builds the wave's LUT for scale block `blk`: entries 0..15 hold U(idx),
// 16..31 hold W(idx) as fp16 (re, im) pairs, each for the wave's 32 rows;
// layout [entry][row] so the 32 lanes of a lookup touch 32 consecutive
// dwords (no bank conflicts).
template <int CB>
__device__ __forceinline__ void build_lut(uint32_t* lut, const float4* params, int64_t n, bool active, int nblk,
                                          int blk, const RotParams& rot, int r, int g) {
    float4 pu = make_float4(0, 0, 0, 0), pw = make_float4(0, 0, 0, 0);
    if (CB != RPFQ_CB_TABLE && active) {
        const float4* p = params + (n * nblk + blk) * 2;
        pu = p[0];
        pw = p[1];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t idx = (uint32_t)(g + 2 * j);
        float2 u, w;
        if constexpr (CB == RPFQ_CB_TABLE) {
            const float2* t = reinterpret_cast<const float2*>(params) + n * 32;
            u = active ? t[idx] : make_float2(0.0f, 0.0f);
            w = active ? t[16 + idx] : make_float2(0.0f, 0.0f);
        } else {
            u = lut_entry<CB>(idx, pu);
            w = lut_entry<CB>(idx, pw);
        }
        if (rot.rotate) {
            u = derotate(u, rot.cu, rot.su);
            w = derotate(w, rot.cw, rot.sw);
        }
        lut[idx * 32 + r] = cvt_pk(u.x, u.y);
        lut[(16 + idx) * 32 + r] = cvt_pk(w.x, w.y);
    }
}

// 8 consecutive activations -> 8 floats (bf16 / f32 sources).
template <int XDT>
__device__ __forceinline__ void load8_f32(const void* base, int64_t off, float* v) {
    if (XDT == RPFQ_BF16) {
        uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + off);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
            v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
        float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

// Widely-linear GEMM.  Workgroup = 4 waves; tile = BM rows of x times 128
// complex output rows (wave w owns complex rows 32w..32w+31 and produces both
// their real and imaginary outputs).  Per k-step of 32 complex columns:
//   * activations: BM x 32 (re, im) pairs staged to LDS (double buffered);
//   * codes: one 128-bit load per lane (16 elements, one byte each);
//   * decode: byte -> U, W from the wave's LUT (fp32), fused coefficients
//     (A11,A12) and (A21,A22) formed in fp32 as the reference does and packed
//     to fp16 pairs that are directly the MFMA B operands (k order re, im);
//   * 2 x MB v_mfma_f32_32x32x16_f16 per 8 complex columns.
template <int BM, int XDT, int YDT, int CB>
__global__ void __launch_bounds__(256, 2) wide_linear_kernel(WideArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int MB = BM / 32;
    constexpr int XSTAGE = BM * kXRow;
    constexpr int CPT = BM >= 64 ? BM / 64 : 1;  // (row, 8-column) chunks per thread per k-step
    constexpr int NCHUNK = BM * 4;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, g = lane >> 5;
    const int tile = xcd_tile(blockIdx.x, a.tiles_m * a.tiles_n);
    const int mt = tile / a.tiles_n, ntl = tile - mt * a.tiles_n;
    const int64_t m0 = (int64_t)mt * BM;
    const int ntw = ntl * 4 + wave;  // this wave's 32-row tile
    const bool active = ntw < a.NT;
    const int64_t n = (int64_t)ntw * 32 + r;
    uint32_t* lut = reinterpret_cast<uint32_t*>(smem + 2 * XSTAGE) + wave * 1024;
    const int64_t ldx = 2 * (int64_t)a.K;

    // Raw activation prefetch: the loads for k-step ks+1 are issued before
    // the MFMAs of k-step ks and converted/interleaved only when stored to
    // LDS afterwards, so their latency overlaps the math.  Out-of-range
    // chunks load a valid address and are zeroed at store time.
    constexpr int RAW = (XDT == RPFQ_F32) ? 4 : 2;  // uint4 per (re|im) chunk pair
    // Two raw buffers: the data of k-step ks+1 waits in one while the loads
    // of k-step ks+2 land in the other (prefetch distance 2 k-steps).
    uint4 xbufA[CPT][RAW], xbufB[CPT][RAW];
    uint32_t okA = 0, okB = 0;
    uint4 cA = make_uint4(0, 0, 0, 0), cB = make_uint4(0, 0, 0, 0);

    // chunk c = tid + 256 j: row c >> 2, columns 8 (c & 3) .. +7 of the k-step
    auto load_x = [&](int ks, uint4 (&xraw)[CPT][RAW], uint32_t& xok) {
        xok = 0;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tid + 256 * j;
            const int row = c >> 2, sub = c & 3;
            const int64_t m = m0 + row;
            const int kk = ks * 32 + sub * 8;
            const bool ok = c < NCHUNK && m < a.M && kk < a.K;
            xok |= (ok ? 1u : 0u) << j;
            const int64_t off = ok ? m * ldx + kk : 0;
            if (XDT == RPFQ_F32) {
                const uint4* pr = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(a.x) + off);
                const uint4* pi = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(a.x) + off + a.K);
                xraw[j][0] = pr[0];
                xraw[j][1] = pr[1];
                xraw[j][RAW - 2] = pi[0];
                xraw[j][RAW - 1] = pi[1];
            } else {
                xraw[j][0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) + off);
                xraw[j][1] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.x) + off + a.K);
            }
        }
    };
    auto store_x = [&](int stage, const uint4 (&xraw)[CPT][RAW], uint32_t xok) {
        char* xs = smem + stage * XSTAGE;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tid + 256 * j;
            if (NCHUNK < 256 && c >= NCHUNK) break;
            const int row = c >> 2, sub = c & 3;
            uint4 o0, o1;
            {
                if (XDT == RPFQ_F16) {
                    const uint4 vr = xraw[j][0], vi = xraw[j][1];
                    // interleave (re, im) halves: perm selects bytes of (vi, vr)
                    o0.x = __builtin_amdgcn_perm(vi.x, vr.x, 0x05040100u);
                    o0.y = __builtin_amdgcn_perm(vi.x, vr.x, 0x07060302u);
                    o0.z = __builtin_amdgcn_perm(vi.y, vr.y, 0x05040100u);
                    o0.w = __builtin_amdgcn_perm(vi.y, vr.y, 0x07060302u);
                    o1.x = __builtin_amdgcn_perm(vi.z, vr.z, 0x05040100u);
                    o1.y = __builtin_amdgcn_perm(vi.z, vr.z, 0x07060302u);
                    o1.z = __builtin_amdgcn_perm(vi.w, vr.w, 0x05040100u);
                    o1.w = __builtin_amdgcn_perm(vi.w, vr.w, 0x07060302u);
                } else {
                    float fr[8], fi[8];
                    if (XDT == RPFQ_BF16) {
                        const uint32_t wr[4] = {xraw[j][0].x, xraw[j][0].y, xraw[j][0].z, xraw[j][0].w};
                        const uint32_t wi[4] = {xraw[j][1].x, xraw[j][1].y, xraw[j][1].z, xraw[j][1].w};
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            fr[2 * t] = bf16_to_f32(wr[t] & 0xffffu);
                            fr[2 * t + 1] = bf16_to_f32(wr[t] >> 16);
                            fi[2 * t] = bf16_to_f32(wi[t] & 0xffffu);
                            fi[2 * t + 1] = bf16_to_f32(wi[t] >> 16);
                        }
                    } else {
#pragma unroll
                        for (int t = 0; t < 2; ++t) {
                            const float4 r4 = __builtin_bit_cast(float4, xraw[j][t]);
                            const float4 i4 = __builtin_bit_cast(float4, xraw[j][RAW - 2 + t]);
                            fr[4 * t] = r4.x; fr[4 * t + 1] = r4.y; fr[4 * t + 2] = r4.z; fr[4 * t + 3] = r4.w;
                            fi[4 * t] = i4.x; fi[4 * t + 1] = i4.y; fi[4 * t + 2] = i4.z; fi[4 * t + 3] = i4.w;
                        }
                    }
                    o0 = make_uint4(cvt_pk(fr[0], fi[0]), cvt_pk(fr[1], fi[1]), cvt_pk(fr[2], fi[2]),
                                    cvt_pk(fr[3], fi[3]));
                    o1 = make_uint4(cvt_pk(fr[4], fi[4]), cvt_pk(fr[5], fi[5]), cvt_pk(fr[6], fi[6]),
                                    cvt_pk(fr[7], fi[7]));
                }
            }
            // branch-free zero fill of out-of-range chunks: the waitcnt pass
            // then sees straight-line code and keeps the prefetch in flight
            const uint32_t keep = 0u - ((xok >> j) & 1u);
            o0 = make_uint4(o0.x & keep, o0.y & keep, o0.z & keep, o0.w & keep);
            o1 = make_uint4(o1.x & keep, o1.y & keep, o1.z & keep, o1.w & keep);
            uint4* dst = reinterpret_cast<uint4*>(xs + row * kXRow + sub * 32);
            dst[0] = o0;
            dst[1] = o1;
        }
    };
    // Inactive waves (past the last 32-row tile) read tile NT-1 and never
    // store: loads stay unconditional so the wait counts stay exact.
    const int ntw_ld = active ? ntw : a.NT - 1;
    auto load_codes = [&](int ks) -> uint4 {
        return a.codes[(((int64_t)ntw_ld * a.KS + ks) * 32 + r) * 2 + g];
    };

    floatx16 acc_re[MB], acc_im[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc_re[i] = acc_im[i] = floatx16{0};

    int cur_blk = 0;
    build_lut<CB>(lut, a.params, n, active, a.nblk, 0, a.rot, r, g);
    load_x(0, xbufA, okA);
    cA = load_codes(0);
    {
        const int k1 = a.KS > 1 ? 1 : 0;
        load_x(k1, xbufB, okB);
        cB = load_codes(k1);
    }
    store_x(0, xbufA, okA);
    __syncthreads();

    // One k-step: prefetch k-step ks+2 into `fill`, run the MFMAs of ks, stage
    // k-step ks+1 (waiting in `next`) into the other LDS buffer.
    auto kstep = [&](int ks, const uint4 cw, uint4 (&next)[CPT][RAW], uint32_t next_ok, uint4 (&fill)[CPT][RAW],
                     uint32_t& fill_ok, uint4& fill_codes) {
        {   // unconditional: past the end the last k-step is reloaded, unused
            const int kp = ks + 2 < a.KS ? ks + 2 : a.KS - 1;
            load_x(kp, fill, fill_ok);
            fill_codes = load_codes(kp);
        }
        const char* xs = smem + (ks & 1) * XSTAGE;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t word = s == 0 ? cw.x : s == 1 ? cw.y : s == 2 ? cw.z : cw.w;
            // issue every LDS read of the substep first: 8 LUT entries, MB operands
            uint32_t U[4], W[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t byte = (word >> (8 * e)) & 0xffu;
                U[e] = lut[(byte & 15u) * 32 + r];
                W[e] = lut[(16u + (byte >> 4)) * 32 + r];
            }
            half8 ax[MB];
#pragma unroll
            for (int i = 0; i < MB; ++i)
                ax[i] = *reinterpret_cast<const half8*>(xs + (i * 32 + r) * kXRow + (8 * s + 4 * g) * 4);
            uint32_t bre[4], bim[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) fuse_h(U[e], W[e], bre[e], bim[e]);  // (A11, A12), (A21, A22)
            const half8 b_re = as_half8(make_uint4(bre[0], bre[1], bre[2], bre[3]));
            const half8 b_im = as_half8(make_uint4(bim[0], bim[1], bim[2], bim[3]));
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                acc_re[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[i], b_re, acc_re[i], 0, 0, 0);
                acc_im[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[i], b_im, acc_im[i], 0, 0, 0);
            }
        }
        if (ks + 1 < a.KS) {
            store_x((ks + 1) & 1, next, next_ok);
            const int nb = (ks + 1) / a.block_ks;
            if (nb != cur_blk) {
                __syncthreads();
                build_lut<CB>(lut, a.params, n, active, a.nblk, nb, a.rot, r, g);
                cur_blk = nb;
            }
        }
        __syncthreads();
    };
    for (int ks = 0; ks < a.KS; ks += 2) {
        const uint4 c0 = cA;
        kstep(ks, c0, xbufB, okB, xbufA, okA, cA);
        if (ks + 1 < a.KS) {
            const uint4 c1 = cB;
            kstep(ks + 1, c1, xbufA, okA, xbufB, okB, cB);
        }
    }

    const bool n_ok = active && n < a.N;
    const float br = (a.bias && n_ok) ? a.bias[n] : 0.0f;
    const float bi = (a.bias && n_ok) ? a.bias[a.N + n] : 0.0f;
    const int64_t ldy = 2 * (int64_t)a.N;
    if (YDT == RPFQ_F32) {
        if (!n_ok) return;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t m = m0 + i * 32 + acc_row(v, g);
                if (m < a.M) {
                    store1<YDT>(a.y, m * ldy + n, with_res<YDT>(act_y<YDT>(acc_re[i][v] + br, a.act), a.res, m * ldy + n));
                    store1<YDT>(a.y, m * ldy + a.N + n,
                                with_res<YDT>(act_y<YDT>(acc_im[i][v] + bi, a.act), a.res, m * ldy + a.N + n));
                }
            }
        }
        return;
    }
    // 16-bit outputs: transpose the wave's [BM x 64] tile through LDS (the
    // staging buffers are free after the final barrier) and write 16-byte
    // chunks: per row, 32 real then 32 imaginary outputs of this wave.
    constexpr int TROW = kTRow;
    uint16_t* tt = reinterpret_cast<uint16_t*>(smem + wave * (BM * TROW));
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = i * 32 + acc_row(v, g);
            uint16_t hr, hi;
            if (YDT == RPFQ_F16) {
                hr = __builtin_bit_cast(uint16_t, (_Float16)(acc_re[i][v] + br));
                hi = __builtin_bit_cast(uint16_t, (_Float16)(acc_im[i][v] + bi));
            } else {
                hr = f32_to_bf16(acc_re[i][v] + br);
                hi = f32_to_bf16(acc_im[i][v] + bi);
            }
            tt[row * (TROW / 2) + r] = hr;
            tt[row * (TROW / 2) + 32 + r] = hi;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
    __builtin_amdgcn_wave_barrier();
    if (!active) return;
    const int64_t nbase = (int64_t)ntw * 32;
    // lane -> (row offset lane >> 3, 16-byte chunk q = lane & 7): chunks 0-3 real, 4-7 imaginary
    const int q = lane & 7;
    const int64_t col0 = (q < 4 ? 0 : a.N) + nbase + 8 * (q & 3);
    const int64_t nfirst = nbase + 8 * (q & 3);
#pragma unroll 4
    for (int row = lane >> 3; row < BM; row += 8) {
        const int64_t m = m0 + row;
        if (m >= a.M) break;
        uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(tt) + row * TROW + q * 16);
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.y) + m * ldy + col0;
        if (a.vec_store && nfirst + 8 <= a.N) {
            if (a.res) v = add_res8<YDT>(v, a.res, m * ldy + col0);
            if (a.act) v = gelu8_y(v, YDT == RPFQ_F16);
            *reinterpret_cast<uint4*>(dst) = v;
        } else {
            const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
            for (int t = 0; t < 8 && nfirst + t < a.N; ++t) {
                uint16_t e = h[t];
                if (a.res) e = (uint16_t)(add2_y(e, reinterpret_cast<const uint16_t*>(a.res)[m * ldy + col0 + t],
                                                 YDT == RPFQ_F16) & 0xffffu);
                if (a.act) e = gelu1_y(e, YDT == RPFQ_F16);
                dst[t] = e;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// widely-linear GEMM, fp16 activations staged by LDS DMA (large M)
// ---------------------------------------------------------------------------
// Workgroup = 4 waves, tile = 128 rows of x times 128 complex output rows;
// wave w owns complex rows 32w..32w+31 (both their real and imaginary
// outputs) for all 128 rows, as in wide_linear_kernel.  Differences:
//   * activations and codes go global -> LDS by DMA (global_load_lds_dwordx4):
//     no registers hold in-flight loads and no VALU work converts them; a
//     3-stage activation ring keeps two k-steps of loads in flight;
//   * an LDS activation row is the k-step's 8 chunks of 16 B (re cols 0-7,
//     8-15, 16-23, 24-31, then im), chunk c stored at slot c ^ ((row>>1)&7)
//     so the MFMA operand reads hit distinct banks;
//   * MFMA k order: substep s covers complex columns c0 = 8s .. 8s+7; lanes
//     0-31 hold re c0..c0+7 and lanes 32-63 im c0..c0+7 (one 16-B read each);
//     the matching B operand is A11 (or A21) of the 8 columns on lanes 0-31
//     and A12 (or A22) on lanes 32-63.  Each lane still decodes the 4 columns
//     c0 + 4g + e of its code word; v_perm_b32 groups the coefficients by kind
//     and v_permlane32_swap_b32 trades the half the other lane group needs;
//   * the LUT is [entry][row] fp16 (re, im) pairs (conflict-free lookups);
//   * outputs leave through an LDS transpose as 16-B non-temporal stores, so
//     the output stream does not evict the activation tiles the other
//     workgroups of the same row tile are about to read from L2;
//   * per substep the 12 LDS reads of substep s+1 are issued before the MFMAs
//     of substep s and its decode runs beside the last 4 of them (fenced with
//     sched_barrier); one raw barrier per k-step with explicit wait counts
//     keeps the DMA prefetch in flight (a __syncthreads fence would drain it).
// Requires K' % 32 == 0 and M >= 128; the last row tile starts at M - 128 so
// every DMA row is inside x (rows shared with the previous tile are written
// twice with the same values).
// Row tile BM = 128 (two workgroups per CU) or 256 (one per CU, accumulators
// in AGPRs, each decoded coefficient feeds twice the MFMAs).
constexpr int kDmaStages = 3;
constexpr int kDmaLutWave = 32 * 32 * 4;                          // [entry][row] fp16 pairs
constexpr int kDmaCodes = 4 * 1024;                               // codes of one k-step, 4 waves
constexpr int kDmaBias = 4 * 64 * 4;                              // bias of the tile's 128 outputs, re | im
template <int BM> constexpr int dma_stage() { return BM * 128; }  // 16/32 KB
// LDS map: LUT of waves 0-1 at [0, 8K), stages, codes, LUT of waves 2-3 at
// [64K, 72K), bias.  The LUT bases are multiples of 64 KB so an entry address
// is base | (index << 8) | (row slot << 2): one v_perm_b32 forms it.
constexpr int kDmaLutPair = 2 * kDmaLutWave;                      // 8 KB: 32 entries x 64 rows
template <int BM> constexpr int dma_stages_at() { return kDmaLutPair; }
template <int BM> constexpr int dma_codes_at() { return kDmaLutPair + kDmaStages * dma_stage<BM>(); }
template <int BM> constexpr int dma_lut1_at() { return dma_codes_at<BM>() + 2 * kDmaCodes <= 65536 ? 65536 : 131072; }
template <int BM> constexpr int dma_bias_at() { return dma_lut1_at<BM>() + kDmaLutPair; }
template <int BM> constexpr int dma_lds() { return dma_bias_at<BM>() + kDmaBias; }  // 74752 B (BM = 128)
static_assert(dma_lds<128>() == 74752, "two workgroups per CU");
static_assert(4 * 64 * kTRow <= kDmaStages * dma_stage<128>(), "epilogue half tile fits the stages");
static_assert(4 * 128 * kTRow <= kDmaStages * dma_stage<256>(), "epilogue half tile fits the stages");

typedef __attribute__((address_space(3))) const uint32_t* lds_u32_t;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const half8* lds_h8_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const char*)p);
}

// LDS DMA: lane l copies 16 B from gbase + voff[l] to LDS address lds + 16 l.
// Written as asm so that the compiler's wait-count pass does not see the LDS
// write (it would otherwise wait for every outstanding DMA before each LDS
// read); every consumer waits explicitly (s_waitcnt vmcnt + s_barrier)
// before reading the destination.
__device__ __forceinline__ void dma_dwordx4(const void* gbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(gbase) : "memory", "m0");
}

// LUT of one output row in the wave-pair layout: entry e (0..15 U, 16..31 W)
// of row slot `slot` at lut_pair[64 e + slot]; lane group g writes the even
// or odd indices.  Same values as build_lut.
template <int CB>
__device__ __forceinline__ void build_lut_slot(uint32_t* lut_pair, int slot, const float4* params, int64_t n,
                                               int nblk, int blk, const RotParams& rot, int g) {
    float4 pu = make_float4(0, 0, 0, 0), pw = make_float4(0, 0, 0, 0);
    if constexpr (CB != RPFQ_CB_TABLE) {
        const float4* p = params + (n * nblk + blk) * 2;
        pu = p[0];
        pw = p[1];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t idx = (uint32_t)(g + 2 * j);
        float2 u, w;
        if constexpr (CB == RPFQ_CB_TABLE) {
            const float2* t = reinterpret_cast<const float2*>(params) + n * 32;
            u = t[idx];
            w = t[16 + idx];
        } else {
            u = lut_entry<CB>(idx, pu);
            w = lut_entry<CB>(idx, pw);
        }
        if (rot.rotate) {
            u = derotate(u, rot.cu, rot.su);
            w = derotate(w, rot.cw, rot.sw);
        }
        lut_pair[idx * 64 + slot] = cvt_pk(u.x, u.y);
        lut_pair[(16 + idx) * 64 + slot] = cvt_pk(w.x, w.y);
    }
}

// ACT (compile time, = WideArgs::act): the fused GELU's code stays out of
// the plain instantiation, whose k-loop runs at the edge of the register file.
template <int BM, int YDT, int CB, int ACT>
__global__ void __launch_bounds__(256, BM == 128 ? 2 : 1) wide_linear_dma_kernel(WideArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int MB = BM / 32;
    constexpr int kDmaStage = dma_stage<BM>();
    constexpr int RPW = BM / 4;          // activation rows each wave loads per k-step
    constexpr int EPI = BM / 2;          // epilogue transposes half a tile
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, g = lane >> 5;

    char* stages = smem + dma_stages_at<BM>();
    char* cbufs = smem + dma_codes_at<BM>();  // two k-steps of codes
    // [entry][64 rows] LUT shared by a wave pair: this lane's row slot is
    // 32 (wave & 1) + r; entry e at +256 e.  lut_slot holds the slot's LDS
    // address of entry 0, whose byte 1 is zero (base is a multiple of 64 KB).
    uint32_t* lut_pair = reinterpret_cast<uint32_t*>(smem + (wave < 2 ? 0 : dma_lut1_at<BM>()));
    const int slot = 32 * (wave & 1) + r;
    float* bias_s = reinterpret_cast<float*>(smem + dma_bias_at<BM>());  // [wave][re 32 | im 32]
    const uint32_t lut_slot = lds_addr(lut_pair + slot);

    // Activation DMA: wave w fills rows RPW w .. RPW w + RPW - 1 of a stage
    // with 1-KB loads of 8 rows; lane l writes row l >> 3, slot l & 7, which
    // holds chunk (l & 7) ^ ((row >> 1) & 7).  The swizzle depends on the
    // load's parity (row >> 1 = RPW w / 2 + 4j + (l >> 4)), hence two lane
    // offsets.
    const int64_t ldx = 2 * (int64_t)a.K;  // fp16 elements per x row
    uint32_t voff[2];
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
        const int chunk = (lane & 7) ^ ((4 * jp + (lane >> 4)) & 7);
        voff[jp] = (uint32_t)((lane >> 3) * ldx * 2 + (chunk >> 2) * (int64_t)a.K * 2 + (chunk & 3) * 16);
    }
    const uint32_t lds_stages = lds_addr(stages) + RPW * wave * 128;
    const char* xw = nullptr;      // this wave's first x row of the current tile
    const char* cw_src = nullptr;  // codes of the current tile's 32-row block
    auto issue_x = [&](int ks, int stage) {
        const char* src = xw + ks * 64;
        const uint32_t dst = lds_stages + stage * kDmaStage;
#pragma unroll
        for (int j = 0; j < RPW / 8; ++j) dma_dwordx4(src + 8 * j * ldx * 2, voff[j & 1], dst + j * 1024);
    };
    // Codes: one 1-KB block per wave and k-step; lane l fetches the uint4 of
    // MFMA lane l (row l & 31, half l >> 5) so the reads are consecutive.
    const uint32_t cw_voff = (uint32_t)((2 * (lane & 31) + (lane >> 5)) * 16);
    const uint32_t lds_codes = lds_addr(cbufs) + wave * 1024;
    auto issue_codes = [&](int ks, int buf) {
        dma_dwordx4(cw_src + (int64_t)ks * 1024, cw_voff, lds_codes + buf * kDmaCodes);
    };
    auto read_codes = [&](int buf) -> uint4 {
        return *reinterpret_cast<const uint4*>(cbufs + buf * kDmaCodes + wave * 1024 + lane * 16);
    };
    // MFMA operand of row R = 32 i + r, substep s: chunk 4 g + s of row R, at
    // slot (4 g + s) ^ ((r >> 1) & 7); the stage and i parts are immediates
    uint32_t aoff[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) aoff[s] = lds_addr(stages) + r * 128 + (((4 * g + s) ^ ((r >> 1) & 7)) * 16);
    (void)kDmaLutWave;

    // Persistent: the grid holds two workgroups per CU and walks the tiles in
    // the same XCD-local order as a one-tile-per-workgroup launch (the grid
    // size is a multiple of 8, so vb & 7 stays this workgroup's XCD).
    // K-step ks of every tile uses activation stage (ks + 2) % 3, so k-step 0
    // sits in stage 2, which (with codes buffer 0) lies outside the epilogue's
    // LDS rows: the next tile's first codes and activations are requested
    // before the epilogue and land while it runs.
    static_assert(4 * ((BM / 2) * kTRow + 64) <= kDmaLutPair + 2 * dma_stage<BM>(),
                  "the epilogue rows end before activation stage 2");
    const int total = a.tiles_m * a.tiles_n;
    auto tile_src = [&](int vb_t) {  // this wave's x rows and code block of tile vb_t
        const int t = xcd_tile(vb_t, total);
        const int mt_t = t / a.tiles_n;
        const int ntw_t = (t - mt_t * a.tiles_n) * 4 + wave;
        const int64_t m0_t = min((int64_t)mt_t * BM, a.M - BM);
        xw = reinterpret_cast<const char*>(a.x) + (m0_t + RPW * wave) * ldx * 2;
        cw_src = reinterpret_cast<const char*>(a.codes + (int64_t)(ntw_t < a.NT ? ntw_t : a.NT - 1) * a.KS * 64);
    };
    for (int vb = blockIdx.x; vb < total; vb += gridDim.x) {
    const int tile = xcd_tile(vb, total);
    const int mt = tile / a.tiles_n, ntl = tile - mt * a.tiles_n;
    // the last m-tile is shifted back to end at row M (M % BM != 0); rows
    // below m_own belong to the previous m-tile and are not stored again, so
    // every output row is read (residual) and written by one workgroup only
    // (y may alias the residual)
    const int64_t m0 = min((int64_t)mt * BM, a.M - BM);
    const int64_t m_own = (int64_t)mt * BM;
    const int ntw = ntl * 4 + wave;
    const bool active = ntw < a.NT;
    const int ntw_ld = active ? ntw : a.NT - 1;  // inactive waves decode a valid tile, store nothing
    tile_src(vb);

    floatx16 acc_re[MB], acc_im[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc_re[i] = acc_im[i] = floatx16{0};

    if (vb == (int)blockIdx.x) {  // later tiles had these requested before the previous epilogue
        issue_codes(0, 0);
        issue_x(0, 2);
    }
    issue_x(a.KS > 1 ? 1 : 0, 0);
    // the LUT and bias are written while the loads are in flight
    int cur_blk = 0;
    build_lut_slot<CB>(lut_pair, slot, a.params, (int64_t)ntw_ld * 32 + r, a.nblk, 0, a.rot, g);
    {   // bias of this wave's 32 output rows (0 past N or without bias), read in the epilogue
        const int64_t nn = (int64_t)ntw * 32 + r;
        const bool ok = a.bias && active && nn < a.N;
        bias_s[wave * 64 + g * 32 + r] = ok ? a.bias[g * (int64_t)a.N + nn] : 0.0f;
    }
    // codes and stage 2 landed (at most the newest k-step's loads in flight), LUT written
    if (RPW == 32)
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // One k-step on stage `st`: first the codes of k-step ks + 1 and the
    // activations of ks + 2 (into the buffers read at ks - 1, free since the
    // last barrier), then the math.  The loop below is unrolled by 3 so stage
    // offsets are static.
    auto kstep = [&](int ks, int st) {
        if (ks + 1 < a.KS) issue_codes(ks + 1, (ks + 1) & 1);
        if (ks + 2 < a.KS) issue_x(ks + 2, st == 0 ? 2 : st - 1);
        const uint4 cw = read_codes(ks & 1);
        const uint32_t words[4] = {cw.x, cw.y, cw.z, cw.w};
        auto read_sub = [&](int s, uint32_t (&U)[4], uint32_t (&W)[4], half8 (&ax)[MB]) {
            const uint32_t word = words[s];
            const uint32_t pu = word & 0x0f0f0f0fu;         // U index of column e in byte e
            const uint32_t pw = (word >> 4) & 0x0f0f0f0fu;  // W index
#pragma unroll
            for (int e = 0; e < 4; ++e) {  // address = lut_slot with byte 1 := index (one v_perm_b32)
                const uint32_t sel = 0x03020000u | ((4u + e) << 8);
                const uint32_t au = __builtin_amdgcn_perm(pu, lut_slot, sel);
                const uint32_t aw = __builtin_amdgcn_perm(pw, lut_slot, sel);
                U[e] = *((lds_u32_t)au);
                W[e] = *((lds_u32_t)aw + 16 * 64);  // W entries follow the 16 U entries
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) ax[i] = *((lds_h8_t)aoff[s] + (st * kDmaStage + i * 4096) / 16);
        };
        auto decode = [&](const uint32_t (&U)[4], const uint32_t (&W)[4], half8& b_re, half8& b_im) {
            uint32_t p1[4], p2[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) fuse_h(U[e], W[e], p1[e], p2[e]);
            // group by kind: x = (A11 | A21) pairs, y = (A12 | A22) pairs of
            // this lane's 4 columns, then trade x of lanes 32-63 for y of
            // lanes 0-31 so lanes 0-31 hold the re-column coefficients of all
            // 8 columns and lanes 32-63 the im-column ones
            uint32_t xr0 = __builtin_amdgcn_perm(p1[1], p1[0], 0x05040100u);
            uint32_t xr1 = __builtin_amdgcn_perm(p1[3], p1[2], 0x05040100u);
            uint32_t yr0 = __builtin_amdgcn_perm(p1[1], p1[0], 0x07060302u);
            uint32_t yr1 = __builtin_amdgcn_perm(p1[3], p1[2], 0x07060302u);
            uint32_t xi0 = __builtin_amdgcn_perm(p2[1], p2[0], 0x05040100u);
            uint32_t xi1 = __builtin_amdgcn_perm(p2[3], p2[2], 0x05040100u);
            uint32_t yi0 = __builtin_amdgcn_perm(p2[1], p2[0], 0x07060302u);
            uint32_t yi1 = __builtin_amdgcn_perm(p2[3], p2[2], 0x07060302u);
            const auto sr0 = __builtin_amdgcn_permlane32_swap(xr0, yr0, false, false);
            const auto sr1 = __builtin_amdgcn_permlane32_swap(xr1, yr1, false, false);
            const auto si0 = __builtin_amdgcn_permlane32_swap(xi0, yi0, false, false);
            const auto si1 = __builtin_amdgcn_permlane32_swap(xi1, yi1, false, false);
            b_re = as_half8(make_uint4(sr0[0], sr1[0], sr0[1], sr1[1]));
            b_im = as_half8(make_uint4(si0[0], si1[0], si0[1], si1[1]));
        };
        uint32_t U[4], W[4];
        half8 ax_c[MB], b_re, b_im;
        read_sub(0, U, W, ax_c);
        decode(U, W, b_re, b_im);
        // Substep pipeline, fenced so the scheduler keeps it: (1) LUT
        // addresses and the 12 LDS reads of substep s+1; (2) 4 MFMAs of
        // substep s, covering the LDS latency; (3) the decode of s+1 next to
        // the other 4 MFMAs of s.
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            half8 ax_n[MB];
            if (s < 3) read_sub(s + 1, U, W, ax_n);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < MB / 2; ++i) {  // transposed product: weights are the A operand
                acc_re[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b_re, ax_c[i], acc_re[i], 0, 0, 0);
                acc_im[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b_im, ax_c[i], acc_im[i], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = MB / 2; i < MB; ++i) {
                acc_re[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b_re, ax_c[i], acc_re[i], 0, 0, 0);
                acc_im[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(b_im, ax_c[i], acc_im[i], 0, 0, 0);
            }
            if (s < 3) {
                decode(U, W, b_re, b_im);
#pragma unroll
                for (int i = 0; i < MB; ++i) ax_c[i] = ax_n[i];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if (ks + 1 < a.KS) {
            const int nb = (ks + 1) / a.block_ks;
            if (nb != cur_blk) {  // new scale block: this wave's LUT rows only
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                build_lut_slot<CB>(lut_pair, slot, a.params, (int64_t)ntw_ld * 32 + r, a.nblk, nb, a.rot, g);
                cur_blk = nb;
            }
        }
        // codes ks + 1 and stage ks + 1 landed: only the newest RPW / 8 loads
        // (activations of ks + 2) may still be in flight; every LDS read of
        // this k-step is complete.  Near the end nothing is prefetched, so
        // everything must land.
        if (ks + 2 < a.KS) {
            if (RPW == 32)
                asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
        } else
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    int ks = 0;
    for (; ks + 3 <= a.KS; ks += 3) {
        kstep(ks, 2);
        kstep(ks + 1, 0);
        kstep(ks + 2, 1);
    }
    if (ks < a.KS) kstep(ks, 2);
    if (ks + 1 < a.KS) kstep(ks + 1, 0);
    // every stage and code buffer is free (the last k-step drained its loads
    // and reads before its barrier): request the next tile's k-step 0
    if (vb + (int)gridDim.x < total) {
        tile_src(vb + (int)gridDim.x);
        issue_codes(0, 0);
        issue_x(0, 2);
    }
    // Epilogue.  The accumulators hold the transposed tile: lane (r, g) of
    // subtile i has, for x row 32 i + r, outputs n = 32 ntw + 8 q + 4 g + t at
    // element 4 q + t.  Each 4 consecutive outputs go to LDS as one 8-B write
    // ([row][re 32 | im 32] fp16 per wave, half a tile at a time); rows are
    // then read back as 16-B chunks, 8 lanes per row, for coalesced stores.
    // The stages are free: the last k-step drained every DMA and LDS read.
    const int64_t ldy = 2 * (int64_t)a.N;
    float bre[16], bim[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 b0 = *reinterpret_cast<const float4*>(bias_s + wave * 64 + 8 * q + 4 * g);
        const float4 b1 = *reinterpret_cast<const float4*>(bias_s + wave * 64 + 32 + 8 * q + 4 * g);
        bre[4 * q] = b0.x; bre[4 * q + 1] = b0.y; bre[4 * q + 2] = b0.z; bre[4 * q + 3] = b0.w;
        bim[4 * q] = b1.x; bim[4 * q + 1] = b1.y; bim[4 * q + 2] = b1.z; bim[4 * q + 3] = b1.w;
    }
    if (YDT == RPFQ_F32) {  // float32 outputs: 4 consecutive outputs = one 16-B store
      if (active) {
        const int64_t nb0 = (int64_t)ntw * 32 + 4 * g;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const int64_t m = m0 + 32 * i + r;
            if (m < m_own) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t n0 = nb0 + 8 * q;
                float vr[4], vi[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    vr[t] = act_y<YDT>(acc_re[i][4 * q + t] + bre[4 * q + t], ACT);
                    vi[t] = act_y<YDT>(acc_im[i][4 * q + t] + bim[4 * q + t], ACT);
                }
                float* yr = reinterpret_cast<float*>(a.y) + m * ldy + n0;
                float* yi = reinterpret_cast<float*>(a.y) + m * ldy + a.N + n0;
                if (a.res) {
                    const float* rr = reinterpret_cast<const float*>(a.res) + m * ldy + n0;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (n0 + t < a.N) {
                            vr[t] = rr[t] + vr[t];
                            vi[t] = rr[a.N + t] + vi[t];
                        }
                    }
                }
                if (a.vec_store && n0 + 4 <= a.N) {
                    __builtin_nontemporal_store((f32x4){vr[0], vr[1], vr[2], vr[3]}, reinterpret_cast<f32x4*>(yr));
                    __builtin_nontemporal_store((f32x4){vi[0], vi[1], vi[2], vi[3]}, reinterpret_cast<f32x4*>(yi));
                } else {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (n0 + t < a.N) {
                            yr[t] = vr[t];
                            yi[t] = vi[t];
                        }
                    }
                }
            }
        }
      }
    } else {
    // Half a tile at a time: each wave writes its 32 output rows to LDS
    // ([row][re 32 | im 32] fp16, wave regions kEpiWave apart), then stores
    // them as 16-B chunks (8 per lane and half) in one of two patterns:
    //  * workgroup-wide (a.wg_epi, whole tiles of 128 output columns and a
    //    k-loop long enough to hide two workgroup barriers per half): after a
    //    barrier each wave stores EPI / 4 token rows across all four waves'
    //    columns, so every store covers whole 128-B lines of y (a row of the
    //    tile is 128 re + 128 im outputs).  Lane l: row 2 j + (l >> 5), chunk
    //    c = l & 31 (c < 16: re outputs 8 c.., else im outputs 8 (c - 16)..);
    //  * per wave: each wave stores its own rows, 8 lanes per row (chunks
    //    0-3 re, 4-7 im), half lines of y, with no workgroup barrier (short
    //    k-loops, where the barriers would cost more than the lines save).
    // The 64-B pad of the wave regions keeps the 8 lanes of a workgroup-wide
    // read on 32 distinct banks.
    constexpr int kEpiWave = EPI * kTRow + 64;
    char* tt = smem + wave * kEpiWave;
    const bool wg = a.wg_epi != 0;
    const int c = wg ? (lane & 31) : (lane & 7);
    const bool im_chunk = wg ? c >= 16 : c >= 4;
    const int64_t ncol = wg ? (int64_t)ntl * 128 + 8 * (c & 15) : (int64_t)ntw * 32 + 8 * (c & 3);
    const int64_t gcol = (im_chunk ? a.N : 0) + ncol;
    const char* tsrc = wg ? smem + ((c & 15) >> 2) * kEpiWave + (im_chunk ? 64 : 0) + (c & 3) * 16 : tt + c * 16;
    const int row0 = wg ? (EPI / 4) * wave + (lane >> 5) : (lane >> 3);
    const int rstep = wg ? 2 : 8;
    const bool chunk_vec = a.vec_store && ncol + 8 <= a.N;
    // residual chunks of this lane's store rows are requested before the
    // half tile goes through LDS, so their latency overlaps the transpose
    const bool res_vec = a.res && chunk_vec;
    constexpr int RPS = EPI / 8;  // store instructions per wave and half
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint4 rres[RPS];
        if (res_vec) {
#pragma unroll
            for (int j = 0; j < RPS; ++j) {
                const int64_t m = m0 + h * EPI + row0 + rstep * j;
                rres[j] = m >= m_own ? *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.res) +
                                                                        m * ldy + gcol)
                                     : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int ii = 0; ii < MB / 2; ++ii) {
            const int i = h * (MB / 2) + ii;
            char* trow = tt + (32 * ii + r) * kTRow;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint2 pr, pi;
                if (YDT == RPFQ_F16) {
                    pr = make_uint2(cvt_pk(acc_re[i][4 * q] + bre[4 * q], acc_re[i][4 * q + 1] + bre[4 * q + 1]),
                                    cvt_pk(acc_re[i][4 * q + 2] + bre[4 * q + 2], acc_re[i][4 * q + 3] + bre[4 * q + 3]));
                    pi = make_uint2(cvt_pk(acc_im[i][4 * q] + bim[4 * q], acc_im[i][4 * q + 1] + bim[4 * q + 1]),
                                    cvt_pk(acc_im[i][4 * q + 2] + bim[4 * q + 2], acc_im[i][4 * q + 3] + bim[4 * q + 3]));
                } else {
                    pr = make_uint2(f32_to_bf16(acc_re[i][4 * q] + bre[4 * q]) |
                                        ((uint32_t)f32_to_bf16(acc_re[i][4 * q + 1] + bre[4 * q + 1]) << 16),
                                    f32_to_bf16(acc_re[i][4 * q + 2] + bre[4 * q + 2]) |
                                        ((uint32_t)f32_to_bf16(acc_re[i][4 * q + 3] + bre[4 * q + 3]) << 16));
                    pi = make_uint2(f32_to_bf16(acc_im[i][4 * q] + bim[4 * q]) |
                                        ((uint32_t)f32_to_bf16(acc_im[i][4 * q + 1] + bim[4 * q + 1]) << 16),
                                    f32_to_bf16(acc_im[i][4 * q + 2] + bim[4 * q + 2]) |
                                        ((uint32_t)f32_to_bf16(acc_im[i][4 * q + 3] + bim[4 * q + 3]) << 16));
                }
                *reinterpret_cast<uint2*>(trow + (8 * q + 4 * g) * 2) = pr;
                *reinterpret_cast<uint2*>(trow + 64 + (8 * q + 4 * g) * 2) = pi;
            }
        }
        // the rows of this half are in LDS (every wave's, or this wave's)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (wg) __builtin_amdgcn_s_barrier(); else __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < RPS; ++j) {
            const int row = row0 + rstep * j;
            const int64_t m = m0 + h * EPI + row;
            if (m < m_own || ncol >= a.N) continue;
            uint4 v = *reinterpret_cast<const uint4*>(tsrc + row * kTRow);
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.y) + m * ldy + gcol;
            if (chunk_vec) {
                if (res_vec) {
                    const bool f16 = YDT == RPFQ_F16;
                    v = make_uint4(add2_y(v.x, rres[j].x, f16), add2_y(v.y, rres[j].y, f16),
                                   add2_y(v.z, rres[j].z, f16), add2_y(v.w, rres[j].w, f16));
                }
                if constexpr (ACT != 0) v = gelu8_rolled(v, YDT == RPFQ_F16);
                __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(dst));
            } else {
                const uint16_t* hv = reinterpret_cast<const uint16_t*>(&v);
                for (int t = 0; t < 8 && ncol + t < a.N; ++t) {
                    uint16_t e = hv[t];
                    if (a.res)
                        e = (uint16_t)(add2_y(e, reinterpret_cast<const uint16_t*>(a.res)[m * ldy + gcol + t],
                                              YDT == RPFQ_F16) & 0xffffu);
                    if constexpr (ACT != 0) e = gelu1_y(e, YDT == RPFQ_F16);
                    dst[t] = e;
                }
            }
        }
        // all reads of this half done before the next half overwrites the rows
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (wg) __builtin_amdgcn_s_barrier(); else __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    }
    }
    // every wave is done with this tile's LDS before the next tile refills it
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    }
}



// ---------------------------------------------------------------------------
// widely-linear layer for small M: weight streaming
// ---------------------------------------------------------------------------
// The packed codes are the only large operand, so each wave streams one
// 32-row tile of them (KS contiguous 1-KB blocks) and contracts it with a
// chunk of up to 16 activation rows on v_mfma_f32_16x16x32_f16 (workgroup
// = chunk x tiles + tile; M <= 16 is one chunk): the decoded weights are the
// A operand (16 output rows x 16 complex columns as (re, im) fp16 pairs),
// the activations the B operand (its 16 columns are the x rows).
//   * codes: lane (r16 = lane & 15, q = lane >> 4) loads 8 B of rows r16 and
//     16 + r16 per k-step: bytes 8q .. 8q+7 of the row's 32, i.e. the dwords
//     s = 2 (q & 1) + t (t = 0, 1) of lane group g = q >> 1, which hold the
//     complex columns 8 s + 4 g + e.  MFMA t takes dword t, so the four lane
//     groups contribute 16 distinct columns per MFMA and 32 per k-step; the
//     decoded pairs (A11, A12) / (A21, A22) of a column are directly the two
//     k slots that meet (x_re, x_im) of the same column in B.
//   * LUT: [entry][64 slots] fp16 (re, im) pairs at LDS address 0 (one tile
//     per workgroup), each row held twice: row 16 h + r16 in slots
//     32 h + 16 c + r16 (c = 0, 1), and lane group q reads copy c = q & 1,
//     so the 32 lanes of a half-wave hit 32 distinct banks modulo 32.
//     Entry e sits at e * 256 + 4 slot: one v_perm_b32 puts the index
//     nibble into byte 1 of the slot address, and the W entries (e >= 16)
//     are reached through the ds_read immediate offset.
//   * activations: lane (m, q) loads the 4 re and 4 im values of its B
//     fragment straight from x (L2-resident) and interleaves them with
//     v_perm_b32.  Rows past M read row M - 1: their MFMA columns are never
//     stored.  Columns past K' (K' % 32 != 0 only) are zeroed.
//   * split K for layers of few tiles: the NW = 2 or 4 waves of a workgroup
//     share one tile and its LUT (each builds 1 / NW of it), each walks
//     1 / NW of the k-steps, and wave 0 sums the partials through LDS (a
//     small layer then covers NW times the SIMDs);
//   * codes and activations of k-step ks + SK_PF are requested before k-step
//     ks is decoded, by unconditional loads in straight-line code (uniform
//     base + constant lane offset) so the wait counts stay exact; occupancy
//     hides the LDS latency of the decode.
#ifndef RPFQ_SK_PF
#define RPFQ_SK_PF 4
#endif
constexpr int SK_PF = RPFQ_SK_PF;   // prefetch distance in k-steps
constexpr int kSkLut = 32 * 64 * 4;  // 8 KB LUT
// LDS of a workgroup of NW waves: the LUT, and with split K the partial sums
// of waves 1 .. NW-1
constexpr int sk_lds(int nw) { return kSkLut + (nw - 1) * 16 * 64 * 4; }

typedef float floatx4 __attribute__((ext_vector_type(4)));

// LUT of the skinny kernel from row R's parameters (pu, pw), R = lane & 31:
// entry idx in slots 32 (R >> 4) + (R & 15) and + 16; lane group g writes
// the even or odd indices.
// NJ of the 8 (even or odd) indices from j0 on: a whole LUT (NJ = 8), or the
// part one wave of a split-K workgroup of NW waves builds (NJ = 8 / NW,
// j0 = NJ wave).
template <int CB, int NJ = 8>
__device__ __forceinline__ void build_lut_sk(uint32_t* lut, const float4* p, const RotParams& rot, int R, int g,
                                             int j0 = 0) {
    const int s0 = 32 * (R >> 4) + (R & 15);
    float4 pu = make_float4(0, 0, 0, 0), pw = make_float4(0, 0, 0, 0);
    if constexpr (CB != RPFQ_CB_TABLE) {
        pu = p[0];
        pw = p[1];
    }
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
        const uint32_t idx = (uint32_t)(g + 2 * (j0 + jj));
        float2 u, w;
        if constexpr (CB == RPFQ_CB_TABLE) {  // p = the row's 32 (re, im) values
            u = reinterpret_cast<const float2*>(p)[idx];
            w = reinterpret_cast<const float2*>(p)[16 + idx];
        } else {
            u = lut_entry<CB>(idx, pu);
            w = lut_entry<CB>(idx, pw);
        }
        if (rot.rotate) {
            u = derotate(u, rot.cu, rot.su);
            w = derotate(w, rot.cw, rot.sw);
        }
        const uint32_t hu = cvt_pk(u.x, u.y), hw = cvt_pk(w.x, w.y);
        lut[idx * 64 + s0] = hu;
        lut[idx * 64 + s0 + 16] = hu;
        lut[(16 + idx) * 64 + s0] = hw;
        lut[(16 + idx) * 64 + s0 + 16] = hw;
    }
}

// 4 consecutive activations at element offset `off`: the raw 16-bit values
// (fp16, bf16; converted at use so the load stays in flight) or, for
// float32, 4 fp16 converted on load.
template <int XDT>
__device__ __forceinline__ uint2 load4_raw(const void* base, int64_t off) {
    if (XDT != RPFQ_F32) return *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + off);
    const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
    return make_uint2(pack_h2(f.x, f.y), pack_h2(f.z, f.w));
}
template <int XDT>
__device__ __forceinline__ uint2 raw4_f16(uint2 v) {
    if (XDT != RPFQ_BF16) return v;
    return make_uint2(pack_h2(bf16_to_f32(v.x & 0xffffu), bf16_to_f32(v.x >> 16)),
                      pack_h2(bf16_to_f32(v.y & 0xffffu), bf16_to_f32(v.y >> 16)));
}

// PB: per-(row, block) scales (the LUT is rebuilt at each block start);
// KT: K' % 32 != 0 (activation columns past K' are zeroed);
// NW (1 with PB): waves per workgroup.  NW = 2 or 4 splits K: the waves
// share the tile's LUT, take 1 / NW of the k-steps each, and wave 0 adds the
// other partial sums (through LDS, in a fixed order) before the epilogue.
// NW = 1: one wave streams the tile's whole K.
#ifndef RPFQ_SK_OCC
#define RPFQ_SK_OCC 4  // waves per SIMD the register budget is sized for
#endif
template <int XDT, int YDT, int CB, bool PB, bool KT, int NW>
__global__ void __launch_bounds__(64 * NW, RPFQ_SK_OCC) wide_linear_skinny_kernel(WideArgs a) {
    extern __shared__ __align__(16) char smem[];
    uint32_t* lut = reinterpret_cast<uint32_t*>(smem);
    const int lane = threadIdx.x & 63;
    const int wave = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, q = lane >> 4;
    const int R = lane & 31, g = lane >> 5;
    // workgroup -> (16-row chunk of x, 32-row tile of the codes), chunk-major
    const int mc = (int)(blockIdx.x / (unsigned)a.NT);
    const int tile = (int)blockIdx.x - mc * a.NT;
    const int KS = a.KS, K = a.K;
    const int64_t m0 = 16 * (int64_t)mc;                  // first x row of the chunk
    const int M = (int)min((int64_t)16, a.M - m0);        // rows of the chunk
    const void* xc = reinterpret_cast<const char*>(a.x) + m0 * 2 * K * (XDT == RPFQ_F32 ? 4 : 2);
    const int chunk = (KS + NW - 1) / NW;
    const int kb = min(wave * chunk, KS), ke = min(kb + chunk, KS);  // this wave's k-steps

    // uniform bases + constant lane offsets (global_load saddr + voffset)
    const uint2* ctile = reinterpret_cast<const uint2*>(a.codes) + (int64_t)tile * KS * 128;
    const int coff = r16 * 4 + q;
    const bool m_ok = r16 < M;
    const int xoff = (m_ok ? r16 : M - 1) * 2 * K + 16 * (q & 1) + 4 * (q >> 1);  // + 32 ks + 8 t
    const int xcol = 16 * (q & 1) + 4 * (q >> 1);
    struct Step {
        uint2 c[2];          // code dwords (t = 0, 1) of rows r16 and 16 + r16
        uint2 xr[2], xi[2];  // activations of MFMA t: 4 re, 4 im (raw 16-bit or fp16)
    };
    auto load_step = [&](int ks, Step& st) {
        const int kc = ks < ke ? ks : (ke > 0 ? ke - 1 : 0);  // past the range: an L1 hit, unused
        const uint2* cp = ctile + kc * 128;
        st.c[0] = cp[coff];
        st.c[1] = cp[coff + 64];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (KT) {
                const int col = 32 * kc + xcol + 8 * t;
                const int off = xoff - xcol + (col < K ? col : 0);  // K' tail: in bounds, zeroed at use
                st.xr[t] = load4_raw<XDT>(xc, off);
                st.xi[t] = load4_raw<XDT>(xc, off + K);
            } else {
                const int64_t xb = 32 * (int64_t)kc + 8 * t;
                st.xr[t] = load4_raw<XDT>(xc, xb + xoff);
                st.xi[t] = load4_raw<XDT>(xc, xb + K + xoff);
            }
        }
    };
    Step ring[SK_PF];
#pragma unroll
    for (int i = 0; i < SK_PF; ++i) load_step(kb + i, ring[i]);

    int blk = 0;
    {  // split K: each wave builds 1 / NW of the shared LUT
        const float4* p = a.params + ((int64_t)tile * 32 + R) * (CB == RPFQ_CB_TABLE ? 16 : a.nblk * 2);
        if (NW == 1)
            build_lut_sk<CB>(lut, p, a.rot, R, g);
        else
            build_lut_sk<CB, 8 / NW>(lut, p, a.rot, R, g, (8 / NW) * wave);
    }
    if (NW > 1) {  // LUT written before any wave reads it; the code loads stay in flight
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }
    // slot of (row group h, copy q & 1, row r16) in byte 0 of the address
    const uint32_t slot0 = (uint32_t)(16 * (q & 1) + r16) * 4;

    floatx4 acc_re[2], acc_im[2];
    acc_re[0] = acc_re[1] = acc_im[0] = acc_im[1] = floatx4{0, 0, 0, 0};
    auto compute = [&](int ks, const Step& st) {
        half8 bx[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint2 re = raw4_f16<XDT>(st.xr[t]), im = raw4_f16<XDT>(st.xi[t]);
            uint4 b = make_uint4(__builtin_amdgcn_perm(im.x, re.x, 0x05040100u),
                                 __builtin_amdgcn_perm(im.x, re.x, 0x07060302u),
                                 __builtin_amdgcn_perm(im.y, re.y, 0x05040100u),
                                 __builtin_amdgcn_perm(im.y, re.y, 0x07060302u));
            if (KT && 32 * ks + xcol + 8 * t >= K) b = make_uint4(0, 0, 0, 0);
            bx[t] = as_half8(b);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t slot = slot0 + 128 * h;
            const uint32_t words[2] = {st.c[h].x, st.c[h].y};
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const uint32_t pu = words[t] & 0x0f0f0f0fu;
                const uint32_t pw = (words[t] >> 4) & 0x0f0f0f0fu;
                uint32_t p1[4], p2[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t sel = 0x03020000u | ((4u + e) << 8);
                    const uint32_t U = *((lds_u32_t)__builtin_amdgcn_perm(pu, slot, sel));
                    const uint32_t W = *((lds_u32_t)__builtin_amdgcn_perm(pw, slot, sel) + 16 * 64);
                    fuse_h(U, W, p1[e], p2[e]);
                }
                const half8 are = as_half8(make_uint4(p1[0], p1[1], p1[2], p1[3]));
                const half8 aim = as_half8(make_uint4(p2[0], p2[1], p2[2], p2[3]));
                acc_re[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(are, bx[t], acc_re[h], 0, 0, 0);
                acc_im[h] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aim, bx[t], acc_im[h], 0, 0, 0);
            }
        }
    };
    for (int ks0 = kb; ks0 < ke; ks0 += SK_PF) {
#pragma unroll
        for (int i = 0; i < SK_PF; ++i) {
            const int ks = ks0 + i;
            if (ks >= ke) break;
            const Step cur = ring[i];
            load_step(ks + SK_PF, ring[i]);  // past the end: reloads the last k-step, unused
            if (PB) {  // per-(row, block) scales: new LUT at each block start
                const int nb = ks / a.block_ks;
                if (nb != blk) {
                    blk = nb;
                    const float4* p = a.params + (((int64_t)tile * 32 + R) * a.nblk + nb) * 2;
                    build_lut_sk<CB>(lut, p, a.rot, R, g);
                }
            }
            compute(ks, cur);
        }
    }

    if (NW > 1) {  // waves 1 .. NW-1 hand their partial sums to wave 0
        float* red = reinterpret_cast<float*>(smem + kSkLut);
        if (wave > 0) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                red[((wave - 1) * 16 + v) * 64 + lane] = acc_re[0][v];
                red[((wave - 1) * 16 + 4 + v) * 64 + lane] = acc_re[1][v];
                red[((wave - 1) * 16 + 8 + v) * 64 + lane] = acc_im[0][v];
                red[((wave - 1) * 16 + 12 + v) * 64 + lane] = acc_im[1][v];
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < NW - 1; ++w) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                acc_re[0][v] += red[(w * 16 + v) * 64 + lane];
                acc_re[1][v] += red[(w * 16 + 4 + v) * 64 + lane];
                acc_im[0][v] += red[(w * 16 + 8 + v) * 64 + lane];
                acc_im[1][v] += red[(w * 16 + 12 + v) * 64 + lane];
            }
        }
    }

    // Epilogue: lane (m = r16, q) holds outputs n = 32 tile + 16 h + 4 q + v
    // of x row m; rows past M and outputs past N' store nothing.
    if (!m_ok) return;
    const int64_t ldy = 2 * (int64_t)a.N;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t n0 = (int64_t)tile * 32 + 16 * h + 4 * q;
        float vr[4], vi[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int64_t n = n0 + v;
            const bool ok = n < a.N;
            vr[v] = acc_re[h][v] + ((a.bias && ok) ? a.bias[n] : 0.0f);
            vi[v] = acc_im[h][v] + ((a.bias && ok) ? a.bias[a.N + n] : 0.0f);
        }
        const int64_t base = (m0 + r16) * ldy + n0;
        if (a.vec_store && n0 + 4 <= a.N && YDT == RPFQ_F16) {
            uint2 hr = make_uint2(cvt_pk(vr[0], vr[1]), cvt_pk(vr[2], vr[3]));
            uint2 hi = make_uint2(cvt_pk(vi[0], vi[1]), cvt_pk(vi[2], vi[3]));
            if (a.res) {
                hr = add_res4<YDT>(hr, a.res, base);
                hi = add_res4<YDT>(hi, a.res, base + a.N);
            }
            if (a.act) {
                hr = make_uint2(gelu2_y(hr.x, true), gelu2_y(hr.y, true));
                hi = make_uint2(gelu2_y(hi.x, true), gelu2_y(hi.y, true));
            }
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.y) + base) = hr;
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.y) + base + a.N) = hi;
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if (n0 + v < a.N) {
                    store1<YDT>(a.y, base + v, with_res<YDT>(act_y<YDT>(vr[v], a.act), a.res, base + v));
                    store1<YDT>(a.y, base + a.N + v, with_res<YDT>(act_y<YDT>(vi[v], a.act), a.res, base + a.N + v));
                }
            }
        }
    }
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
template <int XDT, int YDT>
__global__ void __launch_bounds__(256) act_quant_kernel(const void* __restrict__ x, int64_t K, int bits,
                                                        void* __restrict__ y) {
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
        for (int i = 0; i < 4; ++i) w[i] = (uint32_t)f32_to_bf16(v[2 * i]) | ((uint32_t)f32_to_bf16(v[2 * i + 1]) << 16);
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + off) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <int TPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = TPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int TPR>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = TPR / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

template <int YDT>
__device__ __forceinline__ float round_to(float v) {
    if (YDT == RPFQ_F16) return (float)(_Float16)v;
    if (YDT == RPFQ_BF16) return bf16_to_f32(f32_to_bf16(v));
    return v;
}

// Row kernel for LayerNorm and / or activation fake quantization.
// LN: y = (x - mean) / sqrt(var + eps) * gamma + beta (nn.LayerNorm);
// AQ: per row and per half [0, C/2), [C/2, C): scale = qmax * (1 / max(max|v|,
// 1e-5)), v = clamp(rint(v * scale), qmin, qmax) / scale in float32
// (quant_i.py:438-455), applied to the LN output already rounded to y's
// dtype, so LN + AQ is bit-identical to the two kernels in sequence.
// Requires C % 8 == 0 and (AQ) C/2 % 8 == 0, so no 8-element chunk straddles
// the two halves.
template <int XDT, int YDT, int TPR, int NC, bool LN, bool AQ>
__global__ void __launch_bounds__(256) layer_norm_kernel(const void* __restrict__ x, int64_t M, int C,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float eps, int bits,
                                                         void* y) {
    const int sub = threadIdx.x % TPR;
    const int64_t row = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
    if (row >= M) return;  // whole groups leave together: TPR divides the wave
    const int nch = C >> 3;
    const int64_t base = row * C;
    float v[NC][8];
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = sub + TPR * j;
        if (c < nch) load8_ln<XDT>(x, base + 8 * c, v[j]);
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
                    const float o = (v[j][e] - mean) * rstd * gk[e] + bk[e];
                    v[j][e] = AQ ? round_to<YDT>(o) : o;
                }
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
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const int c = sub + TPR * j;
        if (c < nch) store8_ln<YDT>(y, base + 8 * c, v[j]);
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
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
    if (a.nblk > 1) return phase_go<64, XDT, YDT, true>(a, s);
    return phase_go<64, XDT, YDT, false>(a, s);
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

static RotParams rot_of(const rpfq_wide_desc& d) {
    RotParams r;
    r.rotate = d.rotate;
    r.cu = d.rot_u[0];
    r.su = d.rot_u[1];
    r.cw = d.rot_w[0];
    r.sw = d.rot_w[1];
    return r;
}

// Compute units of the current device (cached per device; 256 on MI355X).
static int device_cus() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cached[dev] <= 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev] & ~3;  // keep the grid a multiple of 8 (XCD-local tile order)
}

template <int BM, int XDT, int YDT, int CB>
static hipError_t wide_go(WideArgs& a, hipStream_t s) {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    constexpr int lds = wide_lds_bytes<BM>();
    std::call_once(once, [] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&wide_linear_kernel<BM, XDT, YDT, CB>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    });
    if (attr_err != hipSuccess) return attr_err;
    a.tiles_m = (int)((a.M + BM - 1) / BM);
    a.tiles_n = (int)((a.NT + 3) / 4);
    hipLaunchKernelGGL((wide_linear_kernel<BM, XDT, YDT, CB>), dim3(a.tiles_m * a.tiles_n), dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int BM, int YDT, int CB, int ACT>
static hipError_t wide_dma_act(WideArgs& a, hipStream_t s) {
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    constexpr int lds = dma_lds<BM>();
    std::call_once(once, [] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&wide_linear_dma_kernel<BM, YDT, CB, ACT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    });
    if (attr_err != hipSuccess) return attr_err;
    a.tiles_m = (int)((a.M + BM - 1) / BM);
    a.tiles_n = (int)((a.NT + 3) / 4);
    const int total = a.tiles_m * a.tiles_n;
    const int slots = (BM == 128 ? 2 : 1) * device_cus();  // workgroups resident per CU
    const int grid = total < slots ? total : slots;
    hipLaunchKernelGGL((wide_linear_dma_kernel<BM, YDT, CB, ACT>), dim3(grid), dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int BM, int YDT, int CB>
static hipError_t wide_dma_go(WideArgs& a, hipStream_t s) {
    if constexpr (YDT == RPFQ_BF16) return wide_dma_act<BM, YDT, CB, 0>(a, s);  // GELU: not routed here
    else return a.act ? wide_dma_act<BM, YDT, CB, 1>(a, s) : wide_dma_act<BM, YDT, CB, 0>(a, s);
}

// Workgroups of the streaming kernel: one per (16-row chunk, 32-row tile).
static int64_t sk_groups(const WideArgs& a) { return a.NT * ((a.M + 15) / 16); }

template <int XDT, int YDT, int CB, bool PB, bool KT, int NW>
static hipError_t wide_sk_go(WideArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((wide_linear_skinny_kernel<XDT, YDT, CB, PB, KT, NW>), dim3((unsigned)sk_groups(a)),
                       dim3(64 * NW), sk_lds(NW), s, a);
    return hipGetLastError();
}

// Split K when the launch has too few workgroups to give every SIMD a few
// waves (a single layer at batch 1): over 4 waves below 400 workgroups, over
// 2 from there (less LUT building and reduction per k-step once the groups
// alone fill the SIMDs; ViT-B/16 batch-1 forward 0.834 -> 0.772 ms, and 2
// waves already from 128 groups measured slower); a long stream of tiles
// runs one wave each.
#ifndef RPFQ_SK_SPLIT_TILES
#define RPFQ_SK_SPLIT_TILES 4096
#endif
#ifndef RPFQ_SK_NW2_GROUPS
#define RPFQ_SK_NW2_GROUPS 400
#endif
template <int XDT, int YDT, int CB>
static hipError_t wide_sk(WideArgs& a, hipStream_t s) {
    const bool pb = a.nblk > 1, kt = a.K % 32 != 0;
    if (pb) return kt ? wide_sk_go<XDT, YDT, CB, true, true, 1>(a, s) : wide_sk_go<XDT, YDT, CB, true, false, 1>(a, s);
    const int64_t groups = sk_groups(a);
    if (groups >= RPFQ_SK_NW2_GROUPS && groups < RPFQ_SK_SPLIT_TILES)
        return kt ? wide_sk_go<XDT, YDT, CB, false, true, 2>(a, s) : wide_sk_go<XDT, YDT, CB, false, false, 2>(a, s);
    if (groups < RPFQ_SK_SPLIT_TILES)
        return kt ? wide_sk_go<XDT, YDT, CB, false, true, 4>(a, s) : wide_sk_go<XDT, YDT, CB, false, false, 4>(a, s);
    return kt ? wide_sk_go<XDT, YDT, CB, false, true, 1>(a, s) : wide_sk_go<XDT, YDT, CB, false, false, 1>(a, s);
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
// The kernel a launch runs (RPFQ_KERNEL_*), from the shape, dtypes and the
// kernel-choice flags (the GELU bit already moved into a.act).
static int choose_kernel(const WideArgs& a, int xdt, int ydt, int flags) {
    if ((flags & RPFQ_FLAG_STREAM) || (!(flags & (RPFQ_FLAG_TILE_M128 | RPFQ_FLAG_NO_STREAM)) && stream_pays(a)))
        return RPFQ_KERNEL_STREAM;
    flags &= ~RPFQ_FLAG_NO_STREAM;
    // (bf16 outputs with the fused GELU: the DMA kernel's instantiation would
    // spill in its k-loop, so they take the register-staged kernel)
    if (xdt == RPFQ_F16 && flags == 0 && a.K % 32 == 0 && a.M >= RPFQ_DMA_MIN_M && !(a.act && ydt == RPFQ_BF16))
        return RPFQ_KERNEL_DMA;
    return RPFQ_KERNEL_TILED;
}

template <int XDT, int YDT, int CB>
static hipError_t wide_bm(WideArgs& a, int flags, hipStream_t s) {
    const int k = choose_kernel(a, XDT, YDT, flags);
    if (k == RPFQ_KERNEL_STREAM) return wide_sk<XDT, YDT, CB>(a, s);
    if (k == RPFQ_KERNEL_DMA) return wide_dma_go<128, YDT, CB>(a, s);
    flags &= ~RPFQ_FLAG_NO_STREAM;
    if (flags & RPFQ_FLAG_TILE_M128) return wide_go<128, XDT, YDT, CB>(a, s);
    if (a.M <= 32) return wide_go<32, XDT, YDT, CB>(a, s);
    if (a.M <= 64) return wide_go<64, XDT, YDT, CB>(a, s);
    return wide_go<128, XDT, YDT, CB>(a, s);
}

template <int XDT, int CB>
static hipError_t wide_y(WideArgs& a, int ydt, int flags, hipStream_t s) {
    switch (ydt) {
        case RPFQ_F32: return wide_bm<XDT, RPFQ_F32, CB>(a, flags, s);
        case RPFQ_F16: return wide_bm<XDT, RPFQ_F16, CB>(a, flags, s);
        default: return wide_bm<XDT, RPFQ_BF16, CB>(a, flags, s);
    }
}

template <int CB>
static hipError_t wide_x(WideArgs& a, int xdt, int ydt, int flags, hipStream_t s) {
    switch (xdt) {
        case RPFQ_F32: return wide_y<RPFQ_F32, CB>(a, ydt, flags, s);
        case RPFQ_F16: return wide_y<RPFQ_F16, CB>(a, ydt, flags, s);
        default: return wide_y<RPFQ_BF16, CB>(a, ydt, flags, s);
    }
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

int wide_linear_kernel_choice(const WideGeom& g, int xdt, int64_t M, int ydt, int flags) {
    return choose_kernel(wide_shape(g, M, flags), xdt, ydt, flags & ~RPFQ_FLAG_GELU);
}

hipError_t launch_wide_linear(const rpfq_wide_desc& d, const WideGeom& g, const void* packed, const void* x,
                              int xdt, int64_t M, const float* bias, const void* res, void* y, int ydt, int flags,
                              hipStream_t s) {
    WideArgs a = wide_shape(g, M, flags);
    flags &= ~RPFQ_FLAG_GELU;
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
    switch (d.codebook) {
        case RPFQ_CB_SIGN: return wide_x<RPFQ_CB_SIGN>(a, xdt, ydt, flags, s);
        case RPFQ_CB_PSK16: return wide_x<RPFQ_CB_PSK16>(a, xdt, ydt, flags, s);
        case RPFQ_CB_TABLE: return wide_x<RPFQ_CB_TABLE>(a, xdt, ydt, flags, s);
        default: return wide_x<RPFQ_CB_AXIS>(a, xdt, ydt, flags, s);
    }
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
                         float eps, int mode, int bits, void* y, int ydt, hipStream_t s);

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
                            int mode, int bits, void* y, hipStream_t s) {
    const dim3 grid((unsigned)((M + 256 / TPR - 1) / (256 / TPR)));
    if (mode == 1)
        hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, true, false>), grid, dim3(256), 0, s, x, M, C, gamma,
                           beta, eps, bits, y);
    else if (mode == 2)
        hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, false, true>), grid, dim3(256), 0, s, x, M, C, gamma,
                           beta, eps, bits, y);
    else
        hipLaunchKernelGGL((layer_norm_kernel<XDT, YDT, TPR, NC, true, true>), grid, dim3(256), 0, s, x, M, C, gamma,
                           beta, eps, bits, y);
    return hipGetLastError();
}

// Lanes per row: the smallest of 8, 16, 32, 64 that keeps every lane at <= 4
// chunks (C <= 2048), else 64 lanes with up to 8 chunks (C <= 4096); 64
// lanes whenever that smallest choice would launch fewer than 256
// workgroups (a batch-1 forward: 197 rows), so the launch spreads over the
// CUs and each lane's chain of loads and reductions is shorter.
// mode: 1 LayerNorm, 2 activation quantization, 3 both.
template <int XDT, int YDT>
static hipError_t ln_go(const void* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                        int mode, int bits, void* y, hipStream_t s) {
    const int nch = C / 8;
    const int tpr = nch <= 32 ? 8 : nch <= 64 ? 16 : nch <= 128 ? 32 : 64;
    if (nch <= 256 && tpr < 64 && M * tpr < 256 * 256)
        return ln_launch<XDT, YDT, 64, 4>(x, M, C, gamma, beta, eps, mode, bits, y, s);
    if (nch <= 32) return ln_launch<XDT, YDT, 8, 4>(x, M, C, gamma, beta, eps, mode, bits, y, s);
    if (nch <= 64) return ln_launch<XDT, YDT, 16, 4>(x, M, C, gamma, beta, eps, mode, bits, y, s);
    if (nch <= 128) return ln_launch<XDT, YDT, 32, 4>(x, M, C, gamma, beta, eps, mode, bits, y, s);
    if (nch <= 256) return ln_launch<XDT, YDT, 64, 4>(x, M, C, gamma, beta, eps, mode, bits, y, s);
    return ln_launch<XDT, YDT, 64, 8>(x, M, C, gamma, beta, eps, mode, bits, y, s);
}

template <int XDT>
static hipError_t ln_y(const void* x, int64_t M, int C, const float* gamma, const float* beta, float eps, int mode,
                       int bits, void* y, int ydt, hipStream_t s) {
    switch (ydt) {
        case RPFQ_F32: return ln_go<XDT, RPFQ_F32>(x, M, C, gamma, beta, eps, mode, bits, y, s);
        case RPFQ_F16: return ln_go<XDT, RPFQ_F16>(x, M, C, gamma, beta, eps, mode, bits, y, s);
        default: return ln_go<XDT, RPFQ_BF16>(x, M, C, gamma, beta, eps, mode, bits, y, s);
    }
}

static hipError_t row_op(const void* x, int xdt, int64_t M, int64_t C, const float* gamma, const float* beta,
                         float eps, int mode, int bits, void* y, int ydt, hipStream_t s) {
    switch (xdt) {
        case RPFQ_F32: return ln_y<RPFQ_F32>(x, M, (int)C, gamma, beta, eps, mode, bits, y, ydt, s);
        case RPFQ_F16: return ln_y<RPFQ_F16>(x, M, (int)C, gamma, beta, eps, mode, bits, y, ydt, s);
        default: return ln_y<RPFQ_BF16>(x, M, (int)C, gamma, beta, eps, mode, bits, y, ydt, s);
    }
}

hipError_t launch_layer_norm(const void* x, int xdt, int64_t M, int64_t C, const float* gamma, const float* beta,
                             float eps, int bits, void* y, int ydt, hipStream_t s) {
    return row_op(x, xdt, M, C, gamma, beta, eps, bits > 0 ? 3 : 1, bits, y, ydt, s);
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
