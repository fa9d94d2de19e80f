// Device helpers shared by the HIP kernel translation units: codebooks,
// element I/O, the fused-coefficient decode and the LUT builders.
//
// Arithmetic order of the decoded coefficients follows the reference exactly
// (RPFQ-ViT-main/quant_models/quant_i.py:111-118 stage sums, :534-544
// recombination) so the float32 coefficient is bit-identical to A_q; it is
// rounded once to fp16 for the MFMA.
#pragma once

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
static __constant__ float kPskCos[16] = {1.0f,    PSK_C1,  PSK_R2,  PSK_S1,  0.0f,    -PSK_S1, -PSK_R2, -PSK_C1,
                                  -1.0f,   -PSK_C1, -PSK_R2, -PSK_S1, 0.0f,    PSK_S1,  PSK_R2,  PSK_C1};
static __constant__ float kPskSin[16] = {0.0f,    PSK_S1,  PSK_R2,  PSK_C1,  1.0f,    PSK_C1,  PSK_R2,  PSK_S1,
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
// 16-PSK unit value e^{i pi idx / 8} from the octant constants by selects
// (no memory access): r = idx & 3 within the quadrant, q = idx >> 2 quarter
// turns.  Negation as 0 - v keeps the zeros +0, so every value equals
// (kPskCos[idx], kPskSin[idx]) bit for bit.
__device__ __forceinline__ float2 psk16_unit(uint32_t idx) {
    const uint32_t r = idx & 3u, q = (idx >> 2) & 3u;
    const float c = r == 0 ? 1.0f : r == 1 ? PSK_C1 : r == 2 ? PSK_R2 : PSK_S1;
    const float s = r == 0 ? 0.0f : r == 1 ? PSK_S1 : r == 2 ? PSK_R2 : PSK_C1;
    float2 v;
    v.x = q == 0 ? c : q == 1 ? 0.0f - s : q == 2 ? 0.0f - c : s;
    v.y = q == 0 ? s : q == 1 ? c : q == 2 ? 0.0f - s : 0.0f - c;
    return v;
}

template <int CB>
__device__ __forceinline__ float2 lut_entry(uint32_t idx, float4 p) {
    if (CB == RPFQ_CB_PSK16) {
        const float2 u = psk16_unit(idx);
        return make_float2(p.x * u.x, p.x * u.y);
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

// lut_entry(even + g, p) for g in {0, 1}: the LUT builders' index pattern
// (lane half g, unrolled even offset).  16-PSK picks between the two unit
// values of the even offset, which fold to constants when it is known.
template <int CB>
__device__ __forceinline__ float2 lut_entry_g(uint32_t even, int g, float4 p) {
    if (CB == RPFQ_CB_PSK16) {
        const float2 ue = psk16_unit(even), uo = psk16_unit(even + 1);
        const float2 u = g ? uo : ue;
        return make_float2(p.x * u.x, p.x * u.y);
    }
    return lut_entry<CB>(even + (uint32_t)g, p);
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

// float32 -> bf16 by gfx950's v_cvt_pk_bf16_f32: round to nearest even, NaN
// kept quiet with its sign and top payload bits, i.e. bit for bit
//   u += 0x7fff + ((u >> 16) & 1), u >> 16   (NaN: (u >> 16) | 0x40)
// for every float32 bit pattern (checked exhaustively on the device).
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// two bf16 in one instruction: lo in bits 0-15, hi in bits 16-31
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){lo, hi}, bf16x2v));
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
    return pack_bf2(lo, hi);
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

// Exact GELU (approximate = 'none') in float32 by the formula of torch's
// GELU kernel, x * 0.5 * (1 + erf(x * sqrt(1/2))): the GELU + act-quant row
// kernel, whose quantized values are bit-exact with torch's GELU followed by
// the reference's act quant.  The empty asm keeps the float32 result: without
// it the backend may fold the last multiply and a following fp16 conversion
// into one v_fma_mixlo_f16 (a single rounding).
__device__ __forceinline__ float gelu_f(float x) {
    float g = x * 0.5f * (1.0f + erff(x * 0.707106781186547524f));
    asm volatile("" : "+v"(g));
    return g;
}

// Fused activation of the GEMM stores (WideArgs::act = 1), applied to the
// output already rounded to y's dtype and rounded again by the store:
// GELU(x) = x Phi(x), ~20 VALU (2 transcendental)
// against ~40-60 for the erff form above.  The normal tail Q(a) =
// P(X > a) = erfc(a / sqrt 2) / 2, a = |x|, is written
//   Q(a) = exp(-a^2 / 2) t S(t),  t = 1 / (1 + p a),
// with S a degree-7 polynomial fitted here (weighted least squares on the
// relative error, Lawson reweighting, over a in [0, 14]) to a relative
// error below 1e-7 in float64; Phi(x) = 1 - Q(a) for x >= 0, Q(a) below.
// Evaluated in float32 the GELU is within 1e-6 relative of x Phi(x) for
// x > -5 (1.8e-6 in the far tail), i.e. correctly rounded to fp16 for all
// but ~0.02% of fp16 inputs; the erff form loses relative accuracy for
// x < -3 to the cancellation in 1 + erf (0.9% of fp16 inputs round
// differently from the exact GELU there).
__device__ __forceinline__ float gelu_fast(float x) {
    constexpr float p = 0.305f;
    constexpr float s0 = 0.12163970644663864f, s1 = 0.12246733368920268f, s2 = 0.10341694433614163f,
                    s3 = 0.1210368392091385f, s4 = -0.038009486079897375f, s5 = 0.1857564848237517f,
                    s6 = -0.15301350130459096f, s7 = 0.03670572580834201f;
    const float a = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(fmaf(p, a, 1.0f));
    float sp = fmaf(s7, t, s6);
    sp = fmaf(sp, t, s5);
    sp = fmaf(sp, t, s4);
    sp = fmaf(sp, t, s3);
    sp = fmaf(sp, t, s2);
    sp = fmaf(sp, t, s1);
    sp = fmaf(sp, t, s0);
    const float e = __builtin_amdgcn_exp2f(a * a * -0.72134752044448170f);  // exp(-a^2 / 2)
    const float q = e * t * sp;
    float g = x * (x >= 0.0f ? 1.0f - q : q);
    asm volatile("" : "+v"(g));  // one rounding to y's dtype after the float32 product
    return g;
}

template <int YDT>
__device__ __forceinline__ float act_y(float v, int act) {
    if (!act) return v;
    if (YDT == RPFQ_F16) v = (float)(_Float16)v;
    if (YDT == RPFQ_BF16) v = bf16_to_f32(f32_to_bf16(v));
    return gelu_fast(v);
}
// two packed 16-bit outputs of y's dtype
__device__ __forceinline__ uint32_t gelu2_y(uint32_t v, bool f16) {
    if (f16) {
        const half2v h = __builtin_bit_cast(half2v, v);
        const half2v o = {(_Float16)gelu_fast((float)h.x), (_Float16)gelu_fast((float)h.y)};
        return __builtin_bit_cast(uint32_t, o);
    }
    return pack_bf2(gelu_fast(bf16_to_f32(v & 0xffffu)), gelu_fast(bf16_to_f32(v >> 16)));
}
__device__ __forceinline__ uint4 gelu8_y(uint4 v, bool f16) {
    return make_uint4(gelu2_y(v.x, f16), gelu2_y(v.y, f16), gelu2_y(v.z, f16), gelu2_y(v.w, f16));
}
__device__ __forceinline__ uint16_t gelu1_y(uint16_t e, bool f16) {
    if (f16) return __builtin_bit_cast(uint16_t, (_Float16)gelu_fast((float)__builtin_bit_cast(_Float16, e)));
    return f32_to_bf16(gelu_fast(bf16_to_f32(e)));
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
            u = lut_entry_g<CB>(2 * j, g, pu);
            w = lut_entry_g<CB>(2 * j, g, pw);
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

// ---------------------------------------------------------------------------
// per-row prescale of float32 / bf16 activations (the forward's range guard)
// ---------------------------------------------------------------------------
// The MFMA takes activations as fp16, whose normal range is [2^-14, 65504].
// A float32 / bf16 row whose largest magnitude is mx is multiplied by
// s = 2^(14 - floor(log2 mx)) before that rounding, so its largest element
// lands in [2^14, 2^15), and the row's outputs are multiplied by 1/s
// (exact) before the bias.  Power-of-two factors commute with every
// rounding that stays inside the formats' ranges (the fp16 conversion, the
// exact fp16 products, the float32 accumulation), so a row that already
// fits gives bit for bit the unscaled result, and any other row keeps the
// relative accuracy of one that fits.  The exponent is clamped to
// [-126, 126] (max|x| in [2^-112, 2^140) scales exactly); zero, NaN and
// infinite maxima keep s = 1.
__device__ __forceinline__ float row_prescale(float mx) {
    if (!(mx > 0.0f) || !(mx <= 3.40282347e38f)) return 1.0f;
    int k = 15 - __builtin_amdgcn_frexp_expf(mx);  // frexp: mx = f 2^e, f in [0.5, 1)
    k = k < -126 ? -126 : (k > 126 ? 126 : k);
    return __builtin_amdgcn_ldexpf(1.0f, k);
}
// 1 / s for a prescale s (a power of two in [2^-126, 2^126]): exact.
__device__ __forceinline__ float row_unscale(float s) { return 1.0f / s; }

// Sum / maximum over the TPR consecutive lanes of a row group (a butterfly:
// every lane of the group ends with the same value).
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

// LDS address-space views and the LDS byte address of a shared pointer.
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
// read); every consumer waits explicitly (s_waitcnt vmcnt, and s_barrier
// when another wave reads the destination) before reading it.  The
// compiler's own waits stay correct: loads it does not count only make
// them wait longer.
__device__ __forceinline__ void dma_dwordx4(const void* gbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(gbase) : "memory", "m0");
}

// LDS DMA of one dword per lane (lane l: 4 B from gbase + voff[l] to lds + 4 l).
__device__ __forceinline__ void dma_dword(const void* gbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff), "s"(gbase) : "memory", "m0");
}

}  // namespace rpfq
