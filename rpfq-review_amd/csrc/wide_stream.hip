// Widely-linear layer for small M: weight streaming.  Compiled once per
// codebook (RPFQ_CB_SEL).
#include "rpfq_device.h"

#ifndef RPFQ_CB_SEL
#error "compile once per codebook with -DRPFQ_CB_SEL=<RPFQ_CB_*>"
#endif

namespace rpfq {



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
            u = lut_entry_g<CB>((uint32_t)(2 * (j0 + jj)), g, pu);
            w = lut_entry_g<CB>((uint32_t)(2 * (j0 + jj)), g, pw);
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

// The same LUT (or the NJ-index share from j0 on) from the row's
// parameters already in registers (not TABLE).
template <int CB, int NJ = 8>
__device__ __forceinline__ void build_lut_sk_regs(uint32_t* lut, float4 pu, float4 pw, const RotParams& rot, int R,
                                                  int g, int j0 = 0) {
    const int s0 = 32 * (R >> 4) + (R & 15);
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
        const uint32_t idx = (uint32_t)(g + 2 * (j0 + jj));
        float2 u = lut_entry_g<CB>((uint32_t)(2 * (j0 + jj)), g, pu);
        float2 w = lut_entry_g<CB>((uint32_t)(2 * (j0 + jj)), g, pw);
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

// 8 activations of a 16-B chunk (fp16 or bf16) as float32.
template <int XDT>
__device__ __forceinline__ void chunk_f32(uint4 v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (XDT == RPFQ_BF16) {
            f[2 * i] = bf16_to_f32(w[i] & 0xffffu);
            f[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        } else {
            const half2v h = __builtin_bit_cast(half2v, w[i]);
            f[2 * i] = (float)h.x;
            f[2 * i + 1] = (float)h.y;
        }
    }
}

// 4 consecutive activations at element offset `off`: the raw 16-bit values
// (fp16, bf16; converted at use so the load stays in flight) or, for
// float32, 4 fp16 converted on load after the row's prescale xs (exact).
template <int XDT>
__device__ __forceinline__ uint2 load4_raw(const void* base, int64_t off, float xs) {
    if (XDT != RPFQ_F32) return *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(base) + off);
    const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
    return make_uint2(pack_h2(f.x * xs, f.y * xs), pack_h2(f.z * xs, f.w * xs));
}
template <int XDT>
__device__ __forceinline__ uint2 raw4_f16(uint2 v, float xs) {
    if (XDT != RPFQ_BF16) return v;
    return make_uint2(pack_h2(bf16_to_f32(v.x & 0xffffu) * xs, bf16_to_f32(v.x >> 16) * xs),
                      pack_h2(bf16_to_f32(v.y & 0xffffu) * xs, bf16_to_f32(v.y >> 16) * xs));
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
// LN, the row prologue (NW = 4, per-row scales, K' % 32 == 0, K' <=
// kLnMaxK, fp16 / bf16 x, not TABLE): the workgroup first prepares its 16
// rows of x -- nn.LayerNorm over the 2K' features (a.ln; float32, two
// passes) and / or the activation fake quantization of each half
// (a.aq_bits), rounded to x's dtype as the separate row kernels round their
// output -- into an LDS tile [16][2K' + 4] fp16, which the k-steps then read
// instead of x.  Rows past M are zero rows (never stored).
template <int XDT, int YDT, int CB, bool PB, bool KT, int NW, bool LN = false>
__global__ void __launch_bounds__(64 * NW, LN ? 2 : RPFQ_SK_OCC) wide_linear_skinny_kernel(WideArgs a) {
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
    // prescale of this lane's x row (float32 / bf16 x with a.xs, else 1); the
    // row prologue computes its own from the prepared rows (xs_tile below)
    const float xsl = (XDT != RPFQ_F16 && !LN && a.xs) ? a.xs[m0 + (m_ok ? r16 : M - 1)] : 1.0f;
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
        if (LN) return;  // activations from the normalized LDS tile
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (KT) {
                const int col = 32 * kc + xcol + 8 * t;
                const int off = xoff - xcol + (col < K ? col : 0);  // K' tail: in bounds, zeroed at use
                st.xr[t] = load4_raw<XDT>(xc, off, xsl);
                st.xi[t] = load4_raw<XDT>(xc, off + K, xsl);
            } else {
                const int64_t xb = 32 * (int64_t)kc + 8 * t;
                st.xr[t] = load4_raw<XDT>(xc, xb + xoff, xsl);
                st.xi[t] = load4_raw<XDT>(xc, xb + K + xoff, xsl);
            }
        }
    };
    // Row prologue tile (LN): rows of xsb bytes after the LUT and the
    // split-K partials.  Wave w prepares rows RW w .. RW w + RW - 1 of the
    // chunk, each with all 64 lanes, lane l holding chunks l + 64 j: the
    // LayerNorm / act-quant row kernel's lane order at 64 lanes per row (its
    // choice for every launch this kernel fuses), so the statistics, the
    // per-half maxima and every value after them are bit-identical to
    // rpfq_layer_norm / rpfq_layer_norm_act_quant / rpfq_act_quant.
    const int C2 = 2 * K, nch = C2 / 8;
    const int xsb = 2 * C2 + 8;  // the 8-B pad puts consecutive rows 2 banks apart
    char* xtile = smem + sk_lds(NW);
    // (LN, bf16 x) the prepared rows' prescales, [16] floats after the tile
    float* xs_tile = reinterpret_cast<float*>(xtile + 16 * xsb);
    constexpr int RW = 16 / NW;                                  // (LN) rows per wave
    constexpr int NCP = LN ? (2 * kLnMaxK / 8 + 63) / 64 : 1;    // chunks per lane and row
    uint4 lnv[RW][NCP];
    float4 gv[NCP][2], bv[NCP][2];
    float4 prm[2];
    if (LN) {  // requested before the code ring: their waits leave the codes in flight
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int row = wave * RW + i;
#pragma unroll
            for (int j = 0; j < NCP; ++j) {
                const int c = lane + 64 * j;
                lnv[i][j] = (c < nch && row < M)
                                ? *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(xc) + row * C2 + 8 * c)
                                : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < NCP; ++j) {
            const int c = lane + 64 * j;
            const bool ok = a.ln && c < nch;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                gv[j][t] = (ok && a.ln_gamma) ? reinterpret_cast<const float4*>(a.ln_gamma)[2 * c + t]
                                              : make_float4(1, 1, 1, 1);
                bv[j][t] = (ok && a.ln_beta) ? reinterpret_cast<const float4*>(a.ln_beta)[2 * c + t]
                                             : make_float4(0, 0, 0, 0);
            }
        }
        const float4* pp = a.params + ((int64_t)tile * 32 + R) * 2;
        prm[0] = pp[0];
        prm[1] = pp[1];
    }

    // The epilogue's bias and residual (wave 0, rows < M).  With split K (a
    // layer at batch 1-2, latency-bound) they are requested before the code
    // ring, so their latency overlaps the k-loop instead of following it
    // (ViT-B/16 batch-1 forward -1%); one wave per tile (many tiles, where
    // occupancy hides the epilogue) loads them at the end, keeping the
    // registers.  The residual read stays before this lane's own store of the
    // same elements, so y may alias it.
    const int64_t ldy = 2 * (int64_t)a.N;
    const bool epi = (NW == 1 || wave == 0) && m_ok;
    float eb[2][2][4];  // [h][re / im][v]
    uint2 er[2][2];     // [h][re / im]: 4 residual values of the vector store
    auto fetch_epi = [&]() {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t n0 = (int64_t)tile * 32 + 16 * h + 4 * q;
            const int64_t base = (m0 + r16) * ldy + n0;
            const bool vec = a.vec_store && n0 + 4 <= a.N && YDT == RPFQ_F16;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const bool ok = epi && a.bias && n0 + v < a.N;
                eb[h][0][v] = ok ? a.bias[n0 + v] : 0.0f;
                eb[h][1][v] = ok ? a.bias[a.N + n0 + v] : 0.0f;
            }
            const bool rv = epi && vec && a.res;
            er[h][0] = rv ? *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.res) + base)
                          : make_uint2(0, 0);
            er[h][1] = rv ? *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(a.res) + base + a.N)
                          : make_uint2(0, 0);
        }
    };
    if (NW > 1) fetch_epi();

    // float32 x holds twice the bytes per ring slot: half the distance keeps
    // the ring in registers
    constexpr int PF = XDT == RPFQ_F32 ? SK_PF / 2 : SK_PF;
    Step ring[PF];
#pragma unroll
    for (int i = 0; i < PF; ++i) load_step(kb + i, ring[i]);

    int blk = 0;
    if (LN) {
        // y = LayerNorm(x) (a.ln) or x, float32, per row i of the wave; the
        // RW rows' reductions interleave so their shuffle chains overlap
        float mean[RW], rstd[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            mean[i] = 0.0f;
            rstd[i] = 1.0f;
        }
        if (a.ln) {
            float sum[RW], s2[RW];
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                sum[i] = 0.0f;
#pragma unroll
                for (int j = 0; j < NCP; ++j) {
                    if (lane + 64 * j < nch) {
                        float f[8];
                        chunk_f32<XDT>(lnv[i][j], f);
#pragma unroll
                        for (int e = 0; e < 8; ++e) sum[i] += f[e];
                    }
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
                for (int i = 0; i < RW; ++i) sum[i] += __shfl_xor(sum[i], o, 64);
            }
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                mean[i] = sum[i] / (float)C2;
                s2[i] = 0.0f;
#pragma unroll
                for (int j = 0; j < NCP; ++j) {
                    if (lane + 64 * j < nch) {
                        float f[8];
                        chunk_f32<XDT>(lnv[i][j], f);
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const float d = f[e] - mean[i];
                            s2[i] += d * d;
                        }
                    }
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
                for (int i = 0; i < RW; ++i) s2[i] += __shfl_xor(s2[i], o, 64);
            }
#pragma unroll
            for (int i = 0; i < RW; ++i) rstd[i] = 1.0f / sqrtf(s2[i] / (float)C2 + a.ln_eps);
        }
        build_lut_sk_regs<CB, 8 / NW>(lut, prm[0], prm[1], a.rot, R, g, (8 / NW) * wave);  // this wave's share
        auto value = [&](int i, int j, float* y) {
            chunk_f32<XDT>(lnv[i][j], y);
            if (a.ln) {
                const float gk[8] = {gv[j][0].x, gv[j][0].y, gv[j][0].z, gv[j][0].w,
                                     gv[j][1].x, gv[j][1].y, gv[j][1].z, gv[j][1].w};
                const float bk[8] = {bv[j][0].x, bv[j][0].y, bv[j][0].z, bv[j][0].w,
                                     bv[j][1].x, bv[j][1].y, bv[j][1].z, bv[j][1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = (y[e] - mean[i]) * rstd[i] * gk[e] + bk[e];
            }
        };
        // activation fake quantization (a.aq_bits): per row and half, scale
        // = qmax * (1 / max(max|y|, 1e-5)), y_q = clamp(rint(y scale)) / scale;
        // for <= 4 bits the quotients of the 16 levels are divided once per
        // row (lane l < 32: level (l & 15) - 8 of half l >> 4) and fetched
        // with ds_bpermute, which every lane takes part in (lanes past the
        // row's chunks hold zeros and store nothing)
        const int bits = a.aq_bits;
        const float qmax = (float)((1 << (bits - 1)) - 1), qmin = -(float)(1 << (bits - 1));
        const int half_ch = nch >> 1;
        float sc0[RW], sc1[RW];
        int tvb[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            sc0[i] = sc1[i] = 1.0f;
            tvb[i] = 0;
        }
        if (bits) {
            float m0[RW], m1[RW];
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                m0[i] = m1[i] = 0.0f;
#pragma unroll
                for (int j = 0; j < NCP; ++j) {
                    const int c = lane + 64 * j;
                    if (c < nch) {
                        float y[8];
                        value(i, j, y);
                        float mx = 0.0f;
#pragma unroll
                        for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(y[e]));
                        if (c < half_ch) m0[i] = fmaxf(m0[i], mx); else m1[i] = fmaxf(m1[i], mx);
                    }
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
                for (int i = 0; i < RW; ++i) {
                    m0[i] = fmaxf(m0[i], __shfl_xor(m0[i], o, 64));
                    m1[i] = fmaxf(m1[i], __shfl_xor(m1[i], o, 64));
                }
            }
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                // torch evaluates `float(qmax) / tensor` as reciprocal(tensor) * qmax
                sc0[i] = (1.0f / fmaxf(m0[i], 1e-5f)) * qmax;
                sc1[i] = (1.0f / fmaxf(m1[i], 1e-5f)) * qmax;
                tvb[i] = __float_as_int((float)((lane & 15) - 8) / ((lane & 16) ? sc1[i] : sc0[i]));
            }
        }
        const bool table = bits > 0 && bits <= 4;
        // the prepared value of chunk j of row i: LayerNorm / act quant, and
        // for bf16 x the rounding to x's dtype (every lane calls it: the
        // ds_bpermute reads take all lanes)
        auto prepared = [&](int i, int j, float* y) {
            const int c = lane + 64 * j;
            value(i, j, y);
            if (bits) {
                const bool hi = c >= half_ch;
                const float sc = hi ? sc1[i] : sc0[i];
                float qv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) qv[e] = fminf(fmaxf(rintf(y[e] * sc), qmin), qmax);
                if (table) {
                    int d[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        d[e] = __builtin_amdgcn_ds_bpermute(((hi ? 16 : 0) + (int)qv[e] + 8) << 2, tvb[i]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) y[e] = copysignf(__int_as_float(d[e]), qv[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) y[e] = qv[e] / sc;
                }
            }
            if (XDT == RPFQ_BF16) {  // rounded to x's dtype (then exactly to fp16 for the MFMA)
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] = bf16_to_f32(f32_to_bf16(y[e]));
            }
        };
        // bf16 x: each prepared row takes the range guard's prescale of its
        // largest magnitude before the fp16 conversion, as rpfq_row_scales
        // and rpfq_wide_linear_scaled apply it to the row kernel's bf16
        // output (a first pass for the maxima; fp16 x is rounded directly)
        float rs[RW];
#pragma unroll
        for (int i = 0; i < RW; ++i) rs[i] = 1.0f;
        if (XDT == RPFQ_BF16) {
            float mx[RW];
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                mx[i] = 0.0f;
#pragma unroll
                for (int j = 0; j < NCP; ++j) {
                    float y[8];
                    prepared(i, j, y);
                    if (lane + 64 * j < nch) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) mx[i] = fmaxf(mx[i], fabsf(y[e]));
                    }
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
                for (int i = 0; i < RW; ++i) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], o, 64));
            }
#pragma unroll
            for (int i = 0; i < RW; ++i) {
                rs[i] = row_prescale(mx[i]);
                if (lane == 0) xs_tile[wave * RW + i] = rs[i];
            }
        }
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int row = wave * RW + i;
#pragma unroll
            for (int j = 0; j < NCP; ++j) {
                const int c = lane + 64 * j;
                float y[8];
                prepared(i, j, y);
                uint32_t o[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) o[t] = row < M ? cvt_pk(y[2 * t] * rs[i], y[2 * t + 1] * rs[i]) : 0u;
                if (c < nch) *reinterpret_cast<uint4*>(xtile + row * xsb + 16 * c) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    } else {  // split K: each wave builds 1 / NW of the shared LUT
        const float4* p = a.params + ((int64_t)tile * 32 + R) * (CB == RPFQ_CB_TABLE ? 16 : a.nblk * 2);
        if (NW == 1)
            build_lut_sk<CB>(lut, p, a.rot, R, g);
        else
            build_lut_sk<CB, 8 / NW>(lut, p, a.rot, R, g, (8 / NW) * wave);
    }
    if (NW > 1) {  // LUT (and the LN tile) written before any wave reads it; the code loads stay in flight
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
            uint2 re, im;
            if (LN) {  // row r16 of the normalized tile (fp16)
                const char* rp = xtile + r16 * xsb + (32 * ks + xcol + 8 * t) * 2;
                re = *reinterpret_cast<const uint2*>(rp);
                im = *reinterpret_cast<const uint2*>(rp + 2 * K);
            } else {
                re = raw4_f16<XDT>(st.xr[t], xsl);
                im = raw4_f16<XDT>(st.xi[t], xsl);
            }
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
    // Whole groups of PF k-steps with a uniform guard around the compute
    // and each ring slot reloaded after its k-step is consumed: the slots keep
    // their registers across iterations (no copies, whose waits would drain
    // every load in flight), and each wait is for the oldest loads only.
    for (int ks0 = kb; ks0 < ke; ks0 += PF) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            const int ks = ks0 + i;
            if (ks < ke) {
                if (PB) {  // per-(row, block) scales: new LUT at each block start
                    const int nb = ks / a.block_ks;
                    if (nb != blk) {
                        blk = nb;
                        const float4* p = a.params + (((int64_t)tile * 32 + R) * a.nblk + nb) * 2;
                        build_lut_sk<CB>(lut, p, a.rot, R, g);
                    }
                }
                compute(ks, ring[i]);
            }
            load_step(ks + PF, ring[i]);  // past the end: reloads the last k-step, unused
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
    if (NW == 1) fetch_epi();
    // undo the row's prescale (exact; 1 without one) before the bias
    const float inv = row_unscale((LN && XDT == RPFQ_BF16) ? xs_tile[r16] : xsl);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t n0 = (int64_t)tile * 32 + 16 * h + 4 * q;
        float vr[4], vi[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            vr[v] = acc_re[h][v] * inv + eb[h][0][v];
            vi[v] = acc_im[h][v] * inv + eb[h][1][v];
        }
        const int64_t base = (m0 + r16) * ldy + n0;
        if (a.vec_store && n0 + 4 <= a.N && YDT == RPFQ_F16) {
            uint2 hr = make_uint2(cvt_pk(vr[0], vr[1]), cvt_pk(vr[2], vr[3]));
            uint2 hi = make_uint2(cvt_pk(vi[0], vi[1]), cvt_pk(vi[2], vi[3]));
            if (a.res) {
                hr = make_uint2(add2_y(hr.x, er[h][0].x, true), add2_y(hr.y, er[h][0].y, true));
                hi = make_uint2(add2_y(hi.x, er[h][1].x, true), add2_y(hi.y, er[h][1].y, true));
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

// ---------------------------------------------------------------------------
// widely-linear layer for M <= 8: weight streaming with re / im as B columns
// ---------------------------------------------------------------------------
// The same code stream and LUT as above, but the fused coefficients A11 ..
// A22 are never formed: the U and W values of a complex column take separate
// k slots of the A operand, [Ure, Uim, Wre, Wim], and the real and the
// imaginary output of x row m are the B columns 2m and 2m + 1:
//   column 2m:     [ xr, -xi,  xr, xi ]  Ure xr - Uim xi + Wre xr + Wim xi = Re(U x + W conj(x))
//   column 2m + 1: [ xi,  xr, -xi, xr ]  Ure xi + Uim xr - Wre xi + Wim xr = Im(U x + W conj(x))
// so a code byte costs two address permutes and two LUT reads, and the sums
// U + W run on the matrix pipe (products of fp16 values are exact in the
// float32 accumulator, where the fused kernels round U + W to fp16 first).
// The B operands depend on x only and are shared by the H row groups.
//   * lane (r16, q) holds the code dwords t = 0, 1 of rows 16 h + r16 as the
//     kernel above (complex columns cq + 8 t + e, cq = 16 (q & 1) + 4 (q >> 1),
//     e = 0..3); MFMA j = 0..3 takes bytes 2 (j & 1) and 2 (j & 1) + 1 of
//     dword t = j >> 1, columns c0 and c0 + 1: A = [U(c0), W(c0), U(c0+1),
//     W(c0+1)].
//   * lane (col = r16, q) of B reads x row min(col / 2, M - 1), columns
//     cq + 8 t .. cq + 8 t + 3, as L1 = re, L2 = im for an even col and
//     swapped for an odd one, so each (L1, L2) pair of a column is one
//     permute with a uniform selector and the two sign patterns are per-lane
//     XOR masks.
//   * H = 2: one packed 32-row tile per workgroup; H = 4: two consecutive
//     tiles (the last one clamped when NT is odd), their LUTs 8 KB apart.
//   * NW = 2 or 4 waves split K and share the LUT (each builds its share),
//     wave 0 adding the partial sums through LDS in a fixed order.
#ifndef RPFQ_GV_OCC
#define RPFQ_GV_OCC 4
#endif
constexpr int GV_XPF = 2;  // prefetch distance of the activations (L2-resident) in k-steps
static_assert(SK_PF % GV_XPF == 0, "the activation ring must divide the code ring");
constexpr int gv_lds(int h, int nw) { return (h / 2) * kSkLut + (nw - 1) * h * 4 * 64 * 4; }

template <int XDT>
__device__ __forceinline__ uint32_t raw2_f16(uint32_t v, float xs) {
    if (XDT != RPFQ_BF16) return v;
    return pack_h2(bf16_to_f32(v & 0xffffu) * xs, bf16_to_f32(v >> 16) * xs);
}

// Lane constants of the column-split kernels.
struct GvLane {
    int r16, q, R, g;
    int coff;             // uint2 index of the lane's codes in a 16-row block
    int p, xrow, cq;      // B lane: part p of x row xrow / 2K, columns cq + 8 t ..
    int off1, off2;       // element offsets of L1 (part p) and L2 (the other part)
    uint32_t m0, m1;      // sign masks of the B dwords (re / im column)
    uint32_t slot0;       // LUT slot of the lane's row in byte 0 of an address
    float xs;             // prescale of the lane's x row (float32 / bf16 x with a.xs, else 1)
};
__device__ __forceinline__ GvLane gv_lane(int lane, int M, int K) {
    GvLane l;
    l.r16 = lane & 15;
    l.q = lane >> 4;
    l.R = lane & 31;
    l.g = lane >> 5;
    l.coff = l.r16 * 4 + l.q;
    l.p = l.r16 & 1;
    l.xrow = min(l.r16 >> 1, M - 1) * 2 * K;
    l.cq = 16 * (l.q & 1) + 4 * (l.q >> 1);
    l.off1 = l.xrow + (l.p ? K : 0) + l.cq;
    l.off2 = l.xrow + (l.p ? 0 : K) + l.cq;
    l.m0 = l.p ? 0u : 0x80000000u;
    l.m1 = l.p ? 0x00008000u : 0u;
    l.slot0 = (uint32_t)(16 * (l.q & 1) + l.r16) * 4;
    l.xs = 1.0f;
    return l;
}

// Activations of k-step ks (raw 16-bit or fp16-converted float32), [t][L1, L2].
template <int XDT, bool KT>
__device__ __forceinline__ void gv_load_x(const WideArgs& a, const GvLane& l, int ks, uint2* xv) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int col = 32 * ks + 8 * t;
        const bool in = !KT || col + l.cq < a.K;  // K' tail: the row's first columns, zeroed at use
        xv[2 * t] = load4_raw<XDT>(a.x, in ? l.off1 + col : l.xrow, l.xs);
        xv[2 * t + 1] = load4_raw<XDT>(a.x, in ? l.off2 + col : l.xrow, l.xs);
    }
}

// One k-step: B operands from the activations, LUT reads of the H row
// groups' U and W values, 4 x H MFMAs (acc[h * NA + j % NA]).
template <int XDT, bool KT, int H, int NA>
__device__ __forceinline__ void gv_kstep(floatx4* acc, const GvLane& l, int ks, int K, const uint2* c,
                                         const uint2* xv) {
    // L1 / L2 dword j: columns c0, c0 + 1 of MFMA j
    const uint32_t l1[4] = {xv[0].x, xv[0].y, xv[2].x, xv[2].y};
    const uint32_t l2[4] = {xv[1].x, xv[1].y, xv[3].x, xv[3].y};
    half8 bx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t u1 = raw2_f16<XDT>(l1[j], l.xs), u2 = raw2_f16<XDT>(l2[j], l.xs);
        const uint32_t p0 = __builtin_amdgcn_perm(u2, u1, 0x05040100u);
        const uint32_t p1 = __builtin_amdgcn_perm(u2, u1, 0x07060302u);
        uint4 b = make_uint4(p0 ^ l.m0, p0 ^ l.m1, p1 ^ l.m0, p1 ^ l.m1);
        if (KT && 32 * ks + l.cq + 8 * (j >> 1) >= K) b = make_uint4(0, 0, 0, 0);
        bx[j] = as_half8(b);
    }
    // index nibbles of every row group, then the MFMAs j-major so that
    // consecutive ones accumulate into different row groups
    uint32_t pu[H][2], pw[H][2];
#pragma unroll
    for (int h = 0; h < H; ++h) {
        pu[h][0] = c[h].x & 0x0f0f0f0fu;
        pw[h][0] = (c[h].x >> 4) & 0x0f0f0f0fu;
        pu[h][1] = c[h].y & 0x0f0f0f0fu;
        pw[h][1] = (c[h].y >> 4) & 0x0f0f0f0fu;
    }
    auto reads = [&](int j, uint32_t (&av)[H][4]) {
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const uint32_t slot = l.slot0 + 128 * (h & 1);
            const int rg = (h >> 1) * (kSkLut / 4);  // LUT of the h-th tile, in dwords
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t sel = 0x03020000u | ((4u + 2 * (j & 1) + e) << 8);
                av[h][2 * e] = *((lds_u32_t)__builtin_amdgcn_perm(pu[h][j >> 1], slot, sel) + rg);
                av[h][2 * e + 1] = *((lds_u32_t)__builtin_amdgcn_perm(pw[h][j >> 1], slot, sel) + rg + 16 * 64);
            }
        }
    };
    // LUT reads of MFMA j + 1 are issued before the MFMAs of j, so each
    // group of MFMAs waits only for reads issued a group earlier
    uint32_t av[2][H][4];
    reads(0, av[0]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (j < 3) reads(j + 1, av[(j + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < H; ++h)
            acc[h * NA + (j % NA)] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                as_half8(make_uint4(av[j & 1][h][0], av[j & 1][h][1], av[j & 1][h][2], av[j & 1][h][3])), bx[j],
                acc[h * NA + (j % NA)], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Epilogue: lane (col = r16, q) holds part p of x row m = col / 2 for the
// outputs n = 32 tile0 + 16 h + 4 q + v; rows past M and outputs past N'
// store nothing.
template <int YDT, int H>
__device__ __forceinline__ void gv_store(const WideArgs& a, const GvLane& l, const floatx4* acc, int tile0, int M) {
    const int m = l.r16 >> 1;
    if (m >= M) return;
    const int64_t ldy = 2 * (int64_t)a.N;
#pragma unroll
    for (int h = 0; h < H; ++h) {
        const int64_t n0 = (int64_t)tile0 * 32 + 16 * h + 4 * l.q;
        if (n0 >= a.N) continue;
        const int64_t base = m * ldy + (l.p ? a.N : 0) + n0;
        const float* bias = a.bias ? a.bias + (l.p ? a.N : 0) : nullptr;
        float v4[4];
        const float inv = row_unscale(l.xs);  // undo the row's prescale (exact) before the bias
#pragma unroll
        for (int v = 0; v < 4; ++v) v4[v] = acc[h][v] * inv + ((bias && n0 + v < a.N) ? bias[n0 + v] : 0.0f);
        if (a.vec_store && n0 + 4 <= a.N && YDT == RPFQ_F16) {
            uint2 o = make_uint2(cvt_pk(v4[0], v4[1]), cvt_pk(v4[2], v4[3]));
            if (a.res) o = add_res4<YDT>(o, a.res, base);
            if (a.act) o = make_uint2(gelu2_y(o.x, true), gelu2_y(o.y, true));
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.y) + base) = o;
        } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (n0 + v < a.N)
                    store1<YDT>(a.y, base + v, with_res<YDT>(act_y<YDT>(v4[v], a.act), a.res, base + v));
        }
    }
}

// LUTs of the TPG tiles from tile0 on, each wave of NW building its share
// of the 8 entry pairs per tile (clamped to the last packed tile).
template <int CB, int TPG, int NW>
__device__ __forceinline__ void gv_build_luts(uint32_t* lut, const WideArgs& a, int tile0, int wave, int R, int g) {
    constexpr int per = 8 * TPG / NW, nj = per < 8 ? per : 8;
#pragma unroll
    for (int f = 0; f < per; f += nj) {
        const int f0 = wave * per + f, region = f0 >> 3;
        const int tile = min(tile0 + region, a.NT - 1);
        const float4* pp = a.params + ((int64_t)tile * 32 + R) * (CB == RPFQ_CB_TABLE ? 16 : a.nblk * 2);
        build_lut_sk<CB, nj>(lut + region * (kSkLut / 4), pp, a.rot, R, g, f0 & 7);
    }
}

template <int XDT, int YDT, int CB, bool KT, int NW, int H>
__global__ void __launch_bounds__(64 * NW, RPFQ_GV_OCC) wide_linear_gemv_kernel(WideArgs a) {
    static_assert(H == 2 || H == 4, "16-row groups per workgroup");
    constexpr int TPG = H / 2;  // packed 32-row tiles per workgroup
    extern __shared__ __align__(16) char smem[];
    uint32_t* lut = reinterpret_cast<uint32_t*>(smem);
    const int lane = threadIdx.x & 63;
    const int wave = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KS = a.KS;
    const int M = (int)a.M;  // 1 .. 8 (host-checked)
    GvLane l = gv_lane(lane, M, a.K);
    if (XDT != RPFQ_F16 && a.xs) l.xs = a.xs[min(l.r16 >> 1, M - 1)];
    const int chunk = (KS + NW - 1) / NW;
    const int kb = min(wave * chunk, KS), ke = min(kb + chunk, KS);  // this wave's k-steps
    const int tile0 = (int)blockIdx.x * TPG;

    // codes of tile tile0 + t (t < TPG), clamped to the last packed tile
    const uint2* ctile[TPG];
#pragma unroll
    for (int t = 0; t < TPG; ++t)
        ctile[t] = reinterpret_cast<const uint2*>(a.codes) + (int64_t)min(tile0 + t, a.NT - 1) * KS * 128;
    uint2 cring[SK_PF][H];
    uint2 xring[GV_XPF][4];
    auto clamp_ks = [&](int ks) { return ks < ke ? ks : (ke > 0 ? ke - 1 : 0); };  // past the range: unused
    auto load_codes = [&](int ks, uint2* c) {
        const int kc = clamp_ks(ks);
#pragma unroll
        for (int h = 0; h < H; ++h) c[h] = ctile[h >> 1][kc * 128 + l.coff + 64 * (h & 1)];
    };
#pragma unroll
    for (int i = 0; i < SK_PF; ++i) load_codes(kb + i, cring[i]);
#pragma unroll
    for (int i = 0; i < GV_XPF; ++i) gv_load_x<XDT, KT>(a, l, clamp_ks(kb + i), xring[i]);
    gv_build_luts<CB, TPG, NW>(lut, a, tile0, wave, l.R, l.g);
    if (NW > 1) {  // LUT written before any wave reads it; the loads stay in flight
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }

    // two accumulators per row group when H = 2 (MFMAs j even / odd), so
    // that four independent chains interleave as with H = 4
    constexpr int NA = H == 2 ? 2 : 1;
    floatx4 acc[H * NA];
#pragma unroll
    for (int h = 0; h < H * NA; ++h) acc[h] = floatx4{0, 0, 0, 0};
    // (the k-step loop of the kernel above)
    for (int ks0 = kb; ks0 < ke; ks0 += SK_PF) {
#pragma unroll
        for (int i = 0; i < SK_PF; ++i) {
            const int ks = ks0 + i;
            if (ks < ke) gv_kstep<XDT, KT, H, NA>(acc, l, ks, a.K, cring[i], xring[i % GV_XPF]);
            // the slots just consumed take k-step ks + SK_PF (ks + GV_XPF)
            load_codes(ks + SK_PF, cring[i]);
            gv_load_x<XDT, KT>(a, l, clamp_ks(ks + GV_XPF), xring[i % GV_XPF]);
        }
    }

    if (NA == 2) {
#pragma unroll
        for (int h = 0; h < H; ++h) acc[h] = acc[h * NA] + acc[h * NA + 1];
    }
    if (NW > 1) {  // waves 1 .. NW-1 hand their partial sums to wave 0
        float* red = reinterpret_cast<float*>(smem + TPG * kSkLut);
        if (wave > 0) {
#pragma unroll
            for (int h = 0; h < H; ++h)
#pragma unroll
                for (int v = 0; v < 4; ++v) red[(((wave - 1) * H + h) * 4 + v) * 64 + lane] = acc[h][v];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < NW - 1; ++w)
#pragma unroll
            for (int h = 0; h < H; ++h)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[h][v] += red[((w * H + h) * 4 + v) * 64 + lane];
    }
    gv_store<YDT, H>(a, l, acc, tile0, M);
}

// Persistent form of the one-wave column-split kernel (H = 4: two packed
// 32-row tiles, a "group", per wave) for long streams of groups below 16
// k-steps: a grid of the resident waves walks the groups; the code ring runs
// on into the next group's first k-steps while the current group's last ones
// decode, the next group's row scales are prefetched into registers and its
// LUT is built from them, so a group's start waits for no global load (the
// one-group-per-wave launch pays the LUT's scale loads and the first code
// loads at every group).  The bias and the residual of a group go to LDS by
// DMA at the group's start, so the epilogue waits for no load issued after
// the ring's (vmcnt counts in issue order: a load the epilogue waited for
// would drain the ring).  Every ring load is issued on every path, so the
// wait counts stay exact across groups; rows past M store row M - 1's values
// (the same bits).  Taken for whole groups (NT even, N' % 32 == 0),
// K' % (32 SK_PF) == 0, per-row scales, not TABLE, 16-bit y (vec_store).
__device__ __align__(16) const float kGvZeroBias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
// LDS bytes past the two LUTs: the group's bias, [part][64 outputs] float,
// and residual, [row][part][64 outputs] 16-bit
constexpr int kGpBias = 2 * 64 * 4, kGpRes = 8 * 2 * 64 * 2;
constexpr int gp_lds(bool res) { return gv_lds(4, 1) + kGpBias + (res ? kGpRes : 0); }

// Three waves per SIMD (168 VGPRs: the next group's scales and the ring
// across the group boundary do not fit 128); the 16.5-KB LDS share caps a CU
// at 9 such waves anyway.
template <int XDT, int YDT, int CB, bool RES>
__global__ void __launch_bounds__(64, 3) wide_linear_gemv_persist_kernel(WideArgs a) {
    constexpr int H = 4, TPG = 2, GN = 64;  // row groups, tiles and output rows per group
    extern __shared__ __align__(16) char smem[];
    uint32_t* lut = reinterpret_cast<uint32_t*>(smem);
    const float* bias_s = reinterpret_cast<const float*>(smem + gv_lds(H, 1));
    const uint16_t* res_s = reinterpret_cast<const uint16_t*>(smem + gv_lds(H, 1) + kGpBias);
    const int lane = threadIdx.x & 63;
    const int KS = a.KS;
    const int M = (int)a.M;  // 1 .. 8 (host-checked)
    GvLane l = gv_lane(lane, M, a.K);
    if (XDT != RPFQ_F16 && a.xs) l.xs = a.xs[min(l.r16 >> 1, M - 1)];
    const int groups = a.NT / TPG, gs = (int)gridDim.x;
    int grp = (int)blockIdx.x;
    const int64_t tile_u2 = (int64_t)KS * 128;  // uint2 of codes per tile
    // step s of group gg: its own for s < KS, else step s - KS of the next
    // group of this wave (past the last group: the last step again)
    auto load_codes = [&](int gg, int s, uint2* c) {
        int g2 = gg, k = s;
        if (s >= KS) {
            g2 = gg + gs;
            k = s - KS;
            if (g2 >= groups) {
                g2 = gg;
                k = KS - 1;
            }
        }
        const uint2* base = reinterpret_cast<const uint2*>(a.codes) + (int64_t)(TPG * g2) * tile_u2 + k * 128;
#pragma unroll
        for (int h = 0; h < H; ++h) c[h] = base[(h >> 1) * tile_u2 + l.coff + 64 * (h & 1)];
    };
    // (pu, pw) of this lane's LUT row in the group's tiles
    auto load_params = [&](int gg, float4 (&pp)[TPG][2]) {
#pragma unroll
        for (int t = 0; t < TPG; ++t) {
            const float4* p = a.params + ((int64_t)(TPG * gg + t) * 32 + l.R) * 2;
            pp[t][0] = p[0];
            pp[t][1] = p[1];
        }
    };
    // bias (both parts) and residual (rows 0 .. M - 1, both parts) of group
    // gg into LDS, one dword per lane and DMA
    const int64_t N = a.N;
    auto stage_epilogue = [&](int gg) {
        const int64_t n0 = (int64_t)gg * GN;
        const bool hb = a.bias != nullptr;
#pragma unroll
        for (int p = 0; p < 2; ++p)  // a part's 64 outputs per DMA
            dma_dword(hb ? (const void*)(a.bias + p * N + n0) : (const void*)kGvZeroBias, hb ? 4u * lane : 0u,
                      lds_addr(bias_s + 64 * p));
        if constexpr (RES) {  // one row per DMA: lane = (part, output pair)
            const uint16_t* r = reinterpret_cast<const uint16_t*>(a.res) + n0;
            const uint32_t voff = (uint32_t)(((lane >> 5) * N + 2 * (lane & 31)) * 2);
#pragma unroll 1
            for (int m = 0; m < M; ++m) dma_dword(r + 2 * N * m, voff, lds_addr(res_s + 128 * m));
        }
    };
    // issue order: the scales, then as in the loop (activations of a k-step
    // before its codes), so that the wait counts merged at the loop heads are
    // the steady state's
    float4 pp[TPG][2];
    uint2 cring[SK_PF][H];
    uint2 xring[GV_XPF][4];
    load_params(grp, pp);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < GV_XPF; ++i) gv_load_x<XDT, false>(a, l, i, xring[i]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < SK_PF; ++i) load_codes(grp, i, cring[i]);
    __builtin_amdgcn_sched_barrier(0);
    const int m = min(l.r16 >> 1, M - 1);  // rows past M store row M - 1's values
    const int64_t ldy = 2 * N;
    const bool f16 = YDT == RPFQ_F16;
#pragma unroll 1
    for (; grp < groups; grp += gs) {
#pragma unroll
        for (int t = 0; t < TPG; ++t)
            build_lut_sk_regs<CB, 8>(lut + t * (kSkLut / 4), pp[t][0], pp[t][1], a.rot, l.R, l.g, 0);
        load_params(grp + gs < groups ? grp + gs : grp, pp);  // the next group's
        // the previous group's epilogue has consumed its LDS reads of the
        // staging area (its stores depend on them)
        stage_epilogue(grp);
        floatx4 acc[H];
#pragma unroll
        for (int h = 0; h < H; ++h) acc[h] = floatx4{0, 0, 0, 0};
        int ks0 = 0;  // KS >= SK_PF: at least one round, so every path has the same loads in flight
#pragma unroll 1
        do {
#pragma unroll
            for (int i = 0; i < SK_PF; ++i) {
                const int ks = ks0 + i;
                gv_kstep<XDT, false, H, 1>(acc, l, ks, a.K, cring[i], xring[i % GV_XPF]);
                const int kx = ks + GV_XPF < KS ? ks + GV_XPF : ks + GV_XPF - KS;
                gv_load_x<XDT, false>(a, l, kx, xring[i % GV_XPF]);
                load_codes(grp, ks + SK_PF, cring[i]);
            }
            ks0 += SK_PF;
        } while (ks0 < KS);
        // the loop issued 8 loads per k-step (4 code, 4 activation) after the
        // staging DMAs, at least 8 SK_PF of them: 32 outstanding at most
        // means the DMAs have landed
        static_assert(8 * SK_PF == 32, "the wait count below");
        asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
        // outputs n = GN grp + 16 h + 4 q + v of part p of row m
        const float inv = row_unscale(l.xs);  // undo the row's prescale (exact) before the bias
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const int j = 16 * h + 4 * l.q;
            const int64_t base = m * ldy + (l.p ? N : 0) + (int64_t)grp * GN + j;
            const float4 bq = *reinterpret_cast<const float4*>(bias_s + GN * l.p + j);
            float v4[4] = {acc[h][0] * inv + bq.x, acc[h][1] * inv + bq.y, acc[h][2] * inv + bq.z,
                           acc[h][3] * inv + bq.w};
            uint2 o;
            if constexpr (YDT == RPFQ_F16) {
                o = make_uint2(cvt_pk(v4[0], v4[1]), cvt_pk(v4[2], v4[3]));
            } else {
                o = make_uint2(pack_bf2(v4[0], v4[1]), pack_bf2(v4[2], v4[3]));
            }
            if constexpr (RES) {
                const uint2 rv = *reinterpret_cast<const uint2*>(res_s + 2 * GN * m + GN * l.p + j);
                o = make_uint2(add2_y(o.x, rv.x, f16), add2_y(o.y, rv.y, f16));
            } else if (a.act) {
                o = make_uint2(gelu2_y(o.x, f16), gelu2_y(o.y, f16));
            }
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.y) + base) = o;
        }
    }
}

template <int XDT, int YDT, int CB, bool RES>
static hipError_t wide_gv_persist_launch(WideArgs& a, hipStream_t s) {
    static std::atomic<int> per_cu{0};  // resident workgroups (one wave) per CU
    const void* kern = reinterpret_cast<const void*>(&wide_linear_gemv_persist_kernel<XDT, YDT, CB, RES>);
    const int lds = gp_lds(RES);
    int wg = per_cu.load(std::memory_order_relaxed);
    if (wg <= 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wg, kern, 64, lds) != hipSuccess || wg < 1) wg = 1;
        per_cu.store(wg, std::memory_order_relaxed);
    }
    const int64_t groups = a.NT / 2;
    const int64_t slots = (int64_t)device_cus() * wg;
    const int grid = (int)(groups < slots ? groups : slots);
    hipLaunchKernelGGL((wide_linear_gemv_persist_kernel<XDT, YDT, CB, RES>), dim3((unsigned)grid), dim3(64), lds, s,
                       a);
    return hipGetLastError();
}
template <int XDT, int YDT, int CB>
static hipError_t wide_gv_persist_go(WideArgs& a, hipStream_t s) {
    return a.res ? wide_gv_persist_launch<XDT, YDT, CB, true>(a, s) : wide_gv_persist_launch<XDT, YDT, CB, false>(a, s);
}

// The persistent form's conditions (above): the launches of the one-wave
// form (12 .. 15 k-steps from 4096 tiles) that it can take.  The longer ones
// stay on the two-wave form: the persistent one-wave kernel measured slower
// there, and so did a one-tile-per-wave persistent form at any length.
static bool gv_persist_ok(const WideArgs& a, int ydt, int cb) {
    return gemv_single_wave(a) && a.NT % 2 == 0 && a.N % 32 == 0 && a.K % 32 == 0 && a.KS % SK_PF == 0 &&
           a.nblk == 1 && cb != RPFQ_CB_TABLE && (ydt == RPFQ_F16 || ydt == RPFQ_BF16) && a.vec_store;
}

template <int XDT, int YDT, int CB, bool KT, int NW, int H>
static hipError_t wide_gv_go(WideArgs& a, hipStream_t s) {
    const int64_t groups = (a.NT + H / 2 - 1) / (H / 2);
    hipLaunchKernelGGL((wide_linear_gemv_kernel<XDT, YDT, CB, KT, NW, H>), dim3((unsigned)groups),
                       dim3(64 * NW), gv_lds(H, NW), s, a);
    return hipGetLastError();
}

template <int XDT, int YDT, int CB, bool PB, bool KT, int NW>
static hipError_t wide_sk_go(WideArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((wide_linear_skinny_kernel<XDT, YDT, CB, PB, KT, NW>), dim3((unsigned)sk_groups(a)),
                       dim3(64 * NW), sk_lds(NW), s, a);
    return hipGetLastError();
}

template <int XDT, int YDT, int CB, int NW>
static hipError_t wide_sk_ln_go(WideArgs& a, hipStream_t s) {
    const int lds = sk_lds(NW) + 16 * (4 * a.K + 8) + 16 * 4;  // + the prepared rows' prescales
    hipLaunchKernelGGL((wide_linear_skinny_kernel<XDT, YDT, CB, false, false, NW, true>), dim3((unsigned)sk_groups(a)),
                       dim3(64 * NW), lds, s, a);
    return hipGetLastError();
}

// Split K when the launch has too few workgroups to give every SIMD a few
// waves (a single layer at batch 1): over 4 waves below 400 workgroups, over
// 2 from there (less LUT building and reduction per k-step once the groups
// alone fill the SIMDs; ViT-B/16 batch-1 forward 0.834 -> 0.772 ms, and 2
// waves already from 128 groups measured slower); a long stream of tiles
// runs one wave each (the column-split kernel: 2 waves per 64 rows, or 1
// below 16 k-steps).
template <int XDT, int YDT, int CB, bool KT>
static hipError_t wide_gv(WideArgs& a, hipStream_t s) {
    if constexpr (!KT && CB != RPFQ_CB_TABLE && YDT != RPFQ_F32) {
        if (gv_persist_ok(a, YDT, CB)) return wide_gv_persist_go<XDT, YDT, CB>(a, s);
    }
    if (gemv_single_wave(a)) return wide_gv_go<XDT, YDT, CB, KT, 1, 4>(a, s);
    if (a.NT >= kSkSplitTiles) return wide_gv_go<XDT, YDT, CB, KT, 2, 4>(a, s);
    if (a.NT >= kSkNw2Groups) return wide_gv_go<XDT, YDT, CB, KT, 2, 2>(a, s);
    return wide_gv_go<XDT, YDT, CB, KT, 4, 2>(a, s);
}

template <int XDT, int YDT, int CB>
static hipError_t wide_sk(WideArgs& a, hipStream_t s) {
    // Fused row prologue, LayerNorm and / or act quant (qualified on the
    // host, layer_norm_wide_fusable): K split over 4 waves at any group
    // count, so each wave prepares 4 of the chunk's 16 rows (ViT-B/16
    // batch-1 forward 0.775 -> 0.712 ms with the LayerNorm; over 2 waves from
    // 400 groups, as without it, 0.781 ms: the prologue's per-wave work sits
    // on every workgroup's critical path).
    if (a.ln || a.aq_bits) {
        if constexpr (CB != RPFQ_CB_TABLE && XDT != RPFQ_F32) return wide_sk_ln_go<XDT, YDT, CB, 4>(a, s);
        return hipErrorInvalidValue;
    }
    const bool pb = a.nblk > 1, kt = a.K % 32 != 0;
    if (gemv_pays(a)) return kt ? wide_gv<XDT, YDT, CB, true>(a, s) : wide_gv<XDT, YDT, CB, false>(a, s);
    if (pb) return kt ? wide_sk_go<XDT, YDT, CB, true, true, 1>(a, s) : wide_sk_go<XDT, YDT, CB, true, false, 1>(a, s);
    const int64_t groups = sk_groups(a);
    if (groups >= kSkNw2Groups && groups < kSkSplitTiles)
        return kt ? wide_sk_go<XDT, YDT, CB, false, true, 2>(a, s) : wide_sk_go<XDT, YDT, CB, false, false, 2>(a, s);
    if (groups < kSkSplitTiles)
        return kt ? wide_sk_go<XDT, YDT, CB, false, true, 4>(a, s) : wide_sk_go<XDT, YDT, CB, false, false, 4>(a, s);
    return kt ? wide_sk_go<XDT, YDT, CB, false, true, 1>(a, s) : wide_sk_go<XDT, YDT, CB, false, false, 1>(a, s);
}

template <int XDT, int CB>
static hipError_t stream_y(WideArgs& a, int ydt, hipStream_t s) {
    switch (ydt) {
        case RPFQ_F32: return wide_sk<XDT, RPFQ_F32, CB>(a, s);
        case RPFQ_F16: return wide_sk<XDT, RPFQ_F16, CB>(a, s);
        default: return wide_sk<XDT, RPFQ_BF16, CB>(a, s);
    }
}

template <int CB>
hipError_t launch_wide_stream(WideArgs& a, int xdt, int ydt, hipStream_t s) {
    switch (xdt) {
        case RPFQ_F32: return stream_y<RPFQ_F32, CB>(a, ydt, s);
        case RPFQ_F16: return stream_y<RPFQ_F16, CB>(a, ydt, s);
        default: return stream_y<RPFQ_BF16, CB>(a, ydt, s);
    }
}

template hipError_t launch_wide_stream<RPFQ_CB_SEL>(WideArgs&, int, int, hipStream_t);

}  // namespace rpfq
