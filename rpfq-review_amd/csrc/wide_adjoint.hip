// Input gradient of a packed widely-linear layer: gx = gy A, the
// contraction over the layer's N' outputs (the backward of F.linear at
// RPFQ-ViT-main/quant_models/quant_i.py:554; kernel.py:585 in the
// reference's Triton autograd).  Register-staged tiles like
// wide_linear_kernel, with the roles of the two code dimensions exchanged:
// the output columns are the layer's K' inputs and the k-loop runs over row
// steps of 32 layer rows, whose codes and U / W tables come from the adjoint
// blob (rpfq_wide_pack_adjoint).  Codebook-independent: the tables hold
// every codebook's entries as fp16 pairs.
#include "rpfq_device.h"

namespace rpfq {

constexpr int kAdjLutRow = 40;                // dwords per LUT row: 16 U + 16 W entries + pad
constexpr int kAdjLutWave = 32 * kAdjLutRow;  // dwords of one 32-row LUT

// LDS bytes per LUT stage: one table per workgroup (per-row scales) or one
// per wave (per-block scales).
__host__ __device__ constexpr int adj_lut_stage(bool per_wave) { return (per_wave ? 4 : 1) * kAdjLutWave * 4; }

// LDS layout: per-row exponents [BM] int, then the gy stages and LUT stages,
// which the epilogue's transpose tile reuses (4 waves x BM rows x kTRow).
template <int BM>
constexpr int adj_lds_bytes(bool per_wave) {
    return BM * 4 + (2 * BM * kXRow + 2 * adj_lut_stage(per_wave) > 4 * BM * kTRow
                         ? 2 * BM * kXRow + 2 * adj_lut_stage(per_wave)
                         : 4 * BM * kTRow);
}

// gx [M, 2K'] = gy [M, 2N'] A with A the layer's fused fp16 coefficients
// (the forward's MFMA operands):
//   gx_re[k] = sum_n A11[n,k] gy_re[n] + A21[n,k] gy_im[n]
//   gx_im[k] = sum_n A12[n,k] gy_re[n] + A22[n,k] gy_im[n]
// Workgroup = 4 waves; tile = BM rows of gy times 128 complex output columns
// (wave w owns columns 32w..32w+31, lane r column r, real and imaginary
// outputs).  Per row step of 32 layer rows:
//   * gy: BM x 32 (re, im) pairs staged to LDS as fp16 (double buffered);
//     float32 / bf16 rows are first scaled by a per-row power of two that
//     puts their largest magnitude in [2^14, 2^15), undone exactly in the
//     epilogue, so the fp16 operands neither overflow nor flush;
//   * codes: one 128-bit load per lane from the adjoint tiles: lane group g
//     gets rows 8 s + 4 g + e of its column, e = 0..3, s = substep;
//   * U / W: the 32 rows' 16 + 16 entries as fp16 (re, im) pairs, copied
//     from the adjoint blob's tables (4 KB per row step, one 16-B load per
//     thread, prefetched a step ahead) into an LDS table [row][entry] (row
//     stride 40 dwords: the two lane groups, 4 rows apart, hit disjoint
//     banks); one table per workgroup with per-row scales, one per wave with
//     per-(row, block) scales (a wave's 32 columns lie in one block);
//   * coefficients (A11, A21) = U + W and (A12, A22) = (Wim - Uim, Ure - Wre),
//     one v_pk_add_f16 each: the same correctly rounded fp16 adds as the
//     forward's, so A is bit for bit the forward's operand.
template <int BM, int GDT, int XDT>
__global__ void __launch_bounds__(256, 2) wide_grad_x_kernel(AdjArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int MB = BM / 32;
    constexpr int XSTAGE = BM * kXRow;
    constexpr int CPT = BM >= 64 ? BM / 64 : 1;
    constexpr int NCHUNK = BM * 4;
    constexpr bool SCALE = GDT != RPFQ_F16;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, g = lane >> 5;
    const int tile = xcd_tile(blockIdx.x, a.tiles_m * a.tiles_k);
    const int mt = tile / a.tiles_k, ktl = tile - mt * a.tiles_k;
    const int64_t m0 = (int64_t)mt * BM;
    const int ktw = ktl * 4 + wave;  // this wave's 32-column tile
    const bool active = ktw < a.KS;
    const int ktw_ld = active ? ktw : a.KS - 1;
    const int64_t ldg = 2 * (int64_t)a.N;
    const bool per_wave = a.nblk > 1;
    int* const row_exp = reinterpret_cast<int*>(smem);
    char* const base = smem + BM * 4;
    char* const lut_base = base + 2 * XSTAGE;
    const int lut_stage = adj_lut_stage(per_wave);
    const bool gvec = (a.N % 8) == 0;

    constexpr int RAW = (GDT == RPFQ_F32) ? 4 : 2;
    uint4 xbufA[CPT][RAW], xbufB[CPT][RAW];
    uint32_t okA = 0, okB = 0;
    uint4 cA = make_uint4(0, 0, 0, 0), cB = make_uint4(0, 0, 0, 0);
    uint4 pA, pB;  // (shared table) this thread's 16 B of the row step's table waiting in each buffer

    // chunk c = tid + 256 j: gy row c >> 2, complex columns 8 (c & 3) .. +7 of the row step
    auto load_g = [&](int ns, uint4 (&xraw)[CPT][RAW], uint32_t& xok) {
        xok = 0;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tid + 256 * j;
            const int row = c >> 2, sub = c & 3;
            const int64_t m = m0 + row;
            const int nn = ns * 32 + sub * 8;
            const bool ok = c < NCHUNK && m < a.M && nn < a.N;
            xok |= (ok ? 1u : 0u) << j;
            const int64_t off = ok ? m * ldg + nn : 0;
            if (gvec) {
                if (GDT == RPFQ_F32) {
                    const uint4* pr = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(a.gy) + off);
                    const uint4* pi = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(a.gy) + off + a.N);
                    xraw[j][0] = pr[0];
                    xraw[j][1] = pr[1];
                    xraw[j][RAW - 2] = pi[0];
                    xraw[j][RAW - 1] = pi[1];
                } else {
                    xraw[j][0] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.gy) + off);
                    xraw[j][1] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(a.gy) + off + a.N);
                }
            } else {  // N' % 8 != 0: element loads, zero past N'
                if (GDT == RPFQ_F32) {
                    const float* p = reinterpret_cast<const float*>(a.gy) + off;
                    float vr[8], vi[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const bool in = ok && nn + t < a.N;
                        vr[t] = in ? p[t] : 0.0f;
                        vi[t] = in ? p[a.N + t] : 0.0f;
                    }
                    xraw[j][0] = make_uint4(__float_as_uint(vr[0]), __float_as_uint(vr[1]), __float_as_uint(vr[2]),
                                            __float_as_uint(vr[3]));
                    xraw[j][1] = make_uint4(__float_as_uint(vr[4]), __float_as_uint(vr[5]), __float_as_uint(vr[6]),
                                            __float_as_uint(vr[7]));
                    xraw[j][RAW - 2] = make_uint4(__float_as_uint(vi[0]), __float_as_uint(vi[1]),
                                                  __float_as_uint(vi[2]), __float_as_uint(vi[3]));
                    xraw[j][RAW - 1] = make_uint4(__float_as_uint(vi[4]), __float_as_uint(vi[5]),
                                                  __float_as_uint(vi[6]), __float_as_uint(vi[7]));
                } else {
                    const uint16_t* p = reinterpret_cast<const uint16_t*>(a.gy) + off;
                    uint32_t hr[8], hi[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const bool in = ok && nn + t < a.N;
                        hr[t] = in ? p[t] : 0u;
                        hi[t] = in ? p[a.N + t] : 0u;
                    }
                    xraw[j][0] = make_uint4(hr[0] | hr[1] << 16, hr[2] | hr[3] << 16, hr[4] | hr[5] << 16,
                                            hr[6] | hr[7] << 16);
                    xraw[j][1] = make_uint4(hi[0] | hi[1] << 16, hi[2] | hi[3] << 16, hi[4] | hi[5] << 16,
                                            hi[6] | hi[7] << 16);
                }
            }
        }
    };
    auto store_g = [&](int stage, const uint4 (&xraw)[CPT][RAW], uint32_t xok) {
        char* xs = base + stage * XSTAGE;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tid + 256 * j;
            if (NCHUNK < 256 && c >= NCHUNK) break;
            const int row = c >> 2, sub = c & 3;
            uint4 o0, o1;
            if (GDT == RPFQ_F16) {
                const uint4 vr = xraw[j][0], vi = xraw[j][1];
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
                if (GDT == RPFQ_BF16) {
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
                const int sh = row_exp[row];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    fr[t] = ldexpf(fr[t], sh);
                    fi[t] = ldexpf(fi[t], sh);
                }
                o0 = make_uint4(cvt_pk(fr[0], fi[0]), cvt_pk(fr[1], fi[1]), cvt_pk(fr[2], fi[2]),
                                cvt_pk(fr[3], fi[3]));
                o1 = make_uint4(cvt_pk(fr[4], fi[4]), cvt_pk(fr[5], fi[5]), cvt_pk(fr[6], fi[6]),
                                cvt_pk(fr[7], fi[7]));
            }
            const uint32_t keep = 0u - ((xok >> j) & 1u);
            o0 = make_uint4(o0.x & keep, o0.y & keep, o0.z & keep, o0.w & keep);
            o1 = make_uint4(o1.x & keep, o1.y & keep, o1.z & keep, o1.w & keep);
            uint4* dst = reinterpret_cast<uint4*>(xs + row * kXRow + sub * 32);
            dst[0] = o0;
            dst[1] = o1;
        }
    };
    // Per-row exponents (float32 / bf16 gy): sh[m] with max|gy[m]| * 2^sh[m]
    // in [2^14, 2^15).  The workgroup reads its rows once ahead of the
    // k-loop, UNR row steps in flight, taking the maximum of the magnitude
    // bits (ordered like the magnitudes; a NaN leaves sh = 0).
    if constexpr (SCALE) {
        constexpr int UNR = GDT == RPFQ_F32 ? 2 : 4;
        constexpr uint32_t MAG = GDT == RPFQ_F32 ? 0x7fffffffu : 0x7fff7fffu;
        uint32_t mx[CPT];
#pragma unroll
        for (int j = 0; j < CPT; ++j) mx[j] = 0;
        for (int ns0 = 0; ns0 < a.NT; ns0 += UNR) {
            uint4 raw[UNR][CPT][RAW];
            uint32_t ok[UNR];
#pragma unroll
            for (int u = 0; u < UNR; ++u) load_g(ns0 + u < a.NT ? ns0 + u : a.NT - 1, raw[u], ok[u]);
#pragma unroll
            for (int u = 0; u < UNR; ++u) {
#pragma unroll
                for (int j = 0; j < CPT; ++j) {
                    const uint32_t keep = 0u - ((ok[u] >> j) & 1u);
#pragma unroll
                    for (int t = 0; t < RAW; ++t) {
                        const uint4 w = raw[u][j][t];
                        const uint32_t v[4] = {w.x & MAG & keep, w.y & MAG & keep, w.z & MAG & keep,
                                               w.w & MAG & keep};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            if (GDT == RPFQ_F32) {
                                mx[j] = max(mx[j], v[q]);
                            } else {
                                mx[j] = max(mx[j], max(v[q] & 0xffffu, v[q] >> 16));
                            }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            uint32_t v = mx[j];
            v = max(v, (uint32_t)__shfl_xor((int)v, 1));
            v = max(v, (uint32_t)__shfl_xor((int)v, 2));
            const float f = __uint_as_float(GDT == RPFQ_F32 ? v : v << 16);
            const int c = tid + 256 * j;
            if (c < NCHUNK && (c & 3) == 0) {
                int ex = 0;
                (void)frexpf(f, &ex);  // f < 2^ex
                row_exp[c >> 2] = (f > 0.0f && f <= 3.402823466e38f) ? 15 - ex : 0;
            }
        }
        __syncthreads();
    }
    auto load_codes = [&](int ns) -> uint4 {
        return a.codes_t[(((int64_t)ktw_ld * a.NT + ns) * 32 + r) * 2 + g];
    };
    // Table copies.  Shared table (per-row scales): thread tid copies dwords
    // 4 (tid & 7) .. + 3 of row tid >> 3, prefetched with the row step's
    // other loads.  Per-wave tables (per-(row, block) scales): lane copies
    // dwords 16 (lane & 1) .. + 15 of row lane >> 1 for the wave's block,
    // loaded when the table is staged.
    const int64_t lblk = per_wave ? ktw_ld / a.block_ks : 0;
    auto load_lut = [&](int ns) -> uint4 {
        if (per_wave) return make_uint4(0, 0, 0, 0);
        return a.lut_t[((int64_t)ns * 32 + (tid >> 3)) * 8 + (tid & 7)];
    };
    auto build = [&](int ns, int stage, const uint4 v) {
        uint32_t* lut = reinterpret_cast<uint32_t*>(lut_base + stage * lut_stage);
        if (!per_wave) {
            *reinterpret_cast<uint4*>(lut + (tid >> 3) * kAdjLutRow + 4 * (tid & 7)) = v;
            return;
        }
        const int row = lane >> 1, h = lane & 1;
        const uint4* src = a.lut_t + (((int64_t)ns * 32 + row) * a.nblk + lblk) * 8 + 4 * h;
        uint4* dst = reinterpret_cast<uint4*>(lut + wave * kAdjLutWave + row * kAdjLutRow + 16 * h);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = src[i];
    };

    floatx16 acc_re[MB], acc_im[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc_re[i] = acc_im[i] = floatx16{0};

    // prologue: row step 0 staged (gy and LUT), row step 1 waiting in registers
    pA = load_lut(0);
    load_g(0, xbufA, okA);
    cA = load_codes(0);
    {
        const int n1 = a.NT > 1 ? 1 : 0;
        load_g(n1, xbufB, okB);
        cB = load_codes(n1);
        pB = load_lut(n1);
    }
    build(0, 0, pA);
    store_g(0, xbufA, okA);
    __syncthreads();

    // One row step: prefetch row step ns+2 into `fill`, run the MFMAs of ns,
    // stage row step ns+1 (waiting in `next`) into the other LDS buffers.
    auto step = [&](int ns, const uint4 cw, uint4 (&next)[CPT][RAW], uint32_t next_ok, const uint4 nlut,
                    uint4 (&fill)[CPT][RAW], uint32_t& fill_ok, uint4& fill_codes, uint4& flut) {
        {
            const int np = ns + 2 < a.NT ? ns + 2 : a.NT - 1;
            load_g(np, fill, fill_ok);
            fill_codes = load_codes(np);
            flut = load_lut(np);
        }
        const char* xs = base + (ns & 1) * XSTAGE;
        const uint32_t* lut = reinterpret_cast<const uint32_t*>(lut_base + (ns & 1) * lut_stage) +
                              (per_wave ? wave * kAdjLutWave : 0);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t word = s == 0 ? cw.x : s == 1 ? cw.y : s == 2 ? cw.z : cw.w;
            uint32_t U[4], W[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t byte = (word >> (8 * e)) & 0xffu;
                const uint32_t* row = lut + (8 * s + 4 * g + e) * kAdjLutRow;
                U[e] = row[byte & 15u];
                W[e] = row[16u + (byte >> 4)];
            }
            half8 ax[MB];
#pragma unroll
            for (int i = 0; i < MB; ++i)
                ax[i] = *reinterpret_cast<const half8*>(xs + (i * 32 + r) * kXRow + (8 * s + 4 * g) * 4);
            uint32_t bre[4], bim[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const half2v u = __builtin_bit_cast(half2v, U[e]), w = __builtin_bit_cast(half2v, W[e]);
                bre[e] = __builtin_bit_cast(uint32_t, u + w);                                  // (A11, A21)
                bim[e] = __builtin_bit_cast(uint32_t, (half2v){w.y, -w.x} + (half2v){-u.y, u.x});  // (A12, A22)
            }
            const half8 b_re = as_half8(make_uint4(bre[0], bre[1], bre[2], bre[3]));
            const half8 b_im = as_half8(make_uint4(bim[0], bim[1], bim[2], bim[3]));
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                acc_re[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[i], b_re, acc_re[i], 0, 0, 0);
                acc_im[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ax[i], b_im, acc_im[i], 0, 0, 0);
            }
        }
        if (ns + 1 < a.NT) {
            store_g((ns + 1) & 1, next, next_ok);
            build(ns + 1, (ns + 1) & 1, nlut);
        }
        __syncthreads();
    };
    for (int ns = 0; ns < a.NT; ns += 2) {
        const uint4 c0 = cA;
        step(ns, c0, xbufB, okB, pB, xbufA, okA, cA, pA);
        if (ns + 1 < a.NT) {
            const uint4 c1 = cB;
            step(ns + 1, c1, xbufA, okA, pA, xbufB, okB, cB, pB);
        }
    }

    const int64_t k = (int64_t)ktw * 32 + r;
    const bool k_ok = active && k < a.K;
    const int64_t ldx = 2 * (int64_t)a.K;
    if (XDT == RPFQ_F32) {
        if (!k_ok) return;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = i * 32 + acc_row(v, g);
                const int64_t m = m0 + row;
                if (m < a.M) {
                    const int sh = SCALE ? row_exp[row] : 0;
                    float* y = reinterpret_cast<float*>(a.gx);
                    y[m * ldx + k] = ldexpf(acc_re[i][v], -sh);
                    y[m * ldx + a.K + k] = ldexpf(acc_im[i][v], -sh);
                }
            }
        }
        return;
    }
    // 16-bit outputs: transpose the wave's [BM x 64] tile through LDS (the
    // staging buffers are free after the final barrier; the per-row
    // exponents lie before them) and write 16-byte chunks.
    uint16_t* tt = reinterpret_cast<uint16_t*>(base + wave * (BM * kTRow));
#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int row = i * 32 + acc_row(v, g);
            const int sh = SCALE ? row_exp[row] : 0;
            const float vr = SCALE ? ldexpf(acc_re[i][v], -sh) : acc_re[i][v];
            const float vi = SCALE ? ldexpf(acc_im[i][v], -sh) : acc_im[i][v];
            uint16_t hr, hi;
            if (XDT == RPFQ_F16) {
                hr = __builtin_bit_cast(uint16_t, (_Float16)vr);
                hi = __builtin_bit_cast(uint16_t, (_Float16)vi);
            } else {
                hr = f32_to_bf16(vr);
                hi = f32_to_bf16(vi);
            }
            tt[row * (kTRow / 2) + r] = hr;
            tt[row * (kTRow / 2) + 32 + r] = hi;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
    __builtin_amdgcn_wave_barrier();
    if (!active) return;
    const int64_t kbase = (int64_t)ktw * 32;
    const int q = lane & 7;
    const int64_t col0 = (q < 4 ? 0 : a.K) + kbase + 8 * (q & 3);
    const int64_t kfirst = kbase + 8 * (q & 3);
#pragma unroll 4
    for (int row = lane >> 3; row < BM; row += 8) {
        const int64_t m = m0 + row;
        if (m >= a.M) break;
        const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(tt) + row * kTRow + q * 16);
        uint16_t* dst = reinterpret_cast<uint16_t*>(a.gx) + m * ldx + col0;
        if (a.vec_store && kfirst + 8 <= a.K) {
            *reinterpret_cast<uint4*>(dst) = v;
        } else {
            const uint16_t* h = reinterpret_cast<const uint16_t*>(&v);
            for (int t = 0; t < 8 && kfirst + t < a.K; ++t) dst[t] = h[t];
        }
    }
}

template <int BM, int GDT, int XDT>
static hipError_t grad_go(AdjArgs& a, hipStream_t s) {
    static std::atomic<uint64_t> attr_done{0};
    const hipError_t e = set_lds_attr_once(reinterpret_cast<const void*>(&wide_grad_x_kernel<BM, GDT, XDT>),
                                           adj_lds_bytes<BM>(true), attr_done);
    if (e != hipSuccess) return e;
    const int lds = adj_lds_bytes<BM>(a.nblk > 1);
    a.tiles_m = (int)((a.M + BM - 1) / BM);
    a.tiles_k = (a.KS + 3) / 4;
    hipLaunchKernelGGL((wide_grad_x_kernel<BM, GDT, XDT>), dim3(a.tiles_m * a.tiles_k), dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int BM, int GDT>
static hipError_t grad_x_dt(AdjArgs& a, int xdt, hipStream_t s) {
    switch (xdt) {
        case RPFQ_F32: return grad_go<BM, GDT, RPFQ_F32>(a, s);
        case RPFQ_F16: return grad_go<BM, GDT, RPFQ_F16>(a, s);
        default: return grad_go<BM, GDT, RPFQ_BF16>(a, s);
    }
}

template <int BM>
static hipError_t grad_g16(AdjArgs& a, int gdt, int xdt, hipStream_t s) {
    if (gdt == RPFQ_F16) return grad_x_dt<BM, RPFQ_F16>(a, xdt, s);
    return grad_x_dt<BM, RPFQ_BF16>(a, xdt, s);
}

hipError_t launch_wide_grad_x(AdjArgs& a, int gdt, int xdt, hipStream_t s) {
    // float32 gy takes 64-row tiles: at 128 rows its raw prefetch buffers
    // (8 x 16 B per chunk) push the k-loop past 256 VGPRs and spill
    if (gdt == RPFQ_F32) return grad_x_dt<64, RPFQ_F32>(a, xdt, s);
    if (a.M <= 64) return grad_g16<64>(a, gdt, xdt, s);
    return grad_g16<128>(a, gdt, xdt, s);
}

}  // namespace rpfq
