// Widely-linear GEMM, register-staged tiles (every case the LDS-DMA and
// streaming kernels do not take: bf16 / float32 x, K' % 32 != 0, small M,
// RPFQ_FLAG_TILE_M128).  Compiled once per codebook (RPFQ_CB_SEL).
#include "rpfq_device.h"

#ifndef RPFQ_CB_SEL
#error "compile once per codebook with -DRPFQ_CB_SEL=<RPFQ_CB_*>"
#endif

namespace rpfq {

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

    // Per-row prescales of float32 / bf16 x (a.xs): this thread's CPT staging
    // rows in registers, the tile's BM rows in LDS past the LUTs for the
    // epilogue (written here, read after the k-loop's barriers)
    float xsr[CPT];
    float* xs_lds = reinterpret_cast<float*>(smem + wide_lds_bytes<BM>());
    if (XDT != RPFQ_F16 && a.xs) {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int64_t m = m0 + ((tid + 256 * j) >> 2);
            xsr[j] = m < a.M ? a.xs[m] : 1.0f;
        }
        if (tid < BM) xs_lds[tid] = m0 + tid < a.M ? a.xs[m0 + tid] : 1.0f;
    } else {
#pragma unroll
        for (int j = 0; j < CPT; ++j) xsr[j] = 1.0f;
    }

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
#pragma unroll
                    for (int t = 0; t < 8; ++t) {  // the row's prescale (1 without a.xs): exact
                        fr[t] *= xsr[j];
                        fi[t] *= xsr[j];
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

    if (XDT != RPFQ_F16 && a.xs) {  // undo the rows' prescales (exact) before the bias
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float inv = row_unscale(xs_lds[i * 32 + acc_row(v, g)]);
                acc_re[i][v] *= inv;
                acc_im[i][v] *= inv;
            }
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

template <int BM, int XDT, int YDT, int CB>
static hipError_t wide_go(WideArgs& a, hipStream_t s) {
    static std::atomic<uint64_t> attr_done{0};
    constexpr int lds = wide_lds_bytes<BM>() + BM * 4;  // + the tile's row prescales
    const hipError_t e = set_lds_attr_once(reinterpret_cast<const void*>(&wide_linear_kernel<BM, XDT, YDT, CB>), lds,
                                           attr_done);
    if (e != hipSuccess) return e;
    a.tiles_m = (int)((a.M + BM - 1) / BM);
    a.tiles_n = (int)((a.NT + 3) / 4);
    hipLaunchKernelGGL((wide_linear_kernel<BM, XDT, YDT, CB>), dim3(a.tiles_m * a.tiles_n), dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int BM, int XDT, int CB>
static hipError_t tiled_y(WideArgs& a, int ydt, hipStream_t s) {
    switch (ydt) {
        case RPFQ_F32: return wide_go<BM, XDT, RPFQ_F32, CB>(a, s);
        case RPFQ_F16: return wide_go<BM, XDT, RPFQ_F16, CB>(a, s);
        default: return wide_go<BM, XDT, RPFQ_BF16, CB>(a, s);
    }
}

template <int BM, int CB>
static hipError_t tiled_x(WideArgs& a, int xdt, int ydt, hipStream_t s) {
    switch (xdt) {
        case RPFQ_F32: return tiled_y<BM, RPFQ_F32, CB>(a, ydt, s);
        case RPFQ_F16: return tiled_y<BM, RPFQ_F16, CB>(a, ydt, s);
        default: return tiled_y<BM, RPFQ_BF16, CB>(a, ydt, s);
    }
}

template <int CB>
hipError_t launch_wide_tiled(WideArgs& a, int bm, int xdt, int ydt, hipStream_t s) {
    if (bm == 32) return tiled_x<32, CB>(a, xdt, ydt, s);
    if (bm == 64) return tiled_x<64, CB>(a, xdt, ydt, s);
    return tiled_x<128, CB>(a, xdt, ydt, s);
}

template hipError_t launch_wide_tiled<RPFQ_CB_SEL>(WideArgs&, int, int, int, hipStream_t);

}  // namespace rpfq
