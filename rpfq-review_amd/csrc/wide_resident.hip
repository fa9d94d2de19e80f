// Widely-linear GEMM for small layers at large M: the decoded layer stays in
// LDS for the whole launch and the waves stream rows of x past it.
// Compiled once per codebook (RPFQ_CB_SEL).
#include "rpfq_device.h"

#ifndef RPFQ_CB_SEL
#error "compile once per codebook with -DRPFQ_CB_SEL=<RPFQ_CB_*>"
#endif

namespace rpfq {

// ---------------------------------------------------------------------------
// Resident-weight kernel (RPFQ_KERNEL_RESIDENT).
//
// The layer is one real GEMM y [M, 2N'] = x [M, 2K'] A_r^T with
//   A_r [2N'][2K'] = [[A11, A12], [A21, A22]]
// (rows n < N' give Re y_n, rows N' + n give Im y_n; columns k < K' multiply
// Re x_k, columns K' + k multiply Im x_k).  A persistent workgroup of
// kResWaves waves (one per CU) decodes all of A_r into LDS once, as the A
// operands of v_mfma_f32_16x16x32_f16: tile (b, c) holds rows 16 b .. +15
// and columns 32 c .. +31, lane l = (o, q) = (l % 16, l / 16) the 8 fp16
// A_r[16 b + o][32 c + 8 q ..] at byte ((b * KC + c) * 64 + l) * 16
// (KC = 2K' / 32 tiles per row block).  Every wave then takes 16-row
// subtiles of x on its own, with no barrier, and holds the whole output row
// block of its subtile in registers (2N' / 16 accumulator tiles):
//   * B operand: lane (r, q) loads row m0 + r, columns 32 c + 8 q .. + 7 of
//     every k-chunk c (16 B; 64 contiguous bytes per row and instruction;
//     bf16 rows converted to fp16 after the row's prescale, as every kernel
//     converts them); a register ring keeps the rows of the wave's next
//     U - 1 subtiles in flight (res_ring);
//   * D: lane (r, q) holds x row r's outputs 16 b + 4 q .. + 3;
//     after bias and rounding, v_permlane16_swap pairs blocks 2p and 2p + 1
//     so that lane (r, q) holds the 8 outputs 32 p + 16 (q & 1) + 8 (q >> 1)
//     .. + 7: one 16-B store, 64 contiguous bytes per row and instruction;
//   * the subtile's rows are stored in one burst of 2N' / 32 instructions
//     (whole rows, so the L2 merges every 128-B line before it writes it back;
//     write-back stores: non-temporal ones reach HBM as partial lines and
//     halve the rate).
// Every coefficient is the fp16 value the other kernels feed the MFMA
// (lut_entry, de-rotation, cvt_pk, fuse_h), and the epilogue rounds as theirs.
// ---------------------------------------------------------------------------
constexpr int kResMaxTasks = 5;  // decode tasks per thread: N' K' / 8 <= 5 * 512 for every layer taken

// Decodes the layer into the LDS tiles above and the bias after them.
// Task (n, k0): complex row n, columns k0 .. k0 + 7 (one 4-byte code word
// in each lane-group half of the row's k-step), giving 8 columns of each of
// A11, A12, A21, A22.  Every global load of the thread is issued first.
template <int CB, int KC>
__device__ __forceinline__ void res_decode(const WideArgs& a, char* smem, float* bias_s) {
    const int k8n = a.K >> 3;
    const int tasks = a.N * k8n;
    uint32_t w0[kResMaxTasks], w1[kResMaxTasks];
    float4 pu[kResMaxTasks], pw[kResMaxTasks];
#pragma unroll
    for (int i = 0; i < kResMaxTasks; ++i) {
        const int t = threadIdx.x + i * (int)blockDim.x;
        if (t >= tasks) break;
        const int n = t / k8n, k0 = (t - n * k8n) * 8;
        // byte 16 g + 4 s + e of (row n, k-step) holds column 32 ks + 8 s + 4 g + e
        const uint8_t* cw = reinterpret_cast<const uint8_t*>(a.codes) +
                            (((int64_t)(n >> 5) * a.KS + (k0 >> 5)) * 32 + (n & 31)) * 32 + 4 * ((k0 >> 3) & 3);
        w0[i] = *reinterpret_cast<const uint32_t*>(cw);       // columns k0 .. k0 + 3
        w1[i] = *reinterpret_cast<const uint32_t*>(cw + 16);  // columns k0 + 4 .. k0 + 7
        if constexpr (CB != RPFQ_CB_TABLE) {
            const int blk = a.nblk > 1 ? k0 / (a.block_ks * 32) : 0;
            const float4* p = a.params + ((int64_t)n * a.nblk + blk) * 2;
            pu[i] = p[0];
            pw[i] = p[1];
        }
    }
    const int nb = 2 * a.N;
    const float bv = (int)threadIdx.x < nb && a.bias ? a.bias[threadIdx.x] : 0.0f;  // 2N' <= 384 < blockDim.x
#pragma unroll
    for (int i = 0; i < kResMaxTasks; ++i) {
        const int t = threadIdx.x + i * (int)blockDim.x;
        if (t >= tasks) break;
        const int n = t / k8n, k0 = (t - n * k8n) * 8;
        const float2* tab = nullptr;
        if constexpr (CB == RPFQ_CB_TABLE) tab = reinterpret_cast<const float2*>(a.params) + (int64_t)n * 32;
        uint32_t p1[8], p2[8];  // (A11, A12) and (A21, A22) fp16 pairs of the 8 columns
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t code = ((j < 4 ? w0[i] : w1[i]) >> (8 * (j & 3))) & 0xffu;
            float2 u, w;
            if constexpr (CB == RPFQ_CB_TABLE) {
                u = tab[code & 15u];
                w = tab[16 + (code >> 4)];
            } else {
                u = lut_entry<CB>(code & 15u, pu[i]);
                w = lut_entry<CB>(code >> 4, pw[i]);
            }
            if (a.rot.rotate) {
                u = derotate(u, a.rot.cu, a.rot.su);
                w = derotate(w, a.rot.cw, a.rot.sw);
            }
            fuse_h(cvt_pk(u.x, u.y), cvt_pk(w.x, w.y), p1[j], p2[j]);
        }
        uint4 a11, a12, a21, a22;  // 8 consecutive columns of each kind
        uint32_t* q11 = &a11.x;
        uint32_t* q12 = &a12.x;
        uint32_t* q21 = &a21.x;
        uint32_t* q22 = &a22.x;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            q11[e] = __builtin_amdgcn_perm(p1[2 * e + 1], p1[2 * e], 0x05040100u);
            q12[e] = __builtin_amdgcn_perm(p1[2 * e + 1], p1[2 * e], 0x07060302u);
            q21[e] = __builtin_amdgcn_perm(p2[2 * e + 1], p2[2 * e], 0x05040100u);
            q22[e] = __builtin_amdgcn_perm(p2[2 * e + 1], p2[2 * e], 0x07060302u);
        }
        // A_r[o][j0 .. j0 + 7] (j0 % 8 == 0) -> tile (o / 16, j0 / 32), lane (o % 16, (j0 / 8) % 4)
        auto at = [&](int o, int j0) -> uint4* {
            return reinterpret_cast<uint4*>(smem) + ((o >> 4) * KC + (j0 >> 5)) * 64 + (o & 15) + 16 * ((j0 >> 3) & 3);
        };
        *at(n, k0) = a11;
        *at(n, a.K + k0) = a12;
        *at(a.N + n, k0) = a21;
        *at(a.N + n, a.K + k0) = a22;
    }
    if ((int)threadIdx.x < nb) bias_s[threadIdx.x] = bv;
}

// 16 B of x (8 fp16 or bf16) -> the fp16 MFMA operand; bf16 after the row's
// prescale sc (1 without one): the same conversion as every other kernel.
template <int XDT>
__device__ __forceinline__ half8 res_x16(uint4 v, float sc) {
    if constexpr (XDT == RPFQ_BF16) {
        uint4 o;
        o.x = pack_h2(bf16_to_f32(v.x & 0xffffu) * sc, bf16_to_f32(v.x >> 16) * sc);
        o.y = pack_h2(bf16_to_f32(v.y & 0xffffu) * sc, bf16_to_f32(v.y >> 16) * sc);
        o.z = pack_h2(bf16_to_f32(v.z & 0xffffu) * sc, bf16_to_f32(v.z >> 16) * sc);
        o.w = pack_h2(bf16_to_f32(v.w & 0xffffu) * sc, bf16_to_f32(v.w >> 16) * sc);
        return as_half8(o);
    } else {
        return as_half8(v);
    }
}

template <int YDT>
__device__ __forceinline__ uint32_t res_pack2(float lo, float hi) {
    if constexpr (YDT == RPFQ_F16) return cvt_pk(lo, hi);
    return pack_bf2(lo, hi);
}

// Subtiles in flight per wave (the register ring).  Deeper rings (4 at
// K' = 48, 3 at K' = 96) measured no faster: 8 waves per CU with two
// subtiles each keep enough rows in flight.  With 24 accumulator tiles one
// slot (each chunk refilled with the next subtile's as its MFMAs issue)
// keeps the registers within 256.
template <int KC, int NB> constexpr int res_ring() { return NB >= 24 ? 1 : 2; }
constexpr int kResWAhead = 4;  // weight tiles read ahead of their MFMA

// prescale of bf16 rows launched without row scales (WideArgs::xs NULL)
__device__ const float kResUnitScale = 1.0f;

// KC: 32-column k-chunks of the real row (2K' / 32); NB: 16-row blocks of
// A_r (2N' / 16); RES: a residual is added in the store (NB <= 12); ACT:
// fused GELU.
//
// Every vector memory instruction of the subtile loop is issued on every
// path (rows past M load and store row M - 1's values, the last round
// refills the ring from the slot's own rows, the prescale of bf16 rows comes
// from a unit constant without row scales): loads and stores share one
// counter on gfx950, and with path-dependent counts the compiler waits for
// every outstanding store and ring load at each slot.
template <int KC, int NB, int RES, int XDT, int YDT, int CB, int ACT>
__global__ __launch_bounds__(kResWaves * 64) void wide_linear_resident_kernel(WideArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int U = res_ring<KC, NB>();
    constexpr int J = NB * KC;  // MFMAs per subtile, chunk-major (j = c NB + b)
    constexpr int D = kResWAhead < J ? kResWAhead : J;
    static_assert(!RES || NB <= 12, "residual layers: N' <= 96");
    float* bias_s = reinterpret_cast<float*>(smem + NB * KC * 1024);
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    // output staging: TR rows of RB bytes per wave after the layer
    constexpr int TR = res_stage_rows(KC, NB);
    constexpr int RB = 32 * NB;                          // bytes of an output row (4N')
    constexpr int RP = res_stage_pitch(NB);              // its pitch in the staging rows
    static_assert(TR > 0, "the shapes taken leave LDS for at least 8 staged rows per wave");
    constexpr int NI = (TR * RB + 1023) / 1024;  // 1-KB stores per staged block
    constexpr int NOUT = NI * (16 / TR);         // 16-B stores per lane and subtile
    char* stage = smem + res_lds_layer(KC, NB) + (threadIdx.x >> 6) * TR * RP;
    // byte offset in the staged rows (as in y) of store i: lane l's 16 B of
    // the i-th KB (the last KB's lanes past the block repeat its last chunk)
    auto stage_off = [&](int i) -> int {
        const int o = 1024 * i + 16 * lane;
        return o < TR * RB ? o : TR * RB - 16;
    };
    auto stage_at = [&](int o) -> int { return (o / RB) * RP + o % RB; };  // its LDS offset
    const int64_t nsub = (a.M + 15) >> 4;
    const int64_t ws = (int64_t)gridDim.x * kResWaves;
    const int64_t t0 = (int64_t)blockIdx.x * kResWaves + (threadIdx.x >> 6);
    const int64_t ldx = 2 * (int64_t)a.K, ldy = 2 * (int64_t)a.N;
    const bool scaled = XDT == RPFQ_BF16 && a.xs != nullptr;
    const int ocol = 16 * (q & 1) + 8 * (q >> 1);  // this lane's 8 outputs within each 32

    // This lane's row of subtile tt (rows past M are row M - 1).  Ring slot
    // s holds subtile t0 + (i U + s) ws of round i; each chunk is refilled
    // with the next round's as soon as the MFMAs that read it are issued, so
    // U - 1 subtiles stay in flight.
    auto row_of = [&](int64_t tt) -> int64_t {
        const int64_t m = tt * 16 + r;
        return m < a.M ? m : a.M - 1;
    };
    auto xptr = [&](int64_t tt) -> const uint16_t* {
        return reinterpret_cast<const uint16_t*>(a.x) + row_of(tt) * ldx + 8 * q;
    };
    auto xsptr = [&](int64_t tt) -> const float* { return scaled ? a.xs + row_of(tt) : &kResUnitScale; };
    // This lane's stores of subtile tt go to out_base(tt) + out_off(tt, k)
    // bytes of y (and read the residual there): byte o = stage_off(i) of the
    // staged rows hh TR .. of the subtile, k = hh NI + i, i.e. row
    // hh TR + o / RB, byte o % RB (rows past M go to row M - 1, whose values
    // they hold).
    auto out_base = [&](int64_t tt) -> int64_t { return 2 * tt * 16 * ldy; };  // bytes
    auto out_off = [&](int64_t tt, int k) -> uint32_t {
        const int last = a.M - 1 - tt * 16 < 15 ? (int)(a.M - 1 - tt * 16) : 15;  // last row in y
        const int hh = k / NI, o = stage_off(k - hh * NI);
        const int row = hh * TR + o / RB;
        return (uint32_t)((row < last ? row : last) * RB + o % RB);
    };
    uint4 xr[U][KC];
    float xsc[U];
#pragma unroll
    for (int s = 0; s < U; ++s) {  // requested before the decode
        const int64_t tt = t0 + s * ws < nsub ? t0 + s * ws : t0;
        const uint16_t* p = xptr(tt);
#pragma unroll
        for (int c = 0; c < KC; ++c) xr[s][c] = *reinterpret_cast<const uint4*>(p + 32 * c);
        xsc[s] = 1.0f;
        if constexpr (XDT == RPFQ_BF16) xsc[s] = *xsptr(tt);
    }
    res_decode<CB, KC>(a, smem, bias_s);
    __syncthreads();

    // weight tile of MFMA j: block j % NB, chunk j / NB
    const uint4* wl = reinterpret_cast<const uint4*>(smem) + lane;
    auto wtile = [&](int j) -> half8 { return as_half8(wl[((j % NB) * KC + j / NB) * 64]); };
    auto slot = [&](int64_t t, uint4 (&xv)[KC], float& xsv) {
        const int64_t tn = t + U * ws;
        const int64_t tl = tn < nsub ? tn : t;  // refill source: the slot's own rows on its last round
        // residual chunks of this lane's stores, all read before any store
        // (in place, residual == y, a chunk stored twice reads the original)
        uint4 rres[RES ? NOUT : 1];
        if constexpr (RES != 0) {
#pragma unroll
            for (int i = 0; i < NOUT; ++i)
                rres[i] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(a.res) + out_base(t) +
                                                          out_off(t, i));
        }
        const float sc = xsv;
        const float inv = scaled ? row_unscale(sc) : 1.0f;
        const uint16_t* pn = xptr(tl);
        f32x4 acc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        // MFMA j reads the weight tile requested D steps earlier; each step
        // is fenced so the schedule keeps that distance (unfenced, every
        // tile's read is hoisted to the top and the registers run out)
        half8 wq[D];
#pragma unroll
        for (int j = 0; j < D; ++j) wq[j] = wtile(j);
        half8 xc = res_x16<XDT>(xv[0], sc);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = j / NB, b = j % NB;
            const half8 w = wq[j % D];
            if (j + D < J) wq[j % D] = wtile(j + D);
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(w, xc, acc[b], 0, 0, 0);
            if (b == NB - 1) {  // chunk c done: refill it with the next subtile's, convert chunk c + 1
                xv[c] = *reinterpret_cast<const uint4*>(pn + 32 * c);
                if (c + 1 < KC) xc = res_x16<XDT>(xv[c + 1], sc);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (XDT == RPFQ_BF16) xsv = *xsptr(tl);
        // epilogue: blocks 2p, 2p + 1 -> 32 outputs, 8 per lane
        auto pair_out = [&](int p) -> uint4 {
            uint32_t d[4];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const f32x4 v = acc[2 * p + hb];
                const float4 bq = *reinterpret_cast<const float4*>(bias_s + 32 * p + 16 * hb + 4 * q);
                float v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
                if (scaled) {  // undo the row's prescale (exact) before the bias
                    v0 *= inv;
                    v1 *= inv;
                    v2 *= inv;
                    v3 *= inv;
                }
                d[2 * hb] = res_pack2<YDT>(v0 + bq.x, v1 + bq.y);
                d[2 * hb + 1] = res_pack2<YDT>(v2 + bq.z, v3 + bq.w);
            }
            // lane row q (16 lanes) holds outputs 4 q .. 4 q + 3 of both blocks;
            // swapping odd rows of block 2p with even rows of block 2p + 1
            // leaves 8 consecutive outputs in each lane
            const auto s0 = __builtin_amdgcn_permlane16_swap(d[0], d[2], false, false);
            const auto s1 = __builtin_amdgcn_permlane16_swap(d[1], d[3], false, false);
            return make_uint4(s0[0], s1[0], s0[1], s1[1]);
        };
        auto finish = [&](uint4 o, int i) -> uint4 {  // residual and GELU of store i
            if constexpr (RES != 0) {
                const bool f16 = YDT == RPFQ_F16;
                const uint4 rv = rres[i];
                o = make_uint4(add2_y(o.x, rv.x, f16), add2_y(o.y, rv.y, f16), add2_y(o.z, rv.z, f16),
                               add2_y(o.w, rv.w, f16));
            }
            // the 8 GELUs unrolled (independent chains; the register file has room here):
            // Swin-T stage-0 fc1 + GELU 193-197 -> 171-177 us against the rolled form
            if constexpr (ACT != 0) o = gelu8_y(o, YDT == RPFQ_F16);
            return o;
        };
        // TR rows at a time through this wave's LDS rows (laid out as in
        // y), then copied out 1 KB per instruction: whole 128-B lines
        uint4 po[NB / 2];  // the packed outputs, computed once (the accumulators die as they go)
#pragma unroll
        for (int p = 0; p < NB / 2; ++p) po[p] = pair_out(p);
#pragma unroll
        for (int hh = 0; hh < 16 / TR; ++hh) {
            // no branch around the writes: with one, the compiler has
            // placed the block's reads below inside the masked region
            // (lanes of the other half kept stale registers); those
            // lanes write the wave's scratch area instead
            const uint32_t mine = (TR == 16 || (r >> 3) == hh) ? ~0u : 0u;
            const uint32_t stage0 = (uint32_t)(stage - smem);
            const uint32_t junk_at = (uint32_t)(res_lds_layer(KC, NB) + kResWaves * TR * RP +
                                                (threadIdx.x >> 6) * 512 + 16 * ((r & 7) + 8 * q));
#pragma unroll
            for (int p = 0; p < NB / 2; ++p) {
                const uint32_t real_at = stage0 + (uint32_t)((r - hh * TR) * RP + 64 * p + 2 * ocol);
                const uint32_t at = (real_at & mine) | (junk_at & ~mine);  // a mask, not a branch
                *reinterpret_cast<uint4*>(smem + at) = po[p];
            }
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint4 o = *reinterpret_cast<const uint4*>(stage + stage_at(stage_off(i)));
                const int k = hh * NI + i;
                *reinterpret_cast<uint4*>(reinterpret_cast<char*>(a.y) + out_base(t) + out_off(t, k)) =
                    finish(o, k);
            }
        }
    };
    // whole rounds without a branch around any slot (so the wait before each
    // chunk counts exactly the U - 1 slots issued since), then the rest
    const int64_t n = t0 < nsub ? (nsub - t0 + ws - 1) / ws : 0;  // this wave's subtiles
    const int64_t full = n / U;
    int64_t tb = t0;
#pragma unroll 1
    for (int64_t i = 0; i < full; ++i, tb += U * ws) {
#pragma unroll
        for (int s = 0; s < U; ++s) slot(tb + s * ws, xr[s], xsc[s]);
    }
    const int rest = (int)(n - full * U);
#pragma unroll
    for (int s = 0; s < U - 1; ++s)
        if (s < rest) slot(tb + s * ws, xr[s], xsc[s]);
}

template <int KC, int NB, int RES, int XDT, int YDT, int CB, int ACT>
static hipError_t wide_res_go(WideArgs& a, hipStream_t s) {
    static std::atomic<uint64_t> attr_done{0};
    static std::atomic<int> per_cu{0};  // resident workgroups per CU (occupancy at the largest LDS)
    const void* kern = reinterpret_cast<const void*>(&wide_linear_resident_kernel<KC, NB, RES, XDT, YDT, CB, ACT>);
    const hipError_t e = set_lds_attr_once(kern, kResLdsMax, attr_done);
    if (e != hipSuccess) return e;
    const int lds = resident_lds(a);
    int wg = per_cu.load(std::memory_order_relaxed);
    if (wg <= 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&wg, kern, kResWaves * 64, lds) != hipSuccess || wg < 1)
            wg = 1;
        per_cu.store(wg, std::memory_order_relaxed);  // lds is fixed per (K', N'): one instantiation per shape
    }
    const int64_t nsub = (a.M + 15) / 16;
    // as few waves as give every wave the same number of subtiles (+- 1) in
    // the fewest rounds: the last round is then full
    const int64_t slots = (int64_t)device_cus() * wg * kResWaves;
    const int64_t rounds = (nsub + slots - 1) / slots;
    const int64_t waves = (nsub + rounds - 1) / rounds;
    const int grid = (int)((waves + kResWaves - 1) / kResWaves);
    hipLaunchKernelGGL((wide_linear_resident_kernel<KC, NB, RES, XDT, YDT, CB, ACT>), dim3(grid), dim3(kResWaves * 64),
                       lds, s, a);
    return hipGetLastError();
}

template <int KC, int NB, int XDT, int YDT, int CB>
static hipError_t wide_res_act(WideArgs& a, hipStream_t s) {
    if constexpr (NB <= 12) {
        if (a.res) return wide_res_go<KC, NB, 1, XDT, YDT, CB, 0>(a, s);  // GELU is never fused with a residual
    }
    return a.act ? wide_res_go<KC, NB, 0, XDT, YDT, CB, 1>(a, s) : wide_res_go<KC, NB, 0, XDT, YDT, CB, 0>(a, s);
}

template <int KC, int NB, int CB>
static hipError_t wide_res_dt(WideArgs& a, int xdt, int ydt, hipStream_t s) {
    if (xdt == RPFQ_BF16)
        return ydt == RPFQ_BF16 ? wide_res_act<KC, NB, RPFQ_BF16, RPFQ_BF16, CB>(a, s)
                                : wide_res_act<KC, NB, RPFQ_BF16, RPFQ_F16, CB>(a, s);
    return ydt == RPFQ_BF16 ? wide_res_act<KC, NB, RPFQ_F16, RPFQ_BF16, CB>(a, s)
                            : wide_res_act<KC, NB, RPFQ_F16, RPFQ_F16, CB>(a, s);
}

// The shapes taken (resident_shape): K' = 48 with N' in {48, 96, 144, 192};
// K' = 96 with N' in {48, 96}; K' = 192 with N' = 48 (Swin-T stage 0, its
// stage-1 proj).  Larger products leave no LDS for the staged stores and
// their instantiations spill.
template <int CB>
hipError_t launch_wide_resident(WideArgs& a, int xdt, int ydt, hipStream_t s) {
    if (a.K == 48) {
        switch (a.N) {
            case 48: return wide_res_dt<3, 6, CB>(a, xdt, ydt, s);
            case 96: return wide_res_dt<3, 12, CB>(a, xdt, ydt, s);
            case 144: return wide_res_dt<3, 18, CB>(a, xdt, ydt, s);
            case 192: return wide_res_dt<3, 24, CB>(a, xdt, ydt, s);
            default: return hipErrorInvalidValue;
        }
    }
    if (a.K == 96) {
        if (a.N == 48) return wide_res_dt<6, 6, CB>(a, xdt, ydt, s);
        if (a.N == 96) return wide_res_dt<6, 12, CB>(a, xdt, ydt, s);
        return hipErrorInvalidValue;
    }
    if (a.K == 192 && a.N == 48) return wide_res_dt<12, 6, CB>(a, xdt, ydt, s);
    return hipErrorInvalidValue;
}

template hipError_t launch_wide_resident<RPFQ_CB_SEL>(WideArgs&, int, int, hipStream_t);

}  // namespace rpfq
