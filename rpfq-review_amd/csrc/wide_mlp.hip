// Fused MLP tail of a transformer block: y = residual + fc2(GELU(fc1(x))),
// both layers packed widely-linear layers, in one launch.  Compiled once per
// codebook (RPFQ_CB_SEL); fp16 activations.
#include "rpfq_device.h"

#ifndef RPFQ_CB_SEL
#error "compile once per codebook with -DRPFQ_CB_SEL=<RPFQ_CB_*>"
#endif

namespace rpfq {

// ---------------------------------------------------------------------------
// One workgroup of NW waves per 64-row tile of x (the last tile shifted back
// to end at row M, its rows below the tile boundary stored by the previous
// tile only).  fc1: K' = 32 NW (so x's tile is NW k-steps and fc2 has 32 NW
// complex outputs, one 32-row block per wave), N1' = a multiple of 32 NW.
//   * x's tile goes to LDS once by DMA (k-step w by wave w), in the LDS
//     activation layout of the DMA kernel: a row of a k-step is 8 chunks of
//     16 B (re columns 0-7 .. 24-31, then im), chunk c at slot c ^ ((row >> 1)
//     & 7); optionally the block's LayerNorm of those rows follows, in place
//     (mlp_layer_norm: the row kernel's bits);
//   * fc1 runs in chunks of 32 NW complex outputs: wave w computes outputs
//     32 w .. 32 w + 31 of the chunk for all 64 rows, adds the bias, rounds
//     to fp16 and applies the GELU of the rounded value (as the GEMM stores
//     do), and writes them to LDS as fc2's activation k-step w of the chunk;
//   * fc2 then contracts the chunk's NW k-steps into its accumulators (wave
//     w: fc2 outputs 32 w .. 32 w + 31), so the hidden activations never
//     reach global memory;
//   * both layers decode as the DMA kernel does (same LUT lookups, fuse adds,
//     lane swap, v_mfma_f32_32x32x16_f16 sequence), so each output equals the
//     DMA kernel's for the same operands bit for bit: fc1 with the fused
//     GELU, then fc2 with the residual.
// LUTs: [entry][64 slots] fp16 (re, im) pairs in 8-KB regions at LDS 0 ..
// 8 NW KB; wave w's fc1 table is virtual table w and its fc2 table NW + w,
// table v at region v / 2, slots 32 (v & 1) ... (two tables per region).
// The region number rides in bits 5-7 of the index byte that v_perm_b32
// writes into the address (entry e of region z at z 8 KB + 256 e), so one
// permute still forms each lookup address.
// ---------------------------------------------------------------------------
// 64 x rows per workgroup (32-row tiles, with twice the decode per MFMA,
// measured slower at DeiT-Ti and Swin-T sizes).
constexpr int kMlpBM = 64;
constexpr int kMlpMB = kMlpBM / 32;
constexpr int kMlpStage = kMlpBM * 128;  // one k-step of the tile's activation rows
__device__ __align__(16) const float kMlpZero[4] = {0.0f, 0.0f, 0.0f, 0.0f};

constexpr int mlp_lut_bytes(int nw) { return nw * 8192; }
constexpr int mlp_x_at(int nw) { return mlp_lut_bytes(nw); }
constexpr int mlp_h_at(int nw) { return mlp_x_at(nw) + nw * kMlpStage; }
constexpr int mlp_bias_at(int nw) { return mlp_h_at(nw) + nw * kMlpStage; }
inline int mlp_lds(int nw, int n1) { return mlp_bias_at(nw) + 8 * n1 + 8 * 32 * nw; }
constexpr int kMlpMaxN1 = 1536;  // LDS: 72 KB + the biases (15 KB at N1' = 1536)

// Wave's LUT rows (32 of them, this lane's row r) from the row's (pu, pw)
// in registers (TABLE: the row's 32 values from the blob), into table slot
// `slot` of region base `lut` ([entry][64 slots]).
template <int CB>
__device__ __forceinline__ void mlp_build_lut(uint32_t* lut, int slot, float4 pu, float4 pw, const float4* params,
                                              int64_t n, const RotParams& rot, int g) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t idx = (uint32_t)(g + 2 * j);
        float2 u, w;
        if constexpr (CB == RPFQ_CB_TABLE) {
            const float2* t = reinterpret_cast<const float2*>(params) + n * 32;
            u = t[idx];
            w = t[16 + idx];
        } else {
            u = lut_entry_g<CB>(2 * j, g, pu);
            w = lut_entry_g<CB>(2 * j, g, pw);
        }
        if (rot.rotate) {
            u = derotate(u, rot.cu, rot.su);
            w = derotate(w, rot.cw, rot.sw);
        }
        lut[idx * 64 + slot] = cvt_pk(u.x, u.y);
        lut[(16 + idx) * 64 + slot] = cvt_pk(w.x, w.y);
    }
}

// LayerNorm of the tile's rows in place in LDS (fp16 in, fp16 out), with
// TPR lanes per row in the row kernel's arithmetic (layer_norm_kernel: lane
// sub of a row holds the 8-feature chunks sub, sub + TPR, ..., sums them in
// that order, then a butterfly over the row's lanes; mean and variance in
// float32; ((x - mean) * rstd) * gamma + beta rounded once), so the rows
// are the bits rpfq_layer_norm writes for the same M.  Feature chunk c of
// [re | im] (K' re features, then K' im) sits at k-step (c mod K'/8) / 4,
// LDS chunk (c mod 4) (+4 for im) of the row.
template <int TPR, int NW>
__device__ __forceinline__ void mlp_layer_norm(uint32_t lds_x, const MlpArgs& a, int wave, int lane) {
    constexpr int RPP = 64 / TPR;  // rows per wave and pass
    const int K = a.K, nch = K / 4, nre = K / 8;
    constexpr int NC = TPR == 8 ? 4 : 1;  // chunks per lane (K' <= 128)
    const float C = (float)(2 * K);
    const int sub = lane % TPR;
    for (int r0 = wave * RPP; r0 < kMlpBM; r0 += NW * RPP) {
        const int row = r0 + lane / TPR;
        const uint32_t swz = (uint32_t)((row >> 1) & 7);
        uint32_t addr[NC];
        float v[NC][8];
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = sub + TPR * j;
            const int cc = c < nre ? c : c - nre;
            const uint32_t q = (uint32_t)((cc & 3) + (c < nre ? 0 : 4));
            addr[j] = lds_x + (uint32_t)(cc >> 2) * kMlpStage + (uint32_t)row * 128u + ((q ^ swz) * 16u);
            if (c < nch) {
                const u32x4 u = *reinterpret_cast<__attribute__((address_space(3))) const u32x4*>(addr[j]);
                const uint32_t w[4] = {u[0], u[1], u[2], u[3]};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const half2v h = __builtin_bit_cast(half2v, w[i]);
                    v[j][2 * i] = (float)h.x;
                    v[j][2 * i + 1] = (float)h.y;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[j][e] = 0.0f;
            }
        }
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j)
            if (sub + TPR * j < nch) {
#pragma unroll
                for (int e = 0; e < 8; ++e) s += v[j][e];
            }
        const float mean = group_sum<TPR>(s) / C;
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < NC; ++j)
            if (sub + TPR * j < nch) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float d = v[j][e] - mean;
                    s2 += d * d;
                }
            }
        const float rstd = 1.0f / sqrtf(group_sum<TPR>(s2) / C + a.ln_eps);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const int c = sub + TPR * j;
            if (c < nch) {
                float gk[8], bk[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    gk[e] = a.ln_gamma ? a.ln_gamma[8 * c + e] : 1.0f;
                    bk[e] = a.ln_beta ? a.ln_beta[8 * c + e] : 0.0f;
                }
                float o[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = (v[j][e] - mean) * rstd * gk[e] + bk[e];
                *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(addr[j]) =
                    (u32x4){cvt_pk(o[0], o[1]), cvt_pk(o[2], o[3]), cvt_pk(o[4], o[5]), cvt_pk(o[6], o[7])};
            }
        }
    }
}

template <int CB, int NW, int LN>
__global__ void __launch_bounds__(64 * NW, 2) wide_mlp_kernel(MlpArgs a) {
    extern __shared__ __align__(16) char smem[];
    constexpr int MB = kMlpMB;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 31, g = lane >> 5;
    const int K = a.K, N1 = a.N1;
    const int KS2 = N1 / 32;  // fc2 k-steps
    const int nch = N1 / (32 * NW);

    // tables: fc1 = virtual table wave, fc2 = NW + wave
    const int v1 = wave, v2 = NW + wave;
    uint32_t* lut1 = reinterpret_cast<uint32_t*>(smem + (v1 >> 1) * 8192);
    uint32_t* lut2 = reinterpret_cast<uint32_t*>(smem + (v2 >> 1) * 8192);
    const int slot1 = 32 * (v1 & 1) + r, slot2 = 32 * (v2 & 1) + r;
    // lookup address = (slot << 2) with byte 1 := index | region << 5
    const uint32_t base1 = (uint32_t)slot1 * 4u, base2 = (uint32_t)slot2 * 4u;
    const uint32_t reg1 = (uint32_t)(v1 >> 1) * 0x20202020u, reg2 = (uint32_t)(v2 >> 1) * 0x20202020u;
    const uint32_t lds_x = lds_addr(smem + mlp_x_at(NW)), lds_h = lds_addr(smem + mlp_h_at(NW));
    char* h_s = smem + mlp_h_at(NW);
    const float* b1_s = reinterpret_cast<const float*>(smem + mlp_bias_at(NW));  // [re N1' | im N1']
    const float* b2_s = b1_s + 2 * N1;                                           // [re K' | im K']

    const int tile = (int)blockIdx.x;
    const int64_t m0 = min((int64_t)tile * kMlpBM, a.M - kMlpBM);
    const int64_t m_own = (int64_t)tile * kMlpBM;
    const int64_t ldx = 2 * (int64_t)K;  // fp16 per row of x, y and the residual

    // x's tile, k-step `wave`, rows in 8 groups of 8 (lane l: row l >> 3,
    // slot l & 7 holding chunk (l & 7) ^ ((row >> 1) & 7): two lane offsets
    // by group parity)
    {
        uint32_t voff[2];
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
            const int chunk = (lane & 7) ^ ((4 * jp + (lane >> 4)) & 7);
            voff[jp] = (uint32_t)((lane >> 3) * ldx * 2 + (chunk >> 2) * (int64_t)K * 2 + (chunk & 3) * 16);
        }
        const char* src = reinterpret_cast<const char*>(a.x) + m0 * ldx * 2 + wave * 64;
#pragma unroll
        for (int j = 0; j < kMlpBM / 8; ++j)
            dma_dwordx4(src + 8 * j * ldx * 2, voff[j & 1], lds_x + wave * kMlpStage + j * 1024);
        // biases: 256 B per DMA, spread over the waves
        const int nb1 = 2 * N1 / 64, nb2 = 2 * K / 64;
        for (int j = wave; j < nb1 + nb2; j += NW) {
            const bool first = j < nb1;
            const float* b = first ? a.bias1 : a.bias2;
            const int e0 = 64 * (first ? j : j - nb1);
            dma_dword(b ? (const void*)(b + e0) : (const void*)kMlpZero, b ? 4u * lane : 0u,
                      lds_addr((first ? b1_s : b2_s) + e0));
        }
    }
    // row scales: fc2's (its LUT, built once) and fc1's of chunk 0
    float4 p2u = make_float4(0, 0, 0, 0), p2w = p2u, p1u = p2u, p1w = p2u;
    const int64_t n2 = (int64_t)32 * wave + r;
    if constexpr (CB != RPFQ_CB_TABLE) {
        p2u = a.params2[n2 * 2];
        p2w = a.params2[n2 * 2 + 1];
        p1u = a.params1[n2 * 2];  // chunk 0: fc1 row 32 wave + r
        p1w = a.params1[n2 * 2 + 1];
    }
    // codes: lane l takes the uint4 of MFMA lane l (row l & 31, half l >> 5)
    // of its wave's 32-row block; fc1 block of chunk c = c NW + wave
    const int cl = 2 * (lane & 31) + (lane >> 5);
    auto codes1_of = [&](int c, uint4 (&cw)[NW]) {
        const uint4* src = a.codes1 + (int64_t)(c * NW + wave) * NW * 64 + cl;  // K' = 32 NW: NW k-steps
#pragma unroll
        for (int k = 0; k < NW; ++k) cw[k] = src[k * 64];
    };
    auto codes2_of = [&](int c, uint4 (&cw)[NW]) {
        const uint4* src = a.codes2 + ((int64_t)wave * KS2 + c * NW) * 64 + cl;
#pragma unroll
        for (int k = 0; k < NW; ++k) cw[k] = src[k * 64];
    };
    uint4 cw1[NW], cw2[NW];
    codes1_of(0, cw1);
    codes2_of(0, cw2);
    mlp_build_lut<CB>(lut2, slot2, p2u, p2w, a.params2, n2, a.rot2, g);

    // one k-step: the codes' 4 words are the 4 substeps (columns 8 s + 4 g
    // + e of row r); activation chunk 4 g + s of row 32 i + r of stage
    // `stage` (LDS byte address)
    const uint32_t swz = (uint32_t)((r >> 1) & 7);
    auto kstep = [&](const uint4 cw, uint32_t stage, uint32_t base, uint32_t reg, floatx16 (&acc_re)[MB],
                     floatx16 (&acc_im)[MB]) {
        const uint32_t words[4] = {cw.x, cw.y, cw.z, cw.w};
        auto read_sub = [&](int s, uint32_t (&U)[4], uint32_t (&W)[4], half8 (&ax)[MB]) {
            const uint32_t pu = (words[s] & 0x0f0f0f0fu) | reg;
            const uint32_t pw = ((words[s] >> 4) & 0x0f0f0f0fu) | reg;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t sel = 0x03020000u | ((4u + e) << 8);
                U[e] = *((lds_u32_t)__builtin_amdgcn_perm(pu, base, sel));
                W[e] = *((lds_u32_t)__builtin_amdgcn_perm(pw, base, sel) + 16 * 64);
            }
            const uint32_t ao = stage + (uint32_t)r * 128u + ((((uint32_t)(4 * g + s)) ^ swz) * 16u);
#pragma unroll
            for (int i = 0; i < MB; ++i) ax[i] = *((lds_h8_t)(ao + i * 4096));
        };
        auto decode = [&](const uint32_t (&U)[4], const uint32_t (&W)[4], half8& b_re, half8& b_im) {
            uint32_t p1[4], p2[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) fuse_h(U[e], W[e], p1[e], p2[e]);
            const uint32_t xr0 = __builtin_amdgcn_perm(p1[1], p1[0], 0x05040100u);
            const uint32_t xr1 = __builtin_amdgcn_perm(p1[3], p1[2], 0x05040100u);
            const uint32_t yr0 = __builtin_amdgcn_perm(p1[1], p1[0], 0x07060302u);
            const uint32_t yr1 = __builtin_amdgcn_perm(p1[3], p1[2], 0x07060302u);
            const uint32_t xi0 = __builtin_amdgcn_perm(p2[1], p2[0], 0x05040100u);
            const uint32_t xi1 = __builtin_amdgcn_perm(p2[3], p2[2], 0x05040100u);
            const uint32_t yi0 = __builtin_amdgcn_perm(p2[1], p2[0], 0x07060302u);
            const uint32_t yi1 = __builtin_amdgcn_perm(p2[3], p2[2], 0x07060302u);
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
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            half8 ax_n[MB];
            if (s < 3) read_sub(s + 1, U, W, ax_n);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < MB; ++i) {  // weights are the A operand: rows = outputs, columns = x rows
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
    };

    // x, the biases and both tables are in LDS
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if constexpr (LN != 0) {  // normalize the rows in place; fc1 reads them after the barrier
        mlp_layer_norm<LN, NW>(lds_x, a, wave, lane);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    }

    floatx16 acc2_re[MB], acc2_im[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc2_re[i] = acc2_im[i] = floatx16{0};
#pragma unroll 1
    for (int c = 0; c < nch; ++c) {
        // fc1 rows 32 (c NW + wave) + r: this chunk's table, then the next
        // chunk's scales
        const int64_t n1 = (int64_t)32 * (c * NW + wave) + r;
        mlp_build_lut<CB>(lut1, slot1, p1u, p1w, a.params1, n1, a.rot1, g);
        if constexpr (CB != RPFQ_CB_TABLE) {
            const int64_t nn = c + 1 < nch ? n1 + 32 * NW : n1;
            p1u = a.params1[nn * 2];
            p1w = a.params1[nn * 2 + 1];
        }
        floatx16 acc1_re[MB], acc1_im[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) acc1_re[i] = acc1_im[i] = floatx16{0};
#pragma unroll
        for (int k = 0; k < NW; ++k) kstep(cw1[k], lds_x + k * kMlpStage, base1, reg1, acc1_re, acc1_im);
        codes1_of(c + 1 < nch ? c + 1 : c, cw1);

        // every wave is past the previous chunk's fc2 reads of h
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // hidden values: output 8 q + 4 g + t of this wave's 32 (= column of
        // fc2's k-step `wave`), x row 32 i + r: fp16 of acc + bias, GELU of
        // the rounded value, re to chunk q and im to chunk 4 + q, 8 B at 8 g
        {
            const int nb = 32 * (c * NW + wave);
            char* hrow = h_s + wave * kMlpStage + r * 128 + 8 * g;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 bre = *reinterpret_cast<const float4*>(b1_s + nb + 8 * q + 4 * g);
                const float4 bim = *reinterpret_cast<const float4*>(b1_s + N1 + nb + 8 * q + 4 * g);
                const uint32_t so_re = ((uint32_t)q ^ swz) * 16u, so_im = ((uint32_t)(4 + q) ^ swz) * 16u;
#pragma unroll
                for (int i = 0; i < MB; ++i) {
                    const uint2 hr = make_uint2(
                        gelu2_y(cvt_pk(acc1_re[i][4 * q] + bre.x, acc1_re[i][4 * q + 1] + bre.y), true),
                        gelu2_y(cvt_pk(acc1_re[i][4 * q + 2] + bre.z, acc1_re[i][4 * q + 3] + bre.w), true));
                    const uint2 hi = make_uint2(
                        gelu2_y(cvt_pk(acc1_im[i][4 * q] + bim.x, acc1_im[i][4 * q + 1] + bim.y), true),
                        gelu2_y(cvt_pk(acc1_im[i][4 * q + 2] + bim.z, acc1_im[i][4 * q + 3] + bim.w), true));
                    *reinterpret_cast<uint2*>(hrow + i * 4096 + so_re) = hr;
                    *reinterpret_cast<uint2*>(hrow + i * 4096 + so_im) = hi;
                }
            }
        }
        // the chunk's hidden activations are complete
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < NW; ++k) kstep(cw2[k], lds_h + k * kMlpStage, base2, reg2, acc2_re, acc2_im);
        codes2_of(c + 1 < nch ? c + 1 : c, cw2);
    }

    // y = fp16(acc + bias) (+ residual in fp16), outputs 32 wave + 8 q + 4 g
    // + t of x row m0 + 32 i + r; rows below m_own belong to the previous tile
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int64_t m = m0 + 32 * i + r;
        if (m < m_own) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n0 = 32 * wave + 8 * q + 4 * g;
            const float4 bre = *reinterpret_cast<const float4*>(b2_s + n0);
            const float4 bim = *reinterpret_cast<const float4*>(b2_s + K + n0);
            uint2 yr = make_uint2(cvt_pk(acc2_re[i][4 * q] + bre.x, acc2_re[i][4 * q + 1] + bre.y),
                                  cvt_pk(acc2_re[i][4 * q + 2] + bre.z, acc2_re[i][4 * q + 3] + bre.w));
            uint2 yi = make_uint2(cvt_pk(acc2_im[i][4 * q] + bim.x, acc2_im[i][4 * q + 1] + bim.y),
                                  cvt_pk(acc2_im[i][4 * q + 2] + bim.z, acc2_im[i][4 * q + 3] + bim.w));
            uint16_t* dst = reinterpret_cast<uint16_t*>(a.y) + m * ldx + n0;
            if (a.res) {
                const uint16_t* rs = reinterpret_cast<const uint16_t*>(a.res) + m * ldx + n0;
                const uint2 rr = *reinterpret_cast<const uint2*>(rs), ri = *reinterpret_cast<const uint2*>(rs + K);
                yr = make_uint2(add2_y(yr.x, rr.x, true), add2_y(yr.y, rr.y, true));
                yi = make_uint2(add2_y(yi.x, ri.x, true), add2_y(yi.y, ri.y, true));
            }
            *reinterpret_cast<uint2*>(dst) = yr;
            *reinterpret_cast<uint2*>(dst + K) = yi;
        }
    }
}

template <int CB, int NW, int LN>
static hipError_t mlp_go(const MlpArgs& a, hipStream_t s) {
    static std::atomic<uint64_t> attr_done{0};
    const void* kern = reinterpret_cast<const void*>(&wide_mlp_kernel<CB, NW, LN>);
    const int lds = mlp_lds(NW, a.N1);
    hipError_t e = set_lds_attr_once(kern, mlp_lds(NW, kMlpMaxN1), attr_done);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((wide_mlp_kernel<CB, NW, LN>), dim3((unsigned)a.tiles), dim3(64 * NW), lds, s, a);
    return hipGetLastError();
}

template <int CB>
hipError_t launch_wide_mlp(const MlpArgs& args, hipStream_t s) {
    MlpArgs a = args;
    a.tiles = (int)((a.M + kMlpBM - 1) / kMlpBM);
    if (!(a.K == 96 && a.N1 % 96 == 0 && a.N1 <= kMlpMaxN1 && a.M >= kMlpBM)) return hipErrorInvalidValue;
    switch (a.ln) {
        case 0: return mlp_go<CB, 3, 0>(a, s);
        case 8: return mlp_go<CB, 3, 8>(a, s);
        case 64: return mlp_go<CB, 3, 64>(a, s);
        default: return hipErrorInvalidValue;
    }
}

template hipError_t launch_wide_mlp<RPFQ_CB_SEL>(const MlpArgs&, hipStream_t);

}  // namespace rpfq
