// Widely-linear GEMM for fp16 or bf16 activations staged by LDS DMA (large M).
// Compiled once per codebook (RPFQ_CB_SEL).
#include <type_traits>

#include "rpfq_device.h"

#ifndef RPFQ_CB_SEL
#error "compile once per codebook with -DRPFQ_CB_SEL=<RPFQ_CB_*>"
#endif

namespace rpfq {

// ---------------------------------------------------------------------------
// widely-linear GEMM, fp16 / bf16 activations staged by LDS DMA (large M)
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
// per-row scales of the next tile, staged by DMA: [wave][32 rows][pu | pw] float4 pairs
constexpr int kDmaParams = 4 * 1024;
template <int BM> constexpr int dma_params_at() { return dma_bias_at<BM>() + kDmaBias; }
// row prescales (WideArgs::xs) of the current and the next tile: [2][BM] floats
template <int BM> constexpr int dma_xs_at() { return dma_params_at<BM>() + kDmaParams; }
template <int BM> constexpr int dma_lds() { return dma_xs_at<BM>() + 2 * BM * 4; }  // 79872 B (BM = 128)
static_assert(2 * dma_lds<128>() <= 160 * 1024, "two workgroups per CU");
static_assert(4 * 64 * kTRow <= kDmaStages * dma_stage<128>(), "epilogue half tile fits the stages");
static_assert(4 * 128 * kTRow <= kDmaStages * dma_stage<256>(), "epilogue half tile fits the stages");


// LUT of one output row in the wave-pair layout: entry e (0..15 U, 16..31 W)
// of row slot `slot` at lut_pair[64 e + slot]; lane group g writes the even
// or odd indices.  Same values as build_lut.
// staged: the row's (pu, pw) at staged[0..1] (LDS) instead of the blob.
template <int CB>
__device__ __forceinline__ void build_lut_slot(uint32_t* lut_pair, int slot, const float4* params, int64_t n,
                                               int nblk, int blk, const RotParams& rot, int g,
                                               const float4* staged = nullptr) {
    float4 pu = make_float4(0, 0, 0, 0), pw = make_float4(0, 0, 0, 0);
    if constexpr (CB != RPFQ_CB_TABLE) {
        const float4* p = staged ? staged : params + (n * nblk + blk) * 2;
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
            u = lut_entry_g<CB>(2 * j, g, pu);
            w = lut_entry_g<CB>(2 * j, g, pw);
        }
        if (rot.rotate) {
            u = derotate(u, rot.cu, rot.su);
            w = derotate(w, rot.cw, rot.sw);
        }
        lut_pair[idx * 64 + slot] = cvt_pk(u.x, u.y);
        lut_pair[(16 + idx) * 64 + slot] = cvt_pk(w.x, w.y);
    }
}

// bf16 activations: the DMA stages raw bf16 and each wave rewrites the rows
// it loaded as fp16 in place once they land (v_cvt_pk_f16_f32 of the exact
// float32 value: exact for |x| in [2^-14, 65504], rounded in the fp16
// subnormal range, +-inf beyond; the conversion every other kernel applies
// on load), mid-k-step for the next stage, before the barrier that
// publishes it.  Costs ~20% of the kernel at ViT-B/16 bs256 (the LDS
// traffic of the rewrite; converting each MFMA operand in registers instead,
// 4 times over, costs ~35%).  srow: LDS byte address of the prescales of
// the NROWS rows (WideArgs::xs), applied before the conversion (exact), or
// 0 for none (address 0 holds a LUT, never the prescales).
template <int XDT, int NROWS>
__device__ __forceinline__ void stage_to_f16(uint32_t rows, int lane, uint32_t srow) {
    if constexpr (XDT == RPFQ_BF16) {
#pragma unroll
        for (int j = 0; j < NROWS * 128 / 1024; ++j) {  // NROWS rows of 128 B: 16-B chunks, 64 lanes
            const uint32_t addr = rows + (uint32_t)(j * 64 + lane) * 16u;
            const u32x4 v = *reinterpret_cast<__attribute__((address_space(3))) const u32x4*>(addr);
            u32x4 o;
            if (srow) {
                // chunk j 64 + lane lies in row 8 j + lane / 8
                const float sc = *reinterpret_cast<__attribute__((address_space(3))) const float*>(
                    srow + (uint32_t)(8 * j + (lane >> 3)) * 4u);
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    o[t] = pack_h2(bf16_to_f32(v[t] & 0xffffu) * sc, bf16_to_f32(v[t] >> 16) * sc);
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t) o[t] = pack_h2(bf16_to_f32(v[t] & 0xffffu), bf16_to_f32(v[t] >> 16));
            }
            *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(addr) = o;
        }
    }
}

// ACT (compile time, = WideArgs::act): the fused GELU's code stays out of
// the plain instantiation, whose k-loop runs at the edge of the register file.
// XDT: RPFQ_F16 or RPFQ_BF16 (converted in LDS, above).
template <int BM, int XDT, int YDT, int CB, int ACT>
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
    float* bias_s = reinterpret_cast<float*>(smem + dma_bias_at<BM>()) + wave * 64;  // [wave][re 32 | im 32]
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
    // Per-row scales (one scale block per row) of a tile are DMA'd into LDS
    // together with its first codes and activations (before the previous
    // tile's epilogue), so the tile start builds its LUT from LDS without a
    // global load whose wait would drain the activation prefetch.
    const float4* pstage = reinterpret_cast<const float4*>(smem + dma_params_at<BM>() + wave * 1024);
    const bool staged = CB != RPFQ_CB_TABLE && a.nblk == 1;
    // bf16 x with row prescales: wave w's RPW rows of a tile, DMA'd with the
    // tile's first loads into buffer (tile iteration & 1), RPW lanes of 4 B
    float* xs_lds = reinterpret_cast<float*>(smem + dma_xs_at<BM>());
    // row prescales: bf16 rows are multiplied in the stage; fp16 rows arrive
    // prescaled (written so by rpfq_layer_norm_prescaled); both unscaled below
    const bool scaled = a.xs != nullptr;
    auto issue_xs = [&](int vb_t, int buf) {
        if (!scaled) return;
        const int t = xcd_tile(vb_t, total);
        const int64_t m0_t = min((int64_t)(t / a.tiles_n) * BM, a.M - BM);
        if (lane < RPW) dma_dword(a.xs + m0_t + RPW * wave, (uint32_t)lane * 4u, lds_addr(xs_lds + buf * BM + RPW * wave));
    };
    int it = 0;  // tile iteration of this workgroup
    auto issue_params = [&](int vb_t) {  // this wave's 32 rows of tile vb_t; lane l: row l / 2, half l % 2
        if (!staged) return;
        const int t = xcd_tile(vb_t, total);
        const int ntw_t = (t - (t / a.tiles_n) * a.tiles_n) * 4 + wave;
        const int nt = ntw_t < a.NT ? ntw_t : a.NT - 1;
        dma_dwordx4(a.params + (int64_t)nt * 64, (uint32_t)lane * 16u, lds_addr(pstage));
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

    const int xb = it & 1;  // this tile's prescale buffer
    const uint32_t srow = scaled ? lds_addr(xs_lds + xb * BM + RPW * wave) : 0u;
    if (vb == (int)blockIdx.x) {  // later tiles had these requested before the previous epilogue
        issue_codes(0, 0);
        if (a.KS > 1) issue_codes(1, 1);
        issue_x(0, 2);
        issue_params(vb);
        issue_xs(vb, xb);
    }
    {   // bias of this wave's 32 output rows (0 past N or without bias), read in the epilogue;
        // loaded before the next k-step's DMA, so its wait covers only loads this tile needs now
        const int64_t nn = (int64_t)ntw * 32 + r;
        const bool ok = a.bias && active && nn < a.N;
        bias_s[g * 32 + r] = ok ? a.bias[g * (int64_t)a.N + nn] : 0.0f;
    }
    issue_x(a.KS > 1 ? 1 : 0, 0);
    int cur_blk = 0;
    if (staged) {
        // staged scales and bias landed (every load but the newest k-step's)
        if (RPW == 32)
            asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        build_lut_slot<CB>(lut_pair, slot, a.params, 0, a.nblk, 0, a.rot, g, pstage + 2 * r);
    } else {
        build_lut_slot<CB>(lut_pair, slot, a.params, (int64_t)ntw_ld * 32 + r, a.nblk, 0, a.rot, g);
    }
    // codes and stage 2 landed (at most the newest k-step's loads in flight), LUT written
    if (RPW == 32)
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    if constexpr (XDT == RPFQ_BF16) {
        stage_to_f16<XDT, RPW>(lds_stages + 2 * kDmaStage, lane, srow);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // One k-step on stage `st`: the lane's codes of k-step ks into
    // registers, which frees their buffer for the codes of ks + 2; then the
    // codes and activations of ks + 2 (the activation stage read at ks - 1,
    // free since the last barrier), so both arrive two k-steps ahead; then
    // the math.  The loop below is unrolled by 3 so stage offsets are static.
    auto kstep = [&](int ks, int st) {
        const uint4 cw = read_codes(ks & 1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // cw landed: its buffer takes k-step ks + 2
        if (ks + 2 < a.KS) {
            issue_codes(ks + 2, ks & 1);
            issue_x(ks + 2, st == 0 ? 2 : st - 1);
        }
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
            if constexpr (XDT == RPFQ_BF16) {
                // mid-step: the activations of ks + 1 (requested two k-steps
                // ago; only this step's codes and activations are younger)
                // have landed; this wave's rows go to fp16 beside the MFMAs
                if (s == 1 && ks + 1 < a.KS) {
                    if (ks + 2 < a.KS) {
                        if (RPW == 32)
                            asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
                        else
                            asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
                    } else {
                        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    }
                    stage_to_f16<XDT, RPW>(lds_stages + (st == 2 ? 0 : st + 1) * kDmaStage, lane, srow);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (ks + 1 < a.KS) {
            const int nb = (ks + 1) / a.block_ks;
            if (nb != cur_blk) {  // new scale block: this wave's LUT rows only
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                build_lut_slot<CB>(lut_pair, slot, a.params, (int64_t)ntw_ld * 32 + r, a.nblk, nb, a.rot, g);
                cur_blk = nb;
            }
        }
        // codes ks + 1 and stage ks + 1 landed: only the newest 1 + RPW / 8
        // loads (codes and activations of ks + 2) may still be in flight;
        // every LDS read of this k-step is complete.  Near the end nothing is
        // prefetched, so everything must land.
        if (ks + 2 < a.KS) {
            if (RPW == 32)
                asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(9) lgkmcnt(0)" ::: "memory");
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
        if (a.KS > 1) issue_codes(1, 1);
        issue_x(0, 2);
        issue_params(vb + (int)gridDim.x);
        issue_xs(vb + (int)gridDim.x, xb ^ 1);
    }
    if (scaled) {  // undo the rows' prescales (exact) before the bias: subtile i, lane r holds x row 32 i + r
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const float inv = row_unscale(xs_lds[xb * BM + 32 * i + r]);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                acc_re[i][v] *= inv;
                acc_im[i][v] *= inv;
            }
        }
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
        const float4 b0 = *reinterpret_cast<const float4*>(bias_s + 8 * q + 4 * g);
        const float4 b1 = *reinterpret_cast<const float4*>(bias_s + 32 + 8 * q + 4 * g);
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
                    // plain stores: each covers 16 B of a 128-B line the wave's
                    // other stores complete, which L2 merges; non-temporal
                    // partial lines went to memory one by one (qkv 523 -> 281 us)
                    *reinterpret_cast<f32x4*>(yr) = (f32x4){vr[0], vr[1], vr[2], vr[3]};
                    *reinterpret_cast<f32x4*>(yi) = (f32x4){vi[0], vi[1], vi[2], vi[3]};
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
    // one half of the tile; h is a compile-time constant so the accumulator
    // indices stay static (a runtime h would move them to scratch memory)
    auto epi_half = [&](auto h_c) {
        constexpr int h = decltype(h_c)::value;
        // zeros where no residual is read: left undefined, the value would
        // flow around the persistent loop and hold ~10 VGPRs through the k-loop
        uint4 rres[RPS] = {};
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
                    pr = make_uint2(pack_bf2(acc_re[i][4 * q] + bre[4 * q], acc_re[i][4 * q + 1] + bre[4 * q + 1]),
                                    pack_bf2(acc_re[i][4 * q + 2] + bre[4 * q + 2], acc_re[i][4 * q + 3] + bre[4 * q + 3]));
                    pi = make_uint2(pack_bf2(acc_im[i][4 * q] + bim[4 * q], acc_im[i][4 * q + 1] + bim[4 * q + 1]),
                                    pack_bf2(acc_im[i][4 * q + 2] + bim[4 * q + 2], acc_im[i][4 * q + 3] + bim[4 * q + 3]));
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
                if constexpr (ACT != 0) v = gelu8_y(v, YDT == RPFQ_F16);
                // whole 128-byte lines stream past the cache; the per-wave half lines are
                // left for L2 to merge (non-temporal partial lines measured slower)
                if (wg)
                    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4*>(dst));
                else
                    *reinterpret_cast<u32x4*>(dst) = __builtin_bit_cast(u32x4, v);
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
        };
    epi_half(std::integral_constant<int, 0>{});
    epi_half(std::integral_constant<int, 1>{});
    }
    // every wave is done with this tile's LDS before the next tile refills it
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    ++it;
    }
}

template <int BM, int XDT, int YDT, int CB, int ACT>
static hipError_t wide_dma_act(WideArgs& a, hipStream_t s) {
    static std::atomic<uint64_t> attr_done{0};
    constexpr int lds = dma_lds<BM>();
    const hipError_t e = set_lds_attr_once(
        reinterpret_cast<const void*>(&wide_linear_dma_kernel<BM, XDT, YDT, CB, ACT>), lds, attr_done);
    if (e != hipSuccess) return e;
    a.tiles_m = (int)((a.M + BM - 1) / BM);
    a.tiles_n = (int)((a.NT + 3) / 4);
    const int total = a.tiles_m * a.tiles_n;
    const int slots = (BM == 128 ? 2 : 1) * device_cus();  // workgroups resident per CU
    const int grid = total < slots ? total : slots;
    hipLaunchKernelGGL((wide_linear_dma_kernel<BM, XDT, YDT, CB, ACT>), dim3(grid), dim3(256), lds, s, a);
    return hipGetLastError();
}

template <int BM, int XDT, int YDT, int CB>
static hipError_t wide_dma_go(WideArgs& a, hipStream_t s) {
    // GELU with bf16 x and y: not routed here (the register-staged kernel measured as fast)
    if constexpr (YDT == RPFQ_BF16 && XDT == RPFQ_BF16) return wide_dma_act<BM, XDT, YDT, CB, 0>(a, s);
    else return a.act ? wide_dma_act<BM, XDT, YDT, CB, 1>(a, s) : wide_dma_act<BM, XDT, YDT, CB, 0>(a, s);
}

template <int XDT, int CB>
static hipError_t wide_dma_y(WideArgs& a, int ydt, hipStream_t s) {
    switch (ydt) {
        case RPFQ_F32: return wide_dma_go<128, XDT, RPFQ_F32, CB>(a, s);
        case RPFQ_F16: return wide_dma_go<128, XDT, RPFQ_F16, CB>(a, s);
        default: return wide_dma_go<128, XDT, RPFQ_BF16, CB>(a, s);
    }
}

template <int CB>
hipError_t launch_wide_dma(WideArgs& a, int xdt, int ydt, hipStream_t s) {
    return xdt == RPFQ_BF16 ? wide_dma_y<RPFQ_BF16, CB>(a, ydt, s) : wide_dma_y<RPFQ_F16, CB>(a, ydt, s);
}

template hipError_t launch_wide_dma<RPFQ_CB_SEL>(WideArgs&, int, int, hipStream_t);

}  // namespace rpfq
