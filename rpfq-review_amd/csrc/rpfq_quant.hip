// Training-semantics weight quantization of one QATLinearComplexPhase weight
// on the GPU (RPFQ-ViT-main/quant_models/quant_i.py:513-544 with the
// quantizers of :29-118 and the rotation of :425-435).
//
// Per element (n, k) of the complex planes the kernels recompute, in float32
// and in the reference's op order:
//   U = 0.5 (A11 + A22) + i 0.5 (A21 - A12),  W = 0.5 (A11 - A22) + i 0.5 (A12 + A21)
//   optional w e^{-i theta}:  (re c + im s, im c - re s)
//   residual stages q += step, r -= step (step from the stage's scale)
//   optional q e^{+i theta}:  (re c - im s, im c + re s)
//   A_q = [[Wre + Ure, Wim - Uim], [Wim + Uim, -Wre + Ure]]
// A stage's scale is a mean over the whole plane, so each stage is one
// reduction launch (per-block float64 partials of the masked |r| sums and
// counts), one single-block finalize launch (fixed-order float64 sum,
// rounded once to float32, then the reference's float32 division and clamp),
// and the last launch writes A_q and the 2-bit code planes.  Nothing is
// stored between launches except the partials and the scales: every launch
// recomputes the earlier stages from the weight (a few VALU per stage), so
// the weight is read once per launch and never written back.
//
// The float64 sums make each scale the float32 rounding of the exact sum
// (the reference sums float32 in torch's order; both agree to ~1 ulp and the
// CPU restatement uses the same float64 convention).  Results are
// deterministic: the partition into blocks and the reduction order are fixed.
#include <mutex>

#include "rpfq_internal.h"

namespace rpfq {
namespace {

constexpr int kQThreads = 256;
constexpr float kAxisFloor = 1e-5f;  // _safe_mean_abs min_val, quant_i.py:29
constexpr float kSignFloor = 1e-6f;  // EPS, quant_i.py:26, :86-87

struct QuantArgs {
    const float* w;    // [2N, 2K] row-major
    const float* rot;  // NULL or [cos_u, sin_u, cos_w, sin_w]
    int64_t N, K;
    int kind[2], steps[2];
    float* scales;     // [2][4][2]: plane (U, W), stage, (re, im)
    double* partial;   // [blocks][8]
    float* aq;         // NULL or [2N, 2K]
    uint8_t* codes;    // NULL or [steps_u + steps_w][N][K/4]
    int stage;         // stage being reduced / finalized
    int nblocks;       // reduction blocks
};

// Axis class of (re, im) as the exporter codes it (quant_i.py:36-62,
// export_rpfq_vit_to_mlx.py:214-218): 1 real_pos, 0 real_neg, 3 imag_pos,
// 2 imag_neg; 4 = no mask set (only for NaN input), stored as code 0.
__device__ __forceinline__ int axis_class(float re, float im) {
    float ar = fabsf(re), ai = fabsf(im);
    if (ar > ai) return re >= 0.0f ? 1 : 0;
    if (ai > ar) return im >= 0.0f ? 3 : 2;
    if (re == 0.0f && im == 0.0f) return 1;  // zero tie -> real_pos
    if (re > 0.0f && im > 0.0f) return 3;    // quadrant I tie -> imag_pos
    if (re < 0.0f && im > 0.0f) return 0;    // quadrant II tie -> real_neg
    if (re < 0.0f && im < 0.0f) return 2;    // quadrant III tie -> imag_neg
    if (re > 0.0f && im < 0.0f) return 1;    // quadrant IV tie -> real_pos
    return 4;
}

// One plane's running state: residual r and accumulated q.
struct Plane {
    float r_re, r_im, q_re, q_im;
};

// Applies stage t with scales (s_re, s_im); returns the code.
template <int KIND>
__device__ __forceinline__ uint32_t apply_stage(Plane& p, float s_re, float s_im) {
    float v_re, v_im;
    uint32_t code;
    if (KIND == RPFQ_QK_SIGN) {  // quant_i.py:84-91
        bool pr = p.r_re >= 0.0f, pi = p.r_im >= 0.0f;
        v_re = pr ? s_re : -s_re;
        v_im = pi ? s_im : -s_im;
        code = (pr ? 1u : 0u) | (pi ? 2u : 0u);
    } else {  // quant_i.py:65-81
        int c = axis_class(p.r_re, p.r_im);
        v_re = c == 1 ? s_re : (c == 0 ? -s_re : 0.0f);
        v_im = c == 3 ? s_im : (c == 2 ? -s_im : 0.0f);
        code = c == 4 ? 0u : (uint32_t)c;
    }
    p.q_re = p.q_re + v_re;  // quant_i.py:114-117
    p.q_im = p.q_im + v_im;
    p.r_re = p.r_re - v_re;
    p.r_im = p.r_im - v_im;
    return code;
}

__device__ __forceinline__ uint32_t apply_stage_k(int kind, Plane& p, float s_re, float s_im) {
    return kind == RPFQ_QK_SIGN ? apply_stage<RPFQ_QK_SIGN>(p, s_re, s_im) : apply_stage<RPFQ_QK_AXIS>(p, s_re, s_im);
}

// U and W of element (n, k), rotated for quantization when rot is set
// (quant_i.py:519-527, :429-430).
__device__ __forceinline__ void load_planes(const QuantArgs& a, int64_t n, int64_t k, Plane& u, Plane& w) {
    const int64_t row = 2 * a.K;
    float a11 = a.w[n * row + k], a12 = a.w[n * row + a.K + k];
    float a21 = a.w[(a.N + n) * row + k], a22 = a.w[(a.N + n) * row + a.K + k];
    u.r_re = 0.5f * (a11 + a22);
    u.r_im = 0.5f * (a21 - a12);
    w.r_re = 0.5f * (a11 - a22);
    w.r_im = 0.5f * (a12 + a21);
    if (a.rot) {
        float cu = a.rot[0], su = a.rot[1], cw = a.rot[2], sw = a.rot[3];
        float ur = u.r_re * cu + u.r_im * su, ui = u.r_im * cu - u.r_re * su;
        float wr = w.r_re * cw + w.r_im * sw, wi = w.r_im * cw - w.r_re * sw;
        u.r_re = ur; u.r_im = ui;
        w.r_re = wr; w.r_im = wi;
    }
    u.q_re = u.q_im = w.q_re = w.q_im = 0.0f;
}

// V consecutive columns k0.. of U and W (V = 4: one 16-B load per quadrant
// of the weight; K % 4 == 0 keeps the loads aligned).
template <int V>
__device__ __forceinline__ void load_planes_v(const QuantArgs& a, int64_t n, int64_t k0, Plane (&u)[V],
                                              Plane (&w)[V]) {
    if constexpr (V == 4) {
        const int64_t row = 2 * a.K;
        const float4 q11 = *reinterpret_cast<const float4*>(a.w + n * row + k0);
        const float4 q12 = *reinterpret_cast<const float4*>(a.w + n * row + a.K + k0);
        const float4 q21 = *reinterpret_cast<const float4*>(a.w + (a.N + n) * row + k0);
        const float4 q22 = *reinterpret_cast<const float4*>(a.w + (a.N + n) * row + a.K + k0);
        const float v11[4] = {q11.x, q11.y, q11.z, q11.w}, v12[4] = {q12.x, q12.y, q12.z, q12.w};
        const float v21[4] = {q21.x, q21.y, q21.z, q21.w}, v22[4] = {q22.x, q22.y, q22.z, q22.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            u[v].r_re = 0.5f * (v11[v] + v22[v]);
            u[v].r_im = 0.5f * (v21[v] - v12[v]);
            w[v].r_re = 0.5f * (v11[v] - v22[v]);
            w[v].r_im = 0.5f * (v12[v] + v21[v]);
            if (a.rot) {
                const float cu = a.rot[0], su = a.rot[1], cw = a.rot[2], sw = a.rot[3];
                const float ur = u[v].r_re * cu + u[v].r_im * su, ui = u[v].r_im * cu - u[v].r_re * su;
                const float wr = w[v].r_re * cw + w[v].r_im * sw, wi = w[v].r_im * cw - w[v].r_re * sw;
                u[v].r_re = ur; u[v].r_im = ui;
                w[v].r_re = wr; w[v].r_im = wi;
            }
            u[v].q_re = u[v].q_im = w[v].q_re = w[v].q_im = 0.0f;
        }
    } else {
        load_planes(a, n, k0, u[0], w[0]);
    }
}

// Row and first column of work item `it` (V columns each); 32-bit division
// when the item count allows it.
template <int V>
__device__ __forceinline__ void item_nk(const QuantArgs& a, int64_t it, bool small, int64_t& n, int64_t& k0) {
    const int64_t kv = a.K / V;
    if (small) {
        const uint32_t ni = (uint32_t)it / (uint32_t)kv;
        n = ni;
        k0 = ((int64_t)((uint32_t)it - ni * (uint32_t)kv)) * V;
    } else {
        n = it / kv;
        k0 = (it - n * kv) * V;
    }
}

// Masked |r| sums and counts of stage a.stage for U (0..3) and W (4..7):
// (sum |re| over the real mask, count, sum |im| over the imaginary mask,
// count); SIGN planes count every element.
template <int V>
__global__ void __launch_bounds__(kQThreads) quant_reduce_kernel(QuantArgs a) {
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int64_t items = a.N * (a.K / V);
    const bool small = items < (1LL << 31);
    const int st = a.stage;
    float sc[16];  // scales of the finished stages (finalized by earlier launches)
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = a.scales[i];
    for (int64_t it = (int64_t)blockIdx.x * kQThreads + threadIdx.x; it < items;
         it += (int64_t)a.nblocks * kQThreads) {
        int64_t n, k0;
        item_nk<V>(a, it, small, n, k0);
        Plane u[V], w[V];
        load_planes_v<V>(a, n, k0, u, w);
#pragma unroll
        for (int v = 0; v < V; ++v) {
            Plane* pl[2] = {&u[v], &w[v]};
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                if (a.steps[p] <= st) continue;
                Plane& q = *pl[p];
#pragma unroll
                for (int t = 0; t < 3; ++t)
                    if (t < st) apply_stage_k(a.kind[p], q, sc[(p * 4 + t) * 2], sc[(p * 4 + t) * 2 + 1]);
                if (a.kind[p] == RPFQ_QK_SIGN) {
                    acc[4 * p + 0] += (double)fabsf(q.r_re);
                    acc[4 * p + 1] += 1.0;
                    acc[4 * p + 2] += (double)fabsf(q.r_im);
                    acc[4 * p + 3] += 1.0;
                } else {
                    const int c = axis_class(q.r_re, q.r_im);
                    if (c == 0 || c == 1) {
                        acc[4 * p + 0] += (double)fabsf(q.r_re);
                        acc[4 * p + 1] += 1.0;
                    } else if (c == 2 || c == 3) {
                        acc[4 * p + 2] += (double)fabsf(q.r_im);
                        acc[4 * p + 3] += 1.0;
                    }
                }
            }
        }
    }
    // fixed-order block reduction: wave butterfly, then the 4 waves in order
    __shared__ double red[kQThreads / 64][8];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        double v = acc[j];
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) red[wv][j] = v;
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        double v = 0.0;
        for (int i = 0; i < kQThreads / 64; ++i) v += red[i][threadIdx.x];
        a.partial[(int64_t)blockIdx.x * 8 + threadIdx.x] = v;
    }
}

// Sums the partials in a fixed order and writes stage a.stage's scales:
// axis: max((float)sum / max((float)count, 1), 1e-5) (quant_i.py:29-33);
// sign: max((float)sum / (float)(N K), 1e-6) (quant_i.py:86-87, torch's CPU
// mean = sum / numel).  Stage 0 also clears every scale slot.
__global__ void __launch_bounds__(kQThreads) quant_finalize_kernel(QuantArgs a) {
    __shared__ double red[kQThreads / 64][8];
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = threadIdx.x; b < a.nblocks; b += kQThreads)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += a.partial[(int64_t)b * 8 + j];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        double v = acc[j];
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if (lane == 0) red[wv][j] = v;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    double tot[8];
    for (int j = 0; j < 8; ++j) {
        double v = 0.0;
        for (int i = 0; i < kQThreads / 64; ++i) v += red[i][j];
        tot[j] = v;
    }
    if (a.stage == 0)
        for (int i = 0; i < 16; ++i) a.scales[i] = 0.0f;
    for (int p = 0; p < 2; ++p) {
        if (a.steps[p] <= a.stage) continue;
        float sc[2];
        for (int h = 0; h < 2; ++h) {
            float num = (float)tot[4 * p + 2 * h];
            float m, floor_v;
            if (a.kind[p] == RPFQ_QK_SIGN) {
                m = num / (float)(a.N * a.K);
                floor_v = kSignFloor;
            } else {
                float den = (float)tot[4 * p + 2 * h + 1];
                m = num / (den < 1.0f ? 1.0f : den);
                floor_v = kAxisFloor;
            }
            sc[h] = m < floor_v ? floor_v : m;  // clamp_min (NaN passes through)
        }
        a.scales[(p * 4 + a.stage) * 2] = sc[0];
        a.scales[(p * 4 + a.stage) * 2 + 1] = sc[1];
    }
}

// All stages with the final scales: A_q (rotated back, recombined) and the
// code planes.  V consecutive columns per thread (V = 4 writes one packed
// code byte per plane and stage).
template <int V>
__global__ void __launch_bounds__(kQThreads) quant_apply_kernel(QuantArgs a) {
    const int64_t items = a.N * (a.K / V);
    const bool small = items < (1LL << 31);
    const int64_t row = 2 * a.K;
    const int64_t plane_bytes = a.N * (a.K / 4);
    float sc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sc[i] = a.scales[i];
    for (int64_t it = (int64_t)blockIdx.x * kQThreads + threadIdx.x; it < items;
         it += (int64_t)gridDim.x * kQThreads) {
        int64_t n, k0;
        item_nk<V>(a, it, small, n, k0);
        Plane u[V], w[V];
        load_planes_v<V>(a, n, k0, u, w);
        uint32_t cbyte[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float o11[V], o12[V], o21[V], o22[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            Plane* pl[2] = {&u[v], &w[v]};
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (t < a.steps[p]) {
                        const uint32_t c = apply_stage_k(a.kind[p], *pl[p], sc[(p * 4 + t) * 2],
                                                         sc[(p * 4 + t) * 2 + 1]);
                        cbyte[p * 4 + t] |= c << (2 * v);
                    }
            float ur = u[v].q_re, ui = u[v].q_im, wr = w[v].q_re, wi = w[v].q_im;
            if (a.rot) {  // quant_i.py:433-434
                const float cu = a.rot[0], su = a.rot[1], cw = a.rot[2], sw = a.rot[3];
                const float r0 = ur * cu - ui * su, i0 = ui * cu + ur * su;
                const float r1 = wr * cw - wi * sw, i1 = wi * cw + wr * sw;
                ur = r0; ui = i0; wr = r1; wi = i1;
            }
            o11[v] = wr + ur;  // quant_i.py:534-544
            o12[v] = wi - ui;
            o21[v] = wi + ui;
            o22[v] = -wr + ur;
        }
        if (a.aq) {
            float* r0p = a.aq + n * row + k0;
            float* r1p = a.aq + (a.N + n) * row + k0;
            if constexpr (V == 4) {
                *reinterpret_cast<float4*>(r0p) = make_float4(o11[0], o11[1], o11[2], o11[3]);
                *reinterpret_cast<float4*>(r0p + a.K) = make_float4(o12[0], o12[1], o12[2], o12[3]);
                *reinterpret_cast<float4*>(r1p) = make_float4(o21[0], o21[1], o21[2], o21[3]);
                *reinterpret_cast<float4*>(r1p + a.K) = make_float4(o22[0], o22[1], o22[2], o22[3]);
            } else {
#pragma unroll
                for (int v = 0; v < V; ++v) {
                    r0p[v] = o11[v];
                    r0p[a.K + v] = o12[v];
                    r1p[v] = o21[v];
                    r1p[a.K + v] = o22[v];
                }
            }
        }
        if (V == 4 && a.codes) {
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (t < a.steps[p]) {
                        const int plane = p * a.steps[0] + t;
                        a.codes[plane * plane_bytes + n * (a.K / 4) + k0 / 4] = (uint8_t)cbyte[p * 4 + t];
                    }
        }
    }
}

// Device scratch of rpfq_quantize_wide_noalloc: the per-block float64
// partials of one stage (kQuantMaxBlocks x 8 doubles = 64 KiB per device,
// held until the process ends).  Host code never passes `scratch` itself to
// a kernel (its name is a host-side stand-in there): quant_scratch_ptr() resolves
// the device address once per device.
static __device__ __align__(256) double scratch[kQuantMaxBlocks * 8];

int reduce_blocks(int64_t total) {
    int64_t b = (total + kQThreads - 1) / kQThreads;
    return (int)(b < kQuantMaxBlocks ? (b < 1 ? 1 : b) : kQuantMaxBlocks);
}

}  // namespace

size_t quant_scratch_bytes() { return sizeof(scratch); }

hipError_t quant_scratch_ptr(void** out) {
    static std::atomic<void*> ptrs[64];  // per device, zero-initialised
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    void* p = ptrs[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(mu);
        p = ptrs[dev].load(std::memory_order_relaxed);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // with device `dev` current
            if (e != hipSuccess) return e;
            ptrs[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

hipError_t launch_quantize_wide(const rpfq_quant_desc& d, const float* weight, const float* rot, float* aq,
                                float* scales, uint8_t* codes, void* work, hipStream_t s) {
    QuantArgs a;
    a.w = weight;
    a.rot = rot;
    a.N = d.n_complex;
    a.K = d.k_complex;
    for (int p = 0; p < 2; ++p) {
        a.kind[p] = d.kind[p];
        a.steps[p] = d.steps[p];
    }
    a.scales = scales;
    a.partial = static_cast<double*>(work);
    a.aq = aq;
    a.codes = codes;
    // four columns per thread (16-B loads and stores) when the rows allow it
    const bool v4 = a.K % 4 == 0 && reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(aq) % 16 == 0;
    a.nblocks = reduce_blocks(a.N * (v4 ? a.K / 4 : a.K));
    const int max_steps = d.steps[0] > d.steps[1] ? d.steps[0] : d.steps[1];
    for (int st = 0; st < max_steps; ++st) {
        a.stage = st;
        if (v4)
            hipLaunchKernelGGL(quant_reduce_kernel<4>, dim3(a.nblocks), dim3(kQThreads), 0, s, a);
        else
            hipLaunchKernelGGL(quant_reduce_kernel<1>, dim3(a.nblocks), dim3(kQThreads), 0, s, a);
        hipLaunchKernelGGL(quant_finalize_kernel, dim3(1), dim3(kQThreads), 0, s, a);
    }
    if (aq || codes) {
        const int64_t items = a.N * (v4 ? a.K / 4 : a.K);
        int64_t blocks = (items + kQThreads - 1) / kQThreads;
        if (blocks > 8 * kQuantMaxBlocks) blocks = 8 * kQuantMaxBlocks;
        if (v4)
            hipLaunchKernelGGL(quant_apply_kernel<4>, dim3((unsigned)blocks), dim3(kQThreads), 0, s, a);
        else
            hipLaunchKernelGGL(quant_apply_kernel<1>, dim3((unsigned)blocks), dim3(kQThreads), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace rpfq
