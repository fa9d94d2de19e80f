// C entry points that drive the reference's Android phase-linear C++ code
// (compiled from /root/reference by oracle/Makefile into oracle/_ref/).
// TEST INFRASTRUCTURE ONLY: used by tests/ to validate the numpy oracle and
// as the optional CPU baseline.  Never linked into the product.
//
// Driven reference functions (paths under RPFQ-ViTAndroid/app/src/main/cpp):
//   loadPhaseParams      ops/phase_linear.cpp:42-88
//   loadWideParams       ops/phase_linear.cpp:90-117  (builds the fp16 cache
//                        of kernels/phase_linear_cache.cpp:84-131)
//   phaseLinearReference ops/phase_linear.cpp:119-164
//   wideLinearReference  ops/phase_linear.cpp:166-207
//   wideLinearFusedCacheFp16Neon kernels/wide_linear_cache_neon.cpp:69-159
//   wideLinearOptimized  kernels/phase_linear_fused.cpp:120-148
#include "ops/phase_linear.h"
#include "kernels/phase_linear_cache.h"
#include "kernels/phase_linear_fused.h"
#include "kernels/wide_linear_cache_neon.h"
#include "runtime/thread_pool.h"
#include "safetensors_loader.h"
#include "tensor.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>

using namespace rpfq_vit;

namespace {

void put_codes(SafeTensorStore& s, const std::string& name, const uint8_t* p, int rows, int cols) {
    UInt8Tensor t;
    t.shape = {rows, cols};
    t.data.assign(p, p + static_cast<size_t>(rows) * cols);
    s.u8[name] = std::move(t);
}

void put_half(SafeTensorStore& s, const std::string& name, const uint16_t* p, int rows, int cols) {
    Tensor t(std::vector<int64_t>{rows, cols});
    for (size_t i = 0; i < t.data.size(); ++i) t.data[i] = halfToFloat(p[i]);
    s.f32[name] = std::move(t);
}

void set_err(char* err, int errlen, const char* msg) {
    if (err && errlen > 0) {
        std::strncpy(err, msg, static_cast<size_t>(errlen) - 1);
        err[errlen - 1] = 0;
    }
}

}  // namespace

extern "C" {

// One packed plane: codes [out_dim, in_dim/4], gammas fp16 bits [out_dim, in_dim/block].
int ref_phase_linear(const float* xr, const float* xi, int tokens, int in_dim, int out_dim, int block,
                     const uint8_t* codes, const uint16_t* gamma_re, const uint16_t* gamma_im,
                     float* out_re, float* out_im, char* err, int errlen) {
    try {
        SafeTensorStore s;
        put_codes(s, "p.codes", codes, out_dim, in_dim / 4);
        put_half(s, "p.gamma_real", gamma_re, out_dim, in_dim / block);
        put_half(s, "p.gamma_imag", gamma_im, out_dim, in_dim / block);
        PhaseLinearParams p = loadPhaseParams(s, "p", in_dim, out_dim, block);
        std::vector<float> re, im;
        phaseLinearReference(xr, xi, tokens, p, re, im);
        std::memcpy(out_re, re.data(), re.size() * sizeof(float));
        std::memcpy(out_im, im.data(), im.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        set_err(err, errlen, e.what());
        return 1;
    }
}

// Widely-linear layer from 4 planes ordered u_s0, u_s1, w_s0, w_s1.
// mode 0: wideLinearReference (fp32); 1: fp16 fused cache (threads);
// 2: wideLinearOptimized (fused scalar, threads).
int ref_wide_linear(const float* x, int tokens, int real_in, int real_out, int complex_in,
                    int complex_out, int original_out_complex, int block,
                    const uint8_t* const* codes, const uint16_t* const* gamma_re,
                    const uint16_t* const* gamma_im, const float* bias, float* y, int mode,
                    int threads, char* err, int errlen) {
    try {
        static const char* names[4] = {"L.u_s0", "L.u_s1", "L.w_s0", "L.w_s1"};
        SafeTensorStore s;
        for (int p = 0; p < 4; ++p) {
            put_codes(s, std::string(names[p]) + ".codes", codes[p], complex_out, complex_in / 4);
            put_half(s, std::string(names[p]) + ".gamma_real", gamma_re[p], complex_out, complex_in / block);
            put_half(s, std::string(names[p]) + ".gamma_imag", gamma_im[p], complex_out, complex_in / block);
        }
        Tensor b(std::vector<int64_t>{real_out});
        std::memcpy(b.data.data(), bias, sizeof(float) * real_out);
        s.f32["L.bias"] = b;
        WideLinearParams p = loadWideParams(s, "L", real_in, real_out, complex_in, complex_out,
                                            original_out_complex, block);
        Tensor xt(std::vector<int64_t>{tokens, real_in});
        std::memcpy(xt.data.data(), x, sizeof(float) * static_cast<size_t>(tokens) * real_in);
        Tensor out;
        if (mode == 0) {
            out = wideLinearReference(xt, p);
        } else if (mode == 1) {
            if (!p.fusedCache || !p.fusedCache->valid) throw std::runtime_error("fp16 cache not built");
            ThreadPool pool(threads);
            out = Tensor(std::vector<int64_t>{tokens, real_out});
            wideLinearFusedCacheFp16Neon(xt, p, out, pool);
        } else {
            out = wideLinearOptimized(xt, p, threads);
        }
        std::memcpy(y, out.data.data(), sizeof(float) * out.data.size());
        return 0;
    } catch (const std::exception& e) {
        set_err(err, errlen, e.what());
        return 1;
    }
}

// The reference's own float -> fp16 rounding used by its coefficient cache.
uint16_t ref_float_to_half_bits(float x) { return floatToHalfBits(x); }

}  // extern "C"
