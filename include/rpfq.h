/*
 * rpfq.h -- C ABI of the MI355X (gfx950) packed complex-phase linear kernels.
 *
 * Contract shared by every entry point:
 *   - all array arguments are caller-owned DEVICE pointers (HIP memory);
 *     nothing is allocated on the hot path;
 *   - work is enqueued asynchronously on `stream` (a hipStream_t passed as
 *     void*; NULL = the default stream) and the call returns without waiting;
 *   - the return value is RPFQ_OK or a positive RPFQ_ERR_* status; the entry
 *     points never abort or throw.  rpfq_last_error() returns a thread-local
 *     message for the last failing call on the calling thread;
 *   - argument validation happens on the host before any HIP call, so every
 *     shape / null / alignment / enum error is reported without a GPU;
 *   - the library holds no mutable global state: calls are reentrant and
 *     may be issued from several threads on different streams (the one
 *     exception, rpfq_quantize_wide_noalloc, says so at its declaration).
 *
 * Feature layout: a "wide" (widely-linear) layer maps x = [x_re | x_im]
 * ([M, 2K'] row-major) to y = [y_re | y_im] ([M, 2N']) with
 * y = U x + W conj(x) + bias, where U and W are complex [N', K'] matrices held
 * as phase codes times scales.  This is the reference layer
 * QATLinearComplexPhase (RPFQ-ViT-main/quant_models/quant_i.py:475-554).
 */
#ifndef RPFQ_H_
#define RPFQ_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RPFQ_ABI_VERSION 1

/* status codes */
#define RPFQ_OK 0
#define RPFQ_ERR_NULL 1      /* a required pointer is NULL */
#define RPFQ_ERR_SHAPE 2     /* non-positive, odd or inconsistent dimensions */
#define RPFQ_ERR_ALIGN 3     /* dimension or pointer not aligned as required */
#define RPFQ_ERR_BITS 4      /* unsupported code width / codebook / planes */
#define RPFQ_ERR_DTYPE 5     /* unsupported element type */
#define RPFQ_ERR_VALUE 6     /* invalid value (e.g. block not a multiple of 32) */
#define RPFQ_ERR_HIP 7       /* the HIP runtime reported an error */

/* element types of activations / outputs */
#define RPFQ_F32 0
#define RPFQ_F16 1
#define RPFQ_BF16 2

/* rpfq_wide_linear flags.  Default (0): the kernel is chosen from the shape
 * (M <= 16, and small-M launches where a cost model predicts it faster --
 * e.g. a ViT-B layer at one image -- stream the packed codes, 32-row tiles
 * against 16-row chunks of x; M >= 32768 with a small layer -- K' = 48 and
 * N' in {48, 96, 144, 192}, K' = 96 and N' in {48, 96}, or K' = 192 and
 * N' = 48, fp16 / bf16 x and y, y 16-byte aligned: Swin-T stage 0 --
 * keeps the decoded layer resident in LDS and streams rows of x; fp16 / bf16
 * x with K' % 32 == 0 and M >= 128 stages activations by LDS DMA; other cases
 * stage them through registers with a 32/64/128-row tile).
 * RPFQ_FLAG_TILE_M128 forces the register-staged 128-row kernel;
 * RPFQ_FLAG_NO_STREAM keeps every M on the tiled kernels (not the resident
 * one);
 * RPFQ_FLAG_STREAM forces the streaming kernel for any M (one workgroup per
 * 16-row chunk of x and 32-row tile of the codes; at most 2^24 of them,
 * else RPFQ_ERR_SHAPE; not combinable with the other two, RPFQ_ERR_VALUE);
 * RPFQ_FLAG_RESIDENT forces the resident-weight kernel for any M (the layer
 * and dtypes as above, N' <= 96 with a residual, else
 * RPFQ_ERR_SHAPE / RPFQ_ERR_DTYPE, y not 16-byte aligned RPFQ_ERR_ALIGN; not
 * combinable with the other three).
 * Every kernel feeds the MFMA the same fp16 coefficients. */
#define RPFQ_FLAG_TILE_M128 1
#define RPFQ_FLAG_NO_STREAM 2
#define RPFQ_FLAG_STREAM 4
#define RPFQ_FLAG_RESIDENT 16
/* RPFQ_FLAG_GELU (rpfq_wide_linear only; the residual entry point rejects
 * it, RPFQ_ERR_VALUE): y = gelu(layer output), exact erf GELU applied in the
 * store to the output rounded to y's dtype, computed in float32 and rounded
 * again -- equal to torch.nn.functional.gelu (approximate='none') of the
 * unfused output, as the ViT MLP applies it after fc1 (timm Mlp, nn.GELU). */
#define RPFQ_FLAG_GELU 8

/* codebooks of the packed planes */
#define RPFQ_CB_AXIS 0   /* 2-bit {-1,+1,-i,+i} axis codes, residual stages
                            (quant_i.py:36-118, export_rpfq_vit_to_mlx.py:189-224) */
#define RPFQ_CB_SIGN 1   /* 2-bit quadrant-sign codes (quant_i.py:84-91):
                            bit0 = (re >= 0), bit1 = (im >= 0) */
#define RPFQ_CB_PSK16 2  /* 4-bit code c -> exp(i 2 pi c / 16); build-defined,
                            no counterpart in the reference */
#define RPFQ_CB_TABLE 3  /* 4-bit index into a per-row table of 16 complex
                            values for U and 16 for W: the learnable grouped
                            codebook of complex_phase_next_v1 (quant_i.py:193-351;
                            index = codeword | (e_re >= 0) << 2 | (e_im >= 0) << 3) */

/* Descriptor of one packed widely-linear layer. */
typedef struct rpfq_wide_desc {
    int64_t n_complex; /* N' = out_features / 2 */
    int64_t k_complex; /* K' = in_features / 2 (multiple of 8) */
    int64_t block;     /* scale block along K' in complex columns: 0 = one
                          scale per row, else a multiple of 32 */
    int32_t codebook;  /* RPFQ_CB_* */
    int32_t stages;    /* residual stages per U/W: 1 or 2 (AXIS/SIGN); 1 (PSK16, TABLE) */
    int32_t rotate;    /* 1: de-rotate the quantized U/W by (cos,sin) below,
                          quant_i.py:425-435 */
    float rot_u[2];    /* cos(theta_u), sin(theta_u) as float32 */
    float rot_w[2];    /* cos(theta_w), sin(theta_w) as float32 */
} rpfq_wide_desc;

/* Library identity. */
int rpfq_abi_version(void);
const char* rpfq_last_error(void);

/*
 * Decode one packed plane to float32 real/imag planes.
 * Replaces the unpack + dequantize of
 *   RPFQ-ViTApple/scripts/export_rpfq_vit_to_mlx.py:227-254 (dequantize_axis)
 *   RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:15-19, :143-154
 * bits = 2: codes [rows, k/4] uint8 (4 codes per byte, low bits first),
 *           code -> {-1, +1, -i, +i};
 * bits = 4: codes [rows, k/2] uint8 (low nibble first), 16-PSK codebook.
 * gamma_re / gamma_im: fp16 bit patterns [rows, ceil(k/block)]; the value is
 * codebook / gamma (as the exporter).  Both NULL: unit codebook values.
 * Bit-exact with the reference.
 */
int rpfq_unpack(const uint8_t* codes, int bits, int64_t rows, int64_t k,
                const uint16_t* gamma_re, const uint16_t* gamma_im, int64_t block,
                float* re, float* im, void* stream);

/*
 * Single packed plane complex linear, the reference primitive
 *   RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:119-164
 *   (phaseLinearReference; also RPFQViTMetalKernels.swift:91-174 prefill):
 *   conj_x = 1:  y = W conj(x):  Re = sum wRe xr + wIm xi, Im = sum wIm xr - wRe xi
 *   conj_x = 0:  y = W x (the U-branch feed (xr, -xi), phase_linear.cpp:189-192)
 * xr, xi: [M, K] planes; codes [N, K/4] uint8; gamma_re/gamma_im fp16 bits
 * [N, ceil(K/block)] (block multiple of 32, or 0 = one per row); yr, yi:
 * [M, N].  K must be a multiple of 32.  Codes are contracted exactly
 * (ternary MFMA operands) and the scales are applied in the epilogue;
 * float32 x is split into two fp16 terms (relative error ~2^-22).
 */
int rpfq_phase_linear(const void* xr, const void* xi, int x_dtype, int conj_x,
                      int64_t M, int64_t K, const uint8_t* codes,
                      const uint16_t* gamma_re, const uint16_t* gamma_im, int64_t block,
                      int64_t N, void* yr, void* yi, int y_dtype, void* stream);

/* Bytes of the device blob that rpfq_wide_pack writes for `desc`. */
size_t rpfq_wide_packed_bytes(const rpfq_wide_desc* desc);

/*
 * Repack a layer's code planes into the MI355X tiled layout.
 * Replaces the loader step of
 *   RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:90-117 (loadWideParams)
 *   and the fused cache of kernels/phase_linear_cache.cpp:84-131.
 * planes (AXIS/SIGN): 2*stages code planes ordered u_s0[, u_s1], w_s0[, w_s1],
 *   each [N', K'/4] uint8 in the exporter's packing (export…py:148-159);
 * planes (PSK16, TABLE): u, w, each [N', K'/2] uint8 (low nibble first).
 * scale_re[p] / scale_im[p]: float32 [N', nblk] multipliers of plane p
 *   (the training scale, or 1/gamma of the exporter); PSK16 uses scale_re
 *   only (magnitude).  nblk = 1 if desc->block == 0 else ceil(K'/block).
 *   TABLE: scale_re[p] / scale_im[p] are the real / imaginary parts of the
 *   [N', 16] float32 value table of plane p (U, W); block and rotate are 0.
 * packed: device buffer of rpfq_wide_packed_bytes(desc) bytes.
 */
int rpfq_wide_pack(const rpfq_wide_desc* desc, const uint8_t* const* planes, int nplanes,
                   const float* const* scale_re, const float* const* scale_im,
                   void* packed, size_t packed_bytes, void* stream);

/*
 * Widely-linear layer y = U x + W conj(x) + bias on [re | im] features.
 * Replaces the contraction F.linear(x, A_q, bias) of quant_i.py:554 and
 *   RPFQ-ViTAndroid/app/src/main/cpp/ops/phase_linear.cpp:166-256
 *   (wideLinearReference / wideLinear; Metal widePrefill
 *   RPFQViTMetalKernels.swift:176-268).
 * x: [M, 2K'] of x_dtype (rows 16-byte aligned); bias: float32 [2N'] or NULL;
 * y: [M, 2N'] of y_dtype.  U and W are formed in float32 exactly as the
 * reference does (stage sums, de-rotation) and rounded to fp16; each fused
 * coefficient (A11 = Wre + Ure, A12 = Wim - Uim, A21 = Wim + Uim,
 * A22 = -Wre + Ure) is one correctly rounded fp16 add of those; the MFMA
 * accumulates in float32.  The RPFQ_KERNEL_GEMV launches (M <= 8) never
 * round the fused coefficients: the fp16 U and W values meet x in separate
 * MFMA products, so their sums are exact in the float32 accumulator.
 * Input range: x is rounded to fp16 for the MFMA as it stands, which is
 * exact for fp16 x and for bf16 x in [2^-14, 65504] and 2^-11 relative for
 * float32 x in that range; larger magnitudes become +-inf and smaller ones
 * lose relative precision.  rpfq_wide_linear_scaled with the row prescales
 * of rpfq_row_scales removes that limit for float32 / bf16 x; with fp16 x
 * and row_scale, the rows are taken as already prescaled (as
 * rpfq_layer_norm_prescaled writes them) and the outputs unscaled (DMA
 * kernel launches only; RPFQ_ERR_VALUE otherwise).
 * flags: the RPFQ_FLAG_* bits above.
 */
int rpfq_wide_linear(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes,
                     const void* x, int x_dtype, int64_t M, const float* bias,
                     void* y, int y_dtype, int flags, void* stream);

/* kernels of rpfq_wide_linear (rpfq_wide_linear_kernel) */
#define RPFQ_KERNEL_STREAM 0  /* weight streaming, 16-row chunks of x */
#define RPFQ_KERNEL_DMA 1     /* 128-row tiles, activations staged by LDS DMA */
#define RPFQ_KERNEL_TILED 2   /* 32/64/128-row tiles staged through registers */
#define RPFQ_KERNEL_GEMV 3    /* weight streaming for M <= 8, U and W as separate MFMA operands */
#define RPFQ_KERNEL_RESIDENT 4 /* decoded layer resident in LDS, 32-row subtiles of x per wave */

/*
 * *kernel := the RPFQ_KERNEL_* that rpfq_wide_linear runs for this layer, M,
 * dtypes and flags (no GPU work; same validation as rpfq_wide_linear minus
 * the buffers).  For callers choosing whether to fuse an epilogue op: the
 * fused GELU pays most on the streaming and resident kernels (HBM-bound,
 * VALU idle); on the DMA kernel it makes the launch ~30% longer, still less
 * than a separate GELU pass over the output.  No counterpart in the
 * reference: the kernel choice is this library's.
 */
int rpfq_wide_linear_kernel(const rpfq_wide_desc* desc, int64_t M, int x_dtype, int y_dtype, int flags,
                            int* kernel);

/*
 * rpfq_wide_linear with the block's residual add fused into the store:
 *   y = residual + (U x + W conj(x) + bias)
 * where the layer output is rounded to y_dtype first and the sum rounded
 * again, so y is bit-identical to rpfq_wide_linear followed by an add in
 * y_dtype (torch's `x + proj(...)`).  residual: [M, 2N'] of y_dtype, rows
 * 16-byte aligned; it may be y itself (in place: every element is read and
 * written by the same thread).  Other arguments as rpfq_wide_linear.
 * Replaces the residual adds after attn.proj and mlp.fc2 of a ViT block
 *   RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:546 and :556
 *   (runtime path :619, :625).
 */
int rpfq_wide_linear_residual(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes,
                              const void* x, int x_dtype, int64_t M, const float* bias,
                              const void* residual, void* y, int y_dtype, int flags, void* stream);

/*
 * The MLP tail of a transformer block in one launch:
 *   y = residual + fc2(GELU(fc1(x) + bias1)) + bias2
 * fc1 (desc1: K' -> N1') and fc2 (desc2: N1' -> K') packed widely-linear
 * layers; the hidden activations stay on chip.  Each hidden value is fc1's
 * output rounded to fp16 and its GELU rounded again, within 1 ulp of the
 * exact GELU (the fused GELU of rpfq_wide_linear's RPFQ_FLAG_GELU), and y is
 * bit-identical to rpfq_wide_linear(fc1, RPFQ_FLAG_GELU) followed by
 * rpfq_wide_linear_residual(fc2) on the large-M kernel.  x, residual, y:
 * fp16 [M, 2K'], rows 16-byte aligned; residual may be NULL or y itself.
 * bias1 [2N1'] / bias2 [2K'] float32 or NULL.  Shapes: K' = 96 (DeiT-Ti,
 * Swin-T stage 1), N1' a multiple of 96 up to 1536, per-row scales
 * (block = 0) on both layers, one codebook, M >= 64; others return
 * RPFQ_ERR_SHAPE.  Replaces the block's
 *   norm2 -> mlp.fc1 -> mlp.act -> mlp.fc2 -> + residual1 sequence
 *   RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:549-556
 * after the LayerNorm (the reference's two QATLinearComplexPhase.forward
 * calls, RPFQ-ViT-main/quant_models/quant_i.py:513-554, and the GELU
 * between them).
 */
int rpfq_wide_mlp(const rpfq_wide_desc* desc1, const void* packed1, size_t packed1_bytes,
                  const rpfq_wide_desc* desc2, const void* packed2, size_t packed2_bytes, const void* x,
                  int64_t M, const float* bias1, const float* bias2, const void* residual, void* y,
                  void* stream);

/*
 * rpfq_wide_mlp with the block's LayerNorm before fc1 and x itself as the
 * residual, one launch:
 *   y = x + fc2(GELU(fc1(LayerNorm(x)) + bias1)) + bias2
 * The normalized rows are the bits rpfq_layer_norm(x, M, 2K', gamma, beta,
 * eps) writes in fp16 (same arithmetic and summation order for this M), so
 * y equals rpfq_layer_norm followed by rpfq_wide_mlp(residual = x) bit for
 * bit.  gamma / beta: float32 [2K'], 16-byte aligned, or NULL (ones /
 * zeros); eps >= 0 (else RPFQ_ERR_VALUE); y may be x.  Shapes and the other
 * arguments as rpfq_wide_mlp.  Replaces
 *   norm2 -> mlp.fc1 -> mlp.act -> mlp.fc2 -> + residual1
 *   RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:548-556.
 */
int rpfq_layer_norm_wide_mlp(const rpfq_wide_desc* desc1, const void* packed1, size_t packed1_bytes,
                             const rpfq_wide_desc* desc2, const void* packed2, size_t packed2_bytes, const void* x,
                             int64_t M, const float* gamma, const float* beta, float eps, const float* bias1,
                             const float* bias2, void* y, void* stream);

/*
 * Per-row prescales of x [M, C] for rpfq_wide_linear_scaled (the forward's
 * range guard): scale[m] = 2^(14 - floor(log2 max_k |x[m, k]|)), clamped to
 * [2^-126, 2^126], so the row's largest element times scale[m] lies in
 * [2^14, 2^15); 1 for rows whose maximum is 0, inf or NaN.  x: any of the
 * three dtypes, element-aligned (C % 8 == 0 with 16-byte aligned rows reads
 * 16-byte chunks); scale: float32 [M].  No counterpart in the reference: its
 * float32 F.linear has float32's range, which this restores around the
 * kernels' fp16 operands.
 */
int rpfq_row_scales(const void* x, int x_dtype, int64_t M, int64_t C, float* scale, void* stream);

/*
 * rpfq_wide_linear (residual = NULL) or rpfq_wide_linear_residual with the
 * rows of a float32 / bf16 x prescaled: row m is multiplied by row_scale[m]
 * before its fp16 rounding and its layer output by 1 / row_scale[m] (exact)
 * before the bias, the GELU and the residual add.  row_scale: float32 [M],
 * 16-byte aligned, powers of two in [2^-126, 2^126] (as rpfq_row_scales
 * writes them), or NULL (no prescale).  fp16 x with a row_scale: rows
 * already prescaled (rpfq_layer_norm_prescaled), only undone in the output;
 * the launch must take the DMA kernel (rpfq_wide_linear_kernel reports
 * RPFQ_KERNEL_DMA), else RPFQ_ERR_VALUE.  Power-of-two factors commute with the roundings of the
 * contraction, so a row inside fp16's range gives the same output as
 * rpfq_wide_linear, and a row of any float32 / bf16 range keeps that
 * relative accuracy (2^-11 of sum |x| |A| for float32 x, exact operands for
 * bf16 x).  Other arguments and flags as rpfq_wide_linear (RPFQ_FLAG_GELU
 * only without a residual).
 * Replaces F.linear(x, A_q, bias) of quant_i.py:554 on float32 activations
 * of any magnitude (the reference layer's dtype).
 */
int rpfq_wide_linear_scaled(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, const void* x,
                            int x_dtype, int64_t M, const float* row_scale, const float* bias, const void* residual,
                            void* y, int y_dtype, int flags, void* stream);

/* Bytes of the adjoint blob that rpfq_wide_pack_adjoint writes for `desc`
 * (0 if the descriptor is invalid). */
size_t rpfq_wide_adjoint_bytes(const rpfq_wide_desc* desc);

/*
 * Adjoint blob of a packed layer, for rpfq_wide_linear_grad_x: its codes
 * with rows and columns exchanged, and each row's U / W value tables as the
 * fp16 (re, im) pairs the kernels contract (de-rotated; every codebook).
 * Run once per packed blob (and again after the blob or the descriptor's
 * rotation changes); both buffers 256-byte aligned.  No counterpart in the
 * reference: it is this library's layout for contractions over N'.
 */
int rpfq_wide_pack_adjoint(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, void* adjoint,
                           size_t adjoint_bytes, void* stream);

/*
 * Input gradient of rpfq_wide_linear: grad_x = grad_y A, where A [2N', 2K']
 * is the real matrix of y = U x + W conj(x) made of the fused fp16
 * coefficients that rpfq_wide_linear feeds its MFMAs (A11 = Wre + Ure,
 * A12 = Wim - Uim, A21 = Wim + Uim, A22 = -Wre + Ure, bit for bit):
 *   gx_re = gy_re A11 + gy_im A21,   gx_im = gy_re A12 + gy_im A22.
 * grad_y: [M, 2N'] of grad_y_dtype (16-byte aligned when N' % 8 == 0);
 * grad_x: [M, 2K'] of grad_x_dtype.  adjoint: the layer's
 * rpfq_wide_pack_adjoint blob.  The products run on fp16 MFMA
 * operands with float32 accumulation; float32 and bf16 grad_y rows are
 * scaled by a power of two per row (largest magnitude in [2^14, 2^15))
 * before the fp16 rounding and unscaled exactly after, so each grad_y
 * element carries one fp16 rounding (relative 2^-11) unless it is below
 * 2^-24 of its row's largest.  The bias gradient is the column sum of
 * grad_y and is left to the caller.
 * Replaces grad_x = einsum('blo, oi -> bli', grad_output, w_quant) of
 *   RPFQ-ViT-main/quant_models/kernel.py:585 (the reference operator's
 *   backward), i.e. the input gradient of F.linear(x, A_q, bias) at
 *   quant_i.py:554 under the straight-through estimator (quant_i.py:128-130).
 */
int rpfq_wide_linear_grad_x(const rpfq_wide_desc* desc, const void* adjoint, size_t adjoint_bytes, const void* grad_y,
                            int grad_y_dtype, int64_t M, void* grad_x, int grad_x_dtype, void* stream);

/*
 * y = layer(LayerNorm(x)) in one launch: the LayerNorm of rpfq_layer_norm
 * over the layer's 2K' input features (float32 statistics and affine map,
 * rounded to x_dtype) runs in the streaming kernel's prologue, and the
 * packed layer of rpfq_wide_linear contracts the normalized rows from LDS;
 * the normalized x is never written to memory.  Equal to rpfq_layer_norm
 * (y_dtype = x_dtype) followed by rpfq_wide_linear up to the order of the
 * statistics' float32 sums.  gamma, beta: float32 [2K'] or NULL (1 / 0),
 * 16-byte aligned.  flags: 0 or RPFQ_FLAG_GELU.  Only for launches that
 * rpfq_layer_norm_wide_linear_fusable accepts (a layer at batch 1-2: the
 * streaming kernel's split-K forms, per-row scales, K' % 32 == 0,
 * K' <= 384, fp16 / bf16 x, not RPFQ_CB_TABLE); RPFQ_ERR_VALUE otherwise.
 * Replaces norm1 -> qkv and norm2 -> fc1 of a ViT block
 *   RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:520-521, :549-550
 *   (RPFQ-ViT-main/quant_models/quant_i.py:554 inside the layer).
 */
int rpfq_layer_norm_wide_linear(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes,
                                const void* x, int x_dtype, int64_t M, const float* gamma, const float* beta,
                                float eps, const float* bias, void* y, int y_dtype, int flags, void* stream);

/*
 * y = layer(act_quant(x)) or, with layer_norm = 1, layer(act_quant(LayerNorm(x)))
 * in one launch, with an optional residual added in the store: the
 * activation fake quantization of rpfq_act_quant (per row and half, scale =
 * qmax * (1 / max(max|v|, 1e-5)), v_q = clamp(rint(v scale), qmin, qmax) /
 * scale, bits 2 .. 16), applied to x or to the float32 LayerNorm output as
 * rpfq_layer_norm_act_quant applies it, rounded to x_dtype, runs in the
 * streaming kernel's prologue, and the packed layer contracts the quantized
 * rows from LDS.  The prepared rows are bit-identical to those of
 * rpfq_act_quant / rpfq_layer_norm_act_quant (same lane order of the
 * statistics), so y is bit-identical to that kernel followed by
 * rpfq_wide_linear (or rpfq_wide_linear_residual) on the same launch.
 * gamma, beta, eps: as rpfq_layer_norm_wide_linear (ignored when
 * layer_norm = 0); residual: [M, 2N'] of y_dtype or NULL, 16-byte aligned,
 * may equal y; flags: 0 or RPFQ_FLAG_GELU (not with a residual).  Only for
 * launches that rpfq_layer_norm_wide_linear_fusable accepts; RPFQ_ERR_VALUE
 * otherwise.
 * Replaces the act quant of the layer's input and the contraction,
 *   RPFQ-ViT-main/quant_models/quant_i.py:546-554 (ActivationQuantSTE then
 *   F.linear), after norm1 / norm2 (audit_rpfq_vit_ios_parity.py:520, :549)
 *   when layer_norm = 1; the Triton analogue kernel.py:449-521.
 */
int rpfq_act_quant_wide_linear(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes, const void* x,
                               int x_dtype, int64_t M, int bits, int layer_norm, const float* gamma, const float* beta,
                               float eps, const float* bias, const void* residual, void* y, int y_dtype, int flags,
                               void* stream);

/* *fusable = 1 if rpfq_layer_norm_wide_linear (and rpfq_act_quant_wide_linear)
 * accepts this launch, else 0 (no GPU work; no counterpart in the reference). */
int rpfq_layer_norm_wide_linear_fusable(const rpfq_wide_desc* desc, int64_t M, int x_dtype, int y_dtype,
                                        int* fusable);

/*
 * LayerNorm over the last dimension (nn.LayerNorm with biased variance):
 *   y = (x - mean) / sqrt(var + eps) * gamma + beta
 * per row of x [M, C], statistics and the affine map in float32, then
 * rounded to y_dtype.  gamma, beta: float32 [C] or NULL (1 / 0).  x, y,
 * gamma and beta must be 16-byte aligned, C a multiple of 8 up to 4096; y
 * may equal x.
 * Replaces the norm1 / norm2 / final norm around the packed layers of a ViT
 * block (RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:520, :549).
 */
int rpfq_layer_norm(const void* x, int x_dtype, int64_t M, int64_t C, const float* gamma, const float* beta,
                    float eps, void* y, int y_dtype, void* stream);

/*
 * rpfq_layer_norm of bf16 / float32 rows handed to a packed layer as
 * prescaled fp16 rows: each row is normalized (and, for bf16 x, rounded to
 * bf16 exactly as rpfq_layer_norm(y_dtype = RPFQ_BF16) rounds it),
 * row_scale[m] is what rpfq_row_scales gives that row in x's dtype (a power
 * of two), and y [M, C] fp16 holds the row times row_scale[m], rounded to
 * fp16 -- the operand the kernels make of the row itself.
 * rpfq_wide_linear_scaled(x = y, x_dtype = RPFQ_F16, row_scale) then undoes
 * the prescale on the DMA kernel (the launch must be one
 * rpfq_wide_linear_kernel reports as RPFQ_KERNEL_DMA): for bf16 x, bit for
 * bit what that launch returns for the bf16 rows with their row scales,
 * without converting them in the kernel; for float32 x, the same fp16
 * operands the register-staged kernel makes of the float32 rows, on the
 * faster DMA kernel.  x_dtype: RPFQ_BF16 or RPFQ_F32; row_scale: float32
 * [M], 16-byte aligned; other arguments as rpfq_layer_norm (y may equal x
 * for bf16 x).  Replaces norm1 / norm2 before qkv / fc1
 * (audit_rpfq_vit_ios_parity.py:520, :549) in a bf16 model; no counterpart
 * in the reference for the prescale (the guard of this library's fp16 MFMA
 * operands).
 */
int rpfq_layer_norm_prescaled(const void* x, int x_dtype, int64_t M, int64_t C, const float* gamma,
                              const float* beta, float eps, void* y, float* row_scale, void* stream);

/*
 * The prescaled fp16 operand rows of bf16 / float32 rows without a
 * LayerNorm: y [M, C] fp16 = x times row_scale[m] (what rpfq_row_scales
 * gives x), rounded to fp16 -- the bits the kernels make of x with those
 * prescales, so rpfq_wide_linear_scaled(y, RPFQ_F16, row_scale) on a
 * DMA-kernel launch equals it on bf16 (x, RPFQ_BF16, row_scale) bit for
 * bit, one pass instead of the row-scale pass plus the in-kernel
 * conversion, and takes float32 rows to the DMA kernel with the
 * register-staged kernel's operands.  x_dtype: RPFQ_BF16 or RPFQ_F32; C a
 * multiple of 8 up to 4096; x, y 16-byte aligned (y may equal x for bf16
 * x); row_scale float32 [M], 16-byte aligned.  No counterpart in the
 * reference (the guard of this library's fp16 MFMA operands).
 */
int rpfq_row_prescale(const void* x, int x_dtype, int64_t M, int64_t C, void* y, float* row_scale, void* stream);

/*
 * rpfq_layer_norm followed by the activation fake quantization of
 * rpfq_act_quant on its output, in one pass over the rows: the float32
 * LayerNorm output is quantized per row and per half (C/2 columns each;
 * C % 16 == 0) and only the quantized value is rounded to y_dtype, as the
 * reference quantizes its float32 LayerNorm output; y is bit-identical to
 * rpfq_layer_norm with float32 output followed by rpfq_act_quant with
 * y_dtype output.  bits: 2 .. 16.  The quantized input of the qkv and fc1 layers
 * of a block with activation quantization on
 *   RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:520, :549 followed by
 *   RPFQ-ViT-main/quant_models/quant_i.py:546-551.
 */
int rpfq_layer_norm_act_quant(const void* x, int x_dtype, int64_t M, int64_t C, const float* gamma,
                              const float* beta, float eps, int bits, void* y, int y_dtype, void* stream);

/*
 * The exact GELU (approximate = 'none') of each element of x [M, C] in
 * float32 followed by the activation fake quantization of rpfq_act_quant,
 * in one pass over the rows: the float32 GELU is quantized per row and per
 * half (C/2 columns each; C % 16 == 0), only the quantized value rounded to
 * y_dtype, as the reference quantizes fc2's float32 input; y is
 * bit-identical to torch's GELU with float32 output followed by
 * rpfq_act_quant with y_dtype output.  bits: 2 .. 16.  x and y 16-byte
 * aligned, C up to 4096; y may equal x.  The fc2 input of a block with
 * activation quantization on:
 *   RPFQ-ViTApple/scripts/audit_rpfq_vit_ios_parity.py:550-553 (act, fc2)
 *   with RPFQ-ViT-main/quant_models/quant_i.py:546-551 inside fc2.
 */
int rpfq_gelu_act_quant(const void* x, int x_dtype, int64_t M, int64_t C, int bits, void* y, int y_dtype,
                        void* stream);

/*
 * Activation fake quantization of a [M, in_features] feature block laid out
 * [re | im]: per row and per half, scale = qmax * (1 / max(max|x|, 1e-5)),
 * y = clamp(round_half_even(x * scale), -2^(bits-1), 2^(bits-1)-1) / scale,
 * in float32 (bit-exact for float32 in/out).
 * Replaces ActivationQuantSTE / ComplexActivationQuantizer
 *   RPFQ-ViT-main/quant_models/quant_i.py:438-472, applied at :546-551.
 */
int rpfq_act_quant(const void* x, int x_dtype, int64_t M, int64_t in_features, int bits,
                   void* y, int y_dtype, void* stream);

/*
 * Write the fused float32 weight A_q [2N', 2K'] that the packed layer
 * represents (quant_i.py:534-544 layout), decoded by the same device code the
 * GEMM uses (bit-identical to the reference's float32 A_q).  round_fp16 = 1
 * writes the fp16 coefficients the MFMA consumes (see rpfq_wide_linear).
 * Replaces export_rpfq_vit_to_mlx.py:336-375 (quantized_forward_weight).
 */
int rpfq_wide_decode(const rpfq_wide_desc* desc, const void* packed, size_t packed_bytes,
                     float* a, int round_fp16, void* stream);

/* weight quantizer kinds (training semantics) */
#define RPFQ_QK_AXIS 0  /* dominant-axis stages, quant_i.py:36-81 (complex_phase_v1..v4) */
#define RPFQ_QK_SIGN 1  /* quadrant-sign stages, quant_i.py:84-91 (complex_phase_new_v2) */

/* Shape and methods of one QATLinearComplexPhase weight for rpfq_quantize_wide. */
typedef struct rpfq_quant_desc {
    int64_t n_complex; /* N' = out_features / 2 */
    int64_t k_complex; /* K' = in_features / 2 */
    int32_t kind[2];   /* RPFQ_QK_* of U and of W */
    int32_t steps[2];  /* residual stages of U and of W, 1..4 */
} rpfq_quant_desc;

/* Bytes of the device workspace rpfq_quantize_wide needs (fixed, 64 KiB). */
size_t rpfq_quantize_workspace_bytes(const rpfq_quant_desc* desc);

/*
 * Quantize one float32 master weight the way the reference's training
 * forward does, on the GPU:
 *   RPFQ-ViT-main/quant_models/quant_i.py:513-544 (2x2 split into U, W;
 *   recombination into A_q) with ComplexWeightQuantizer.forward (:418-435,
 *   optional rotation) over _residual_quantize (:94-118) of
 *   _quantize_phase_axis (:65-81) or _quantize_sign_phase (:84-91).
 * weight: float32 [2N', 2K'] row-major.
 * rot:    NULL (no rotation) or float32 [4] = cos theta_u, sin theta_u,
 *         cos theta_w, sin theta_w (device memory).
 * a_q:    NULL or float32 [2N', 2K'] output: the quantized weight.
 * scales: float32 [2][4][2] output: (U, W) x stage x (re, im) multipliers;
 *         slots past a plane's stages are 0.
 * codes:  NULL or uint8 [steps_u + steps_w][N'][K'/4] output: each stage's
 *         2-bit codes in the exporter's packing (export…py:148-159; AXIS:
 *         real_pos 1, imag_neg 2, imag_pos 3, else 0; SIGN: bit0 re >= 0,
 *         bit1 im >= 0), ordered u_s0.., w_s0..; needs K' % 4 == 0.
 *         With scale_re/scale_im of these planes taken from `scales`, they
 *         are the input of rpfq_wide_pack (the rotation goes in the desc);
 *         codes also need 16-byte aligned weight and a_q.
 * work:   device buffer of rpfq_quantize_workspace_bytes(desc) bytes.
 * Each scale is the reference's masked mean with the sum accumulated in
 * float64 and rounded once to float32 (torch sums float32 in its own order:
 * the two agree to about 1 ulp); codes and A_q follow from the scales
 * bit-exactly.  Deterministic.  Asynchronous on `stream`; the buffers must
 * not overlap.
 */
int rpfq_quantize_wide(const rpfq_quant_desc* desc, const float* weight, const float* rot, float* a_q,
                       float* scales, uint8_t* codes, void* work, size_t work_bytes, void* stream);

/*
 * rpfq_quantize_wide without a workspace argument and without any device
 * allocation: the float64 partials live in a static device array of this
 * library (64 KiB per GPU, held until the process ends), so the call makes
 * no hipMalloc / hipFree and calls no allocating routine.  Inputs, outputs
 * and results are those of rpfq_quantize_wide (bit-identical); shapes whose
 * workspace would exceed the array are rejected (RPFQ_ERR_SHAPE).  Every
 * call on a GPU shares that GPU's array, so calls that overlap on one GPU
 * (concurrent streams, several host threads) race; calls ordered on one
 * stream do not.  No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, tight serving or training
 * loops, harnesses that forbid allocation).
 */
int rpfq_quantize_wide_noalloc(const rpfq_quant_desc* desc, const float* weight, const float* rot, float* a_q,
                               float* scales, uint8_t* codes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RPFQ_H_ */
