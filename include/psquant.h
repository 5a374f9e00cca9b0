/*
 * psquant.h -- C ABI of libpsquant.so, the MI355X (gfx950) quantized linear library.
 *
 * Plain pointers and sizes only; the caller (PyTorch) owns every buffer.  The library
 * never allocates or frees device memory on these entry points.  Every launch goes to the
 * caller's stream (`stream` is a hipStream_t passed as void*; NULL = the null stream).
 * Every function returns 0 on success and a negative PSQ_E* code on failure, after which
 * psq_last_error() returns a message for the calling thread.  Entry points are re-entrant
 * and hold no per-call state.  A problem with no rows or no columns (M or N zero) is a no-op
 * that succeeds whatever its data pointers (empty tensors may have null ones).
 *
 * Reference interfaces replaced (ComfyUI-PowerShard 0.6.0):
 *   - powershard/quant_linear.py:230-242 native_linear() -> comfy-kitchen ops
 *     int8_linear / torch._scaled_mm / w4a8_int8_linear (NATIVE table, quant_linear.py:32-35)
 *   - powershard/quant_linear.py:245-265 native_support()
 *   - powershard/quant_linear.py:219-220 qt.dequantize() of the dequantize branch
 *   - powershard/operations.py:84-93   dequantize_rows()
 * Arithmetic conventions (bit-exact where stated) are those of the CPU oracle,
 * oracle/psq_oracle.c, restated in the comments below.
 */
#ifndef PSQUANT_H
#define PSQUANT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PSQ_ABI_VERSION 1

#if defined(__GNUC__)
#define PSQ_API __attribute__((visibility("default")))
#else
#define PSQ_API
#endif

/* element types of activations, bias and outputs */
enum psq_dtype { PSQ_BF16 = 0, PSQ_F16 = 1, PSQ_F32 = 2 };

/* error codes */
enum psq_status {
    PSQ_OK = 0,
    PSQ_E_ARG = -1,         /* bad argument (null pointer, negative size, bad dtype) */
    PSQ_E_SHAPE = -2,       /* shape/stride/alignment outside what the kernel supports */
    PSQ_E_DEVICE = -3,      /* no gfx950 device current, or a HIP runtime error */
    PSQ_E_LAUNCH = -4       /* kernel launch failed */
};

/* ABI version (PSQ_ABI_VERSION). */
PSQ_API int psq_abi_version(void);

/* Message of the last failing call on this thread ("" if none).  Never NULL. */
PSQ_API const char *psq_last_error(void);

/* 1 if HIP device `device` is a gfx950 (MI355X-class) GPU the kernels are built for, else 0.
 * Replaces native_support()'s capability probe (powershard/quant_linear.py:245-265). */
PSQ_API int psq_device_supported(int device);

/* ---------------------------------------------------------------- activations
 * Fused ConvRot rotation + per-row (token) absmax + quantize.  Replaces the activation
 * side of comfy-kitchen's int8_linear / QuantizedTensor.from_float(rows, layout, scale)
 * (powershard/quant_linear.py:233-236).
 *   x      [M, K] bf16/f16 (x_dtype), row stride ldx elements, 16-byte aligned rows
 *   rot_group  0 (no rotation) or a power of 4 in [4, 1024] dividing K: each group of
 *          rot_group consecutive elements is multiplied by the regular Hadamard
 *          H4^{(x)k}/sqrt(g) (powershard/operations.py:72-81) with the fixed-order fast
 *          transform of the oracle.
 *   static_scale  NULL for dynamic per-row scale, or a device pointer to one fp32 value
 *          (the module's input_scale, powershard/quant_linear.py:28-30)
 *   q      [M, K] int8 / e4m3fn codes, row stride ldq bytes
 *   scale  [M] fp32 per-row scale (s = absmax/127 or absmax/448; 0 -> 1)
 * A row holding a NaN gets a NaN scale (the absmax propagates NaN, as torch's amax does), so its
 * GEMM output row is NaN; a NaN product takes the lower code bound (-127, or -448 in e4m3).
 * K must be a multiple of 16 and at most 32768.  Bit-exact with the oracle. */
PSQ_API int psq_quantize_rows_i8(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                         int rot_group, const float *static_scale, int8_t *q, int64_t ldq,
                         float *scale, void *stream);
PSQ_API int psq_quantize_rows_fp8(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                          int rot_group, const float *static_scale, uint8_t *q, int64_t ldq,
                          float *scale, void *stream);

/* Rotation only: y = round_out(x H) per group of rot_group elements, the same fixed-order fast
 * transform in fp32 as above (H the normalized regular Hadamard), one rounding to y_dtype
 * (bf16/f16/f32, ldy elements).  rot_group 0 converts only.  The activation side of the ConvRot
 * int8 weight-only linear: x W^T = (x H)(q s)^T for weights stored as W H, so Int8Linear
 * (powershard/operations.py:96-132, dequantize_rows 84-93) runs as psq_rotate_rows +
 * psq_gemm_w8a16 instead of N/rows tile dequantizations.  K as above.  Bit-exact with the oracle. */
PSQ_API int psq_rotate_rows(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int rot_group,
                    void *y, int y_dtype, int64_t ldy, void *stream);

/* ---------------------------------------------------------------------- GEMMs
 * W8A8: y[m][n] = round_out(fmaf((float)acc, a_scale[m] * w_scale[n], bias[n])),
 * acc = sum_k a[m][k] * w[n][k] in int32.  Replaces comfy-kitchen int8_linear behind
 * F.linear(QuantizedTensor, QuantizedTensor, bias) (powershard/quant_linear.py:236-237).
 *   a [M, K] int8 (lda), w [N, K] int8 (ldw), a_scale [M] fp32, w_scale [N] fp32,
 *   bias [N] (bias_dtype) or NULL, y [M, N] (y_dtype, ldy elements).
 * K % 128 == 0; lda, ldw multiples of 16; 16-byte aligned a, w. */
PSQ_API int psq_gemm_i8(const int8_t *a, int64_t lda, const float *a_scale, const int8_t *w,
                int64_t ldw, const float *w_scale, const void *bias, int bias_dtype, void *y,
                int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream);

/* Same GEMM, raw int32 accumulators c[m][n] (ldc elements); for bit-exact checking. */
PSQ_API int psq_gemm_i8_i32(const int8_t *a, int64_t lda, const int8_t *w, int64_t ldw, int32_t *c,
                    int64_t ldc, int64_t M, int64_t N, int64_t K, void *stream);

/* psq_gemm_i8 with bf16 output, scheduled as 8 waves per workgroup (two per SIMD, 128 x 64 wave
 * tiles) instead of 4: the same outputs bit for bit.  A comparison schedule with no counterpart in
 * the reference, not used by the module path (it measures slower than psq_gemm_i8 on every shape
 * tried); kept so that the comparison can be re-run.  N % 256 == 0, K % 256 == 0, y_dtype
 * PSQ_BF16, 16-byte aligned a, w, y; ldy a multiple of 8. */
PSQ_API int psq_gemm_i8_8wave(const int8_t *a, int64_t lda, const float *a_scale, const int8_t *w,
                      int64_t ldw, const float *w_scale, const void *bias, int bias_dtype, void *y,
                      int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream);

/* FP8 e4m3fn x e4m3fn -> fp32 accumulate on the gfx950 f8f6f4 MFMA, same epilogue.
 * w_scale is one fp32 (w_scale_per_row = 0) or [N] (1).  Replaces torch._scaled_mm for
 * float8_e4m3fn (powershard/quant_linear.py:32, 236-237). */
PSQ_API int psq_gemm_fp8(const uint8_t *a, int64_t lda, const float *a_scale, const uint8_t *w,
                 int64_t ldw, const float *w_scale, int w_scale_per_row, const void *bias,
                 int bias_dtype, void *y, int y_dtype, int64_t ldy, int64_t M, int64_t N,
                 int64_t K, void *stream);

/* FP8 with float8_e5m2 weights: e4m3fn activation codes (psq_quantize_rows_fp8) x e5m2 weight
 * codes -> fp32 accumulate on the same f8f6f4 MFMA (A-operand format bf8), same epilogue and
 * arguments as psq_gemm_fp8.  Replaces the native GEMM of comfy_quant "float8_e5m2"
 * (powershard/quant_linear.py:32, 230-242), whose weights keep their e5m2 codes; the activations
 * are quantized to e4m3fn, the finer of the two formats (3 mantissa bits against 2). */
PSQ_API int psq_gemm_fp8_e5m2w(const uint8_t *a, int64_t lda, const float *a_scale,
                 const uint8_t *w, int64_t ldw, const float *w_scale, int w_scale_per_row,
                 const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy, int64_t M,
                 int64_t N, int64_t K, void *stream);

/* GEMM epilogue activations (the *_act entry points). */
enum psq_activation {
    PSQ_ACT_NONE = 0,
    PSQ_ACT_GELU_TANH = 1,  /* gelu(v) = v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))) / 2 */
    PSQ_ACT_SILU_GATE = 2   /* h[j] = silu(v[j]) v[H + j], H = N / 2; y is [M, H] */
};

/* W8A8 / FP8 GEMM with an activation fused into the epilogue:
 *   y[m][n] = round_out(act(round_out(fmaf((float)acc, a_scale[m] * w_scale[n], bias[n]))))
 * act in fp32 on the rounded linear output: the numerics of the Wan FFN's
 * F.gelu(fc1(rows).float(), approximate="tanh") (powershard/wan_model.py:626, chunked_mlp
 * 589-630) followed by the .to(compute dtype) of fc2's QuantLinear.forward
 * (powershard/quant_linear.py:197), with the fp32 hidden never written: the up-projection writes
 * the down-projection's input directly.  GELU is evaluated as v / (1 + exp(-2 z)), the same
 * function as the tanh form without its cancellation: results are within one output ulp of the
 * exact function, and of torch's fp32 F.gelu up to 1e-6 absolute (the fp32 tanh form loses
 * relative precision below v = -3); below v = -9.6 (|gelu| < 1e-37) they are -0.  Arguments as in
 * psq_gemm_i8 / psq_gemm_fp8; y_dtype bf16, f16 or f32 (f32: no inner rounding).
 * activation PSQ_ACT_NONE gives exactly psq_gemm_i8 / psq_gemm_fp8.
 * PSQ_ACT_SILU_GATE is the H3 MLP's gate (powershard/fp16_safe.py:165-167:
 * gate, up = fc1(rows).chunk(2, -1); F.silu(gate.float()) * up.float()): the weight's N rows are
 * the gate rows, then the up rows, N a multiple of 128 and N ldw + K < 2^32; y is [M, N / 2]
 * (ldy >= N / 2) with y[m][j] = round_out(silu(g) u), g and u the rounded linear outputs of
 * columns j and N / 2 + j, silu(g) = g / (1 + exp(-g)) in fp32 (-0 for g < -88.7, where
 * |silu| < 1e-36).  The pairs meet in registers: a tile's W rows are read as 64 gate rows
 * followed by their 64 up rows, so the N x K weight is used as stored. */
PSQ_API int psq_gemm_i8_act(const int8_t *a, int64_t lda, const float *a_scale, const int8_t *w,
                    int64_t ldw, const float *w_scale, const void *bias, int bias_dtype, int activation,
                    void *y, int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream);
PSQ_API int psq_gemm_fp8_act(const uint8_t *a, int64_t lda, const float *a_scale, const uint8_t *w,
                     int64_t ldw, const float *w_scale, int w_scale_per_row, const void *bias,
                     int bias_dtype, int activation, void *y, int y_dtype, int64_t ldy, int64_t M,
                     int64_t N, int64_t K, void *stream);

/* W4A16: uint4 asymmetric group weights dequantized in registers,
 * w = round_bf16((float(q) - float(zero)) * float(scale)), multiplied on bf16 MFMA with
 * fp32 accumulation; y = round_out(acc + bias).  Replaces the int4 F.linear dispatch
 * (powershard/quant_linear.py:239, weight-only formats) and matches the dequantize
 * branch F.linear(rows, qt.dequantize().to(bf16), bias) (quant_linear.py:219-220).
 * The decode kernel (M <= 8 whose activations fit in LDS beside the weight rings, group_size
 * a multiple of 128, K a multiple of 512), the
 * weight-streaming kernel (M <= 64, group_size a multiple of 128) and the tiled kernel (M > 64)
 * form w = round_bf16(fmaf(q, scale, -(zero * scale))), which differs from the formula above by
 * one bf16 ulp on about 2^-16 of the weights; all are within the fp32-accumulation bar.
 *   x [M, K] bf16 (ldx), wq [N, K/2] bytes (low nibble = even k), scale/zero [N, K/group]
 *   fp16, group_size a multiple of 64 dividing K. */
PSQ_API int psq_gemm_w4a16(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq,
                   const uint16_t *w_scale, const uint16_t *w_zero, int group_size,
                   const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy,
                   int64_t M, int64_t N, int64_t K, void *stream);

/* W8A16 (int8 weight-only, per-row fp32 scale): y = round_out(fmaf(sum x*q, w_scale[n],
 * bias[n])), x bf16, q exact in bf16.  Int8 weight-only linear of
 * powershard/operations.py:96-132 (Int8Linear, non-ConvRot storage). */
PSQ_API int psq_gemm_w8a16(const void *x, int x_dtype, int64_t ldx, const int8_t *wq,
                   const float *w_scale, const void *bias, int bias_dtype, void *y,
                   int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream);

/* Split-K workspace of the weight-only GEMMs.  When M, N and K leave CUs idle under the tiled
 * kernel (M > 64; e.g. M = 128 at N = 25600: 100 output tiles of 128 x 256 for 256 CUs, or M = 1024
 * at N = K = 5120: 160 tiles), the *_ws entry points split K across workgroups (stream-K): each
 * tile's K range in a few equal parts, or the (tile, K stage) units of all tiles in equal runs
 * that cross tile boundaries.  A workgroup holding part of a tile writes its fp32 partial tile to
 * the workspace and counts itself in the tile's counter there; the last one to finish adds the
 * partials in K order (a fixed order: results do not depend on timing) and applies the epilogue.
 * Same outputs and bars as psq_gemm_w4a16 / psq_gemm_w8a16 (a different fp32 summation order).
 * No counterpart in the reference (the caller-allocated workspace follows the ownership rule
 * above); the callers are the int4 and int8 weight-only linears of the text encoder and
 * Int8Linear.
 *   workspace        NULL: no split (exactly psq_gemm_w4a16 / psq_gemm_w8a16); else 256-byte
 *                    aligned and at least psq_gemm_wonly_workspace_bytes() bytes, all zero when
 *                    first passed (hipMemset once after allocating it).  Its first 64 KB hold the
 *                    tiles' arrival counters, which every call leaves zero again (the last
 *                    workgroup of a tile resets them); the rest holds partials that a call
 *                    writes before it reads them.  Keep it for this use only, and do not let
 *                    calls that share it overlap (use one workspace per stream). */
enum psq_weight_kind { PSQ_W_UINT4 = 0, PSQ_W_INT8 = 1 };

/* Bytes of workspace a *_ws call of this shape uses on the current device (0: no split). */
PSQ_API int64_t psq_gemm_wonly_workspace_bytes(int weight_kind, int64_t ldx, int64_t M, int64_t N, int64_t K,
                                               int group_size);
PSQ_API int psq_gemm_w4a16_ws(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq,
                      const uint16_t *w_scale, const uint16_t *w_zero, int group_size,
                      const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy,
                      int64_t M, int64_t N, int64_t K, void *workspace, int64_t workspace_bytes,
                      void *stream);
PSQ_API int psq_gemm_w8a16_ws(const void *x, int x_dtype, int64_t ldx, const int8_t *wq,
                      const float *w_scale, const void *bias, int bias_dtype, void *y,
                      int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *workspace,
                      int64_t workspace_bytes, void *stream);

/* psq_gemm_w4a16_ws without the workspace argument: the split-K counters and partial tiles live in
 * a static device array of the library (64 MB + 64 KB on each GPU it runs on, held until the
 * process ends), so the call allocates nothing -- no hipMalloc, no hipFree, no allocating library
 * routine.  No counterpart in the reference; it is for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid allocation.
 * Same arguments and results as psq_gemm_w4a16_ws with a large enough workspace.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU race.  A shape whose split plan
 * needs more than the array is refused with PSQ_E_SHAPE (no plan asks for more). */
PSQ_API int psq_gemm_w4a16_noalloc(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq,
                           const uint16_t *w_scale, const uint16_t *w_zero, int group_size,
                           const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy,
                           int64_t M, int64_t N, int64_t K, void *stream);

/* ---------------------------------------------------------------- dequantize
 * GPU implementations of QuantizedTensor.dequantize() for the dequantize compute mode
 * (powershard/quant_linear.py:216-220) and of dequantize_rows (operations.py:84-93). */

/* out[n][k] = round_out((float(q) - float(zero)) * float(scale)), uint4 layout as above. */
PSQ_API int psq_dequant_uint4(const uint8_t *wq, const uint16_t *w_scale, const uint16_t *w_zero,
                      int group_size, int64_t N, int64_t K, void *out, int out_dtype,
                      void *stream);

/* out = round_out((float)q * scale[n]) then, when rot_group > 0, each group of rot_group
 * values multiplied by H^T (= H) with the oracle's fixed-order fast transform, in fp32.
 * K a multiple of 16, at most 32768. */
PSQ_API int psq_dequant_i8_rows(const int8_t *q, const float *w_scale, int64_t N, int64_t K,
                        int rot_group, void *out, int out_dtype, void *stream);

/* out = round_out(e4m3_to_f32(q) * scale[n or 0]). */
PSQ_API int psq_dequant_fp8(const uint8_t *q, const float *w_scale, int w_scale_per_row, int64_t N,
                    int64_t K, void *out, int out_dtype, void *stream);

/* out = round_out(e5m2_to_f32(q) * scale[n or 0]): the float8_e5m2 weights' decode
 * (powershard/quant_linear.py:387-404 for an F8_E5M2 file weight; comfy_quant "float8_e5m2",
 * quant_linear.py:32).  e5m2_to_f32 is exact (the code is the high byte of an fp16). */
PSQ_API int psq_dequant_e5m2(const uint8_t *q, const float *w_scale, int w_scale_per_row, int64_t N,
                    int64_t K, void *out, int out_dtype, void *stream);

/* ---------------------------------------------------------------- checks */

/* Raises *flag (a device word) to max(*flag, ticket) when any of the n elements of x (bf16 / f16
 * / f32, element-aligned) is NaN or +-Inf; one pass over x.  The device side of the output check
 * that closes Int8Linear.forward (powershard/operations.py:130-131: `not torch.isfinite(out).all()`
 * raises FloatingPointError), in place of torch's two kernels.  The flag is never cleared: keep one
 * per stream, zero once, and pass increasing tickets (from 1); the call's elements were all finite
 * exactly when the flag read after it is below its ticket.  No hipMemsetAsync, so a captured
 * launch replays correctly. */
PSQ_API int psq_flag_nonfinite(const void *x, int dtype, int64_t n, unsigned long long *flag,
                               unsigned long long ticket, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* PSQUANT_H */
