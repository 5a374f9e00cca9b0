// dequant.hip -- GPU QuantizedTensor.dequantize() for the three weight layouts, and
// dequantize_rows (powershard/operations.py:84-93) with the ConvRot inverse.
//
// Used by the dequantize compute mode of QuantLinear (powershard/quant_linear.py:216-220) on a
// GPU, and as the bit-exact probe of the in-register uint4 dequantization of gemm_w4a16
// (same formula: round_out((float(q) - float(z)) * float(s))).  All HBM-bound elementwise
// passes: one thread per 16 output elements, vector loads and stores.
#include "psq_common.hpp"

namespace psq {
namespace {

constexpr int NT = 256;

template <int ODT>
__device__ __forceinline__ void store16(void *out, int64_t base, const float (&v)[16])
{
    if constexpr (ODT == PSQ_F32) {
        v4f *o = (v4f *)((float *)out + base);
#pragma unroll
        for (int i = 0; i < 4; i++) o[i] = v4f{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
    } else {
        uint32_t h[8];
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = f32_to_half<ODT>(v[2 * i]) | (f32_to_half<ODT>(v[2 * i + 1]) << 16);
        v4i *o = (v4i *)((uint16_t *)out + base);
        o[0] = v4i{(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
        o[1] = v4i{(int)h[4], (int)h[5], (int)h[6], (int)h[7]};
    }
}

// uint4: thread handles 16 consecutive k of one row (8 bytes of packed nibbles)
template <int ODT>
__global__ void __launch_bounds__(NT)
dequant_uint4_kernel(const uint8_t *__restrict__ wq, const uint16_t *__restrict__ sc, const uint16_t *__restrict__ zp,
                     int gs, int64_t N, int64_t K, void *__restrict__ out)
{
    const int64_t per_row = K / 16;
    const int64_t id = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (id >= N * per_row) return;
    const int64_t n = id / per_row, k0 = (id % per_row) * 16;
    const v2i p = *(const v2i *)(wq + n * (K / 2) + k0 / 2);
    float v[16];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        // a group boundary can fall inside these 16 values only when gs < 16 (gs >= 16 enforced)
        const int64_t gi = n * (K / gs) + (k0 + 8 * h) / gs;
        const float s = f16_to_f32(sc[gi]), z = f16_to_f32(zp[gi]);
        const uint32_t w = (uint32_t)p[h];
#pragma unroll
        for (int e = 0; e < 8; e++) v[8 * h + e] = ((float)((w >> (4 * e)) & 15u) - z) * s;
    }
    store16<ODT>(out, n * K + k0, v);
}

// fp8 weights: E5M2 false decodes e4m3fn codes, true e5m2 codes
template <int ODT, bool E5M2>
__global__ void __launch_bounds__(NT)
dequant_fp8_kernel(const uint8_t *__restrict__ q, const float *__restrict__ sc, int per_row, int64_t N, int64_t K,
                   void *__restrict__ out)
{
    const int64_t per_row_t = K / 16;
    const int64_t id = (int64_t)blockIdx.x * NT + threadIdx.x;
    if (id >= N * per_row_t) return;
    const int64_t n = id / per_row_t, k0 = (id % per_row_t) * 16;
    const v4i p = *(const v4i *)(q + n * K + k0);
    const float s = sc[per_row ? n : 0];
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t c = ((uint32_t)p[i >> 2] >> (8 * (i & 3))) & 0xffu;
        v[i] = (E5M2 ? e5m2_to_f32(c) : e4m3_to_f32(c)) * s;
    }
    store16<ODT>(out, n * K + k0, v);
}

// int8 rows: one workgroup per row; thread t owns P chunks of 16 consecutive values, chunk c at
// elements [(c T + t) 16, +16) (T = blockDim.x, a multiple of 64), so each wave covers 1024
// consecutive values per chunk and ConvRot groups (at most 1024, dividing K) never straddle waves.
// The ConvRot inverse is the quantizer's transform (H is symmetric, so v @ H^T = 2^-k T(v)).
// Lanes past K carry zeros through the cross-lane stages: their groups lie wholly past K.
template <int ODT, int ROTK, int P>
__global__ void __launch_bounds__(1024)
dequant_i8_rows_kernel(const int8_t *__restrict__ q, const float *__restrict__ sc, int64_t K, void *__restrict__ out)
{
    const int64_t n = blockIdx.x;
    const int t = threadIdx.x, T = blockDim.x;
    const float s = sc[n];
#pragma unroll
    for (int c = 0; c < P; c++) {
        const int64_t e0 = (int64_t)(c * T + t) * 16;
        const bool active = e0 < K;
        float v[16];
        v4i p = {0, 0, 0, 0};
        if (active) p = *(const v4i *)(q + n * K + e0);
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = (float)(int8_t)(((uint32_t)p[i >> 2] >> (8 * (i & 3))) & 0xffu) * s;
        if constexpr (ROTK >= 1) {
#pragma unroll
            for (int b = 0; b < 16; b += 4) radix4(v[b], v[b + 1], v[b + 2], v[b + 3]);
        }
        if constexpr (ROTK >= 2) {
#pragma unroll
            for (int a = 0; a < 4; a++) radix4(v[a], v[a + 4], v[a + 8], v[a + 12]);
        }
        if constexpr (ROTK >= 3) {
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = radix4_lanes<1>(v[j]);
        }
        if constexpr (ROTK >= 4) {
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = radix4_lanes<4>(v[j]);
        }
        if constexpr (ROTK >= 5) {
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = radix4_lanes<16>(v[j]);
        }
        if constexpr (ROTK > 0) {
            const float post = __builtin_ldexpf(1.0f, -ROTK);
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = v[j] * post;
        }
        if (active) store16<ODT>(out, n * K + e0, v);
    }
}

int check_out(const char *name, int64_t N, int64_t K, const void *out, int out_dtype)
{
    if (N < 0 || K < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    if (!out) return set_error(PSQ_E_ARG, "%s: null output", name);
    if (!valid_dtype(out_dtype)) return set_error(PSQ_E_ARG, "%s: bad dtype", name);
    if (K % 16) return set_error(PSQ_E_SHAPE, "%s: K=%lld must be a multiple of 16", name, (long long)K);
    if ((uintptr_t)out & 15) return set_error(PSQ_E_SHAPE, "%s: output must be 16-byte aligned", name);
    return PSQ_OK;
}

unsigned blocks_for(int64_t n) { return (unsigned)((n + NT - 1) / NT); }

template <bool E5M2>
int dequant_fp8_any(const uint8_t *q, const float *w_scale, int w_scale_per_row, int64_t N, int64_t K, void *out,
                    int out_dtype, void *stream, const char *name)
{
    if (int e = check_out(name, N, K, out, out_dtype)) return e;
    if (N == 0 || K == 0) return PSQ_OK;
    if (!q || !w_scale) return set_error(PSQ_E_ARG, "%s: null pointer", name);
    if ((uintptr_t)q & 15) return set_error(PSQ_E_SHAPE, "%s: weights must be 16-byte aligned", name);
    if (int e = require_device()) return e;
    const unsigned nb = blocks_for(N * (K / 16));
    hipStream_t st = (hipStream_t)stream;
    const int pr = w_scale_per_row ? 1 : 0;
    if (out_dtype == PSQ_BF16) dequant_fp8_kernel<PSQ_BF16, E5M2><<<nb, NT, 0, st>>>(q, w_scale, pr, N, K, out);
    else if (out_dtype == PSQ_F16) dequant_fp8_kernel<PSQ_F16, E5M2><<<nb, NT, 0, st>>>(q, w_scale, pr, N, K, out);
    else dequant_fp8_kernel<PSQ_F32, E5M2><<<nb, NT, 0, st>>>(q, w_scale, pr, N, K, out);
    return check_launch(name);
}

}  // namespace
}  // namespace psq

extern "C" {

int psq_dequant_uint4(const uint8_t *wq, const uint16_t *w_scale, const uint16_t *w_zero, int group_size, int64_t N,
                      int64_t K, void *out, int out_dtype, void *stream)
{
    using namespace psq;
    if (int e = check_out("dequant_uint4", N, K, out, out_dtype)) return e;
    if (N == 0 || K == 0) return PSQ_OK;
    if (!wq || !w_scale || !w_zero) return set_error(PSQ_E_ARG, "dequant_uint4: null pointer");
    if (group_size < 16 || group_size % 8 || K % group_size)
        return set_error(PSQ_E_SHAPE, "dequant_uint4: group size %d must be >= 16, a multiple of 8 dividing K",
                         group_size);
    if ((uintptr_t)wq & 7) return set_error(PSQ_E_SHAPE, "dequant_uint4: weights must be 8-byte aligned");
    if (int e = require_device()) return e;
    const unsigned nb = blocks_for(N * (K / 16));
    hipStream_t st = (hipStream_t)stream;
    if (out_dtype == PSQ_BF16) dequant_uint4_kernel<PSQ_BF16><<<nb, NT, 0, st>>>(wq, w_scale, w_zero, group_size, N, K, out);
    else if (out_dtype == PSQ_F16) dequant_uint4_kernel<PSQ_F16><<<nb, NT, 0, st>>>(wq, w_scale, w_zero, group_size, N, K, out);
    else dequant_uint4_kernel<PSQ_F32><<<nb, NT, 0, st>>>(wq, w_scale, w_zero, group_size, N, K, out);
    return check_launch("dequant_uint4");
}

int psq_dequant_fp8(const uint8_t *q, const float *w_scale, int w_scale_per_row, int64_t N, int64_t K, void *out,
                    int out_dtype, void *stream)
{
    return psq::dequant_fp8_any<false>(q, w_scale, w_scale_per_row, N, K, out, out_dtype, stream, "dequant_fp8");
}

int psq_dequant_e5m2(const uint8_t *q, const float *w_scale, int w_scale_per_row, int64_t N, int64_t K, void *out,
                     int out_dtype, void *stream)
{
    return psq::dequant_fp8_any<true>(q, w_scale, w_scale_per_row, N, K, out, out_dtype, stream, "dequant_e5m2");
}

int psq_dequant_i8_rows(const int8_t *q, const float *w_scale, int64_t N, int64_t K, int rot_group, void *out,
                        int out_dtype, void *stream)
{
    using namespace psq;
    if (int e = check_out("dequant_i8_rows", N, K, out, out_dtype)) return e;
    if (N == 0 || K == 0) return PSQ_OK;
    if (!q || !w_scale) return set_error(PSQ_E_ARG, "dequant_i8_rows: null pointer");
    if (K > 32 * 1024) return set_error(PSQ_E_SHAPE, "dequant_i8_rows: K=%lld > 32768", (long long)K);
    if ((uintptr_t)q & 15) return set_error(PSQ_E_SHAPE, "dequant_i8_rows: weights must be 16-byte aligned");
    if (N > 0x7fffffffLL) return set_error(PSQ_E_SHAPE, "dequant_i8_rows: N too large");
    int rotk = 0;
    if (rot_group) {
        int g = rot_group;
        while (g > 1 && (g & 3) == 0) { g >>= 2; rotk++; }
        if (g != 1 || rotk < 1 || rotk > 5 || K % rot_group)
            return set_error(PSQ_E_SHAPE, "dequant_i8_rows: rotation group %d must be a power of 4 in [4,1024] dividing K",
                             rot_group);
    }
    if (int e = require_device()) return e;
    // one 16-value chunk per thread up to K = 16384, two up to 32768
    const int64_t chunks16 = K / 16;
    const int P = chunks16 <= 1024 ? 1 : 2;
    const int threads = (int)(((chunks16 + P - 1) / P + 63) / 64 * 64);
    hipStream_t st = (hipStream_t)stream;
#define PSQ_DQ(ODT, RK)                                                                                     \
    (P == 1 ? dequant_i8_rows_kernel<ODT, RK, 1><<<dim3((unsigned)N), dim3(threads), 0, st>>>(q, w_scale, K, out) \
            : dequant_i8_rows_kernel<ODT, RK, 2><<<dim3((unsigned)N), dim3(threads), 0, st>>>(q, w_scale, K, out))
#define PSQ_DQ_ALL(ODT)                                                                                     \
    switch (rotk) {                                                                                         \
    case 0: PSQ_DQ(ODT, 0); break;                                                                          \
    case 1: PSQ_DQ(ODT, 1); break;                                                                          \
    case 2: PSQ_DQ(ODT, 2); break;                                                                          \
    case 3: PSQ_DQ(ODT, 3); break;                                                                          \
    case 4: PSQ_DQ(ODT, 4); break;                                                                          \
    default: PSQ_DQ(ODT, 5); break;                                                                         \
    }
    if (out_dtype == PSQ_BF16) { PSQ_DQ_ALL(PSQ_BF16) }
    else if (out_dtype == PSQ_F16) { PSQ_DQ_ALL(PSQ_F16) }
    else { PSQ_DQ_ALL(PSQ_F32) }
#undef PSQ_DQ_ALL
#undef PSQ_DQ
    return check_launch("dequant_i8_rows");
}

}  // extern "C"
