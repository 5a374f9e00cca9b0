// quantize_rows.hip -- fused ConvRot rotation + per-token absmax + int8 / fp8 quantization.
//
// The activation side of W8A8 (comfy-kitchen int8_linear / QuantizedTensor.from_float,
// reached from powershard/quant_linear.py:233-236) and of the fp8 scaled-mm path.
// Conventions (bit-exact with the CPU oracle):
//   u = T(x): unnormalized regular-Hadamard transform per group of g = 4^k elements
//     (x H = 2^-k T(x), H from powershard/operations.py:72-81), radix-4 stages over base-4
//     digits, least significant digit first, S = (x0 + x1) + (x2 + x3), y_j = fmaf(-2, x_{3-j}, S);
//   a = max |u| over the row; a == 0 -> s = 1, q = 0; else r = LIM / a, s = (a / LIM) 2^-k;
//   static input scale: s = s_in, r = (1 / s_in) 2^-k;
//   int8: q = clamp(rint(u r), -127, 127);  fp8: q = e4m3_rne(clamp(u r, -448, 448)).
//
// Layout: a workgroup quantizes R rows (tokens) side by side (R = 1 in use); a thread owns chunks of 16
// consecutive elements (32 bytes of bf16 in, 16 bytes of codes out; both fully coalesced), one
// chunk per 1024 threads of the row.  Base-4
// digits 0 and 1 of the element index live inside a thread, digit 2 on lane bits 0-1 (DPP quad
// permutes), digit 3 on lane bits 2-3 with its two bits swapped (DPP row rotates), digit 4 on lane
// bits 4-5 (cross-lane shuffle; g = 1024 only).  The lane stages of digits 2 and 3 leave their
// outputs in reversed digit order (each lane keeps the output its own input enters with -2), so a
// thread stores its results at the chunk of lane t ^ rev_lanes: same values, one exchange fewer per
// stage.  The row's absmax is reduced across the wave with DPP and row swaps and across waves
// through LDS.  2 bytes read + 1 byte written per element (+4 bytes per row).
#include "psq_common.hpp"

namespace psq {
namespace {

constexpr int kElemsPerThread = 16;
constexpr int kMaxThreads = 1024;
constexpr int kMaxChunks = 2;                                      // 16-element chunks per thread
constexpr int kMaxK = kElemsPerThread * kMaxThreads * kMaxChunks;  // 32768


template <int DT>
__device__ __forceinline__ void to_f32(const v4i (&raw)[2], float (&v)[16])
{
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t a = (uint32_t)raw[0][i], b = (uint32_t)raw[1][i];
        v[2 * i] = half_to_f32<DT>(a);
        v[2 * i + 1] = half_to_f32<DT>(a >> 16);
        v[8 + 2 * i] = half_to_f32<DT>(b);
        v[8 + 2 * i + 1] = half_to_f32<DT>(b >> 16);
    }
}

// Largest |v| over the 16 values, NaN if any is NaN (IEEE maximum: gfx950's v_maximum3_f32 with
// |.| source modifiers, two values per instruction).  A row holding a NaN thereby gets a NaN scale,
// as torch's amax gives, and its dequantized output is NaN.
__device__ __forceinline__ float absmax16(const float (&v)[16])
{
    float m = __builtin_elementwise_maximum(__builtin_fabsf(v[0]), __builtin_fabsf(v[1]));
#pragma unroll
    for (int j = 2; j < 16; j += 2)
        m = __builtin_elementwise_maximum(m, __builtin_elementwise_maximum(__builtin_fabsf(v[j]), __builtin_fabsf(v[j + 1])));
    return m;
}

// Wave-wide max of non-negative values (a NaN wins): the bit patterns of non-negative floats order
// as unsigned integers like their values, and a positive NaN's pattern lies above +inf's.  DPP within
// rows of 16 lanes, then the gfx950 row swaps across rows (no LDS, no index arithmetic).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ uint32_t wave_max_bits(uint32_t u)
{
    u = max(u, dpp_u32<DPP_QUAD_XOR1>(u));
    u = max(u, dpp_u32<DPP_QUAD_XOR2>(u));
    u = max(u, dpp_u32<DPP_ROW_HALF_MIRROR>(u));   // lane ^ 7: the other quad of the 8
    u = max(u, dpp_u32<DPP_ROW_MIRROR>(u));        // lane ^ 15: the other 8 of the row
    const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);   // rows 0 <-> 1, 2 <-> 3
    u = max((uint32_t)a[0], (uint32_t)a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);   // halves
    return max((uint32_t)b[0], (uint32_t)b[1]);
}

// int8 code of u r: clamp to [-127, 127] (equal to clamping after rounding, the bounds being
// integers), then + 1.5 * 2^23, which rounds to the nearest integer (ties to even) and leaves the
// code's two's complement in the low byte of the sum.  A NaN clamps to -127, as fmax(NaN, -127)
// does in the rounding-first order.
constexpr float kRoundMagic = 12582912.0f;

__device__ __forceinline__ float i8_clamp(float u) { return __builtin_fminf(__builtin_fmaxf(u, -127.0f), 127.0f); }

// Four codes packed into one word by the adds that round them: the first add writes the whole word
// (its low byte is code 0), the other three are v_add_f32 with an SDWA destination, which writes
// the low byte of the sum into byte B of the word and keeps the other bytes.  No separate pack.
template <int B>
__device__ __forceinline__ void add_into_byte(uint32_t &w, float u, float magic)
{
    static_assert(B >= 1 && B <= 3, "byte 1-3");
    if constexpr (B == 1)
        asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_1 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
            : "+v"(w) : "v"(u), "v"(magic));
    else if constexpr (B == 2)
        asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_2 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
            : "+v"(w) : "v"(u), "v"(magic));
    else
        asm("v_add_f32_sdwa %0, %1, %2 dst_sel:BYTE_3 dst_unused:UNUSED_PRESERVE src0_sel:DWORD src1_sel:DWORD"
            : "+v"(w) : "v"(u), "v"(magic));
}

__device__ __forceinline__ uint32_t i8_codes4(float u0, float u1, float u2, float u3, float magic)
{
    uint32_t w = __float_as_uint(i8_clamp(u0) + magic);
    add_into_byte<1>(w, i8_clamp(u1), magic);
    add_into_byte<2>(w, i8_clamp(u2), magic);
    add_into_byte<3>(w, i8_clamp(u3), magic);
    return w;
}

// Unnormalized transform of the 16 values of this thread (in-thread digits) and of the
// cross-lane digits, for a group size of 4^ROTK.  Digits 2 and 3 (lane bits 0-1 and 2-3) come out
// reversed (radix4_lanes_rev): the thread's 16 results belong to the chunk of thread t ^ rev_lanes.
template <int ROTK>
constexpr int rev_lanes() { return (ROTK >= 3 ? 3 : 0) | (ROTK >= 4 ? 12 : 0); }

// Chunk (within its wave's 64) that lane t loads: lane bits 2 and 3 swapped when digit 3 lives on
// them (see radix4_lanes_rev_sw4), so the chunk's digit-3 bit 0 sits on lane bit 3.  The wave's
// loads and stores cover the same 2 KB and 1 KB as in lane order.
template <int ROTK>
__device__ __forceinline__ int lane_chunk(int t)
{
    if constexpr (ROTK >= 4) return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1);
    else return t;
}

template <int ROTK>
__device__ __forceinline__ void rotate16(float (&v)[16])
{
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
        for (int j = 0; j < 16; j++) v[j] = radix4_lanes_rev<1>(v[j]);
    }
    if constexpr (ROTK >= 4) {
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = radix4_lanes_rev_sw4(v[j]);
    }
    if constexpr (ROTK >= 5) {
#pragma unroll
        for (int j = 0; j < 16; j++) v[j] = radix4_lanes<16>(v[j]);
    }
}

// A workgroup quantizes R consecutive rows side by side (all their loads issued up front, one
// shared barrier for the absmax reductions).  Thread t owns P chunks of 16 consecutive elements
// of each row: chunk c = elements [(c T + lane_chunk(t)) 16, +16), T = blockDim.x (a multiple of
// 64), so every wave covers 1024 consecutive elements per chunk and rotation groups (at most 1024,
// dividing K) never straddle waves.  TAIL: some chunk lies past K (P T 16 > K); without it every
// load and store is unconditional.
template <int DT, int ROTK, bool FP8, int P, int R, bool TAIL>
__global__ void __launch_bounds__(kMaxThreads)
quantize_rows_kernel(const uint16_t *__restrict__ x, int64_t ldx, int M, int K,
                     const float *__restrict__ static_scale, uint8_t *__restrict__ q, int64_t ldq,
                     float *__restrict__ scale)
{
    __shared__ uint32_t wave_amax[R][kMaxThreads / 64];
    const int t = threadIdx.x, T = blockDim.x, lc = lane_chunk<ROTK>(t);
    const int row0 = blockIdx.x * R;
    constexpr float LIM = FP8 ? 448.0f : 127.0f;
    const float post = ROTK ? __builtin_ldexpf(1.0f, -ROTK) : 1.0f;
    bool act[P];
#pragma unroll
    for (int c = 0; c < P; c++) act[c] = !TAIL || (c * T + lc) * kElemsPerThread < K;

    // The activations are read once, non-temporally: streamed through with normal loads they evict
    // the codes this kernel writes, and the weights, from the 256 MB memory-side cache just before
    // the GEMM reads them (M=32760 x K=5120: rotate+quantize then the int8 GEMM 1929 -> 1869 us,
    // the GEMM in that sequence 1836 -> 1775 us, the quantizer alone 92 -> 97 us).
    float v[R][P][16];
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const int row = min(row0 + rr, M - 1);
        const uint16_t *src = x + (int64_t)row * ldx + (int64_t)lc * kElemsPerThread;
#pragma unroll
        for (int c = 0; c < P; c++) {
            v4i raw[2] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
            if (act[c]) {
                raw[0] = __builtin_nontemporal_load((const v4i *)(src + (int64_t)c * T * kElemsPerThread));
                raw[1] = __builtin_nontemporal_load((const v4i *)(src + (int64_t)c * T * kElemsPerThread + 8));
            }
            to_f32<DT>(raw, v[rr][c]);
        }
    }
#pragma unroll
    for (int rr = 0; rr < R; rr++)
#pragma unroll
        for (int c = 0; c < P; c++) rotate16<ROTK>(v[rr][c]);

    // r multiplies the transformed values; the row scale s is only stored (by thread 0), so its
    // division runs in wave 0 alone
    float r[R], amax[R];
    if (static_scale) {
#pragma unroll
        for (int rr = 0; rr < R; rr++) r[rr] = (1.0f / *static_scale) * post;
    } else {
        const int nw = T >> 6;
#pragma unroll
        for (int rr = 0; rr < R; rr++) {
            float m = absmax16(v[rr][0]);
#pragma unroll
            for (int c = 1; c < P; c++) m = __builtin_elementwise_maximum(m, absmax16(v[rr][c]));
            const uint32_t bits = wave_max_bits(__float_as_uint(m));
            if ((t & 63) == 0) wave_amax[rr][t >> 6] = bits;
        }
        __syncthreads();
#pragma unroll
        for (int rr = 0; rr < R; rr++) {
            uint32_t bits = wave_amax[rr][0];
            for (int w = 1; w < nw; w++) bits = max(bits, wave_amax[rr][w]);
            amax[rr] = __uint_as_float(bits);
            r[rr] = amax[rr] == 0.0f ? 1.0f : LIM / amax[rr];
        }
    }
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const int row = row0 + rr;
        if (row >= M) break;
        if (t == 0)
            scale[row] = static_scale ? *static_scale : amax[rr] == 0.0f ? 1.0f : (amax[rr] / LIM) * post;
#pragma unroll
        for (int c = 0; c < P; c++) {
            if (!act[c]) continue;
            uint32_t packed[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float *u = &v[rr][c][4 * i];
                if constexpr (FP8) {
                    // gfx950's v_cvt_pk_fp8_f32 is the OCP e4m3fn encode with round to nearest
                    // even (subnormals included); the clamp keeps it off the overflow path and, as
                    // in the int8 codes, takes a NaN product to the lower bound
                    float uc[4];
#pragma unroll
                    for (int b = 0; b < 4; b++) uc[b] = __builtin_fminf(__builtin_fmaxf(u[b] * r[rr], -448.0f), 448.0f);
                    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(uc[0], uc[1], 0, false);
                    packed[i] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(uc[2], uc[3], lo, true);
                } else {
                    packed[i] = i8_codes4(u[0] * r[rr], u[1] * r[rr], u[2] * r[rr], u[3] * r[rr], kRoundMagic);
                }
            }
            *(v4i *)(q + (int64_t)row * ldq + (int64_t)(c * T + (lc ^ rev_lanes<ROTK>())) * kElemsPerThread) =
                v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
        }
    }
}

// Rotation only: y = round_out(2^-k T(x)) per group (x H with H the normalized regular Hadamard),
// the activation side of a ConvRot weight-only linear, x W^T = (x H)(q s)^T for weights stored as
// W H.  Same thread layout and transform as the quantizer; no reduction, so no barrier.
template <int DT, int ROTK, int OUT, int P>
__global__ void __launch_bounds__(kMaxThreads)
rotate_rows_kernel(const uint16_t *__restrict__ x, int64_t ldx, int K, void *__restrict__ y, int64_t ldy)
{
    const int t = threadIdx.x, T = blockDim.x, row = blockIdx.x, lc = lane_chunk<ROTK>(t);
    const float post = ROTK ? __builtin_ldexpf(1.0f, -ROTK) : 1.0f;
    const uint16_t *src = x + (int64_t)row * ldx + (int64_t)lc * kElemsPerThread;
#pragma unroll
    for (int c = 0; c < P; c++) {
        if ((c * T + lc) * kElemsPerThread >= K) break;
        const int64_t off = (int64_t)c * T * kElemsPerThread;
        v4i raw[2] = {*(const v4i *)(src + off), *(const v4i *)(src + off + 8)};
        float v[16];
        to_f32<DT>(raw, v);
        rotate16<ROTK>(v);
        const int64_t e0 = (int64_t)row * ldy + (int64_t)(c * T + (lc ^ rev_lanes<ROTK>())) * kElemsPerThread;
        if constexpr (OUT == PSQ_F32) {
            float *o = (float *)y + e0;
#pragma unroll
            for (int i = 0; i < 4; i++)
                *(v4f *)(o + 4 * i) = v4f{v[4 * i] * post, v[4 * i + 1] * post, v[4 * i + 2] * post, v[4 * i + 3] * post};
        } else {
            uint32_t w[8];
#pragma unroll
            for (int i = 0; i < 8; i++) w[i] = pack_half2<OUT>(v[2 * i] * post, v[2 * i + 1] * post);
            uint16_t *o = (uint16_t *)y + e0;
            *(v4i *)o = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            *(v4i *)(o + 8) = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
        }
    }
}

template <int DT, int OUT, int P>
int launch_rotate_p(const uint16_t *xp, int64_t M, int64_t K, int64_t ldx, int rotk, int threads, void *y,
                    int64_t ldy, hipStream_t st)
{
    const dim3 grid((unsigned)M), block(threads);
    switch (rotk) {
#define PSQ_CASE(RK)                                                                                    \
    case RK: rotate_rows_kernel<DT, RK, OUT, P><<<grid, block, 0, st>>>(xp, ldx, (int)K, y, ldy); break;
        PSQ_CASE(0) PSQ_CASE(1) PSQ_CASE(2) PSQ_CASE(3) PSQ_CASE(4) PSQ_CASE(5)
#undef PSQ_CASE
    default:
        return set_error(PSQ_E_SHAPE, "rotation group 4^%d unsupported", rotk);
    }
    return check_launch("rotate_rows");
}

template <int DT, int OUT>
int launch_rotate(const void *x, int64_t M, int64_t K, int64_t ldx, int rotk, void *y, int64_t ldy, hipStream_t st)
{
    const int64_t chunks16 = K / kElemsPerThread;
    const int P = chunks16 <= kMaxThreads ? 1 : 2;
    const int threads = (int)((chunks16 + P - 1) / P + 63) / 64 * 64;
    const uint16_t *xp = (const uint16_t *)x;
    if (P == 2) return launch_rotate_p<DT, OUT, 2>(xp, M, K, ldx, rotk, threads, y, ldy, st);
    return launch_rotate_p<DT, OUT, 1>(xp, M, K, ldx, rotk, threads, y, ldy, st);
}

template <int DT, bool FP8, int P, int R, bool TAIL>
int launch_quant_p(const uint16_t *xp, int64_t M, int64_t K, int64_t ldx, int rotk, int threads,
                   const float *static_scale, uint8_t *q, int64_t ldq, float *scale, hipStream_t st)
{
    const dim3 grid((unsigned)((M + R - 1) / R)), block(threads);
    switch (rotk) {
#define PSQ_CASE(RK)                                                                                \
    case RK:                                                                                        \
        quantize_rows_kernel<DT, RK, FP8, P, R, TAIL><<<grid, block, 0, st>>>(xp, ldx, (int)M, (int)K, \
                                                                              static_scale, q, ldq, scale); \
        break;
        PSQ_CASE(0) PSQ_CASE(1) PSQ_CASE(2) PSQ_CASE(3) PSQ_CASE(4) PSQ_CASE(5)
#undef PSQ_CASE
    default:
        return set_error(PSQ_E_SHAPE, "rotation group 4^%d unsupported", rotk);
    }
    return check_launch(FP8 ? "quantize_rows_fp8" : "quantize_rows_i8");
}

template <int DT, bool FP8>
int launch_quant(const void *x, int64_t M, int64_t K, int64_t ldx, int rotk,
                 const float *static_scale, uint8_t *q, int64_t ldq, float *scale, hipStream_t st)
{
    // chunks per thread: 1 up to 8192 elements, else 2 (up to 32768); one row per workgroup
    // (two rows side by side measured slower: 160 vs 138 us at 32760 x 5120).  Past 8192 the
    // smaller workgroups of two chunks per thread overlap their loads, reduction barrier and
    // stores better: 32760 x 13824 270 -> 238 us; at K = 5120 one chunk stays ahead (95 vs 100 us).
    const int64_t chunks16 = K / kElemsPerThread;
    const int P = chunks16 <= 512 ? 1 : 2;
    const int threads = (int)((chunks16 + P - 1) / P + 63) / 64 * 64;
    const uint16_t *xp = (const uint16_t *)x;
    const bool tail = (int64_t)P * threads * kElemsPerThread != K;
    if (P == 2)
        return tail ? launch_quant_p<DT, FP8, 2, 1, true>(xp, M, K, ldx, rotk, threads, static_scale, q, ldq, scale, st)
                    : launch_quant_p<DT, FP8, 2, 1, false>(xp, M, K, ldx, rotk, threads, static_scale, q, ldq, scale, st);
    return tail ? launch_quant_p<DT, FP8, 1, 1, true>(xp, M, K, ldx, rotk, threads, static_scale, q, ldq, scale, st)
                : launch_quant_p<DT, FP8, 1, 1, false>(xp, M, K, ldx, rotk, threads, static_scale, q, ldq, scale, st);
}

// rot_group 0 (rotk 0) or a power of 4 in [4, 1024] dividing K (rotk = its base-4 log)
int rot_log4(int rot_group, int64_t K, int &rotk)
{
    rotk = 0;
    if (!rot_group) return PSQ_OK;
    int g = rot_group;
    while (g > 1 && (g & 3) == 0) { g >>= 2; rotk++; }
    if (g != 1 || rotk < 1 || rotk > 5 || K % rot_group)
        return set_error(PSQ_E_SHAPE, "rotation group %d must be a power of 4 in [4,1024] dividing K=%lld", rot_group,
                         (long long)K);
    return PSQ_OK;
}

int rotate_rows(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int rot_group, void *y, int y_dtype,
                int64_t ldy, void *stream)
{
    if (M < 0 || K < 0) return set_error(PSQ_E_ARG, "negative size M=%lld K=%lld", (long long)M, (long long)K);
    if (M == 0) return PSQ_OK;
    if (!x || !y) return set_error(PSQ_E_ARG, "null pointer");
    if (x_dtype != PSQ_BF16 && x_dtype != PSQ_F16)
        return set_error(PSQ_E_ARG, "activations must be bf16 or f16 (dtype %d)", x_dtype);
    if (!valid_dtype(y_dtype)) return set_error(PSQ_E_ARG, "bad output dtype %d", y_dtype);
    if (K == 0 || K % kElemsPerThread || K > kMaxK)
        return set_error(PSQ_E_SHAPE, "K=%lld must be a positive multiple of 16 and <= %d", (long long)K, kMaxK);
    if (ldx < K || ldy < K || ldx % 8 || ldy % 8)
        return set_error(PSQ_E_SHAPE, "strides ldx=%lld ldy=%lld must be multiples of 8 covering K=%lld",
                         (long long)ldx, (long long)ldy, (long long)K);
    if (((uintptr_t)x & 15) || ((uintptr_t)y & 15)) return set_error(PSQ_E_SHAPE, "x and y must be 16-byte aligned");
    if (M > 0x7fffffffLL) return set_error(PSQ_E_SHAPE, "M=%lld too large", (long long)M);
    int rotk = 0;
    if (int e = rot_log4(rot_group, K, rotk)) return e;
    if (int e = require_device()) return e;
    hipStream_t st = (hipStream_t)stream;
    auto go = [&](auto dtc) {
        constexpr int DT = decltype(dtc)::value;
        if (y_dtype == PSQ_BF16) return launch_rotate<DT, PSQ_BF16>(x, M, K, ldx, rotk, y, ldy, st);
        if (y_dtype == PSQ_F16) return launch_rotate<DT, PSQ_F16>(x, M, K, ldx, rotk, y, ldy, st);
        return launch_rotate<DT, PSQ_F32>(x, M, K, ldx, rotk, y, ldy, st);
    };
    return x_dtype == PSQ_BF16 ? go(std::integral_constant<int, PSQ_BF16>{}) : go(std::integral_constant<int, PSQ_F16>{});
}

int quantize_rows(bool fp8, const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                  int rot_group, const float *static_scale, uint8_t *q, int64_t ldq, float *scale,
                  void *stream)
{
    if (M < 0 || K < 0) return set_error(PSQ_E_ARG, "negative size M=%lld K=%lld", (long long)M, (long long)K);
    if (M == 0) return PSQ_OK;
    if (!x || !q || !scale) return set_error(PSQ_E_ARG, "null pointer");
    if (x_dtype != PSQ_BF16 && x_dtype != PSQ_F16)
        return set_error(PSQ_E_ARG, "activations must be bf16 or f16 (dtype %d)", x_dtype);
    if (K == 0 || K % kElemsPerThread || K > kMaxK)
        return set_error(PSQ_E_SHAPE, "K=%lld must be a positive multiple of 16 and <= %d", (long long)K, kMaxK);
    if (ldx < K || ldq < K || ldx % 8 || ldq % 16)
        return set_error(PSQ_E_SHAPE, "strides ldx=%lld (mult. of 8) ldq=%lld (mult. of 16) must cover K=%lld",
                         (long long)ldx, (long long)ldq, (long long)K);
    if (((uintptr_t)x & 15) || ((uintptr_t)q & 15))
        return set_error(PSQ_E_SHAPE, "x and q must be 16-byte aligned");
    if (M > 0x7fffffffLL) return set_error(PSQ_E_SHAPE, "M=%lld too large", (long long)M);
    int rotk = 0;
    if (int e = rot_log4(rot_group, K, rotk)) return e;
    if (int e = require_device()) return e;
    hipStream_t st = (hipStream_t)stream;
    if (fp8)
        return x_dtype == PSQ_BF16 ? launch_quant<PSQ_BF16, true>(x, M, K, ldx, rotk, static_scale, q, ldq, scale, st)
                                   : launch_quant<PSQ_F16, true>(x, M, K, ldx, rotk, static_scale, q, ldq, scale, st);
    return x_dtype == PSQ_BF16 ? launch_quant<PSQ_BF16, false>(x, M, K, ldx, rotk, static_scale, q, ldq, scale, st)
                               : launch_quant<PSQ_F16, false>(x, M, K, ldx, rotk, static_scale, q, ldq, scale, st);
}

}  // namespace
}  // namespace psq

extern "C" {

int psq_quantize_rows_i8(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int rot_group,
                         const float *static_scale, int8_t *q, int64_t ldq, float *scale, void *stream)
{
    return psq::quantize_rows(false, x, x_dtype, M, K, ldx, rot_group, static_scale, (uint8_t *)q, ldq,
                              scale, stream);
}

int psq_quantize_rows_fp8(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int rot_group,
                          const float *static_scale, uint8_t *q, int64_t ldq, float *scale, void *stream)
{
    return psq::quantize_rows(true, x, x_dtype, M, K, ldx, rot_group, static_scale, q, ldq, scale, stream);
}

int psq_rotate_rows(const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int rot_group, void *y,
                    int y_dtype, int64_t ldy, void *stream)
{
    return psq::rotate_rows(x, x_dtype, M, K, ldx, rot_group, y, y_dtype, ldy, stream);
}

}  // extern "C"
