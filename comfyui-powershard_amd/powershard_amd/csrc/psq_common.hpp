// psq_common.hpp -- shared device helpers of libpsquant (gfx950 only).
//
// Scalar formats follow the conventions of the library's C ABI (include/psquant.h):
// bf16 / fp16 round-to-nearest-even, OCP fp8 e4m3fn with saturation to +-448.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdarg.h>
#include <utility>
#include <type_traits>

#include "../../../include/psquant.h"

namespace psq {

// ------------------------------------------------------------------ host-side errors
// Records the message of the last failure on this thread and returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Checks the launch of the kernel just issued.
int check_launch(const char *what);

// Validates the current device (gfx950) once per device; 0 or PSQ_E_DEVICE.
int require_device();

// Compute units of device `dev` (256 if it cannot be queried), cached.
int cu_count(int dev);

inline bool valid_dtype(int dt) { return dt == PSQ_BF16 || dt == PSQ_F16 || dt == PSQ_F32; }

// ------------------------------------------------------------------ vector types
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------ scalar formats
__device__ __forceinline__ float bf16_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x0040u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t h16)
{
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)h16);
    return (float)h;
}

// Forces `x` to be materialized as an fp32 value: the backend otherwise folds an fma or mul
// feeding an f16 conversion into v_fma_mix / v_mad_mix, rounding once instead of twice.
__device__ __forceinline__ float opaque(float x)
{
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ uint32_t f32_to_f16(float f)
{
    _Float16 h = (_Float16)opaque(f);  // v_cvt_f16_f32, round to nearest even
    return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Convert one 16-bit element of dtype DT (bf16 or f16) held in the low half of `h`.
template <int DT>
__device__ __forceinline__ float half_to_f32(uint32_t h)
{
    if constexpr (DT == PSQ_BF16) return bf16_to_f32(h & 0xffffu);
    else return f16_to_f32(h & 0xffffu);
}

template <int DT>
__device__ __forceinline__ uint32_t f32_to_half(float f)
{
    if constexpr (DT == PSQ_BF16) return f32_to_bf16(f);
    else return f32_to_f16(f);
}

// Two fp32 values rounded (nearest even) to a packed pair of DT (bf16 or f16), low half first:
// one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32.  Finite results equal f32_to_half's, subnormals
// included; a NaN input gives a quiet NaN.  opaque() keeps the backend from folding a producing
// fma / mul into a mixed-precision instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ uint32_t pack_half2(float lo, float hi)
{
    const f32x2_t v{opaque(lo), opaque(hi)};
    if constexpr (DT == PSQ_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}

// OCP e4m3fn decode.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c)
{
    uint32_t e = (c >> 3) & 0xfu, m = c & 7u;
    float v;
    if (e == 0) v = (float)m * 0x1p-9f;
    else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
    if (e == 0xf && m == 7) v = __builtin_nanf("");
    return (c & 0x80u) ? -v : v;
}

// OCP e5m2 (bf8) code to fp32: the code is the high byte of the fp16 with the same value (1 sign,
// 5 exponent bits of bias 15, 2 mantissa bits; subnormals, infinities and NaNs included), so the
// decode is exact.
__device__ __forceinline__ float e5m2_to_f32(uint32_t c)
{
    return f16_to_f32((c & 0xffu) << 8);
}

// ------------------------------------------------------------------ activations
// GELU, tanh approximation: gelu(x) = x (1 + tanh z) / 2 with z = sqrt(2/pi) (x + 0.044715 x^3).
// (1 + tanh z) / 2 is the logistic function of 2 z, so gelu(x) = x / (1 + 2^(x (k0 + k1 x^2)))
// with k0 = -2 sqrt(2/pi) log2(e), k1 = 0.044715 k0: the same function without the cancellation
// of 1 + tanh z for negative x.  v_exp_f32 and v_rcp_f32 (about 1 ulp each).  Saturates to x for
// large x and to -0 for large negative x; +-inf and NaN give what the tanh form gives.
__device__ __forceinline__ float gelu_tanh(float x)
{
    constexpr float k0 = (float)(-2.0 * 0.79788456080286535588 * 1.44269504088896340736);
    constexpr float k1 = (float)(-2.0 * 0.79788456080286535588 * 1.44269504088896340736 * 0.044715);
    const float w = x * __builtin_fmaf(x * x, k1, k0);
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(w));
}

// silu(x) = x / (1 + e^-x) = x / (1 + 2^(-x log2 e)); exp2 overflows to +inf for x < -88.7 and the
// result is then -0 (|silu| < 1e-36 there).
__device__ __forceinline__ float silu(float x)
{
    constexpr float k = (float)(-1.44269504088896340736);
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * k));
}

enum { ACT_NONE = PSQ_ACT_NONE, ACT_GELU_TANH = PSQ_ACT_GELU_TANH, ACT_SILU_GATE = PSQ_ACT_SILU_GATE };

// ------------------------------------------------------------------ stores
// Store one fp32 value as element i of an output of dtype dt.
__device__ __forceinline__ void store_elem(void *p, int64_t i, int dt, float v)
{
    if (dt == PSQ_BF16) ((uint16_t *)p)[i] = (uint16_t)f32_to_bf16(v);
    else if (dt == PSQ_F16) ((uint16_t *)p)[i] = (uint16_t)f32_to_f16(v);
    else ((float *)p)[i] = v;
}

__device__ __forceinline__ float load_elem(const void *p, int64_t i, int dt)
{
    if (dt == PSQ_BF16) return bf16_to_f32(((const uint16_t *)p)[i]);
    if (dt == PSQ_F16) return f16_to_f32(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

// ------------------------------------------------------------------ cross-lane moves
// DPP permutations inside a row of 16 lanes (no LDS traffic).
enum : int {
    DPP_QUAD_XOR1 = 0xB1,        // quad_perm [1,0,3,2]
    DPP_QUAD_XOR2 = 0x4E,        // quad_perm [2,3,0,1]
    DPP_QUAD_XOR3 = 0x1B,        // quad_perm [3,2,1,0]
    DPP_ROW_MIRROR = 0x140,      // lane ^ 15 within a row of 16
    DPP_ROW_HALF_MIRROR = 0x141, // lane ^ 7 within a half row of 8
    DPP_ROW_ROR4 = 0x124,        // lane (l + 4) mod 16 within a row of 16
    DPP_ROW_ROR8 = 0x128         // lane ^ 8 within a row of 16
};

template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

// value of lane ^ (m * L) for the three radix-4 partners at lane stride L in {1, 4}
template <int L, int M_>
__device__ __forceinline__ float lane_xor(float v)
{
    if constexpr (L == 1) {
        if constexpr (M_ == 1) return dpp<DPP_QUAD_XOR1>(v);
        else if constexpr (M_ == 2) return dpp<DPP_QUAD_XOR2>(v);
        else return dpp<DPP_QUAD_XOR3>(v);
    } else if constexpr (L == 4) {
        if constexpr (M_ == 1) return dpp<DPP_QUAD_XOR3>(dpp<DPP_ROW_HALF_MIRROR>(v));  // ^7 ^3 = ^4
        else if constexpr (M_ == 2) return dpp<DPP_ROW_ROR8>(v);                          // ^8
        else return dpp<DPP_QUAD_XOR3>(dpp<DPP_ROW_MIRROR>(v));                           // ^15 ^3 = ^12
    } else {
        return __shfl_xor(v, L * M_, 64);
    }
}

// ------------------------------------------------------------------ radix-4 ConvRot stage
// y_j = S - 2 x_{3-j} with S = (x0 + x1) + (x2 + x3): one stage of the unnormalized regular
// Hadamard transform (H4[a][b] = -1 iff a + b == 3).  S - 2 x is one fma (2 x is exact, so it is
// the once-rounded difference), one VALU op per output.
__device__ __forceinline__ void radix4(float &x0, float &x1, float &x2, float &x3)
{
    float s01 = x0 + x1;
    float s23 = x2 + x3;
    float s = s01 + s23;
    float y0 = __builtin_fmaf(-2.0f, x3, s);
    float y1 = __builtin_fmaf(-2.0f, x2, s);
    float y2 = __builtin_fmaf(-2.0f, x1, s);
    float y3 = __builtin_fmaf(-2.0f, x0, s);
    x0 = y0; x1 = y1; x2 = y2; x3 = y3;
}

// Same stage across the four lanes whose lane index differs in the base-4 digit of weight L.
template <int L>
__device__ __forceinline__ float radix4_lanes(float x)
{
    float t = x + lane_xor<L, 1>(x);   // x_{d} + x_{d^1}: (x0+x1) or (x2+x3), commutative
    float s = t + lane_xor<L, 2>(t);   // (x0+x1) + (x2+x3)
    float r = lane_xor<L, 3>(x);       // x_{3-d}
    return __builtin_fmaf(-2.0f, r, s);
}

// The same stage with the outputs of the digit reversed: lane d keeps y_{3-d} = S - 2 x_d, its
// own value, so no third exchange.  The caller stores the lane's elements at digit 3 - d (lane
// index bits of weight L complemented).
template <int L>
__device__ __forceinline__ float radix4_lanes_rev(float x)
{
    float t = x + lane_xor<L, 1>(x);
    float s = t + lane_xor<L, 2>(t);
    return __builtin_fmaf(-2.0f, x, s);
}

// The reversed stage over lane bits 2-3 for a digit stored with its bits swapped (digit bit 0 on lane
// bit 3, digit bit 1 on lane bit 2).  The pair partner (digit ^ 1) is then lane ^ 8, and the other
// pair's sum, the same value on both of its lanes, sits at lane + 4 mod 16: two DPP adds (row_ror:8,
// row_ror:4) and the fma, where the unswapped digit needs a DPP move for lane ^ 4 as well.  Same
// operations in the same order as radix4_lanes_rev<4>, so the same bits.
__device__ __forceinline__ float radix4_lanes_rev_sw4(float x)
{
    float t = x + dpp<DPP_ROW_ROR8>(x);
    float s = t + dpp<DPP_ROW_ROR4>(t);
    return __builtin_fmaf(-2.0f, x, s);
}

// ------------------------------------------------------------------ XCD-aware tile order
// Rank of workgroup pid among n when the ranks of each XCD (pid % 8) are consecutive: a bijection
// of [0, n) for any n.
__device__ __forceinline__ int xcd_rank(int pid, int n)
{
    const int xcd = pid & 7, per = n >> 3, rem = n & 7;
    return xcd * per + (xcd < rem ? xcd : rem) + (pid >> 3);
}

// gfx950 dispatches workgroup i to XCD (i % 8).  Re-number so that each XCD receives a
// contiguous range of logical tiles, then walk tiles in groups of `group_m` tile rows so
// that concurrently resident tiles of one XCD share A rows and W rows in its L2.
__device__ __forceinline__ void tile_order(int pid, int nbm, int nbn, int group_m, int &pm, int &pn)
{
    const int nblk = nbm * nbn;
    const int xcd = pid & 7, per = nblk >> 3, rem = nblk & 7;
    int lid = xcd * per + (xcd < rem ? xcd : rem) + (pid >> 3);
    const int in_group = group_m * nbn;
    const int gid = lid / in_group;
    const int first_m = gid * group_m;
    const int gsz = (nbm - first_m) < group_m ? (nbm - first_m) : group_m;
    const int r = lid - gid * in_group;
    pm = first_m + r % gsz;
    pn = r / gsz;
}

// ------------------------------------------------------------------ buffer descriptors
// Raw buffer descriptor over `base` (no stride, no range limit, 32-bit data format): a buffer load
// reads base + vector offset + scalar offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void *base)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, -1, 0x00020000);
}

// ------------------------------------------------------------------ GEMM pipelines
typedef __attribute__((address_space(3))) uint8_t *lds_ptr;
typedef const __attribute__((address_space(1))) void *glb_ptr;

// Global -> LDS load through a buffer descriptor: 16 bytes per lane from descriptor base + voff +
// soff into dst + 16 * lane (dst wave-uniform; it goes to M0).
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rs, lds_ptr dst, uint32_t voff, int soff)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, dst, 16, voff, soff, 0, 0);
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4]<<14)
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for the K loop.  __syncthreads() carries a workgroup fence, which makes the
// compiler drain every outstanding global->LDS load (vmcnt(0)) -- including the stages just put
// in flight.  The loop instead waits explicitly for the stage it needs (wait_vmcnt) and for its
// own LDS reads (lgkmcnt(0)), then meets the other waves; the asm memory clobber keeps the
// compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void stage_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Reads an accumulator element through an AGPR operand.  The epilogue's arithmetic cannot take
// AGPRs, and left to itself the register allocator then keeps the whole accumulator array in
// VGPRs (and spills everything else); reading each element with an explicit AGPR-to-VGPR move
// keeps the accumulators in the AGPR file for the MFMAs.
__device__ __forceinline__ int agpr_read(int a)
{
    int v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
    return v;
}
__device__ __forceinline__ int agpr_read(float a)
{
    int v;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
    return v;
}
// agpr_read for a value that goes straight into a store.  A VMEM store of more than 8 bytes reads
// its data registers after issue, and a VALU write of those registers must wait first: two wait
// states on the gfx940 family, gfx950 included (one on earlier gfx9).  The compiler does not
// reliably count an inline-asm move as such a write, and re-used one store's data registers for
// the next store's moves at once (the store then wrote the next value for the lanes it had not
// read yet).  The leading `s_nop 1` (two wait states) is that wait, whatever the schedule.
__device__ __forceinline__ int agpr_read_for_store(float a)
{
    int v;
    asm volatile("s_nop 1\n\tv_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
    return v;
}

// Calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1, expanded at compile time (an unroll
// the optimizer cannot decline: register arrays indexed by I stay in registers).
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f)
{
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (f(std::integral_constant<int, I>{}), ...);
    }(std::make_integer_sequence<int, N>{});
}

}  // namespace psq
