// gemm_q8.hip -- W8A8 int8 and fp8-e4m3 GEMMs on gfx950 MFMA with a fused dequant epilogue.
//
// Replaces comfy-kitchen int8_linear and torch._scaled_mm behind
// F.linear(QuantizedTensor, QuantizedTensor, bias) (powershard/quant_linear.py:230-242).
//   y[m][n] = round_out(fmaf((float)acc[m][n], a_scale[m] * w_scale[n], bias[n]))
//   int8: acc = sum_k a[m][k] w[n][k] in int32 (v_mfma_i32_32x32x32_i8, exact)
//   fp8 : acc = the same in fp32 (v_mfma_f32_32x32x64_f8f6f4, e4m3 x e4m3)
//
// Tiling (MI355X-first): a 256 x 256 output tile per workgroup of 8 waves (2 along M x 4
// along N, each wave 128 x 64 = 4 x 2 MFMA tiles of 32 x 32), K in stages of 128 bytes
// double-buffered in LDS (2 x 64 KB) and filled by direct global->LDS loads
// (global_load_lds_dwordx4: no staging registers, no LDS write instructions).  A stage row of
// 128 bytes is eight 16-byte chunks stored XOR-swizzled (chunk ^ (row & 7)) so that the
// 16-byte fragment reads of a wave hit distinct banks.  Workgroups are renumbered so each XCD owns a contiguous, L2-friendly
// group of tiles.  MFMA-bound: 2 M N K ops per launch.
#include "psq_common.hpp"

namespace psq {
namespace {

constexpr int BM = 256, BN = 256, BK = 128;   // BK in bytes (= elements for int8/fp8)
constexpr int NTHREADS = 512;
constexpr int WAVE_M = 128, WAVE_N = 64;
constexpr int TM = WAVE_M / 32, TN = WAVE_N / 32;   // 4 x 2 MFMA tiles per wave
constexpr int STAGE_BYTES = BM * BK;                 // one operand, one stage (32 KB)
constexpr int LOADS = (BM * BK / 1024) / (NTHREADS / 64);   // 1 KB wave loads per operand per wave (4)
constexpr int GROUP_M = 8;

enum { OUT_EPILOGUE = 0, OUT_I32 = 1 };

struct Epi {
    const float *a_scale;
    const float *w_scale;
    int w_per_row;
    const void *bias;
    int bias_dtype;
    void *y;
    int y_dtype;
    int64_t ldy;
};

typedef __attribute__((address_space(3))) uint8_t *lds_ptr;
typedef const __attribute__((address_space(1))) void *glb_ptr;

__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ (row & 7)) << 4); }

template <bool FP8, int OUT>
__global__ void __launch_bounds__(NTHREADS, 1)
gemm_q8_kernel(const uint8_t *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W, int64_t ldw,
               int M, int N, int K, Epi ep)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];   // [2 stages][A | W]
    using Acc = typename std::conditional<FP8, v16f, v16i>::type;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int pm, pn;
    tile_order(blockIdx.x, nbm, nbn, GROUP_M, pm, pn);
    const int m0 = pm * BM, n0 = pn * BN;

    // global -> LDS: a wave load moves 1 KB = 8 rows x 8 chunks; lane L fills physical slot
    // L of the block (row 8 b + L / 8, physical chunk L % 8) and therefore reads logical
    // chunk (L % 8) ^ (row & 7) of that row.
    const uint8_t *pa[LOADS];
    const uint8_t *pw[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; j++) {
        const int b = j * (NTHREADS / 64) + wave;
        const int r = 8 * b + (lane >> 3);
        const int c = (lane & 7) ^ (r & 7);
        const int ga = min(m0 + r, M - 1), gw = min(n0 + r, N - 1);
        pa[j] = A + (int64_t)ga * lda + c * 16;
        pw[j] = W + (int64_t)gw * ldw + c * 16;
    }
    auto issue_stage = [&](int kt, int buf) {
        const int64_t koff = (int64_t)kt * BK;
        lds_ptr dA = (lds_ptr)(smem + buf * 2 * STAGE_BYTES);
#pragma unroll
        for (int j = 0; j < LOADS; j++) {
            const int b = j * (NTHREADS / 64) + wave;
            __builtin_amdgcn_global_load_lds((glb_ptr)(pa[j] + koff), dA + 1024 * b, 16, 0, 0);
            __builtin_amdgcn_global_load_lds((glb_ptr)(pw[j] + koff), dA + STAGE_BYTES + 1024 * b, 16, 0, 0);
        }
    };

    Acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0;

    const int nk = K / BK;
    issue_stage(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // MFMA operand layout (32 x 32 tiles): lane holds row (lane & 31) of A / of W and the
    // k-slice (lane >> 5) of the instruction's K; A and W use the same slice, so the dot
    // products are complete whatever order the hardware sums the slice in.
    const int frow = lane & 31, fk = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const uint8_t *sA = smem + cur * 2 * STAGE_BYTES;
        const uint8_t *sW = sA + STAGE_BYTES;
        // the other buffer was last read before the barrier that ended the previous step
        if (kt + 1 < nk) issue_stage(kt + 1, cur ^ 1);
        if constexpr (FP8) {
            // two K=64 steps per stage: lane holds 32 bytes = chunks 4 ks + 2 fk, + 1
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                v8i fa[TM], fw[TN];
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const int r = wm * WAVE_M + i * 32 + frow;
                    v4i lo = *(const v4i *)(sA + swz(r, 4 * ks + 2 * fk));
                    v4i hi = *(const v4i *)(sA + swz(r, 4 * ks + 2 * fk + 1));
                    fa[i] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int r = wn * WAVE_N + j * 32 + frow;
                    v4i lo = *(const v4i *)(sW + swz(r, 4 * ks + 2 * fk));
                    v4i hi = *(const v4i *)(sW + swz(r, 4 * ks + 2 * fk + 1));
                    fw[j] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                            fa[i], fw[j], acc[i][j], 0, 0, 0, 127, 0, 127);
            }
        } else {
            // four K=32 steps per stage: lane holds 16 bytes = chunk 2 ks + fk
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                v4i fa[TM], fw[TN];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    fa[i] = *(const v4i *)(sA + swz(wm * WAVE_M + i * 32 + frow, 2 * ks + fk));
#pragma unroll
                for (int j = 0; j < TN; j++)
                    fw[j] = *(const v4i *)(sW + swz(wn * WAVE_N + j * 32 + frow, 2 * ks + fk));
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fw[j], acc[i][j], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);   // this wave's loads of the next stage have landed
        __syncthreads();
    }

    // epilogue: in each 32 x 32 tile, lane holds column (lane & 31) and, for register r,
    // row 8 (r / 4) + 4 (lane / 32) + (r % 4)
    const int rbase = m0 + wm * WAVE_M + 4 * (lane >> 5);
    const int cbase = n0 + wn * WAVE_N + (lane & 31);
    if constexpr (OUT == OUT_I32) {
        int32_t *C = (int32_t *)ep.y;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = cbase + j * 32;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = rbase + i * 32 + 8 * (r >> 2) + (r & 3);
                    if (m < M && n < N) C[(int64_t)m * ep.ldy + n] = (int32_t)acc[i][j][r];
                }
            }
    } else {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int n = cbase + j * 32;
            const int nc = min(n, N - 1);
            const float ws = ep.w_scale[ep.w_per_row ? nc : 0];
            const float b = ep.bias ? load_elem(ep.bias, nc, ep.bias_dtype) : 0.0f;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = rbase + i * 32 + 8 * (r >> 2) + (r & 3);
                    if (m < M && n < N) {
                        const float as = ep.a_scale[m];
                        float y = __builtin_fmaf((float)acc[i][j][r], as * ws, b);
                        store_elem(ep.y, (int64_t)m * ep.ldy + n, ep.y_dtype, y);
                    }
                }
        }
    }
}

constexpr size_t kSmemBytes = 2 * 2 * STAGE_BYTES;   // 128 KB

template <bool FP8, int OUT>
int launch(const uint8_t *a, int64_t lda, const uint8_t *w, int64_t ldw, int64_t M, int64_t N, int64_t K,
           const Epi &ep, hipStream_t st, const char *name)
{
    auto kern = gemm_q8_kernel<FP8, OUT>;
    static bool attr_set = false;   // attribute is per function, idempotent
    if (!attr_set) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSmemBytes) !=
            hipSuccess)
            return set_error(PSQ_E_DEVICE, "%s: cannot reserve %zu bytes of LDS", name, kSmemBytes);
        attr_set = true;
    }
    const int64_t nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    kern<<<dim3((unsigned)nblk), dim3(NTHREADS), kSmemBytes, st>>>(a, lda, w, ldw, (int)M, (int)N, (int)K, ep);
    return check_launch(name);
}

int check_shapes(const char *name, const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M, int64_t N,
                 int64_t K)
{
    if (M < 0 || N < 0 || K < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    if (!a || !w) return set_error(PSQ_E_ARG, "%s: null operand", name);
    if (K == 0 || K % BK)
        return set_error(PSQ_E_SHAPE, "%s: K=%lld must be a positive multiple of %d", name, (long long)K, BK);
    if (lda < K || ldw < K || lda % 16 || ldw % 16)
        return set_error(PSQ_E_SHAPE, "%s: lda=%lld ldw=%lld must be multiples of 16 covering K", name,
                         (long long)lda, (long long)ldw);
    if (((uintptr_t)a & 15) || ((uintptr_t)w & 15)) return set_error(PSQ_E_SHAPE, "%s: operands must be 16-byte aligned", name);
    if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30))
        return set_error(PSQ_E_SHAPE, "%s: size too large", name);
    return PSQ_OK;
}

}  // namespace
}  // namespace psq

extern "C" {

int psq_gemm_i8(const int8_t *a, int64_t lda, const float *a_scale, const int8_t *w, int64_t ldw,
                const float *w_scale, const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy,
                int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_shapes("gemm_i8", a, lda, w, ldw, M, N, K)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!a_scale || !w_scale || !y) return set_error(PSQ_E_ARG, "gemm_i8: null scale or output");
    if (!valid_dtype(y_dtype) || (bias && !valid_dtype(bias_dtype))) return set_error(PSQ_E_ARG, "gemm_i8: bad dtype");
    if (ldy < N) return set_error(PSQ_E_SHAPE, "gemm_i8: ldy < N");
    if (int e = require_device()) return e;
    Epi ep{a_scale, w_scale, 1, bias, bias_dtype, y, y_dtype, ldy};
    return launch<false, OUT_EPILOGUE>((const uint8_t *)a, lda, (const uint8_t *)w, ldw, M, N, K, ep,
                                       (hipStream_t)stream, "gemm_i8");
}

int psq_gemm_i8_i32(const int8_t *a, int64_t lda, const int8_t *w, int64_t ldw, int32_t *c, int64_t ldc,
                    int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_shapes("gemm_i8_i32", a, lda, w, ldw, M, N, K)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!c) return set_error(PSQ_E_ARG, "gemm_i8_i32: null output");
    if (ldc < N) return set_error(PSQ_E_SHAPE, "gemm_i8_i32: ldc < N");
    if (int e = require_device()) return e;
    Epi ep{nullptr, nullptr, 0, nullptr, 0, c, PSQ_F32, ldc};
    return launch<false, OUT_I32>((const uint8_t *)a, lda, (const uint8_t *)w, ldw, M, N, K, ep,
                                  (hipStream_t)stream, "gemm_i8_i32");
}

int psq_gemm_fp8(const uint8_t *a, int64_t lda, const float *a_scale, const uint8_t *w, int64_t ldw,
                 const float *w_scale, int w_scale_per_row, const void *bias, int bias_dtype, void *y, int y_dtype,
                 int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_shapes("gemm_fp8", a, lda, w, ldw, M, N, K)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!a_scale || !w_scale || !y) return set_error(PSQ_E_ARG, "gemm_fp8: null scale or output");
    if (!valid_dtype(y_dtype) || (bias && !valid_dtype(bias_dtype))) return set_error(PSQ_E_ARG, "gemm_fp8: bad dtype");
    if (ldy < N) return set_error(PSQ_E_SHAPE, "gemm_fp8: ldy < N");
    if (int e = require_device()) return e;
    Epi ep{a_scale, w_scale, w_scale_per_row ? 1 : 0, bias, bias_dtype, y, y_dtype, ldy};
    return launch<true, OUT_EPILOGUE>(a, lda, w, ldw, M, N, K, ep, (hipStream_t)stream, "gemm_fp8");
}

}  // extern "C"
