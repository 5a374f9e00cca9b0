// gemm_wonly.hip -- weight-only quantized GEMMs: uint4 asymmetric groups (W4A16) and int8 rows
// (W8A16), dequantized in registers and fed to the bf16 / f16 MFMA (v_mfma_f32_16x16x32_*).
//
// W4A16 reproduces the dequantize branch of QuantLinear.forward,
//   F.linear(rows, qt.dequantize().to(bf16), bias)   (powershard/quant_linear.py:219-220),
// without materializing the weight: w = round_bf16((float(q) - float(z)) * float(s)),
// y = round_out(acc + bias) with fp32 accumulation.
// W8A16: int8 values are exact in bf16, the per-row scale is applied in the epilogue,
// y = round_out(fmaf(acc, s[n], bias[n])) (Int8Linear storage, powershard/operations.py:96-132).
//
// Tiling: 128 x 128 output tile per workgroup of 4 waves (2 x 2, wave tile 64 x 64 = 4 x 4
// MFMA tiles), K in stages of 64 elements double-buffered in LDS: activations as 128-byte
// rows (XOR-swizzled 16-byte chunks), packed weights as padded rows (bank-conflict free
// 4/8-byte fragment reads), group scale and zero per weight row and stage.
#include "psq_common.hpp"

namespace psq {
namespace {

constexpr int BM = 128, BN = 128, BK = 64;     // BK in elements
constexpr int NTHREADS = 256;
constexpr int WAVE_M = 64, WAVE_N = 64;
constexpr int TM = WAVE_M / 16, TN = WAVE_N / 16;
constexpr int XROW = BK * 2;                   // bytes per activation row in LDS (128)
constexpr int X_STAGE = BM * XROW;             // 16 KB
constexpr int GROUP_M = 4;

enum { W_UINT4 = 0, W_INT8 = 1 };

template <int WK> struct WTraits;
template <> struct WTraits<W_UINT4> {
    static constexpr int ROW_BYTES = BK / 2;     // 32 bytes of packed nibbles per row per stage
    static constexpr int PITCH = 36;             // padded LDS pitch (9 words: conflict free)
};
template <> struct WTraits<W_INT8> {
    static constexpr int ROW_BYTES = BK;         // 64 bytes per row per stage
    static constexpr int PITCH = 72;             // padded LDS pitch (18 words)
};

struct WArgs {
    const uint8_t *wq;          // uint4 [N, K/2] or int8 [N, K]
    const uint16_t *scale16;    // uint4: fp16 [N, K/gs]
    const uint16_t *zero16;     // uint4: fp16 [N, K/gs]
    const float *scale32;       // int8: fp32 [N]
    int gs;                     // uint4 group size
    const void *bias;
    int bias_dtype;
    void *y;
    int y_dtype;
    int64_t ldy;
};

__device__ __forceinline__ int xswz(int row, int chunk) { return row * XROW + ((chunk ^ (row & 7)) << 4); }

template <int XDT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi)
{
    return pack_half2<XDT>(lo, hi);
}

template <int XDT, int WK>
__global__ void __launch_bounds__(NTHREADS, 2)
gemm_wonly_kernel(const uint16_t *__restrict__ X, int64_t ldx, int M, int N, int K, WArgs wa)
{
    using WT = WTraits<WK>;
    __shared__ __attribute__((aligned(16))) uint8_t sx[2][X_STAGE];
    __shared__ __attribute__((aligned(16))) uint8_t sw[2][BN * WT::PITCH];
    __shared__ float2 ssz[2][BN];     // uint4: (scale, zero) of the stage's group per row

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int pm, pn;
    tile_order(blockIdx.x, nbm, nbn, GROUP_M, pm, pn);
    const int m0 = pm * BM, n0 = pn * BN;

    // activations: 128 rows x 8 chunks = 1024 chunks, 4 per thread
    const int xchunk = tid & 7;
    const uint16_t *px[4];
    int xoff[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = (tid >> 3) + 32 * j;
        px[j] = X + (int64_t)min(m0 + r, M - 1) * ldx + xchunk * 8;
        xoff[j] = xswz(r, xchunk);
    }
    // weights: uint4 -> 128 rows x 2 chunks (1 per thread); int8 -> 128 rows x 4 chunks (2 per thread)
    constexpr int WCH = WT::ROW_BYTES / 16;            // 16-byte chunks per row per stage
    constexpr int WLOADS = BN * WCH / NTHREADS;
    const uint8_t *pw[WLOADS];
    int woff[WLOADS];
    const int64_t wrow_bytes = (WK == W_UINT4) ? (int64_t)K / 2 : (int64_t)K;
#pragma unroll
    for (int j = 0; j < WLOADS; j++) {
        const int id = tid + j * NTHREADS;
        const int r = id / WCH, c = id % WCH;
        pw[j] = wa.wq + (int64_t)min(n0 + r, N - 1) * wrow_bytes + c * 16;
        woff[j] = r * WT::PITCH + c * 16;
    }
    const int G = (WK == W_UINT4) ? K / wa.gs : 1;
    const int szrow = min(n0 + tid, N - 1);

    v4f acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    v4i rx[4], rw[WLOADS];
    float rs = 0.f, rz = 0.f;
    auto gload = [&](int kt) {
        const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
        for (int j = 0; j < 4; j++) rx[j] = *(const v4i *)(px[j] + k0);
#pragma unroll
        for (int j = 0; j < WLOADS; j++)
            rw[j] = *(const v4i *)(pw[j] + (WK == W_UINT4 ? k0 / 2 : k0));
        if constexpr (WK == W_UINT4) {
            if (tid < BN) {
                const int64_t gi = (int64_t)szrow * G + k0 / wa.gs;
                rs = f16_to_f32(wa.scale16[gi]);
                rz = f16_to_f32(wa.zero16[gi]);
            }
        }
    };
    auto sstore = [&](int st) {
#pragma unroll
        for (int j = 0; j < 4; j++) *(v4i *)(&sx[st][xoff[j]]) = rx[j];
#pragma unroll
        for (int j = 0; j < WLOADS; j++) {
            // padded pitch is not 16-byte aligned for every row: store as dwords
            uint32_t *d = (uint32_t *)(&sw[st][woff[j]]);
            d[0] = rw[j][0]; d[1] = rw[j][1]; d[2] = rw[j][2]; d[3] = rw[j][3];
        }
        if constexpr (WK == W_UINT4) {
            if (tid < BN) ssz[st][tid] = make_float2(rs, rz);
        }
    };

    const int nk = K / BK;
    gload(0);
    sstore(0);
    __syncthreads();

    const int frow = lane & 15, fk = lane >> 4;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 32; ks++) {
            v8bf fx[TM];
            v8bf fwv[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                v4i t = *(const v4i *)(&sx[cur][xswz(wm * WAVE_M + i * 16 + frow, ks * 4 + fk)]);
                fx[i] = __builtin_bit_cast(v8bf, t);
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int r = wn * WAVE_N + j * 16 + frow;   // weight row (output column)
                uint32_t h[4];
                if constexpr (WK == W_UINT4) {
                    // 8 nibbles of k = ks*32 + fk*8 + 0..7, low nibble first
                    const uint32_t p = *(const uint32_t *)(&sw[cur][r * WT::PITCH + ks * 16 + fk * 4]);
                    const float2 sz = ssz[cur][r];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float q0 = (float)((p >> (8 * e)) & 15u);
                        const float q1 = (float)((p >> (8 * e + 4)) & 15u);
                        h[e] = pack2<XDT>((q0 - sz.y) * sz.x, (q1 - sz.y) * sz.x);
                    }
                } else {
                    const uint32_t *src = (const uint32_t *)(&sw[cur][r * WT::PITCH + ks * 32 + fk * 8]);
                    const uint32_t p0 = src[0], p1 = src[1];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t p = e ? p1 : p0;
                        const float q0 = (float)(int8_t)(p & 0xffu);
                        const float q1 = (float)(int8_t)((p >> 8) & 0xffu);
                        const float q2 = (float)(int8_t)((p >> 16) & 0xffu);
                        const float q3 = (float)(int8_t)(p >> 24);
                        h[2 * e] = pack2<XDT>(q0, q1);
                        h[2 * e + 1] = pack2<XDT>(q2, q3);
                    }
                }
                v4i t = {(int)h[0], (int)h[1], (int)h[2], (int)h[3]};
                fwv[j] = __builtin_bit_cast(v8bf, t);
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    if constexpr (XDT == PSQ_BF16)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fx[i], fwv[j], acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, fx[i]),
                                                                           __builtin_bit_cast(v8h, fwv[j]),
                                                                           acc[i][j], 0, 0, 0);
                }
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    const int rbase = m0 + wm * WAVE_M + (lane >> 4) * 4;
    const int cbase = n0 + wn * WAVE_N + (lane & 15);
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int n = cbase + j * 16;
        const int nc = min(n, N - 1);
        const float cs = (WK == W_INT8) ? wa.scale32[nc] : 1.0f;
        const float b = wa.bias ? load_elem(wa.bias, nc, wa.bias_dtype) : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = rbase + i * 16 + v;
                if (m < M && n < N) store_elem(wa.y, (int64_t)m * wa.ldy + n, wa.y_dtype, __builtin_fmaf(acc[i][j][v], cs, b));
            }
    }
}

// Skinny weight-only GEMM (M <= 64, the decode / text-encoder shapes, bound by the weight stream):
// one workgroup per 16 weight rows (output columns) whose 4 waves split K by 128-element blocks
// round-robin.  Per block a lane streams the 32 consecutive k of one weight row that belong to its
// lane group (16 bytes of nibbles / 32 bytes of int8), dequantizes them in registers for four
// 16x16x32 MFMA k-steps, and reads the matching 16-byte activation fragments straight from memory
// (the activations are small and stay in L2).  The MFMA sums over a k set per lane group; both
// operands use the same assignment, so every dot product is complete.  The four waves' partial
// tiles are added through LDS in a fixed order, then the epilogue of the tiled kernel applies.
constexpr int SK_BLOCK = 128;                  // k per block: 4 lane groups x 32

template <int XDT, int WK, int MT>
__global__ void __launch_bounds__(NTHREADS)
gemm_wonly_skinny(const uint16_t *__restrict__ x, int64_t ldx, int M, int N, int K, WArgs wa)
{
    __shared__ float red[4][MT][16][17];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * 16;
    const int nr = lane & 15, h = lane >> 4;
    const int n = min(n0 + nr, N - 1);
    constexpr int WROW_DIV = WK == W_UINT4 ? 2 : 1;
    const uint8_t *wrow = wa.wq + (int64_t)n * (K / WROW_DIV);
    const uint16_t *xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) xrow[mt] = x + (int64_t)min(16 * mt + nr, M - 1) * ldx;
    const int G = WK == W_UINT4 ? K / wa.gs : 1;
    using XV = typename std::conditional<XDT == PSQ_BF16, v8bf, v8h>::type;

    v4f acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

    constexpr int NW = WK == W_UINT4 ? 4 : 8;       // weight words per lane per block
    const int nblk = K / SK_BLOCK;
    // The weight stream is software-pipelined one block deep (the next block's words and group
    // scale / zero load while this block computes); the activation fragments, L2 hits, load at the
    // top of each block.
    struct WBlock { uint32_t w[NW]; float s, z; };
    auto load_w = [&](int b, WBlock &r) {
        const int kb = b * SK_BLOCK + 32 * h;
        const v4i t0 = *(const v4i *)(wrow + kb / WROW_DIV);
#pragma unroll
        for (int c = 0; c < 4; c++) r.w[c] = (uint32_t)t0[c];
        if constexpr (WK == W_INT8) {
            const v4i t1 = *(const v4i *)(wrow + kb + 16);
#pragma unroll
            for (int c = 0; c < 4; c++) r.w[4 + c] = (uint32_t)t1[c];
            r.s = 1.0f;
            r.z = 0.0f;
        } else {
            const int64_t gi = (int64_t)n * G + kb / wa.gs;
            r.s = f16_to_f32(wa.scale16[gi]);
            r.z = f16_to_f32(wa.zero16[gi]);
        }
    };
    auto compute = [&](int b, const WBlock &r) {
        const int kb = b * SK_BLOCK + 32 * h;        // the lane group's first k
        v4i xv[4][MT];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) xv[t][mt] = *(const v4i *)(xrow[mt] + kb + 8 * t);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // weights of k = kb + 8t .. kb + 8t + 7
            uint32_t hw[4];
            if constexpr (WK == W_UINT4) {
                const uint32_t p = r.w[t];
                const uint32_t lo = p & 0x0f0f0f0fu, hi = (p >> 4) & 0x0f0f0f0fu;   // even / odd k
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float q0 = (float)((lo >> (8 * e)) & 0xffu);
                    const float q1 = (float)((hi >> (8 * e)) & 0xffu);
                    hw[e] = pack2<XDT>((q0 - r.z) * r.s, (q1 - r.z) * r.s);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t p = r.w[2 * t + e];
                    hw[2 * e] = pack2<XDT>((float)(int8_t)(p & 0xffu), (float)(int8_t)((p >> 8) & 0xffu));
                    hw[2 * e + 1] = pack2<XDT>((float)(int8_t)((p >> 16) & 0xffu), (float)(int8_t)(p >> 24));
                }
            }
            const XV wf = __builtin_bit_cast(XV, v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]});
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const XV xf = __builtin_bit_cast(XV, xv[t][mt]);
                if constexpr (XDT == PSQ_BF16)
                    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xf, acc[mt], 0, 0, 0);
                else
                    acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf, xf, acc[mt], 0, 0, 0);
            }
        }
    };
    WBlock cur, nxt;
    if (wave < nblk) load_w(wave, cur);
    for (int b = wave; b < nblk; b += 4) {
        if (b + 4 < nblk) load_w(b + 4, nxt);
        compute(b, cur);
        cur = nxt;
    }
    // acc[mt] is the 16 x 16 tile C[n][m]: lane holds m = 16 mt + (lane & 15), n = 4 (lane >> 4) + v
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int v = 0; v < 4; v++) red[wave][mt][4 * h + v][nr] = acc[mt][v];
    __syncthreads();
#pragma unroll
    for (int o = tid; o < MT * 256; o += NTHREADS) {
        const int mt = o >> 8, ml = (o >> 4) & 15, nl = o & 15;
        const int m = 16 * mt + ml, nn = n0 + nl;
        if (m >= M || nn >= N) continue;
        const float sum = ((red[0][mt][nl][ml] + red[1][mt][nl][ml]) + red[2][mt][nl][ml]) + red[3][mt][nl][ml];
        const float cs = (WK == W_INT8) ? wa.scale32[nn] : 1.0f;
        const float bb = wa.bias ? load_elem(wa.bias, nn, wa.bias_dtype) : 0.0f;
        store_elem(wa.y, (int64_t)m * wa.ldy + nn, wa.y_dtype, __builtin_fmaf(sum, cs, bb));
    }
}

template <int XDT, int WK>
void launch_skinny(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa, hipStream_t st)
{
    const dim3 grid((unsigned)((N + 15) / 16)), block(NTHREADS);
    const int mt = (int)((M + 15) / 16);
    if (mt == 1) gemm_wonly_skinny<XDT, WK, 1><<<grid, block, 0, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
    else if (mt == 2) gemm_wonly_skinny<XDT, WK, 2><<<grid, block, 0, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
    else if (mt == 3) gemm_wonly_skinny<XDT, WK, 3><<<grid, block, 0, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
    else gemm_wonly_skinny<XDT, WK, 4><<<grid, block, 0, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
}

// The skinny kernel takes M <= SKINNY_MAX_M when K is a whole number of 128-element blocks (and,
// for uint4, the groups hold whole 32-element lane runs); the tiled kernel takes the rest.
constexpr int64_t SKINNY_MAX_M = 64;

template <int WK>
int launch(const void *x, int x_dtype, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa,
           hipStream_t st, const char *name)
{
    if (M <= SKINNY_MAX_M && K % SK_BLOCK == 0 && (WK != W_UINT4 || wa.gs % 32 == 0)) {
        if (x_dtype == PSQ_BF16) launch_skinny<PSQ_BF16, WK>((const uint16_t *)x, ldx, M, N, K, wa, st);
        else launch_skinny<PSQ_F16, WK>((const uint16_t *)x, ldx, M, N, K, wa, st);
        return check_launch(name);
    }
    const int64_t nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const dim3 grid((unsigned)nblk), block(NTHREADS);
    if (x_dtype == PSQ_BF16)
        gemm_wonly_kernel<PSQ_BF16, WK><<<grid, block, 0, st>>>((const uint16_t *)x, ldx, (int)M, (int)N, (int)K, wa);
    else
        gemm_wonly_kernel<PSQ_F16, WK><<<grid, block, 0, st>>>((const uint16_t *)x, ldx, (int)M, (int)N, (int)K, wa);
    return check_launch(name);
}

int check_common(const char *name, const void *x, int x_dtype, int64_t ldx, const void *wq, const void *y, int y_dtype,
                 int64_t ldy, const void *bias, int bias_dtype, int64_t M, int64_t N, int64_t K)
{
    if (M < 0 || N < 0 || K < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    if (!x || !wq || !y) return set_error(PSQ_E_ARG, "%s: null pointer", name);
    if (x_dtype != PSQ_BF16 && x_dtype != PSQ_F16) return set_error(PSQ_E_ARG, "%s: activations must be bf16/f16", name);
    if (!valid_dtype(y_dtype) || (bias && !valid_dtype(bias_dtype))) return set_error(PSQ_E_ARG, "%s: bad dtype", name);
    if (K == 0 || K % BK) return set_error(PSQ_E_SHAPE, "%s: K=%lld must be a positive multiple of %d", name, (long long)K, BK);
    if (ldx < K || ldx % 8 || ((uintptr_t)x & 15)) return set_error(PSQ_E_SHAPE, "%s: x rows must be 16-byte aligned", name);
    if (((uintptr_t)wq & 15)) return set_error(PSQ_E_SHAPE, "%s: weights must be 16-byte aligned", name);
    if (ldy < N) return set_error(PSQ_E_SHAPE, "%s: ldy < N", name);
    if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30)) return set_error(PSQ_E_SHAPE, "%s: size too large", name);
    return PSQ_OK;
}

}  // namespace
}  // namespace psq

extern "C" {

int psq_gemm_w4a16(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq, const uint16_t *w_scale,
                   const uint16_t *w_zero, int group_size, const void *bias, int bias_dtype, void *y, int y_dtype,
                   int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_common("gemm_w4a16", x, x_dtype, ldx, wq, y, y_dtype, ldy, bias, bias_dtype, M, N, K)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!w_scale || !w_zero) return set_error(PSQ_E_ARG, "gemm_w4a16: null scale/zero");
    if (group_size <= 0 || group_size % BK || K % group_size)
        return set_error(PSQ_E_SHAPE, "gemm_w4a16: group size %d must be a multiple of %d dividing K", group_size, BK);
    if (int e = require_device()) return e;
    WArgs wa{wq, w_scale, w_zero, nullptr, group_size, bias, bias_dtype, y, y_dtype, ldy};
    return launch<W_UINT4>(x, x_dtype, ldx, M, N, K, wa, (hipStream_t)stream, "gemm_w4a16");
}

int psq_gemm_w8a16(const void *x, int x_dtype, int64_t ldx, const int8_t *wq, const float *w_scale, const void *bias,
                   int bias_dtype, void *y, int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_common("gemm_w8a16", x, x_dtype, ldx, wq, y, y_dtype, ldy, bias, bias_dtype, M, N, K)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!w_scale) return set_error(PSQ_E_ARG, "gemm_w8a16: null scale");
    if (int e = require_device()) return e;
    WArgs wa{(const uint8_t *)wq, nullptr, nullptr, w_scale, 0, bias, bias_dtype, y, y_dtype, ldy};
    return launch<W_INT8>(x, x_dtype, ldx, M, N, K, wa, (hipStream_t)stream, "gemm_w8a16");
}

}  // extern "C"
