// gemm_q8_8wave.hip -- the W8A8 int8 GEMM (bf16 output, no activation) with two waves per SIMD:
// a comparison schedule for gemm_q8.hip, not on the module path.
//
// Same tile, ring and arithmetic as gemm_q8_kernel: a persistent workgroup per CU walks 256 x 256
// output tiles, K in 128-byte stages through the same 2-slot LDS ring (direct global->LDS loads),
// y = round_bf16(fmaf((float)acc, a_scale[m] * w_scale[n], bias[n])) -- the outputs are
// bit-identical.  The workgroup is 8 waves instead of 4: two per SIMD, each a 128 x 64 wave tile
// (2 x 4 waves, 4 x 2 MFMA tiles of 32 x 32, 128 accumulator registers), so a SIMD holds a second
// wave to issue while the first waits on LDS, a barrier or its stores.  The price is 1.5x the
// fragment reads per MFMA (6 per 8 MFMAs against 8 per 16) and, with the ring shared, both waves
// of a SIMD reach their epilogue together: a wave's epilogue cannot run beside the other wave's
// MFMAs.  Measured against gemm_q8_kernel on the same host, alternating launches, it is slower on
// every shape tried; the entry point stays so that the comparison can be re-run.
#include "psq_common.hpp"

namespace psq {
namespace w8 {

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int NSTAGE = 2;
constexpr int NW = 8, NTHREADS = 64 * NW;
constexpr int WAVE_M = 128, WAVE_N = 64;
constexpr int TM = WAVE_M / 32, TN = WAVE_N / 32;    // 4 x 2
constexpr int STAGE_BYTES = BM * BK;
constexpr int LOADS = (BM * BK / 1024) / NW;         // 4
constexpr int LPS = 2 * LOADS;                        // 8
constexpr int GROUP_M = 8;
constexpr int KS = 4;

struct Epi {
    const float *a_scale;
    const float *w_scale;
    int w_per_row;
    const void *bias;
    int bias_dtype;
    void *y;
    int64_t ldy;
    int vec;
};

constexpr size_t kRingBytes = NSTAGE * 2 * STAGE_BYTES;
__device__ __forceinline__ int chunk_xor(int row) { return ((row ^ (row >> 3)) & 3) | (row & 4); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ chunk_xor(row)) << 4); }

// ring loads: t = 3 (after the barrier): loads 0-2 of stage kt+2 behind MFMAs 1, 3, 5;
// t = 0: loads 3, 4 behind MFMAs 2, 5; t = 1: loads 5-7 behind MFMAs 1, 4, 7
constexpr int dma_slot(int t, int p)
{
    if (t == 3) return (p == 1 || p == 3 || p == 5) ? p / 2 : -1;
    if (t == 0) return p == 2 ? 3 : p == 5 ? 4 : -1;
    if (t == 1) return p == 1 ? 5 : p == 4 ? 6 : p == 7 ? 7 : -1;
    return -1;
}
constexpr int LATE = 3;

constexpr int NSCALEBUF = 3;
constexpr int SCALE_WORDS = BM + 2 * BN;
constexpr int EPI_WAVE_BYTES = 32 * 64;     // 32 rows x 64 bytes (32 bf16 columns)
constexpr size_t kEpiOffset = kRingBytes + NSCALEBUF * SCALE_WORDS * sizeof(float);
constexpr size_t kSmemBytes = kEpiOffset + NW * EPI_WAVE_BYTES;
static_assert(kSmemBytes <= 160 * 1024, "LDS");

// Tile order and ring swizzle as in gemm_q8.hip (restated here: that file keeps them private).
__device__ __forceinline__ void tile_range(int b, int G, int T, int &v, int &step, int &end)
{
    const int x = b & 7, slot = b >> 3;
    int pre = 0;
    for (int y = 0; y < x; y++) pre += (G - y + 7) >> 3;
    const int wx = (G - x + 7) >> 3;
    v = (int)((int64_t)T * pre / G) + slot;
    step = wx;
    end = (int)((int64_t)T * (pre + wx) / G);
}

__device__ __forceinline__ void tile_coords(int v, int nbm, int nbn, int &m0, int &n0)
{
    const int per_group = GROUP_M * nbn;
    const int g = v / per_group, first = g * GROUP_M;
    const int h = min(nbm - first, GROUP_M);
    const int r = v - g * per_group;
    m0 = (first + r % h) * BM;
    n0 = (r / h) * BN;
}

// staging chunk swizzle for 64-byte rows: rows r, r + 4, r + 8, r + 12 share banks
__device__ __forceinline__ int ex(int row) { return (row >> 2) & 3; }

__global__ void __launch_bounds__(NTHREADS, 1)
gemm_i8_8wave_kernel(const uint8_t *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W, int64_t ldw,
                  int M, int N, int K, Epi ep)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    using Acc = v16i;
    using FT = v4i;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 2, wn = wave & 3;
    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int v, step, vend;
    tile_range(blockIdx.x, gridDim.x, nbm * nbn, v, step, vend);
    if (v >= vend) return;
    const int nk = K / BK;
    uint32_t *const scale_lds = (uint32_t *)(smem + kRingBytes);

    const uint8_t *ba = nullptr, *bw = nullptr;
    const uint8_t *nba = nullptr, *nbw = nullptr;
    uint32_t oa[LOADS], ow[LOADS];
    int32_t doa[LOADS] = {}, dow[LOADS] = {};
    auto point_at = [&](int tv, int buf, const uint8_t *&pa, const uint8_t *&pw, uint32_t (&qa)[LOADS],
                        uint32_t (&qw)[LOADS]) {
        int m0, n0;
        tile_coords(tv, nbm, nbn, m0, n0);
        pa = A + (int64_t)m0 * lda;
        pw = W + (int64_t)n0 * ldw;
#pragma unroll
        for (int j = 0; j < LOADS; j++) {
            const int b = j * NW + wave;
            const int r = 8 * b + (lane >> 3);
            const int c = (lane & 7) ^ chunk_xor(r);
            qa[j] = (uint32_t)(min(r, M - 1 - m0) * lda + c * 16);
            qw[j] = (uint32_t)(min(r, N - 1 - n0) * ldw + c * 16);
        }
        if (wave < 4) {
            lds_ptr dst = (lds_ptr)(scale_lds + buf * SCALE_WORDS + 64 * wave);
            const int m = min(m0 + 64 * wave + lane, M - 1), n = min(n0 + 64 * wave + lane, N - 1);
            __builtin_amdgcn_global_load_lds((glb_ptr)(ep.a_scale + m), dst, 4, 0, 0);
            __builtin_amdgcn_global_load_lds((glb_ptr)(ep.w_scale + (ep.w_per_row ? n : 0)), dst + 4 * BM, 4, 0, 0);
            if (ep.bias) {
                const uint8_t *bp = (const uint8_t *)ep.bias + (int64_t)n * (ep.bias_dtype == PSQ_F32 ? 4 : 2);
                if (ep.bias_dtype == PSQ_F32) __builtin_amdgcn_global_load_lds((glb_ptr)bp, dst + 4 * (BM + BN), 4, 0, 0);
                else __builtin_amdgcn_global_load_lds((glb_ptr)bp, dst + 4 * (BM + BN), 2, 0, 0);
            }
        }
    };
    bool has_next = false;
    auto source = [&](int s, bool &same, int64_t &koff) {
        same = s < nk || !has_next;
        koff = (int64_t)(s < nk ? s : (has_next ? s - nk : nk - 1)) * BK;
    };
    auto issue_one = [&](int slot, bool same, int64_t koff, int q) {
        const int j = q % LOADS, b = j * NW + wave;
        lds_ptr d = (lds_ptr)(smem + (q < LOADS ? 0 : NSTAGE * STAGE_BYTES) + slot * STAGE_BYTES + 1024 * b);
        const int32_t mask = same ? 0 : -1;
        const uint8_t *base = (q < LOADS ? (same ? ba : nba) : (same ? bw : nbw)) + koff;
        const uint32_t off = q < LOADS ? oa[j] + (uint32_t)(doa[j] & mask) : ow[j] + (uint32_t)(dow[j] & mask);
        __builtin_amdgcn_global_load_lds((glb_ptr)(base + off), d, 16, 0, 0);
    };
    __amdgpu_buffer_rsrc_t rsa, rsw;
    auto set_rsrc = [&] {
        rsa = raw_rsrc(ba);
        rsw = raw_rsrc(bw);
    };
    auto issue_fast = [&](auto slotc, int64_t koff, auto qc) {
        constexpr int slot = decltype(slotc)::value, q = decltype(qc)::value, j = q % LOADS;
        const int b = j * NW + wave;
        lds_ptr d = (lds_ptr)(smem + (q < LOADS ? 0 : NSTAGE * STAGE_BYTES) + slot * STAGE_BYTES + 1024 * b);
        if constexpr (q < LOADS) buffer_load_lds16(rsa, d, oa[j], (int)koff);
        else buffer_load_lds16(rsw, d, ow[j], (int)koff);
    };

    const int frow = lane & 31, fk = lane >> 5;
    auto read_frag = [&](int slot, int ks, int q, FT (&fa)[TM], FT (&fw)[TN]) {
        const uint8_t *base = smem + (q < TM ? 0 : NSTAGE * STAGE_BYTES) + slot * STAGE_BYTES;
        const int r = (q < TM ? wm * WAVE_M + q * 32 : wn * WAVE_N + (q - TM) * 32) + frow;
        const v4i f = *(const v4i *)(base + swz(r, 2 * ks + fk));
        if (q < TM) fa[q] = f;
        else fw[q - TM] = f;
    };
    uint32_t lof[2][KS];
    auto set_lof = [&] {
#pragma unroll
        for (int o = 0; o < 2; o++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const int c = 2 * ks + fk;
                lof[o][ks] = (uint32_t)((o ? NSTAGE * STAGE_BYTES + wn * WAVE_N * BK : wm * WAVE_M * BK) + frow * BK +
                                        ((c ^ chunk_xor(frow)) << 4));
            }
    };
    auto read_frag_c = [&](auto slotc, auto ksc, auto qc, FT (&fa)[TM], FT (&fw)[TN]) {
        constexpr int slot = decltype(slotc)::value, ks = decltype(ksc)::value, q = decltype(qc)::value;
        constexpr int o = q < TM ? 0 : 1, ql = q < TM ? q : q - TM;
        constexpr uint32_t imm = slot * STAGE_BYTES + ql * 32 * BK;
        const v4i f = *(const v4i *)(smem + lof[o][ks] + imm);
        if constexpr (q < TM) fa[q] = f;
        else fw[q - TM] = f;
    };
    Acc acc[TM][TN];
    auto mfma = [&](int i, int j, const FT (&fa)[TM], const FT (&fw)[TN]) {
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], acc[i][j], 0, 0, 0);
    };
    // MFMA order row-major over (i, j): A0 W0 | W1 | A1 | - | A2 | - | A3
    constexpr int kReadOrder[TM + TN] = {0, 4, 5, 1, 2, 3};

    // epilogue: bf16, full-width tile, aligned rows
    auto epilogue = [&](int m0, int n0, int buf) {
        const uint32_t *sc = scale_lds + buf * SCALE_WORDS;
        const int nl0 = wn * WAVE_N + 4 * (lane >> 5);
        float as[TM];
#pragma unroll
        for (int i = 0; i < TM; i++) as[i] = __uint_as_float(sc[wm * WAVE_M + 32 * i + frow]);
        auto operands = [&](int nc, float (&ws)[4], float (&bs)[4]) {
            const v4i wv = *(const v4i *)(sc + BM + nl0 + nc);
#pragma unroll
            for (int c = 0; c < 4; c++) ws[c] = __int_as_float(wv[c]);
            const v4i bv = *(const v4i *)(sc + BM + BN + nl0 + nc);
            if (!ep.bias) {
#pragma unroll
                for (int c = 0; c < 4; c++) bs[c] = 0.0f;
            } else if (ep.bias_dtype == PSQ_BF16) {
#pragma unroll
                for (int c = 0; c < 4; c++) bs[c] = __uint_as_float((uint32_t)bv[c] << 16);
            } else if (ep.bias_dtype == PSQ_F16) {
#pragma unroll
                for (int c = 0; c < 4; c++) bs[c] = f16_to_f32((uint32_t)bv[c]);
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++) bs[c] = __int_as_float(bv[c]);
            }
        };
        auto value = [&](int i, int j, int r, float w, float b) {
            const int x = agpr_read(acc[i][j][r]);
            return __builtin_fmaf((float)x, as[i] * w, b);
        };
        uint8_t *const eb = smem + kEpiOffset + wave * EPI_WAVE_BYTES;
        const int h = lane >> 5;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            float hws[2][2][4], hbs[2][2][4];
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                const int nc = 32 * j + 16 * pr;
                operands(nc, hws[pr][0], hbs[pr][0]);
                operands(nc + 8, hws[pr][1], hbs[pr][1]);
            }
#pragma unroll
            for (int i = 0; i < TM; i++) {
#pragma unroll
                for (int pr = 0; pr < 2; pr++) {
                    const float (&ws)[2][4] = hws[pr];
                    const float (&bs)[2][4] = hbs[pr];
                    uint32_t x[2], y[2];
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        uint32_t *o = hh == 0 ? x : y;
                        const int r = 8 * pr + 4 * hh;
                        o[0] = pack_half2<PSQ_BF16>(value(i, j, r, ws[hh][0], bs[hh][0]), value(i, j, r + 1, ws[hh][1], bs[hh][1]));
                        o[1] = pack_half2<PSQ_BF16>(value(i, j, r + 2, ws[hh][2], bs[hh][2]), value(i, j, r + 3, ws[hh][3], bs[hh][3]));
                    }
                    uint32_t lo[2], hi[2];
#pragma unroll
                    for (int d = 0; d < 2; d++) {
                        const auto sw = __builtin_amdgcn_permlane32_swap(x[d], y[d], false, false);
                        lo[d] = sw[0];
                        hi[d] = sw[1];
                    }
                    // lane h holds columns 16 pr + 8 h .. + 7 of the 32-column block: chunk 2 pr + h
                    const int ch = 2 * pr + h;
                    *(v4i *)(eb + frow * 64 + ((ch ^ ex(frow)) << 4)) = v4i{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
                }
                v4i val[2];
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int row = 16 * q + (lane >> 2), ch = lane & 3;
                    val[q] = *(const v4i *)(eb + row * 64 + ((ch ^ ex(row)) << 4));
                }
                const int mb = m0 + wm * WAVE_M + 32 * i;
                const int64_t ubase = ((int64_t)mb * ep.ldy + n0 + wn * WAVE_N + 32 * j) * 2;
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int row = 16 * q + (lane >> 2);
                    if (mb + row < M) {
                        const uint32_t loff = (uint32_t)((row * ep.ldy + 8 * (lane & 3)) * 2);
                        __builtin_nontemporal_store(val[q], (v4i *)((uint8_t *)ep.y + ubase + loff));
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    point_at(v, 0, ba, bw, oa, ow);
    has_next = v + step < vend;
    {
        bool same;
        int64_t koff;
        source(0, same, koff);
#pragma unroll
        for (int q = 0; q < LPS; q++) issue_one(0, same, koff, q);
        source(1, same, koff);
#pragma unroll
        for (int q = 0; q < LATE; q++) issue_one(1, same, koff, q);
    }
    wait_vmcnt<LATE>();
    stage_barrier();

    FT fa0[TM], fw0[TN], fa1[TM], fw1[TN];
    int rs = 0;
    int buf = 0;
#pragma unroll
    for (int q = 0; q < TM + TN; q++) read_frag(0, 0, q, fa0, fw0);

    auto kstep = [&](auto tc, FT (&ca)[TM], FT (&cw)[TN], FT (&na)[TM], FT (&nw)[TN], bool s1, int64_t k1,
                     bool s2, int64_t k2) {
        constexpr int t = decltype(tc)::value;
        constexpr bool last = t == KS - 1;
        static_for<TM * TN>([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            mfma(p / TN, p % TN, ca, cw);
            if constexpr (p < TM + TN) read_frag(last ? rs ^ 1 : rs, last ? 0 : t + 1, kReadOrder[p], na, nw);
            constexpr int d = dma_slot(t, p);
            if constexpr (d >= 0) {
                if constexpr (last) issue_one(rs, s2, k2, d);
                else issue_one(rs ^ 1, s1, k1, d);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    auto kstep_fast = [&](auto tc, auto slc, FT (&ca)[TM], FT (&cw)[TN], FT (&na)[TM], FT (&nw)[TN], int64_t k1,
                          int64_t k2) {
        constexpr int t = decltype(tc)::value, SL = decltype(slc)::value;
        constexpr bool last = t == KS - 1;
        static_for<TM * TN>([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            mfma(p / TN, p % TN, ca, cw);
            if constexpr (p < TM + TN)
                read_frag_c(std::integral_constant<int, last ? (SL ^ 1) : SL>{},
                            std::integral_constant<int, last ? 0 : t + 1>{},
                            std::integral_constant<int, kReadOrder[p]>{}, na, nw);
            constexpr int d = dma_slot(t, p);
            if constexpr (d >= 0) {
                if constexpr (last) issue_fast(std::integral_constant<int, SL>{}, k2, std::integral_constant<int, d>{});
                else issue_fast(std::integral_constant<int, SL ^ 1>{}, k1, std::integral_constant<int, d>{});
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    auto stage_fast = [&](auto slc, int kt) {
        const int64_t k1 = (int64_t)(kt + 1) * BK, k2 = (int64_t)(kt + 2) * BK;
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        kstep_fast(I0{}, slc, fa0, fw0, fa1, fw1, k1, k2);
        kstep_fast(I1{}, slc, fa1, fw1, fa0, fw0, k1, k2);
        kstep_fast(std::integral_constant<int, 2>{}, slc, fa0, fw0, fa1, fw1, k1, k2);
        wait_vmcnt<0>();
        stage_barrier();
        kstep_fast(std::integral_constant<int, 3>{}, slc, fa1, fw1, fa0, fw0, k1, k2);
    };
    auto stage = [&](int kt) {
        bool s1, s2;
        int64_t k1, k2;
        source(kt + 1, s1, k1);
        source(kt + 2, s2, k2);
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        kstep(I0{}, fa0, fw0, fa1, fw1, s1, k1, s2, k2);
        kstep(I1{}, fa1, fw1, fa0, fw0, s1, k1, s2, k2);
        kstep(std::integral_constant<int, 2>{}, fa0, fw0, fa1, fw1, s1, k1, s2, k2);
        wait_vmcnt<0>();
        stage_barrier();
        kstep(std::integral_constant<int, 3>{}, fa1, fw1, fa0, fw0, s1, k1, s2, k2);
        rs ^= 1;
    };
#pragma clang loop unroll(disable)
    for (;;) {
        int m0, n0;
        tile_coords(v, nbm, nbn, m0, n0);
        if (has_next) {
            uint32_t qa[LOADS], qw[LOADS];
            point_at(v + step, buf == NSCALEBUF - 1 ? 0 : buf + 1, nba, nbw, qa, qw);
#pragma unroll
            for (int j = 0; j < LOADS; j++) {
                doa[j] = (int32_t)(qa[j] - oa[j]);
                dow[j] = (int32_t)(qw[j] - ow[j]);
            }
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
        int kt0 = 0;
        if ((nk & 1) == 0) {
            set_lof();
            set_rsrc();
#pragma clang loop unroll(disable)
            for (; kt0 + 3 < nk; kt0 += 2) {
                stage_fast(std::integral_constant<int, 0>{}, kt0);
                stage_fast(std::integral_constant<int, 1>{}, kt0 + 1);
            }
        }
#pragma clang loop unroll(disable)
        for (int kt = kt0; kt < nk; kt++) stage(kt);
        epilogue(m0, n0, buf);
        buf = buf == NSCALEBUF - 1 ? 0 : buf + 1;
        if (!has_next) break;
        ba = nba;
        bw = nbw;
#pragma unroll
        for (int j = 0; j < LOADS; j++) {
            oa[j] += (uint32_t)doa[j];
            ow[j] += (uint32_t)dow[j];
        }
        v += step;
        has_next = v + step < vend;
    }
    wait_vmcnt<0>();
}

}  // namespace w8
}  // namespace psq

extern "C" {

int psq_gemm_i8_8wave(const int8_t *a, int64_t lda, const float *a_scale, const int8_t *w, int64_t ldw,
                      const float *w_scale, const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy,
                      int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    using namespace psq::w8;
    const char *name = "gemm_i8_8wave";
    if (M < 0 || N < 0 || K < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    if (M == 0 || N == 0) return PSQ_OK;
    if (!a || !w || !a_scale || !w_scale || !y) return set_error(PSQ_E_ARG, "%s: null operand", name);
    if (y_dtype != PSQ_BF16 || (bias && !valid_dtype(bias_dtype)))
        return set_error(PSQ_E_ARG, "%s: bf16 output only, bias bf16 / f16 / f32", name);
    // whole 256-column tiles, an even stage count (the compile-time ring slots), aligned rows
    if (N % BN || K % (2 * BK) || M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30))
        return set_error(PSQ_E_SHAPE, "%s: N=%lld must be a multiple of 256 and K=%lld of 256", name, (long long)N,
                         (long long)K);
    if (lda < K || ldw < K || lda % 16 || ldw % 16 || lda > (1LL << 23) || ldw > (1LL << 23) || ldy < N ||
        ldy % 8 || ldy >= (1LL << 26))
        return set_error(PSQ_E_SHAPE, "%s: bad strides lda=%lld ldw=%lld ldy=%lld", name, (long long)lda,
                         (long long)ldw, (long long)ldy);
    if (((uintptr_t)a & 15) || ((uintptr_t)w & 15) || ((uintptr_t)y & 15))
        return set_error(PSQ_E_SHAPE, "%s: a, w and y must be 16-byte aligned", name);
    if (int e = require_device()) return e;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(PSQ_E_DEVICE, "%s: no device", name);
    static bool attr_set[64] = {};
    if (dev < 64 && !attr_set[dev]) {
        if (hipFuncSetAttribute((const void *)gemm_i8_8wave_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)kSmemBytes) != hipSuccess)
            return set_error(PSQ_E_DEVICE, "%s: cannot reserve %zu bytes of LDS", name, kSmemBytes);
        attr_set[dev] = true;
    }
    Epi ep{a_scale, w_scale, 1, bias, bias_dtype, y, ldy, 1};
    const int64_t tiles = ((M + BM - 1) / BM) * (N / BN);
    const int64_t grid = tiles < cu_count(dev) ? tiles : cu_count(dev);
    gemm_i8_8wave_kernel<<<dim3((unsigned)grid), dim3(NTHREADS), kSmemBytes, (hipStream_t)stream>>>(
        (const uint8_t *)a, lda, (const uint8_t *)w, ldw, (int)M, (int)N, (int)K, ep);
    return check_launch(name);
}

}  // extern "C"
