// gemm_q8.hip -- W8A8 int8 and fp8-e4m3 GEMMs on gfx950 MFMA with a fused dequant epilogue.
//
// Replaces comfy-kitchen int8_linear and torch._scaled_mm behind
// F.linear(QuantizedTensor, QuantizedTensor, bias) (powershard/quant_linear.py:230-242).
//   y[m][n] = round_out(fmaf((float)acc[m][n], a_scale[m] * w_scale[n], bias[n]))
//   int8: acc = sum_k a[m][k] w[n][k] in int32 (v_mfma_i32_32x32x32_i8, exact)
//   fp8 : acc = the same in fp32 (v_mfma_f32_32x32x64_f8f6f4, e4m3 x e4m3)
//
// Tiling (MI355X-first): a persistent grid of one workgroup per CU walks 256 x 256 output tiles;
// a workgroup is 4 waves, one per SIMD (2 x 2, each wave 128 x 128 = 4 x 4 MFMA tiles of 32 x 32,
// accumulators in the AGPR half of the register file).  K runs in stages of 64 bytes through a
// 4-deep LDS ring (4 x 32 KB) filled by direct global->LDS loads (global_load_lds_dwordx4: no
// staging registers, no LDS write instructions), three stages in flight, continuously across the
// tiles of a workgroup.  Fragments are double-buffered in registers so the LDS reads of the next
// k-step overlap the MFMAs of the current one; one barrier per stage.  The epilogue converts the
// accumulators in registers and stores them without an LDS round trip while the next tile's first
// stages load.  MFMA-bound: 2 M N K ops per launch.
#include "psq_common.hpp"

namespace psq {
namespace {

// Tuning knobs (compile-time): the int8 LDS swizzle and the tile grouping.
#ifndef PSQ_Q8_SWZ
#define PSQ_Q8_SWZ 1
#endif
#ifndef PSQ_Q8_SCHED
#define PSQ_Q8_SCHED 1
#endif
#ifndef PSQ_Q8_GROUP_M
#define PSQ_Q8_GROUP_M 8
#endif

constexpr int BM = 256, BN = 256, BK = 64;    // BK in bytes (= elements for int8/fp8)
// LDS ring depth (NSTAGE - 1 stages in flight): 4 for int8; 3 for fp8, whose fragment sets
// alternate per stage and so need an even number of stages between tile switches.
#ifndef PSQ_Q8_RING_I8
#define PSQ_Q8_RING_I8 4
#endif
template <bool FP8> constexpr int ring_depth() { return FP8 ? 3 : PSQ_Q8_RING_I8; }
constexpr int NTHREADS = 256;                  // 4 waves, one per SIMD
constexpr int WAVE_M = 128, WAVE_N = 128;
constexpr int TM = WAVE_M / 32, TN = WAVE_N / 32;   // 4 x 4 MFMA tiles of 32 x 32 per wave
constexpr int STAGE_BYTES = BM * BK;                 // one operand, one stage (16 KB)
constexpr int LOADS = (BM * BK / 1024) / (NTHREADS / 64);   // 1 KB wave loads per operand per stage (4)
constexpr int GROUP_M = PSQ_Q8_GROUP_M;

enum { OUT_BF16 = PSQ_BF16, OUT_F16 = PSQ_F16, OUT_F32 = PSQ_F32, OUT_I32 = 3 };

struct Epi {
    const float *a_scale;
    const float *w_scale;
    int w_per_row;
    const void *bias;
    int bias_dtype;
    void *y;
    int64_t ldy;
    int vec;          // rows of y are 16-byte aligned: 4-element vector stores allowed
};

// Two outputs packed for a vector store (round to nearest even).
template <int OUT>
__device__ __forceinline__ uint32_t pack2(float a, float b)
{
    return pack_half2<OUT == OUT_BF16 ? PSQ_BF16 : PSQ_F16>(a, b);
}

// One output element (the slow path of partial tiles and unaligned outputs).
template <int OUT>
__device__ __forceinline__ void store1(void *p, int c, float v)
{
    if constexpr (OUT == OUT_F32) ((float *)p)[c] = v;
    else ((uint16_t *)p)[c] = (uint16_t)f32_to_half<OUT>(v);
}

// LDS: the K-loop ring, then the epilogue operands.
constexpr size_t kRingBytes = 4 * 2 * STAGE_BYTES;   // the deeper (int8) ring

// Stage rows are 64 bytes = four 16-byte chunks; a 32-lane MFMA fragment read touches 32
// consecutive rows at one logical chunk.  int8 stores chunk ^ x(row) with x = (r1 ^ r3, r2) (bits
// of the row): bijective in (r1, r2) and in (r2, r3), so both 8 consecutive rows (a 32-bank,
// 128-byte LDS cycle) and 16 consecutive rows (a 64-bank, 256-byte cycle) hit distinct banks.
// fp8 reads 32 bytes (two chunks) per lane, so it swaps whole 32-byte halves,
// chunk ^ (((row >> 1) & 1) << 1), which keeps each lane's fragment contiguous and in k order.
__device__ __forceinline__ int swz_i8(int r)
{
#if PSQ_Q8_SWZ == 0
    return (r >> 1) & 3;
#elif PSQ_Q8_SWZ == 1
    return (((r >> 1) ^ (r >> 3)) & 1) | (r & 4) >> 1;
#else
    return (r >> 2) & 3;
#endif
}

template <bool FP8>
__device__ __forceinline__ int swz(int row, int chunk)
{
    const int x = FP8 ? (((row >> 1) & 1) << 1) : swz_i8(row);
    return row * BK + ((chunk ^ x) << 4);
}

template <bool FP8> struct Frag;
template <> struct Frag<false> { typedef v4i T; static constexpr int KSTEP = 32; };   // 32x32x32 i8
template <> struct Frag<true> { typedef v8i T; static constexpr int KSTEP = 64; };    // 32x32x64 f8f6f4

// Epilogue operands of a tile in LDS past the ring: row scales, column scales and raw bias words
// (one 32-bit word per column: the bias element zero-extended, or the fp32 bits), three buffers
// used round-robin by consecutive tiles of a workgroup.
constexpr int NSCALEBUF = 3;
constexpr int SCALE_WORDS = BM + 2 * BN;
constexpr size_t kSmemBytes = kRingBytes + NSCALEBUF * SCALE_WORDS * sizeof(float);

// Tiles of a persistent workgroup.  Hardware dispatches workgroup b to XCD b % 8; the tile
// sequence (grouped raster order, GROUP_M row tiles per group) is cut into one contiguous chunk
// per XCD, sized by its number of workgroups, and a workgroup takes every wx-th tile of its XCD's
// chunk.  The workgroups of one XCD therefore work on GROUP_M x (wx / GROUP_M) neighbouring tiles
// at a time and share their A and W rows in that XCD's L2.
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

// Bias word (see above) to fp32.
__device__ __forceinline__ float bias_word(uint32_t w, int dt)
{
    if (dt == PSQ_BF16) return __uint_as_float(w << 16);
    if (dt == PSQ_F16) return f16_to_f32(w);
    return __uint_as_float(w);
}

// Persistent kernel: one workgroup per CU walks its tiles; the LDS ring streams continuously
// across tile boundaries, so the first stages of the next tile load while the current tile's
// epilogue runs.  The MFMAs compute the transposed tile (W fragment as the first operand), which
// gives each lane one output row and, per 32 x 32 tile, four runs of 4 consecutive columns: the
// epilogue converts the accumulators in registers and stores them directly.
template <bool FP8, int OUT>
__global__ void __launch_bounds__(NTHREADS, 1)
gemm_q8_kernel(const uint8_t *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W, int64_t ldw,
               int M, int N, int K, Epi ep)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];   // ring [NSTAGE][A | W], scales
    using Acc = typename std::conditional<FP8, v16f, v16i>::type;
    using FT = typename Frag<FP8>::T;
    static_assert(BK / Frag<FP8>::KSTEP == (FP8 ? 1 : 2), "k-steps per stage: 2 for int8, 1 for fp8");
    constexpr int LPS = 2 * LOADS;                 // ring DMA instructions per wave per stage
    constexpr bool SCALED = OUT != OUT_I32;
    constexpr int NSTAGE = ring_depth<FP8>();

    // wave-uniform values in scalar registers: the LDS destination of every global->LDS load (M0)
    // is then computed without a VALU -> SGPR round trip
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int v, step, vend;
    tile_range(blockIdx.x, gridDim.x, nbm * nbn, v, step, vend);
    if (v >= vend) return;
    const int nk = K / BK;
    uint32_t *const scale_lds = (uint32_t *)(smem + kRingBytes);

    // ---------------------------------------------------------------- ring loads
    // global -> LDS: a wave load moves 1 KB = 16 rows x 4 chunks; lane L fills physical slot L of
    // the block (row 16 b + L / 4, physical chunk L % 4) and reads the logical chunk stored there.
    // The loads run NSTAGE - 1 stages ahead of the computation: during the last NSTAGE - 1 stages
    // of a tile they fetch the first stages of the workgroup's next tile (pointer set `nx`); after
    // its last tile a workgroup re-issues the tile's last stage, a load into a ring slot nobody
    // reads again, so every stage issues the same number of loads and the waits are static.
    // A tile's rows are addressed as a wave-uniform base (A + m0 lda, W + n0 ldw: scalar
    // registers) plus a per-lane 32-bit offset -- the scalar-base form of global_load_lds, so a
    // load costs no 64-bit vector address arithmetic.  Rows past M (N) are clamped to the last
    // row; the tile's stores skip them.
    const uint8_t *ba = nullptr, *bw = nullptr;       // current tile
    const uint8_t *nba = nullptr, *nbw = nullptr;     // next tile
    uint32_t oa[LOADS], ow[LOADS];                    // current tile's lane offsets
    int32_t doa[LOADS] = {}, dow[LOADS] = {};         // next tile's offsets minus the current ones
    auto point_at = [&](int tv, int buf, const uint8_t *&pa, const uint8_t *&pw, uint32_t (&qa)[LOADS],
                        uint32_t (&qw)[LOADS]) {
        int m0, n0;
        tile_coords(tv, nbm, nbn, m0, n0);
        pa = A + (int64_t)m0 * lda;
        pw = W + (int64_t)n0 * ldw;
#pragma unroll
        for (int j = 0; j < LOADS; j++) {
            const int b = j * (NTHREADS / 64) + wave;
            const int r = 16 * b + (lane >> 2);
            const int c = (lane & 3) ^ (FP8 ? (((r >> 1) & 1) << 1) : swz_i8(r));
            qa[j] = (uint32_t)(min(r, M - 1 - m0) * lda + c * 16);
            qw[j] = (uint32_t)(min(r, N - 1 - n0) * ldw + c * 16);
        }
        if constexpr (SCALED) {
            // the tile's row scales, column scales and bias words: 64 entries of each per wave
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
    // ring load q of a stage (q < LOADS: A block q, else W block q - LOADS), from the current tile
    // (same) or the next one, at byte offset koff along K, into ring slot `slot`.  The next tile's
    // lane offset is the current one plus a masked delta (a select between two offset arrays is
    // turned into a load from a selected address, which sends both arrays to scratch memory).
    auto issue_one = [&](int slot, bool same, int64_t koff, int q) {
        const int j = q % LOADS, b = j * (NTHREADS / 64) + wave;
        lds_ptr d = (lds_ptr)(smem + slot * 2 * STAGE_BYTES + (q < LOADS ? 0 : STAGE_BYTES) + 1024 * b);
        const int32_t mask = same ? 0 : -1;
        const uint8_t *base = (q < LOADS ? (same ? ba : nba) : (same ? bw : nbw)) + koff;
        const uint32_t off = q < LOADS ? oa[j] + (uint32_t)(doa[j] & mask) : ow[j] + (uint32_t)(dow[j] & mask);
        __builtin_amdgcn_global_load_lds((glb_ptr)(base + off), d, 16, 0, 0);
    };
    auto issue_stage = [&](int slot, bool same, int64_t koff) {
#pragma unroll
        for (int q = 0; q < LPS; q++) issue_one(slot, same, koff, q);
    };

    // MFMA operand layout (32 x 32 tiles): lane holds row (lane & 31) of W / of A and the k-slice
    // (lane >> 5) of the instruction's K; both operands use the same slice, so the dot products are
    // complete whatever order the hardware sums a slice in.
    const int frow = lane & 31, fk = lane >> 5;
    // fragment q of a k-step: q < TM is A fragment q, else W fragment q - TM
    auto read_frag = [&](int slot, int ks, int q, FT (&fa)[TM], FT (&fw)[TN]) {
        const uint8_t *base = smem + slot * 2 * STAGE_BYTES + (q < TM ? 0 : STAGE_BYTES);
        const int r = (q < TM ? wm * WAVE_M + q * 32 : wn * WAVE_N + (q - TM) * 32) + frow;
        if constexpr (FP8) {
            // two 16-byte reads: the compiler otherwise makes every 32-byte read wait for all
            // global->LDS loads in flight (vmcnt(0)), whose completion the stage wait and barrier
            // already order
            const v4i lo = *(const v4i *)(base + swz<true>(r, 2 * fk));
            const v4i hi = *(const v4i *)(base + swz<true>(r, 2 * fk) + 16);
            const v8i f = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (q < TM) fa[q] = f;
            else fw[q - TM] = f;
        } else {
            const v4i f = *(const v4i *)(base + swz<false>(r, 2 * ks + fk));
            if (q < TM) fa[q] = f;
            else fw[q - TM] = f;
        }
    };
    // acc[i][j] is the transposed 32 x 32 tile: W rows (output columns) x A rows (output rows).
    Acc acc[TM][TN];
    auto mfma = [&](int i, int j, const FT (&fa)[TM], const FT (&fw)[TN]) {
        if constexpr (FP8)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw[j], fa[i], acc[i][j], 0, 0, 0, 127, 0, 127);
        else
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], acc[i][j], 0, 0, 0);
    };
    // Reads in the order the MFMAs (row-major over i, j) first need them: A0, W0..W3, A1..A3.
    constexpr int kReadOrder[TM + TN] = {0, 4, 5, 6, 7, 1, 2, 3};
    // int8 half-stage schedules: behind MFMA q, fragment read kSchedRead[q] and ring load
    // kSchedLoadA[q] (first half) / kSchedLoadB[q] (second half); -1 = none.  Global->LDS loads
    // issued back to back stall the wave's MFMA issue, so they are spaced out; the reads go first.
#if PSQ_Q8_SCHED == 0
    constexpr int kSchedRead[16] = {0, 1, 2, 3, 4, 5, 6, 7, -1, -1, -1, -1, -1, -1, -1, -1};
    constexpr int kSchedLoadA[16] = {-1, -1, -1, -1, -1, -1, -1, -1, 0, 1, 2, 3, 4, 5, 6, 7};
    constexpr int kSchedLoadB[16] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1};
#elif PSQ_Q8_SCHED == 1
    constexpr int kSchedRead[16] = {0, 1, 2, 3, 4, 5, 6, 7, -1, -1, -1, -1, -1, -1, -1, -1};
    constexpr int kSchedLoadA[16] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, 0, -1, 1, -1, 2, -1, 3};
    constexpr int kSchedLoadB[16] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, 4, -1, 5, -1, 6, -1, 7};
#elif PSQ_Q8_SCHED == 2
    constexpr int kSchedRead[16] = {0, -1, 1, -1, 2, -1, 3, -1, 4, -1, 5, -1, 6, -1, 7, -1};
    constexpr int kSchedLoadA[16] = {-1, 0, -1, 1, -1, 2, -1, 3, -1, 4, -1, 5, -1, 6, -1, 7};
    constexpr int kSchedLoadB[16] = {-1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1};
#elif PSQ_Q8_SCHED == 3
    constexpr int kSchedRead[16] = {0, 1, 2, 3, 4, 5, 6, 7, -1, -1, -1, -1, -1, -1, -1, -1};
    constexpr int kSchedLoadA[16] = {-1, -1, -1, 0, -1, -1, -1, 1, -1, -1, -1, 2, -1, -1, -1, 3};
    constexpr int kSchedLoadB[16] = {-1, -1, -1, 4, -1, -1, -1, 5, -1, -1, -1, 6, -1, -1, -1, 7};
#elif PSQ_Q8_SCHED == 4
    constexpr int kSchedRead[16] = {0, 1, 2, 3, 4, 5, 6, 7, -1, -1, -1, -1, -1, -1, -1, -1};
    constexpr int kSchedLoadA[16] = {-1, -1, -1, -1, -1, -1, -1, -1, 0, -1, 1, -1, 2, -1, 3, -1};
    constexpr int kSchedLoadB[16] = {-1, -1, -1, -1, -1, -1, -1, -1, 4, -1, 5, -1, 6, -1, 7, -1};
#elif PSQ_Q8_SCHED == 5
    constexpr int kSchedRead[16] = {0, 1, 2, 3, 4, 5, 6, 7, -1, -1, -1, -1, -1, -1, -1, -1};
    constexpr int kSchedLoadA[16] = {-1, 0, -1, -1, -1, 1, -1, -1, -1, 2, -1, -1, -1, 3, -1, -1};
    constexpr int kSchedLoadB[16] = {-1, 4, -1, -1, -1, 5, -1, -1, -1, 6, -1, -1, -1, 7, -1, -1};
#else
    constexpr int kSchedRead[16] = {0, -1, 1, -1, 2, -1, 3, -1, 4, -1, 5, -1, 6, -1, 7, -1};
    constexpr int kSchedLoadA[16] = {-1, -1, -1, 0, -1, -1, -1, 1, -1, -1, -1, 2, -1, -1, -1, 3};
    constexpr int kSchedLoadB[16] = {-1, -1, -1, 4, -1, -1, -1, 5, -1, -1, -1, 6, -1, -1, -1, 7};
#endif
    constexpr int kLoadsB = [] {
        int n = 0;
        for (int q = 0; q < 16; q++) n += kSchedLoadB[q] >= 0;
        return n;
    }();

    // ---------------------------------------------------------------- epilogue
    // Lane (l & 31) owns output row m = m0 + 128 wm + 32 i + (l & 31); register 4 g + c of
    // acc[i][j] is column n0 + 128 wn + 32 j + 8 g + 4 (l >> 5) + c.
    //   y = round_out(fmaf((float)acc, a_scale[m] * w_scale[n], bias[n]))
    auto epilogue = [&](int m0, int n0, int buf) {
        const uint32_t *sc = scale_lds + buf * SCALE_WORDS;
        constexpr int esz = OUT == OUT_F32 || OUT == OUT_I32 ? 4 : 2;
        const int nl0 = wn * WAVE_N + 4 * (lane >> 5);
        uint8_t *rowp[TM];
        bool live[TM];
        float as[TM];
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int ml = wm * WAVE_M + 32 * i + frow;
            live[i] = m0 + ml < M;
            rowp[i] = (uint8_t *)ep.y + ((int64_t)min(m0 + ml, M - 1) * ep.ldy + n0 + nl0) * esz;
            as[i] = SCALED ? __uint_as_float(sc[ml]) : 0.0f;
        }
        // the scale / bias operands of the lane's 4 columns at offset nc from its first column
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
        auto raw = [&](int i, int j, int r) { return agpr_read(acc[i][j][r]); };
        auto value = [&](int i, int j, int r, float w, float b) {
            const int x = raw(i, j, r);
            const float a = FP8 ? __int_as_float(x) : (float)x;
            return __builtin_fmaf(a, as[i] * w, b);
        };
        if (ep.vec && n0 + BN <= N) {
            // Full-width tile, aligned rows.  Lanes l and l + 32 hold the same row: for column
            // groups g = 2p and 2p + 1 lane l has columns 16p + {0-3, 8-11} and lane l + 32 has
            // 16p + {4-7, 12-15}.  One v_permlane32_swap per word gives lane l columns 16p + 0-7
            // and lane l + 32 columns 16p + 8-15, so each store writes 8 consecutive outputs and a
            // row's 16 columns take one instruction (half the stores, twice the bytes per line).
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int pr = 0; pr < 2; pr++) {
                    const int nc = 32 * j + 16 * pr;
                    float ws[2][4] = {{1.0f, 1.0f, 1.0f, 1.0f}, {1.0f, 1.0f, 1.0f, 1.0f}};
                    float bs[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
                    if constexpr (SCALED) {
                        operands(nc, ws[0], bs[0]);
                        operands(nc + 8, ws[1], bs[1]);
                    }
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        // words of the two groups: x (g = 2 pr), y (g = 2 pr + 1)
                        constexpr int NW = esz == 4 ? 4 : 2;
                        uint32_t x[NW], y[NW];
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            uint32_t *o = h == 0 ? x : y;
                            const int r = 8 * pr + 4 * h;
                            if constexpr (OUT == OUT_I32) {
#pragma unroll
                                for (int c = 0; c < 4; c++) o[c] = (uint32_t)raw(i, j, r + c);
                            } else if constexpr (OUT == OUT_F32) {
#pragma unroll
                                for (int c = 0; c < 4; c++) o[c] = __float_as_uint(value(i, j, r + c, ws[h][c], bs[h][c]));
                            } else {
                                o[0] = pack2<OUT>(value(i, j, r, ws[h][0], bs[h][0]), value(i, j, r + 1, ws[h][1], bs[h][1]));
                                o[1] = pack2<OUT>(value(i, j, r + 2, ws[h][2], bs[h][2]), value(i, j, r + 3, ws[h][3], bs[h][3]));
                            }
                        }
                        uint32_t lo[NW], hi[NW];
#pragma unroll
                        for (int d = 0; d < NW; d++) {
                            const auto sw = __builtin_amdgcn_permlane32_swap(x[d], y[d], false, false);
                            lo[d] = sw[0];
                            hi[d] = sw[1];
                        }
                        // lane l < 32 stores at column nc, lane l + 32 at nc + 8 (rowp already holds 4 h)
                        uint8_t *p = rowp[i] + (nc + 4 * (lane >> 5)) * esz;
                        if (live[i]) {
                            if constexpr (NW == 2) {
                                *(v4i *)p = v4i{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
                            } else {
                                *(v4i *)p = v4i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3]};
                                *(v4i *)(p + 16) = v4i{(int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
                            }
                        }
                    }
                    // one column pair at a time: keeps the scheduler from hoisting every group's
                    // operand reads (and their registers) to the top of the epilogue
                    __builtin_amdgcn_sched_barrier(0);
                }
        } else {
            // partial tile or unaligned rows: element stores bounded by the row's remaining columns
            const int n_left0 = N - (n0 + nl0);
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int nc = 32 * j + 8 * g;
                    float ws[4] = {1.0f, 1.0f, 1.0f, 1.0f}, bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (SCALED) operands(nc, ws, bs);
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        void *p = rowp[i] + nc * esz;
#pragma unroll
                        for (int c = 0; c < 4; c++) {
                            if (!live[i] || c >= n_left0 - nc) continue;
                            if constexpr (OUT == OUT_I32) ((int32_t *)p)[c] = raw(i, j, 4 * g + c);
                            else store1<OUT>(p, c, value(i, j, 4 * g + c, ws[c], bs[c]));
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
    };

    // ---------------------------------------------------------------- main loop
    point_at(v, 0, ba, bw, oa, ow);
#pragma unroll
    for (int s = 0; s < NSTAGE - 1; s++) issue_stage(s, true, (int64_t)min(s, nk - 1) * BK);
    wait_vmcnt<(NSTAGE - 2) * LPS>();
    stage_barrier();

    FT fa0[TM], fw0[TN], fa1[TM], fw1[TN];
    int rs = 0;                      // ring slot of the stage being computed
    int buf = 0;                     // epilogue-operand buffer of the tile being computed
#pragma unroll
    for (int q = 0; q < TM + TN; q++) read_frag(0, 0, q, fa0, fw0);
    // Stage kt loads stage kt + NSTAGE - 1: of this tile while that exists, else of the next
    // tile (a K shorter than the lookahead gets one tile per workgroup, so it never gets there).
    bool has_next = false;
    // The instruction order inside a stage is fixed explicitly (sched_barrier after every step):
    // with one wave per SIMD every issue slot not spent on an MFMA idles the matrix core, and the
    // wave stalls wherever it waits for LDS reads still in flight.  So each half-stage first slots
    // the fragment reads the next half-stage consumes behind its first MFMAs (they then have the
    // rest of the half-stage to land), then the refill loads behind the following ones.
    //   int8, one stage = two k-steps.  Half A: MFMAs of k-step 0 on (ca, cw); behind them the
    //   reads of k-step 1 into (na, nw) and the refill of the ring slot read in the previous stage
    //   (every wave passed the barrier that ended it).  Wait for the next stage, barrier.  Half B:
    //   MFMAs of k-step 1 on (na, nw); behind them the next stage's k-step 0 reads into (ca, cw).
    //   fp8, one k-step per stage.  Half A: MFMAs of rows 0-1 on (ca, cw) with the refill loads;
    //   wait, barrier; half B: MFMAs of rows 2-3 with the next stage's reads into (na, nw).
    auto stage = [&](int kt, FT (&ca)[TM], FT (&cw)[TN], FT (&na)[TM], FT (&nw)[TN]) {
        const int t = kt + NSTAGE - 1;
        const bool same = t < nk || !has_next;
        const int64_t koff = (int64_t)(t < nk ? t : (has_next ? t - nk : nk - 1)) * BK;
        const int slot = rs == 0 ? NSTAGE - 1 : rs - 1;
        if constexpr (!FP8) {
#pragma unroll
            for (int q = 0; q < TM * TN; q++) {
                mfma(q / TN, q % TN, ca, cw);
                if (kSchedRead[q] >= 0) read_frag(rs, 1, kReadOrder[kSchedRead[q]], na, nw);
                if (kSchedLoadA[q] >= 0) issue_one(slot, same, koff, kSchedLoadA[q]);
                __builtin_amdgcn_sched_barrier(0);
            }
            wait_vmcnt<(NSTAGE - 2) * LPS - kLoadsB>();
            stage_barrier();
            rs = rs == NSTAGE - 1 ? 0 : rs + 1;
#pragma unroll
            for (int q = 0; q < TM * TN; q++) {
                mfma(q / TN, q % TN, na, nw);
                if (kSchedRead[q] >= 0) read_frag(rs, 0, kReadOrder[kSchedRead[q]], ca, cw);
                if (kSchedLoadB[q] >= 0) issue_one(slot, same, koff, kSchedLoadB[q]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
#pragma unroll
            for (int q = 0; q < TM * TN / 2; q++) {
                mfma(q / TN, q % TN, ca, cw);
                issue_one(slot, same, koff, q);
                __builtin_amdgcn_sched_barrier(0);
            }
            wait_vmcnt<(NSTAGE - 2) * LPS>();
            stage_barrier();
            rs = rs == NSTAGE - 1 ? 0 : rs + 1;
#pragma unroll
            for (int q = 0; q < TM * TN / 2; q++) {
                mfma(TM / 2 + q / TN, q % TN, ca, cw);
                read_frag(rs, 0, kReadOrder[q], na, nw);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
#pragma clang loop unroll(disable)
    for (; v < vend; v += step) {
        int m0, n0;
        tile_coords(v, nbm, nbn, m0, n0);
        has_next = v + step < vend;
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
        if constexpr (!FP8) {
            // int8 keeps fragment set 0 current at every stage boundary
#pragma clang loop unroll(disable)
            for (int kt = 0; kt < nk; kt++) stage(kt, fa0, fw0, fa1, fw1);
        } else {
            // fp8 swaps the sets per stage: pairs of stages (nk is even: K % 128 == 0)
#pragma clang loop unroll(disable)
            for (int kt = 0; kt < nk; kt += 2) {
                stage(kt, fa0, fw0, fa1, fw1);
                stage(kt + 1, fa1, fw1, fa0, fw0);
            }
        }
        epilogue(m0, n0, buf);
        buf = buf == NSCALEBUF - 1 ? 0 : buf + 1;
        if (has_next) {
            ba = nba;
            bw = nbw;
#pragma unroll
            for (int j = 0; j < LOADS; j++) {
                oa[j] += (uint32_t)doa[j];
                ow[j] += (uint32_t)dow[j];
            }
        }
    }
    // the re-issued loads past the last tile must land before the workgroup's LDS is released
    wait_vmcnt<0>();
}

// CUs of each device (the persistent grid size), cached per device.
int cu_count(int dev)
{
    static int cus[64] = {};
    if (dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

template <bool FP8, int OUT>
int launch_one(const uint8_t *a, int64_t lda, const uint8_t *w, int64_t ldw, int64_t M, int64_t N, int64_t K,
               const Epi &ep, hipStream_t st, const char *name)
{
    auto kern = gemm_q8_kernel<FP8, OUT>;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(PSQ_E_DEVICE, "%s: no device", name);
    static bool attr_set[64] = {};   // per device; the attribute is idempotent
    if (dev < 64 && !attr_set[dev]) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSmemBytes) !=
            hipSuccess)
            return set_error(PSQ_E_DEVICE, "%s: cannot reserve %zu bytes of LDS", name, kSmemBytes);
        attr_set[dev] = true;
    }
    // persistent grid of one workgroup per CU; a K shorter than the ring's lookahead gets one
    // workgroup per tile (the kernel's loads then never cross into another tile)
    const int64_t tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    const bool short_k = K / BK < ring_depth<FP8>() - 1;
    const int64_t grid = (short_k || tiles < cu_count(dev)) ? tiles : cu_count(dev);
    kern<<<dim3((unsigned)grid), dim3(NTHREADS), kSmemBytes, st>>>(a, lda, w, ldw, (int)M, (int)N, (int)K, ep);
    return check_launch(name);
}

template <bool FP8>
int launch(int out, const uint8_t *a, int64_t lda, const uint8_t *w, int64_t ldw, int64_t M, int64_t N, int64_t K,
           const Epi &ep, hipStream_t st, const char *name)
{
    switch (out) {
    case OUT_BF16: return launch_one<FP8, OUT_BF16>(a, lda, w, ldw, M, N, K, ep, st, name);
    case OUT_F16: return launch_one<FP8, OUT_F16>(a, lda, w, ldw, M, N, K, ep, st, name);
    case OUT_F32: return launch_one<FP8, OUT_F32>(a, lda, w, ldw, M, N, K, ep, st, name);
    default: return launch_one<FP8, OUT_I32>(a, lda, w, ldw, M, N, K, ep, st, name);
    }
}

int vec_ok(const void *y, int64_t ldy, int elem)
{
    return (((uintptr_t)y & 15) == 0 && (ldy * elem) % 16 == 0) ? 1 : 0;
}

int check_shapes(const char *name, const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M, int64_t N,
                 int64_t K)
{
    if (M < 0 || N < 0 || K < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    if (!a || !w) return set_error(PSQ_E_ARG, "%s: null operand", name);
    if (K == 0 || K % 128)
        return set_error(PSQ_E_SHAPE, "%s: K=%lld must be a positive multiple of 128", name, (long long)K);
    if (lda < K || ldw < K || lda % 16 || ldw % 16)
        return set_error(PSQ_E_SHAPE, "%s: lda=%lld ldw=%lld must be multiples of 16 covering K", name,
                         (long long)lda, (long long)ldw);
    if (((uintptr_t)a & 15) || ((uintptr_t)w & 15)) return set_error(PSQ_E_SHAPE, "%s: operands must be 16-byte aligned", name);
    if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30))
        return set_error(PSQ_E_SHAPE, "%s: size too large", name);
    if (lda > (1LL << 23) || ldw > (1LL << 23))   // a tile's row offsets (256 rows) fit in 31 bits
        return set_error(PSQ_E_SHAPE, "%s: lda/ldw above 2^23", name);
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
    Epi ep{a_scale, w_scale, 1, bias, bias_dtype, y, ldy, vec_ok(y, ldy, y_dtype == PSQ_F32 ? 4 : 2)};
    return launch<false>(y_dtype, (const uint8_t *)a, lda, (const uint8_t *)w, ldw, M, N, K, ep,
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
    Epi ep{nullptr, nullptr, 0, nullptr, 0, c, ldc, vec_ok(c, ldc, 4)};
    return launch<false>(OUT_I32, (const uint8_t *)a, lda, (const uint8_t *)w, ldw, M, N, K, ep,
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
    Epi ep{a_scale, w_scale, w_scale_per_row ? 1 : 0, bias, bias_dtype, y, ldy, vec_ok(y, ldy, y_dtype == PSQ_F32 ? 4 : 2)};
    return launch<true>(y_dtype, a, lda, w, ldw, M, N, K, ep, (hipStream_t)stream, "gemm_fp8");
}

}  // extern "C"
