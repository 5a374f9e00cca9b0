// gemm_q8.hip -- W8A8 int8 and fp8-e4m3 GEMMs on gfx950 MFMA with a fused dequant epilogue.
//
// Replaces comfy-kitchen int8_linear and torch._scaled_mm behind
// F.linear(QuantizedTensor, QuantizedTensor, bias) (powershard/quant_linear.py:230-242).
//   y[m][n] = round_out(fmaf((float)acc[m][n], a_scale[m] * w_scale[n], bias[n]))
//   int8: acc = sum_k a[m][k] w[n][k] in int32 (v_mfma_i32_32x32x32_i8, exact)
//   fp8 : acc = the same in fp32 (v_mfma_f32_32x32x64_f8f6f4, e4m3 x e4m3; or e5m2 weights x
//         e4m3 activations, the instruction's A-operand format selector set to bf8)
// With an epilogue activation (GELU, tanh form; the Wan FFN's F.gelu(fc1(x).float(),
// approximate="tanh"), powershard/wan_model.py:626) the store writes round_out(act(round_out(y))):
// the GELU of the rounded linear output, rounded to the dtype the next layer casts it to.
// With the SiLU gate (the H3 MLP's silu(gate) * up, powershard/fp16_safe.py:165-167) the weight's
// N rows are N / 2 gate rows followed by N / 2 up rows; a tile reads its W rows as 64 gate rows
// and their 64 up rows per wave-column block, so each gate value meets its up value in the same
// lane and register, and the store writes round_out(silu(round_out(g)) round_out(u)) to [M, N / 2].
//
// Tiling (MI355X-first): a persistent grid of one workgroup per CU walks 256 x 256 output tiles;
// a workgroup is 4 waves, one per SIMD (2 x 2, each wave 128 x 128 = 4 x 4 MFMA tiles of 32 x 32,
// accumulators in the AGPR half of the register file).  K runs in stages of 128 bytes -- one full
// cache line of every row -- through a 2-slot LDS ring (2 x 64 KB) filled by direct global->LDS
// loads (no staging registers, no LDS write instructions); a stage loads while the previous one
// computes, continuously across the tiles of a workgroup.  Fragments are double-buffered in
// registers so the LDS reads of the next k-step overlap the MFMAs of the current one; one barrier
// per stage.  In the steady state of a tile (pairs of stages with the ring slot known at compile
// time) a k-step issues no address arithmetic: fragment reads use per-tile lane offsets plus
// immediates, and the ring loads are buffer loads with the tile base in a descriptor, the k
// offset as scalar offset and the lane's row offset as vector offset.  The epilogue converts the
// accumulators in registers and stages 32 x 64 blocks through LDS for whole-line stores while the
// next tile's first stage loads.  MFMA-bound: 2 M N K ops per launch.
#include "psq_common.hpp"

namespace psq {
namespace {

constexpr int BM = 256, BN = 256, BK = 128;   // BK in bytes (= elements for int8/fp8)
constexpr int NSTAGE = 2;                      // LDS ring slots: the stage computed, the stage loading
constexpr int NTHREADS = 256;                  // 4 waves, one per SIMD
constexpr int WAVE_M = 128, WAVE_N = 128;
constexpr int TM = WAVE_M / 32, TN = WAVE_N / 32;   // 4 x 4 MFMA tiles of 32 x 32 per wave
constexpr int STAGE_BYTES = BM * BK;                 // one operand, one stage (32 KB)
constexpr int LOADS = (BM * BK / 1024) / (NTHREADS / 64);   // 1 KB wave loads per operand per stage (8)
constexpr int LPS = 2 * LOADS;                       // ring loads per wave per stage (16)
constexpr int GROUP_M = 8;                           // tile rows per raster group

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

// The epilogue's activation, applied to the output rounded to its dtype (fp32 outputs: unrounded);
// the store rounds the result again.
template <int OUT, int ACT>
__device__ __forceinline__ float act1(float v)
{
    if constexpr (ACT != ACT_GELU_TANH || OUT == OUT_I32) return v;
    else if constexpr (OUT == OUT_F32) return gelu_tanh(v);
    else {
        constexpr int DT = OUT == OUT_BF16 ? PSQ_BF16 : PSQ_F16;
        return gelu_tanh(half_to_f32<DT>(f32_to_half<DT>(v)));
    }
}

// Two outputs activated (as act1) and packed: the inner rounding is the same packed conversion.
template <int OUT, int ACT>
__device__ __forceinline__ uint32_t pack2a(float a, float b)
{
    if constexpr (ACT != ACT_GELU_TANH) {
        return pack2<OUT>(a, b);
    } else {
        const uint32_t p = pack2<OUT>(a, b);
        float ra, rb;
        if constexpr (OUT == OUT_BF16) {
            ra = __uint_as_float(p << 16);
            rb = __uint_as_float(p & 0xffff0000u);
        } else {
            ra = f16_to_f32(p & 0xffffu);
            rb = f16_to_f32(p >> 16);
        }
        return pack2<OUT>(gelu_tanh(ra), gelu_tanh(rb));
    }
}

// The gate: silu(g) u on the outputs rounded to their dtype (fp32 outputs: unrounded).
template <int OUT>
__device__ __forceinline__ float gate1(float g, float u)
{
    if constexpr (OUT == OUT_F32) return silu(g) * u;
    else {
        constexpr int DT = OUT == OUT_BF16 ? PSQ_BF16 : PSQ_F16;
        return silu(half_to_f32<DT>(f32_to_half<DT>(g))) * half_to_f32<DT>(f32_to_half<DT>(u));
    }
}

// Two gated outputs packed (as gate1): the inner roundings are the same packed conversion.
template <int OUT>
__device__ __forceinline__ uint32_t pack2g(float g0, float u0, float g1, float u1)
{
    const uint32_t pg = pack2<OUT>(g0, g1), pu = pack2<OUT>(u0, u1);
    float rg0, rg1, ru0, ru1;
    if constexpr (OUT == OUT_BF16) {
        rg0 = __uint_as_float(pg << 16);
        rg1 = __uint_as_float(pg & 0xffff0000u);
        ru0 = __uint_as_float(pu << 16);
        ru1 = __uint_as_float(pu & 0xffff0000u);
    } else {
        rg0 = f16_to_f32(pg & 0xffffu);
        rg1 = f16_to_f32(pg >> 16);
        ru0 = f16_to_f32(pu & 0xffffu);
        ru1 = f16_to_f32(pu >> 16);
    }
    return pack2<OUT>(silu(rg0) * ru0, silu(rg1) * ru1);
}

// One output element (the slow path of partial tiles and unaligned outputs).
template <int OUT>
__device__ __forceinline__ void store1(void *p, int c, float v)
{
    if constexpr (OUT == OUT_F32) ((float *)p)[c] = v;
    else ((uint16_t *)p)[c] = (uint16_t)f32_to_half<OUT>(v);
}

// LDS: the K-loop ring, then the epilogue operands.
constexpr size_t kRingBytes = NSTAGE * 2 * STAGE_BYTES;

// Stage rows are 128 bytes = eight 16-byte chunks.  A fragment read touches 32 consecutive rows at
// one logical chunk, 16 lanes (256 bytes, all 64 banks) per LDS cycle: bank group 8 (r & 1) +
// physical chunk.  Chunk c of row r is stored at c ^ f(r), f(r) = (r0 ^ r3, r1 ^ r4, r2) in bits,
// which is bijective in row bits 0-2 (8 consecutive rows: distinct chunks) and, for a fixed bit 0,
// in bits 1-3 (the 8 rows of one parity among 16 consecutive rows), so every read is conflict
// free.  f ignores row bit 5 and up, so the fragments of all 32-row blocks share one swizzle.  fp8
// reads two consecutive chunks per lane, each its own conflict-free read.
__device__ __forceinline__ int chunk_xor(int row) { return ((row ^ (row >> 3)) & 3) | (row & 4); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ chunk_xor(row)) << 4); }

// Ring-load schedule: dma_slot(t, p) is the ring load (0-15: A blocks, then W blocks) issued
// behind MFMA p (0-15) of k-step t, or -1.  Loads behind the last k-step (after the barrier) fill
// the slot just freed with stage kt + 2 and are numbered first; loads behind the earlier k-steps
// complete stage kt + 1 in the other slot before the barrier.  The fragment reads of the next
// k-step go behind MFMAs 0-7.  int8: 6 loads behind the even MFMAs 2-12 of the last k-step, 5
// behind MFMAs 1, 4, 7, 10, 13 of k-steps 0 and 1 (measured 1% ahead of spreading them evenly or
// of bunching them behind one k-step).  fp8 (two k-steps per stage): the whole of stage kt + 2
// behind k-step 1, one load per MFMA.
template <bool FP8>
constexpr int dma_slot(int t, int p)
{
    if constexpr (!FP8) {
        if (t == 3) return (p >= 2 && p <= 12 && !(p & 1)) ? (p - 2) / 2 : -1;
        if (t < 2) return (p % 3 == 1) ? 6 + 5 * t + p / 3 : -1;
        return -1;
    } else {
        return t == 1 ? p : -1;
    }
}
template <bool FP8>
constexpr int late_loads()
{
    int n = 0;
    for (int p = 0; p < 16; p++) n += dma_slot<FP8>(FP8 ? 1 : 3, p) >= 0;
    return n;
}

template <bool FP8> struct Frag;
template <> struct Frag<false> { typedef v4i T; static constexpr int KSTEP = 32; };   // 32x32x32 i8
template <> struct Frag<true> { typedef v8i T; static constexpr int KSTEP = 64; };    // 32x32x64 f8f6f4

// Epilogue operands of a tile in LDS past the ring: row scales, column scales and raw bias words
// (one 32-bit word per column: the bias element zero-extended, or the fp32 bits), three buffers
// used round-robin by consecutive tiles of a workgroup.
constexpr int NSCALEBUF = 3;
constexpr int SCALE_WORDS = BM + 2 * BN;
// then, per wave, the staging buffer of the bf16 / f16 epilogue: 32 rows x 128 bytes
constexpr int EPI_WAVE_BYTES = 32 * 128;
constexpr size_t kEpiOffset = kRingBytes + NSCALEBUF * SCALE_WORDS * sizeof(float);
constexpr size_t kSmemBytes = kEpiOffset + (NTHREADS / 64) * EPI_WAVE_BYTES;

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
// WF: the fp8 weights' format (0: e4m3fn, 1: e5m2), the f8f6f4 MFMA's A-operand format code.
template <bool FP8, int OUT, int ACT, int WF = 0>
__global__ void __launch_bounds__(NTHREADS, 1)
gemm_q8_kernel(const uint8_t *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W, int64_t ldw,
               int M, int N, int K, Epi ep)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];   // ring A[NSTAGE] | W[NSTAGE], scales
    using Acc = typename std::conditional<FP8, v16f, v16i>::type;
    using FT = typename Frag<FP8>::T;
    constexpr int KS = BK / Frag<FP8>::KSTEP;      // k-steps per stage: 4 (int8), 2 (fp8)
    constexpr bool SCALED = OUT != OUT_I32;
    constexpr int LATE = late_loads<FP8>();         // loads of stage kt + 2 behind the last k-step
    constexpr bool GATED = ACT == ACT_SILU_GATE;

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
    // global -> LDS: a wave load moves 1 KB = 8 rows x 8 chunks (every row a full 128-byte cache
    // line); lane L fills physical slot L of the block (row 8 b + L / 8, physical chunk L % 8) and
    // reads the logical chunk stored there.  Stage s of a workgroup's sequence comes from its
    // current tile while s < nk, then from its next tile (pointer set `n*`); past its last tile a
    // workgroup re-loads the tile's last stage into the slot nobody reads any more.
    // A tile's rows are addressed as a wave-uniform base (A + m0 lda, W + n0 ldw: scalar
    // registers) plus a per-lane 32-bit offset -- the scalar-base form of global_load_lds, so a
    // load costs no 64-bit vector address arithmetic.  Rows past M (N) are clamped to the last
    // row; the tile's stores skip them.
    // With the gate, column n of the GEMM (W row) is stored row wrow(n): within each 128-column
    // block, 64 gate rows and then the same 64 columns' up rows, N / 2 rows further on.
    const int half_n = N >> 1;
    auto wrow = [&](int n) { return GATED ? ((n & 127) >> 6) * half_n + ((n >> 7) << 6) + (n & 63) : n; };
    const uint8_t *ba = nullptr, *bw = nullptr;       // current tile
    const uint8_t *nba = nullptr, *nbw = nullptr;     // next tile
    uint32_t oa[LOADS], ow[LOADS];                    // current tile's lane offsets
    int32_t doa[LOADS] = {}, dow[LOADS] = {};         // next tile's offsets minus the current ones
    auto point_at = [&](int tv, int buf, const uint8_t *&pa, const uint8_t *&pw, uint32_t (&qa)[LOADS],
                        uint32_t (&qw)[LOADS]) {
        int m0, n0;
        tile_coords(tv, nbm, nbn, m0, n0);
        pa = A + (int64_t)m0 * lda;
        pw = GATED ? W : W + (int64_t)n0 * ldw;   // gated: offsets from the weight's first row
#pragma unroll
        for (int j = 0; j < LOADS; j++) {
            const int b = j * (NTHREADS / 64) + wave;
            const int r = 8 * b + (lane >> 3);
            const int c = (lane & 7) ^ chunk_xor(r);
            qa[j] = (uint32_t)(min(r, M - 1 - m0) * lda + c * 16);
            if constexpr (GATED) qw[j] = (uint32_t)wrow(n0 + min(r, N - 1 - n0)) * (uint32_t)ldw + (uint32_t)(c * 16);
            else qw[j] = (uint32_t)(min(r, N - 1 - n0) * ldw + c * 16);
        }
        if constexpr (SCALED) {
            // the tile's row scales, column scales and bias words: 64 entries of each per wave
            lds_ptr dst = (lds_ptr)(scale_lds + buf * SCALE_WORDS + 64 * wave);
            const int m = min(m0 + 64 * wave + lane, M - 1), n = wrow(min(n0 + 64 * wave + lane, N - 1));
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
    // where stage s of the current tile's sequence comes from (see above)
    auto source = [&](int s, bool &same, int64_t &koff) {
        same = s < nk || !has_next;
        koff = (int64_t)(s < nk ? s : (has_next ? s - nk : nk - 1)) * BK;
    };
    // ring load q of a stage (q < LOADS: A block q, else W block q - LOADS), from the current tile
    // (same) or the next one, at byte offset koff along K, into ring slot `slot`.  The next tile's
    // lane offset is the current one plus a masked delta (a select between two offset arrays is
    // turned into a load from a selected address, which sends both arrays to scratch memory).
    auto issue_one = [&](int slot, bool same, int64_t koff, int q) {
        const int j = q % LOADS, b = j * (NTHREADS / 64) + wave;
        lds_ptr d = (lds_ptr)(smem + (q < LOADS ? 0 : NSTAGE * STAGE_BYTES) + slot * STAGE_BYTES + 1024 * b);
        const int32_t mask = same ? 0 : -1;
        const uint8_t *base = (q < LOADS ? (same ? ba : nba) : (same ? bw : nbw)) + koff;
        const uint32_t off = q < LOADS ? oa[j] + (uint32_t)(doa[j] & mask) : ow[j] + (uint32_t)(dow[j] & mask);
        __builtin_amdgcn_global_load_lds((glb_ptr)(base + off), d, 16, 0, 0);
    };

    // the same with the slot and load index known at compile time and the load from the current
    // tile: the scalar base plus the lane's offset, no select
    // (buffer form: the tile's operand base in a descriptor, the k offset as the scalar offset and
    // the lane's row offset as the vector offset -- no address arithmetic per load)
    __amdgpu_buffer_rsrc_t rsa, rsw;
    auto set_rsrc = [&] {
        rsa = raw_rsrc(ba);
        rsw = raw_rsrc(bw);
    };
    auto issue_fast = [&](auto slotc, int64_t koff, auto qc) {
        constexpr int slot = decltype(slotc)::value, q = decltype(qc)::value, j = q % LOADS;
        const int b = j * (NTHREADS / 64) + wave;
        lds_ptr d = (lds_ptr)(smem + (q < LOADS ? 0 : NSTAGE * STAGE_BYTES) + slot * STAGE_BYTES + 1024 * b);
        if constexpr (q < LOADS) buffer_load_lds16(rsa, d, oa[j], (int)koff);
        else buffer_load_lds16(rsw, d, ow[j], (int)koff);
    };

    // MFMA operand layout (32 x 32 tiles): lane holds row (lane & 31) of W / of A and the k-slice
    // (lane >> 5) of the instruction's K; both operands use the same slice, so the dot products are
    // complete whatever order the hardware sums a slice in.
    const int frow = lane & 31, fk = lane >> 5;
    // fragment q of k-step ks of the stage in `slot`: q < TM is A fragment q, else W fragment q - TM
    auto read_frag = [&](int slot, int ks, int q, FT (&fa)[TM], FT (&fw)[TN]) {
        const uint8_t *base = smem + (q < TM ? 0 : NSTAGE * STAGE_BYTES) + slot * STAGE_BYTES;
        const int r = (q < TM ? wm * WAVE_M + q * 32 : wn * WAVE_N + (q - TM) * 32) + frow;
        if constexpr (FP8) {
            // the lane's 32 bytes are chunks 4 ks + 2 fk and + 1: two 16-byte reads (a 32-byte
            // read also makes the compiler wait for every global->LDS load in flight)
            const v4i lo = *(const v4i *)(base + swz(r, 4 * ks + 2 * fk));
            const v4i hi = *(const v4i *)(base + swz(r, 4 * ks + 2 * fk + 1));
            const v8i f = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if (q < TM) fa[q] = f;
            else fw[q - TM] = f;
        } else {
            const v4i f = *(const v4i *)(base + swz(r, 2 * ks + fk));
            if (q < TM) fa[q] = f;
            else fw[q - TM] = f;
        }
    };
    // Fragment reads with the slot known at compile time: the lane's swizzled byte offset depends
    // only on the operand, the k-step and the read half (fp8), so 2 x KS x NH offsets per lane
    // (set per tile, dead during the epilogue) cover every read; the slot and the fragment's
    // 32-row block are immediates of the ds_read.
    constexpr int KSC = BK / Frag<FP8>::KSTEP, NHC = FP8 ? 2 : 1;
    uint32_t lof[2][KSC][NHC];
    auto set_lof = [&] {
#pragma unroll
        for (int o = 0; o < 2; o++)
#pragma unroll
            for (int ks = 0; ks < KSC; ks++)
#pragma unroll
                for (int hh = 0; hh < NHC; hh++) {
                    const int c = FP8 ? 4 * ks + 2 * fk + hh : 2 * ks + fk;
                    lof[o][ks][hh] = (uint32_t)((o ? NSTAGE * STAGE_BYTES + wn * WAVE_N * BK : wm * WAVE_M * BK) +
                                                frow * BK + ((c ^ chunk_xor(frow)) << 4));
                }
    };
    auto read_frag_c = [&](auto slotc, auto ksc, auto qc, FT (&fa)[TM], FT (&fw)[TN]) {
        constexpr int slot = decltype(slotc)::value, ks = decltype(ksc)::value, q = decltype(qc)::value;
        constexpr int o = q < TM ? 0 : 1, ql = q < TM ? q : q - TM;
        constexpr uint32_t imm = slot * STAGE_BYTES + ql * 32 * BK;
        if constexpr (FP8) {
            const v4i lo = *(const v4i *)(smem + lof[o][ks][0] + imm);
            const v4i hi = *(const v4i *)(smem + lof[o][ks][1] + imm);
            const v8i f = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            if constexpr (q < TM) fa[q] = f;
            else fw[q - TM] = f;
        } else {
            const v4i f = *(const v4i *)(smem + lof[o][ks][0] + imm);
            if constexpr (q < TM) fa[q] = f;
            else fw[q - TM] = f;
        }
    };
    // acc[i][j] is the transposed 32 x 32 tile: W rows (output columns) x A rows (output rows).
    Acc acc[TM][TN];
    auto mfma = [&](int i, int j, const FT (&fa)[TM], const FT (&fw)[TN]) {
        if constexpr (FP8)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw[j], fa[i], acc[i][j], WF, 0, 0, 127, 0, 127);
        else
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], acc[i][j], 0, 0, 0);
    };
    // the same with a zero accumulator input (inline constant 0): a tile's first k-step, so the
    // 256 accumulator registers need no clearing writes before the tile
    auto mfma_first = [&](int i, int j, const FT (&fa)[TM], const FT (&fw)[TN]) {
        if constexpr (FP8)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fw[j], fa[i], Acc{}, WF, 0, 0, 127, 0, 127);
        else
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[j], fa[i], Acc{}, 0, 0, 0);
    };
    // Reads in the order the MFMAs (row-major over i, j) first need them: A0, W0..W3, A1..A3.
    constexpr int kReadOrder[TM + TN] = {0, 4, 5, 6, 7, 1, 2, 3};

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
        if constexpr (GATED) {
            // The wave's 128 GEMM columns are 64 gate columns (acc[i][0..1]) and their up columns
            // (acc[i][2..3]): register 4 g + c of acc[i][jj] and of acc[i][jj + 2] is output column
            // ob + 32 jj + 8 g + 4 (l >> 5) + c, ob = (n0 + 128 wn) / 2.  N is a multiple of 128,
            // so a wave's block is whole or past N.
            const int nb = n0 + wn * WAVE_N;
            if (nb >= N) return;
            const int ob = nb >> 1;
            if constexpr (OUT == OUT_BF16 || OUT == OUT_F16) {
                if (ep.vec) {
                    // one 32 x 64 block per row block i, staged through LDS as in the ungated
                    // epilogue below: whole-line stores
                    uint8_t *const eb = smem + kEpiOffset + wave * EPI_WAVE_BYTES;
                    const int h = lane >> 5;
                    // the operand words of column group (jj, pr) (scales and bias words of columns
                    // nc, nc + 8 of the gate and nc + 64, nc + 72 of the up half), read one group
                    // ahead so that their LDS latency overlaps the current group's conversion
                    auto graw = [&](int g, v4i (&w)[8]) {
                        const int nc = 32 * ((g >> 1) & 1) + 16 * (g & 1);
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int off = nc + 8 * (q & 1) + 64 * (q >> 1);
                            w[q] = *(const v4i *)(sc + BM + nl0 + off);
                            w[4 + q] = *(const v4i *)(sc + BM + BN + nl0 + off);
                        }
                    };
                    auto gconv = [&](const v4i (&w)[8], float (&ws)[4][4], float (&bs)[4][4]) {
#pragma unroll
                        for (int q = 0; q < 4; q++)
#pragma unroll
                            for (int c = 0; c < 4; c++) ws[q][c] = __int_as_float(w[q][c]);
                        if (!ep.bias) {
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int c = 0; c < 4; c++) bs[q][c] = 0.0f;
                        } else if (ep.bias_dtype == PSQ_BF16) {
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int c = 0; c < 4; c++) bs[q][c] = __uint_as_float((uint32_t)w[4 + q][c] << 16);
                        } else if (ep.bias_dtype == PSQ_F16) {
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int c = 0; c < 4; c++) bs[q][c] = f16_to_f32((uint32_t)w[4 + q][c]);
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int c = 0; c < 4; c++) bs[q][c] = __int_as_float(w[4 + q][c]);
                        }
                    };
                    v4i graw_buf[2][8];
                    graw(0, graw_buf[0]);
#pragma unroll
                    for (int i = 0; i < TM; i++) {
#pragma unroll
                        for (int jj = 0; jj < 2; jj++)
#pragma unroll
                            for (int pr = 0; pr < 2; pr++) {
                                const int g = 4 * i + 2 * jj + pr;
                                float ws4[4][4], bs4[4][4];
                                gconv(graw_buf[g & 1], ws4, bs4);
                                if (g + 1 < 4 * TM) graw(g + 1, graw_buf[(g + 1) & 1]);
                                float (&wg)[2][4] = *reinterpret_cast<float (*)[2][4]>(&ws4[0]);
                                float (&bg)[2][4] = *reinterpret_cast<float (*)[2][4]>(&bs4[0]);
                                float (&wu)[2][4] = *reinterpret_cast<float (*)[2][4]>(&ws4[2]);
                                float (&bu)[2][4] = *reinterpret_cast<float (*)[2][4]>(&bs4[2]);
                                uint32_t x[2], y[2];
#pragma unroll
                                for (int hh = 0; hh < 2; hh++) {
                                    uint32_t *o = hh == 0 ? x : y;
                                    const int r = 8 * pr + 4 * hh;
#pragma unroll
                                    for (int e = 0; e < 2; e++)
                                        o[e] = pack2g<OUT>(value(i, jj, r + 2 * e, wg[hh][2 * e], bg[hh][2 * e]),
                                                           value(i, jj + 2, r + 2 * e, wu[hh][2 * e], bu[hh][2 * e]),
                                                           value(i, jj, r + 2 * e + 1, wg[hh][2 * e + 1], bg[hh][2 * e + 1]),
                                                           value(i, jj + 2, r + 2 * e + 1, wu[hh][2 * e + 1], bu[hh][2 * e + 1]));
                                }
                                uint32_t lo[2], hi[2];
#pragma unroll
                                for (int d = 0; d < 2; d++) {
                                    const auto sw = __builtin_amdgcn_permlane32_swap(x[d], y[d], false, false);
                                    lo[d] = sw[0];
                                    hi[d] = sw[1];
                                }
                                const int ch = 4 * jj + 2 * pr + h;
                                *(v4i *)(eb + frow * 128 + ((ch ^ chunk_xor(frow)) << 4)) =
                                    v4i{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
                                __builtin_amdgcn_sched_barrier(0);
                            }
                        v4i val[4];
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int row = 8 * q + (lane >> 3), ch = lane & 7;
                            val[q] = *(const v4i *)(eb + row * 128 + ((ch ^ chunk_xor(row)) << 4));
                        }
                        const int mb = m0 + wm * WAVE_M + 32 * i;
                        const int64_t ubase = ((int64_t)mb * ep.ldy + ob) * 2;
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int row = 8 * q + (lane >> 3);
                            if (mb + row < M) {
                                const uint32_t loff = (uint32_t)((row * ep.ldy + 8 * (lane & 7)) * 2);
                                v4i *dst = (v4i *)((uint8_t *)ep.y + ubase + loff);
                                __builtin_nontemporal_store(val[q], dst);
                            }
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    return;
                }
            }
            // fp32 outputs and unaligned rows: element stores
#pragma unroll
            for (int jj = 0; jj < 2; jj++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int nc = 32 * jj + 8 * g;
                    float wg[4], bg[4], wu[4], bu[4];
                    operands(nc, wg, bg);
                    operands(nc + 64, wu, bu);
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        if (!live[i]) continue;
                        const int m = m0 + wm * WAVE_M + 32 * i + frow;
                        void *p = (uint8_t *)ep.y + ((int64_t)m * ep.ldy + ob + nc + 4 * (lane >> 5)) * esz;
#pragma unroll
                        for (int c = 0; c < 4; c++)
                            store1<OUT>(p, c, gate1<OUT>(value(i, jj, 4 * g + c, wg[c], bg[c]),
                                                         value(i, jj + 2, 4 * g + c, wu[c], bu[c])));
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            return;
        }
        if constexpr (OUT == OUT_BF16 || OUT == OUT_F16) {
            if (ep.vec && n0 + BN <= N) {
                // Full-width tile, aligned rows, 16-bit outputs: the wave's 128 x 128 block leaves
                // in blocks of 32 rows x 64 columns through its private 4 KB LDS buffer (chunk
                // swizzle as in the ring), so each store writes 8 rows x 128 bytes -- whole cache
                // lines -- where a store straight from the registers writes 32 rows x 32 bytes.
                // Within a block the lane pair (l, l + 32) first merges its column groups with one
                // v_permlane32_swap per word (as in the direct path below).  LDS accesses of a
                // wave execute in order, so the buffer needs no barrier.
                uint8_t *const eb = smem + kEpiOffset + wave * EPI_WAVE_BYTES;
                const int h = lane >> 5;
                // The half's column operands are read once for all four row blocks (fp8 too: at
                // M=32760, N=15360, K=5120 that leaves two VGPRs to scratch in the epilogue, and
                // still runs 4% faster than reading the operands per row block).
#pragma unroll
                for (int hj = 0; hj < 2; hj++) {
                    float hws[2][2][2][4], hbs[2][2][2][4];
#pragma unroll
                    for (int jj = 0; jj < 2; jj++)
#pragma unroll
                        for (int pr = 0; pr < 2; pr++) {
                            const int nc = 32 * (2 * hj + jj) + 16 * pr;
                            operands(nc, hws[jj][pr][0], hbs[jj][pr][0]);
                            operands(nc + 8, hws[jj][pr][1], hbs[jj][pr][1]);
                        }
#pragma unroll
                    for (int i = 0; i < TM; i++) {
#pragma unroll
                        for (int jj = 0; jj < 2; jj++)
#pragma unroll
                            for (int pr = 0; pr < 2; pr++) {
                                const int j = 2 * hj + jj;
                                const float (&ws)[2][4] = hws[jj][pr];
                                const float (&bs)[2][4] = hbs[jj][pr];
                                uint32_t x[2], y[2];
#pragma unroll
                                for (int hh = 0; hh < 2; hh++) {
                                    uint32_t *o = hh == 0 ? x : y;
                                    const int r = 8 * pr + 4 * hh;
                                    o[0] = pack2a<OUT, ACT>(value(i, j, r, ws[hh][0], bs[hh][0]), value(i, j, r + 1, ws[hh][1], bs[hh][1]));
                                    o[1] = pack2a<OUT, ACT>(value(i, j, r + 2, ws[hh][2], bs[hh][2]), value(i, j, r + 3, ws[hh][3], bs[hh][3]));
                                }
                                uint32_t lo[2], hi[2];
#pragma unroll
                                for (int d = 0; d < 2; d++) {
                                    const auto sw = __builtin_amdgcn_permlane32_swap(x[d], y[d], false, false);
                                    lo[d] = sw[0];
                                    hi[d] = sw[1];
                                }
                                // lane h now holds columns 32 jj + 16 pr + 8 h .. + 7 of the block
                                const int ch = 4 * jj + 2 * pr + h;
                                *(v4i *)(eb + frow * 128 + ((ch ^ chunk_xor(frow)) << 4)) =
                                    v4i{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
                            }
                        // all four reads first (one LDS round trip), then the stores; a block of
                        // whole rows stores without per-row tests from a wave-uniform base plus a
                        // 32-bit lane offset
                        v4i val[4];
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const int row = 8 * q + (lane >> 3), ch = lane & 7;
                            val[q] = *(const v4i *)(eb + row * 128 + ((ch ^ chunk_xor(row)) << 4));
                        }
                        const int mb = m0 + wm * WAVE_M + 32 * i;   // first row of the block
                        const int64_t ubase = ((int64_t)mb * ep.ldy + n0 + wn * WAVE_N + 64 * hj) * 2;
                        if (mb + 32 <= M) {
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                const uint32_t loff = (uint32_t)(((8 * q + (lane >> 3)) * ep.ldy + 8 * (lane & 7)) * 2);
                                v4i *dst = (v4i *)((uint8_t *)ep.y + ubase + loff);
                                __builtin_nontemporal_store(val[q], dst);
                            }
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                const int row = 8 * q + (lane >> 3);
                                if (mb + row < M) {
                                    const uint32_t loff = (uint32_t)((row * ep.ldy + 8 * (lane & 7)) * 2);
                                    v4i *dst = (v4i *)((uint8_t *)ep.y + ubase + loff);
                                    __builtin_nontemporal_store(val[q], dst);
                                }
                            }
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                return;
            }
        }
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
                                for (int c = 0; c < 4; c++) o[c] = __float_as_uint(act1<OUT, ACT>(value(i, j, r + c, ws[h][c], bs[h][c])));
                            } else {
                                o[0] = pack2a<OUT, ACT>(value(i, j, r, ws[h][0], bs[h][0]), value(i, j, r + 1, ws[h][1], bs[h][1]));
                                o[1] = pack2a<OUT, ACT>(value(i, j, r + 2, ws[h][2], bs[h][2]), value(i, j, r + 3, ws[h][3], bs[h][3]));
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
                            else store1<OUT>(p, c, act1<OUT, ACT>(value(i, j, 4 * g + c, ws[c], bs[c])));
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
    };

    // ---------------------------------------------------------------- main loop
    // Ring slot rs holds stage kt, slot rs ^ 1 stage kt + 1 (landed at the barrier before the last
    // k-step of stage kt) and then stage kt + 2, whose loads start after that barrier: every wave
    // has read its last fragments of stage kt by then.
    // Prologue: stage 0 and (the A half of) stage 1 in flight, stage 0 landed, its first fragments.
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
    int rs = 0;                      // ring slot of the stage being computed
    int buf = 0;                     // epilogue-operand buffer of the tile being computed
#pragma unroll
    for (int q = 0; q < TM + TN; q++) read_frag(0, 0, q, fa0, fw0);

    // One k-step: the 16 MFMAs of k-step t on (ca, cw); behind MFMAs 0-7 the fragment reads of
    // the next k-step into (na, nw) (after the last k-step: k-step 0 of the next stage, from the
    // other slot); the ring loads dma_slot places.
    // The instruction order is fixed explicitly (sched_barrier after every MFMA): with one wave per
    // SIMD every issue slot not spent on an MFMA idles the matrix core.
    auto kstep = [&](auto tc, FT (&ca)[TM], FT (&cw)[TN], FT (&na)[TM], FT (&nw)[TN], bool s1, int64_t k1,
                     bool s2, int64_t k2) {
        constexpr int t = decltype(tc)::value;
        constexpr bool last = t == KS - 1;
        static_for<TM * TN>([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            mfma(p / TN, p % TN, ca, cw);
            if constexpr (p < TM + TN) read_frag(last ? rs ^ 1 : rs, last ? 0 : t + 1, kReadOrder[p], na, nw);
            constexpr int d = dma_slot<FP8>(t, p);
            if constexpr (d >= 0) {
                if constexpr (last) issue_one(rs, s2, k2, d);
                else issue_one(rs ^ 1, s1, k1, d);
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    // k-step / stage of the steady state: stage kt + 2 still in the current tile, ring slot SL
    // known at compile time
    auto kstep_fast = [&](auto tc, auto slc, FT (&ca)[TM], FT (&cw)[TN], FT (&na)[TM], FT (&nw)[TN], int64_t k1,
                          int64_t k2, auto firstc) {
        constexpr int t = decltype(tc)::value, SL = decltype(slc)::value;
        constexpr bool last = t == KS - 1;
        static_for<TM * TN>([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            if constexpr (decltype(firstc)::value) mfma_first(p / TN, p % TN, ca, cw);
            else mfma(p / TN, p % TN, ca, cw);
            if constexpr (p < TM + TN)
                read_frag_c(std::integral_constant<int, last ? (SL ^ 1) : SL>{},
                            std::integral_constant<int, last ? 0 : t + 1>{},
                            std::integral_constant<int, kReadOrder[p]>{}, na, nw);
            constexpr int d = dma_slot<FP8>(t, p);
            if constexpr (d >= 0) {
                if constexpr (last) issue_fast(std::integral_constant<int, SL>{}, k2, std::integral_constant<int, d>{});
                else issue_fast(std::integral_constant<int, SL ^ 1>{}, k1, std::integral_constant<int, d>{});
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    // firstc: the tile's first stage (its first k-step starts the accumulators from zero)
    auto stage_fast = [&](auto slc, int kt, auto firstc) {
        const int64_t k1 = (int64_t)(kt + 1) * BK, k2 = (int64_t)(kt + 2) * BK;
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using NO = std::false_type;
        if constexpr (!FP8) {
            kstep_fast(I0{}, slc, fa0, fw0, fa1, fw1, k1, k2, firstc);
            kstep_fast(I1{}, slc, fa1, fw1, fa0, fw0, k1, k2, NO{});
            kstep_fast(std::integral_constant<int, 2>{}, slc, fa0, fw0, fa1, fw1, k1, k2, NO{});
            wait_vmcnt<0>();
            stage_barrier();
            kstep_fast(std::integral_constant<int, 3>{}, slc, fa1, fw1, fa0, fw0, k1, k2, NO{});
        } else {
            kstep_fast(I0{}, slc, fa0, fw0, fa1, fw1, k1, k2, firstc);
            wait_vmcnt<0>();
            stage_barrier();
            kstep_fast(I1{}, slc, fa1, fw1, fa0, fw0, k1, k2, NO{});
        }
    };
    auto stage = [&](int kt) {
        bool s1, s2;
        int64_t k1, k2;
        source(kt + 1, s1, k1);
        source(kt + 2, s2, k2);
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        if constexpr (!FP8) {
            kstep(I0{}, fa0, fw0, fa1, fw1, s1, k1, s2, k2);
            kstep(I1{}, fa1, fw1, fa0, fw0, s1, k1, s2, k2);
            kstep(std::integral_constant<int, 2>{}, fa0, fw0, fa1, fw1, s1, k1, s2, k2);
            // stage kt + 1 landed for every wave; nobody reads stage kt's slot any more
            wait_vmcnt<0>();
            stage_barrier();
            kstep(std::integral_constant<int, 3>{}, fa1, fw1, fa0, fw0, s1, k1, s2, k2);
        } else {
            kstep(I0{}, fa0, fw0, fa1, fw1, s1, k1, s2, k2);
            wait_vmcnt<0>();
            stage_barrier();
            kstep(I1{}, fa1, fw1, fa0, fw0, s1, k1, s2, k2);
        }
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
        // an even stage count brings the ring back to slot 0 at every tile start: the steady state
        // runs in pairs of stages with compile-time slots, the last two the general way.  int8:
        // the first pair starts the accumulators from zero (c1 GEMM 1.789 -> 1.775 ms); fp8 clears
        // them (its first-pair copy measured 0.9% slower at c3)
        auto clear_acc = [&] {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
        };
        int kt0 = 0;
        if constexpr (!FP8) {
            if ((nk & 1) == 0 && nk >= 4) {
                set_lof();
                set_rsrc();
                stage_fast(std::integral_constant<int, 0>{}, 0, std::true_type{});
                stage_fast(std::integral_constant<int, 1>{}, 1, std::false_type{});
#pragma clang loop unroll(disable)
                for (kt0 = 2; kt0 + 3 < nk; kt0 += 2) {
                    stage_fast(std::integral_constant<int, 0>{}, kt0, std::false_type{});
                    stage_fast(std::integral_constant<int, 1>{}, kt0 + 1, std::false_type{});
                }
            } else {
                clear_acc();
            }
        } else {
            clear_acc();
            if ((nk & 1) == 0) {
                set_lof();
                set_rsrc();
#pragma clang loop unroll(disable)
                for (; kt0 + 3 < nk; kt0 += 2) {
                    stage_fast(std::integral_constant<int, 0>{}, kt0, std::false_type{});
                    stage_fast(std::integral_constant<int, 1>{}, kt0 + 1, std::false_type{});
                }
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
    // the re-issued loads past the last tile must land before the workgroup's LDS is released
    wait_vmcnt<0>();
}

template <bool FP8, int OUT, int ACT, int WF = 0>
int launch_one(const uint8_t *a, int64_t lda, const uint8_t *w, int64_t ldw, int64_t M, int64_t N, int64_t K,
               const Epi &ep, hipStream_t st, const char *name)
{
    auto kern = gemm_q8_kernel<FP8, OUT, ACT, WF>;
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
    const bool short_k = K / BK < NSTAGE;
    const int64_t grid = (short_k || tiles < cu_count(dev)) ? tiles : cu_count(dev);
    kern<<<dim3((unsigned)grid), dim3(NTHREADS), kSmemBytes, st>>>(a, lda, w, ldw, (int)M, (int)N, (int)K, ep);
    return check_launch(name);
}

template <bool FP8>
int launch(int out, int act, const uint8_t *a, int64_t lda, const uint8_t *w, int64_t ldw, int64_t M, int64_t N,
           int64_t K, const Epi &ep, hipStream_t st, const char *name)
{
    if (act == ACT_SILU_GATE) {
        switch (out) {
        case OUT_BF16: return launch_one<FP8, OUT_BF16, ACT_SILU_GATE>(a, lda, w, ldw, M, N, K, ep, st, name);
        case OUT_F16: return launch_one<FP8, OUT_F16, ACT_SILU_GATE>(a, lda, w, ldw, M, N, K, ep, st, name);
        default: return launch_one<FP8, OUT_F32, ACT_SILU_GATE>(a, lda, w, ldw, M, N, K, ep, st, name);
        }
    }
    if (act == ACT_GELU_TANH) {
        switch (out) {
        case OUT_BF16: return launch_one<FP8, OUT_BF16, ACT_GELU_TANH>(a, lda, w, ldw, M, N, K, ep, st, name);
        case OUT_F16: return launch_one<FP8, OUT_F16, ACT_GELU_TANH>(a, lda, w, ldw, M, N, K, ep, st, name);
        default: return launch_one<FP8, OUT_F32, ACT_GELU_TANH>(a, lda, w, ldw, M, N, K, ep, st, name);
        }
    }
    switch (out) {
    case OUT_BF16: return launch_one<FP8, OUT_BF16, ACT_NONE>(a, lda, w, ldw, M, N, K, ep, st, name);
    case OUT_F16: return launch_one<FP8, OUT_F16, ACT_NONE>(a, lda, w, ldw, M, N, K, ep, st, name);
    case OUT_F32: return launch_one<FP8, OUT_F32, ACT_NONE>(a, lda, w, ldw, M, N, K, ep, st, name);
    default: return launch_one<FP8, OUT_I32, ACT_NONE>(a, lda, w, ldw, M, N, K, ep, st, name);
    }
}

// Vector stores need 16-byte-aligned rows; the staged stores also address a 32-row block with a
// 32-bit lane offset, which holds for ldy < 2^26.  Other outputs take the element-store path.
int vec_ok(const void *y, int64_t ldy, int elem)
{
    return (((uintptr_t)y & 15) == 0 && (ldy * elem) % 16 == 0 && ldy < (1LL << 26)) ? 1 : 0;
}

int check_shapes(const char *name, const void *a, int64_t lda, const void *w, int64_t ldw, int64_t M, int64_t N,
                 int64_t K)
{
    if (M < 0 || N < 0 || K < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    // an empty problem reads nothing: empty tensors may come with null data pointers
    if (M > 0 && N > 0 && (!a || !w)) return set_error(PSQ_E_ARG, "%s: null operand", name);
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

// Activation codes, and the gate's shape rules: N = 2 H rows with H a multiple of 64, an output of
// H columns, and every W row offset (row ldw, 32-bit lane offsets from the weight's first row)
// plus the k offset below 2^32.
int check_act(const char *name, int activation, int64_t N, int64_t ldw, int64_t K, int64_t ldy)
{
    if (activation != ACT_NONE && activation != ACT_GELU_TANH && activation != ACT_SILU_GATE)
        return set_error(PSQ_E_ARG, "%s: bad activation %d", name, activation);
    if (activation == ACT_SILU_GATE) {
        if (N % 128) return set_error(PSQ_E_SHAPE, "%s: the SiLU gate needs N a multiple of 128, got %lld", name, (long long)N);
        if (N * ldw + K >= (1LL << 32)) return set_error(PSQ_E_SHAPE, "%s: the SiLU gate needs N ldw + K < 2^32", name);
        if (ldy < N / 2) return set_error(PSQ_E_SHAPE, "%s: ldy < N / 2", name);
    } else if (ldy < N) {
        return set_error(PSQ_E_SHAPE, "%s: ldy < N", name);
    }
    return PSQ_OK;
}

}  // namespace
}  // namespace psq

extern "C" {

int psq_gemm_i8_act(const int8_t *a, int64_t lda, const float *a_scale, const int8_t *w, int64_t ldw,
                    const float *w_scale, const void *bias, int bias_dtype, int activation, void *y, int y_dtype,
                    int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_shapes("gemm_i8", a, lda, w, ldw, M, N, K)) return e;
    if (int e = check_act("gemm_i8", activation, N, ldw, K, ldy)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!a_scale || !w_scale || !y) return set_error(PSQ_E_ARG, "gemm_i8: null scale or output");
    if (!valid_dtype(y_dtype) || (bias && !valid_dtype(bias_dtype))) return set_error(PSQ_E_ARG, "gemm_i8: bad dtype");
    if (int e = require_device()) return e;
    Epi ep{a_scale, w_scale, 1, bias, bias_dtype, y, ldy, vec_ok(y, ldy, y_dtype == PSQ_F32 ? 4 : 2)};
    return launch<false>(y_dtype, activation, (const uint8_t *)a, lda, (const uint8_t *)w, ldw, M, N, K, ep,
                         (hipStream_t)stream, "gemm_i8");
}

int psq_gemm_i8(const int8_t *a, int64_t lda, const float *a_scale, const int8_t *w, int64_t ldw,
                const float *w_scale, const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy,
                int64_t M, int64_t N, int64_t K, void *stream)
{
    return psq_gemm_i8_act(a, lda, a_scale, w, ldw, w_scale, bias, bias_dtype, PSQ_ACT_NONE, y, y_dtype, ldy, M, N,
                           K, stream);
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
    return launch<false>(OUT_I32, ACT_NONE, (const uint8_t *)a, lda, (const uint8_t *)w, ldw, M, N, K, ep,
                         (hipStream_t)stream, "gemm_i8_i32");
}

int psq_gemm_fp8_act(const uint8_t *a, int64_t lda, const float *a_scale, const uint8_t *w, int64_t ldw,
                     const float *w_scale, int w_scale_per_row, const void *bias, int bias_dtype, int activation,
                     void *y, int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_shapes("gemm_fp8", a, lda, w, ldw, M, N, K)) return e;
    if (int e = check_act("gemm_fp8", activation, N, ldw, K, ldy)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!a_scale || !w_scale || !y) return set_error(PSQ_E_ARG, "gemm_fp8: null scale or output");
    if (!valid_dtype(y_dtype) || (bias && !valid_dtype(bias_dtype))) return set_error(PSQ_E_ARG, "gemm_fp8: bad dtype");
    if (int e = require_device()) return e;
    Epi ep{a_scale, w_scale, w_scale_per_row ? 1 : 0, bias, bias_dtype, y, ldy, vec_ok(y, ldy, y_dtype == PSQ_F32 ? 4 : 2)};
    return launch<true>(y_dtype, activation, a, lda, w, ldw, M, N, K, ep, (hipStream_t)stream, "gemm_fp8");
}

int psq_gemm_fp8(const uint8_t *a, int64_t lda, const float *a_scale, const uint8_t *w, int64_t ldw,
                 const float *w_scale, int w_scale_per_row, const void *bias, int bias_dtype, void *y, int y_dtype,
                 int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    return psq_gemm_fp8_act(a, lda, a_scale, w, ldw, w_scale, w_scale_per_row, bias, bias_dtype, PSQ_ACT_NONE, y,
                            y_dtype, ldy, M, N, K, stream);
}

int psq_gemm_fp8_e5m2w(const uint8_t *a, int64_t lda, const float *a_scale, const uint8_t *w, int64_t ldw,
                       const float *w_scale, int w_scale_per_row, const void *bias, int bias_dtype, void *y,
                       int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (int e = check_shapes("gemm_fp8_e5m2w", a, lda, w, ldw, M, N, K)) return e;
    if (int e = check_act("gemm_fp8_e5m2w", PSQ_ACT_NONE, N, ldw, K, ldy)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!a_scale || !w_scale || !y) return set_error(PSQ_E_ARG, "gemm_fp8_e5m2w: null scale or output");
    if (!valid_dtype(y_dtype) || (bias && !valid_dtype(bias_dtype)))
        return set_error(PSQ_E_ARG, "gemm_fp8_e5m2w: bad dtype");
    if (int e = require_device()) return e;
    Epi ep{a_scale, w_scale, w_scale_per_row ? 1 : 0, bias, bias_dtype, y, ldy, vec_ok(y, ldy, y_dtype == PSQ_F32 ? 4 : 2)};
    hipStream_t st = (hipStream_t)stream;
    const char *name = "gemm_fp8_e5m2w";
    switch (y_dtype) {
    case OUT_BF16: return launch_one<true, OUT_BF16, ACT_NONE, 1>(a, lda, w, ldw, M, N, K, ep, st, name);
    case OUT_F16: return launch_one<true, OUT_F16, ACT_NONE, 1>(a, lda, w, ldw, M, N, K, ep, st, name);
    default: return launch_one<true, OUT_F32, ACT_NONE, 1>(a, lda, w, ldw, M, N, K, ep, st, name);
    }
}

}  // extern "C"
