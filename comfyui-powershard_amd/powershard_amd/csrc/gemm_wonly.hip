// gemm_wonly.hip -- weight-only quantized GEMMs: uint4 asymmetric groups (W4A16) and int8 rows
// (W8A16), dequantized in registers and fed to the bf16 / f16 MFMA.
//
// W4A16 reproduces the dequantize branch of QuantLinear.forward,
//   F.linear(rows, qt.dequantize().to(bf16), bias)   (powershard/quant_linear.py:219-220),
// without materializing the weight: w = round_bf16((float(q) - float(z)) * float(s)),
// y = round_out(acc + bias) with fp32 accumulation.
// W8A16: int8 values are exact in bf16, the per-row scale is applied in the epilogue,
// y = round_out(fmaf(acc, s[n], bias[n])) (Int8Linear storage, powershard/operations.py:96-132).
//
// Two kernels: a weight-streaming one for M <= 64 (decode / short prompts: HBM-bound) and a
// 256 x 256-tile one for larger M (MFMA-bound), both described where they are defined.
#include "psq_common.hpp"

#include <mutex>

namespace psq {
namespace {

constexpr int NTHREADS = 256;
constexpr int KSTAGE = 64;                     // K granularity of every path

enum { W_UINT4 = 0, W_INT8 = 1 };

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
    // stream-K of the tiled kernel (sk > 0): the (tile, K stage) units of all tiles, tile after
    // tile, are cut into sk equal contiguous ranges, one per workgroup; a workgroup whose range
    // holds part of a tile's stages writes its fp32 partial tile to `part`, and the last of the
    // tile's workgroups to finish adds the partials in K order and applies the epilogue
    int sk = 0;
    float *part = nullptr;      // [2 sk][BM][256] fp32: the first and the last partial of each workgroup
    uint32_t *cnt = nullptr;    // [tiles] finished workgroups per tile: zero at launch, left zero
};

template <int XDT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi)
{
    return pack_half2<XDT>(lo, hi);
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

// The four bytes of w as floats: v_cvt_f32_ubyte0..3, one instruction each (the compiler would
// otherwise extract each nibble-masked byte with a bitfield op first).
__device__ __forceinline__ void ubytes_to_f32(uint32_t w, float (&f)[4])
{
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f[0]) : "v"(w));
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f[1]) : "v"(w));
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f[2]) : "v"(w));
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f[3]) : "v"(w));
}

// uint4 dequantization without an int -> float step.  A nibble q alone in a 16-bit half is the
// fp16 subnormal q * 2^-24, and v_fma_mix_f32 takes an fp16 operand as is, so
//   fma_mix(q * 2^-24, s * 2^24, c) = fmaf(q, s, c)
// exactly: s * 2^24 is an exact fp32 scaling of the fp16 scale and the fma's product is exact
// (tests/test_parity_gpu.py::test_w4a16_dequantized_weights_exact checks every kernel's weights
// bit for bit against round_16(fmaf(q, s, -z s)), fp16-subnormal scales included).
// The eight nibbles of a word (nibble i = k offset i) are split into four such pairs with 5 ops:
// nibbles 0, 4 and (after one shift by 8) 2, 6 masked to the bottom of their halves, nibbles 1, 5
// and 3, 7 masked where they stand, four bits up: 16 q 2^-24, still an fp16 subnormal, taken with
// s 2^20 instead of s 2^24 (also exact).  With one fma_mix per weight and the packs: 17 VALU ops
// per 8 weights, against 19 with four shifted masks and 23 for v_cvt_f32_ubyte + v_fma_f32.
struct Nib4 { uint32_t a, b, c, d; };   // halves (lo, hi): a = k (0, 4), b = 16 (1, 5), c = (2, 6), d = 16 (3, 7)
__device__ __forceinline__ Nib4 nib_split(uint32_t p)
{
    const uint32_t t = p >> 8;
    return Nib4{p & 0x000f000fu, p & 0x00f000f0u, t & 0x000f000fu, t & 0x00f000f0u};
}
__device__ __forceinline__ float mix_lo(uint32_t h2, float s24, float c)
{
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s24), "v"(c));
    return r;
}
__device__ __forceinline__ float mix_hi(uint32_t h2, float s24, float c)
{
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(s24), "v"(c));
    return r;
}
// packed weights of k offsets 2e, 2e + 1: round_16(fmaf(q, s, c)) each, s24 = s * 2^24,
// s20 = s * 2^20
template <int XDT>
__device__ __forceinline__ uint32_t dq_pair_u4(const Nib4 &v, int e, float s24, float s20, float c)
{
    switch (e) {
    case 0: return pack_half2<XDT>(mix_lo(v.a, s24, c), mix_lo(v.b, s20, c));
    case 1: return pack_half2<XDT>(mix_lo(v.c, s24, c), mix_lo(v.d, s20, c));
    case 2: return pack_half2<XDT>(mix_hi(v.a, s24, c), mix_hi(v.b, s20, c));
    default: return pack_half2<XDT>(mix_hi(v.c, s24, c), mix_hi(v.d, s20, c));
    }
}
constexpr float kTwo24 = 16777216.0f, kTwo20 = 1048576.0f;

// Two int8 weights (bytes 2 hi and 2 hi + 1 of p) as an exact f16 pair without conversions: each
// byte, biased by 128, under the f16 exponent of 1024 (0x64bb = 1024 + bb) is 1152 + q, and one
// packed f16 subtraction of 1152 leaves q (integers below 2048 are exact in f16).  A v_perm_b32
// and a v_pk_add_f16 per pair, where the conversion takes two extracts, two conversions and a pack.
__device__ __forceinline__ uint32_t i8pair_f16(uint32_t p, int hi)
{
    const uint32_t h = __builtin_amdgcn_perm(0x64646464u, p ^ 0x80808080u, hi ? 0x04030402u : 0x04010400u);
    const f16x2_t q = __builtin_bit_cast(f16x2_t, h) - f16x2_t{(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, q);
}

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
    // Activation fragments of MT <= 2 row tiles ride in the same pipeline (they are L2 hits, but
    // their latency would otherwise be exposed once per block).
    constexpr bool XPRE = MT <= 2;
    struct WBlock { uint32_t w[NW]; float s, z; v4i x[XPRE ? 4 : 1][XPRE ? MT : 1]; };
    auto load_x = [&](int kb, v4i (&xv)[4][MT]) {
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) xv[t][mt] = *(const v4i *)(xrow[mt] + kb + 8 * t);
    };
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
        if constexpr (XPRE) load_x(kb, r.x);
    };
    auto compute = [&](int b, const WBlock &r) {
        const int kb = b * SK_BLOCK + 32 * h;        // the lane group's first k
        v4i xl[4][MT];
        if constexpr (!XPRE) load_x(kb, xl);
        auto xfrag = [&](int t, int mt) -> v4i {
            if constexpr (XPRE) return r.x[t][mt];
            else return xl[t][mt];
        };
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // weights of k = kb + 8t .. kb + 8t + 7
            uint32_t hw[4];
            if constexpr (WK == W_UINT4) {
                const uint32_t p = r.w[t];
                const uint32_t lo = p & 0x0f0f0f0fu, hi = (p >> 4) & 0x0f0f0f0fu;   // even / odd k
                float q0[4], q1[4];
                ubytes_to_f32(lo, q0);
                ubytes_to_f32(hi, q1);
#pragma unroll
                for (int e = 0; e < 4; e++) hw[e] = pack2<XDT>((q0[e] - r.z) * r.s, (q1[e] - r.z) * r.s);
            } else {
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t p = r.w[2 * t + e];
                    if constexpr (XDT == PSQ_F16) {
                        hw[2 * e] = i8pair_f16(p, 0);
                        hw[2 * e + 1] = i8pair_f16(p, 1);
                    } else {
                        hw[2 * e] = pack2<XDT>((float)(int8_t)(p & 0xffu), (float)(int8_t)((p >> 8) & 0xffu));
                        hw[2 * e + 1] = pack2<XDT>((float)(int8_t)((p >> 16) & 0xffu), (float)(int8_t)(p >> 24));
                    }
                }
            }
            const XV wf = __builtin_bit_cast(XV, v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]});
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const XV xf = __builtin_bit_cast(XV, xfrag(t, mt));
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

// ------------------------------------------------------------------ tiled kernel (M > 64)
// A BM x 256 output tile (BM = 256, or 128 when that fills more of the GPU) per workgroup of 8
// waves, two per SIMD.  Wave w owns all BM rows (tokens) and the 32 weight rows (output columns)
// 32w .. 32w + 31: BM/32 MFMA tiles of 32 x 32 on v_mfma_f32_32x32x16_bf16 / f16 with the
// accumulators in AGPRs.  So every weight element is dequantized once per workgroup, by the one
// wave that multiplies it, for BM rows.  Two waves per SIMD because the dequantization is VALU
// work that one wave cannot issue fast enough beside its own MFMAs: on gfx950 a single wave issues
// a v_fma_f32 every ~5.3 cycles and a v_cvt_f32_ubyte / v_cvt_pk_bf16_f32 every 8, two waves of a
// SIMD together one every ~3.3 / ~4.5, and the other wave's MFMAs run meanwhile.  K runs in
// stages of 64 through a 3-deep LDS ring filled by global->LDS loads: per stage the activations
// (BM rows x 128 bytes, XOR-swizzled 16-byte chunks), the packed weights (256 rows x 32 bytes of
// nibbles, or 64 bytes of int8) and, for uint4, each weight row's group scale and zero (one
// 32-bit word each, zero-extended fp16; waves 0-3 load the scales of 64 columns each, waves 4-7
// the zeros).  Inside a stage the MFMAs of k-step t run beside the
// activation fragment reads and the weight dequantization of k-step t + 1; the stage's one
// barrier sits before its last k-step, whose MFMAs cover the next stage's first reads and
// dequantization.  Lane-half h of every fragment carries k = 32 h + 8 t .. + 7 of the stage in
// k-step t, for both operands, so a lane's weights of a stage are 16 contiguous bytes of nibbles.
namespace wt {
constexpr int BN = 256, BK = 64;
constexpr int TN = 1;                              // 32 x 32 tiles per wave: BM rows x 32 columns
constexpr int WCOLS = 32 * TN;                     // output columns per wave
constexpr int NWAVE = BN / WCOLS;                  // waves per workgroup (8: two per SIMD)
constexpr int THREADS = NWAVE * 64;
constexpr int XROW = BK * 2;                       // activation bytes per row per stage
template <int BM> constexpr int xbytes() { return BM * XROW; }                        // 32 / 16 KB
template <int BM> constexpr int xdma() { return xbytes<BM>() / 1024 / NWAVE; }        // activation loads per wave (4 / 2)
template <int WK> constexpr int wrow() { return WK == W_UINT4 ? BK / 2 : BK; }         // 32 / 64 B
template <int WK> constexpr int wdma() { return BN * wrow<WK>() / 1024 / NWAVE; }      // 1 / 2
template <int WK> constexpr int szdma() { return WK == W_UINT4 ? 1 : 0; }
template <int WK, int BM> constexpr int lps() { return xdma<BM>() + wdma<WK>() + szdma<WK>(); }   // 6 / 6 (BM 256)
template <int WK, int BM> constexpr int slot_bytes() { return xbytes<BM>() + BN * wrow<WK>() + (WK == W_UINT4 ? 2 * BN * 4 : 0); }
// ring depth: 3 slots of 256-row stages, and of the half-size 128-row ones too (deeper rings of
// 128-row stages measured no faster)
template <int WK, int BM> constexpr int nstage()
{
    return 163840 / slot_bytes<WK, BM>() < 3 ? 163840 / slot_bytes<WK, BM>() : 3;
}
// uint4 group scales and zeros in blocks of SZG groups: per block and column 16 bytes of scales and
// 16 of zeros (one dense 16-byte load per lane), two blocks buffered past the ring
constexpr int SZG = 8;
constexpr int SZB_BYTES = 2 * BN * 16;
template <int WK, int BM> constexpr int lds_bytes()
{
    return nstage<WK, BM>() * slot_bytes<WK, BM>() + (WK == W_UINT4 ? 2 * SZB_BYTES : 0);   // 142 KB (uint4, BM 256)
}
// activation chunk swizzle: bijective on 8 consecutive rows (32 banks) and on each parity class
// of 16 consecutive rows (64 banks), so a fragment read (32 rows, one logical chunk) is conflict free
__device__ __forceinline__ int xsw(int r) { return ((r >> 1) ^ (r << 2)) & 7; }
// weight chunk swizzle: chunk c of weight row r (2 chunks of a 32-byte uint4 row, 4 of a 64-byte
// int8 row) sits at c ^ wsw(r).  ds_read_b128 on gfx950 serves a wave in four groups of 16 lanes,
// the group of lane l given by l >> 5 and the parity of its bits 2-4 (fitted to two in-bounds
// probes of 22 address patterns, every measured time predicted); the 32 lanes of a fragment read
// (rows 32 w .. + 31, one chunk) then fall on distinct banks, where the unswizzled rows conflicted
// two ways (uint4) and four ways (int8).
template <int WK> __device__ __forceinline__ int wsw(int r) { return WK == W_UINT4 ? (r >> 4) & 1 : (r >> 3) & 3; }
// Stream-K over U units and G workgroup ranges, range l = [floor(l U / G), floor((l + 1) U / G)):
// the range holding unit u (the largest l with floor(l U / G) <= u; ranges are never empty when
// U >= G) ...
__host__ __device__ inline int sk_owner(int64_t u, int64_t U, int G) { return (int)(((u + 1) * G + U - 1) / U) - 1; }
// ... and the partial-tile slot of range l's segment of tile t: 2 l for the range's first tile,
// 2 l + 1 for its last (a range's other tiles are whole and need none)
__host__ __device__ inline int sk_slot(int l, int t, int64_t U, int G, int nk)
{
    return 2 * l + (t == (int)((int64_t)l * U / G / nk) ? 0 : 1);
}
}  // namespace wt

template <int XDT, int WK, int BM, bool SKM>
__global__ void __launch_bounds__(wt::THREADS, 1)
gemm_wonly_tiled(const uint16_t *__restrict__ x, int64_t ldx, int M, int N, int K, WArgs wa)
{
    using namespace wt;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    using XV = typename std::conditional<XDT == PSQ_BF16, v8bf, v8h>::type;
    constexpr int TM = BM / 32;                    // 32-row MFMA tiles per wave
    constexpr int XBYTES = xbytes<BM>(), XDMA = xdma<BM>();
    constexpr int SLOT = slot_bytes<WK, BM>();
    constexpr int NSTAGE = nstage<WK, BM>();       // ring slots: NSTAGE - 1 stages in flight
    constexpr int LPS = lps<WK, BM>();
    constexpr int NQ = TM * TN;                    // MFMAs per k-step
    constexpr int LPK = (LPS + 2) / 3;             // refill loads behind each of the first three k-steps
    constexpr int RB = wrow<WK>();
    constexpr int WDMA = wdma<WK>();
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int frow = lane & 31, h = lane >> 5;
    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    const int nk_all = K / BK;
    const int G = WK == W_UINT4 ? K / wa.gs : 1;
    const int64_t wld = WK == W_UINT4 ? K / 2 : K;          // weight row bytes
    // Stream-K: the workgroup's units [u0, u1) (unit = (tile, K stage); tile-major, the tiles of a
    // column of tiles, which share their weights, consecutive), taken as segments of one tile
    // each, from the last to the first.  A range's first segment is the end of a tile that other
    // workgroups began earlier in their runs, so the workgroup that finishes a tile, and adds it
    // up, is most often the one that holds that segment.  Without stream-K one segment: every
    // stage of tile blockIdx.x.
    const int SK = SKM ? wa.sk : 0;
    const int64_t U = (int64_t)nbm * nbn * nk_all;
    const int lw = SK ? xcd_rank((int)blockIdx.x, SK) : 0;   // consecutive ranges on one XCD
    const int64_t u0 = SK ? (int64_t)lw * U / SK : 0;
    int64_t ue = SK ? (int64_t)(lw + 1) * U / SK : nk_all;
    bool first_seg = true;
#pragma clang loop unroll(disable)
    while (ue > u0) {
        int tile, kb, nk, pm, pn;   // this segment: K stages [kb, kb + nk) of tile (pm, pn)
        if (SK) {
            tile = (int)((ue - 1) / nk_all);
            const int64_t tb = (int64_t)tile * nk_all;
            kb = (int)((u0 > tb ? u0 : tb) - tb);
            nk = (int)(ue - tb) - kb;
            ue = tb + kb;
            pm = tile % nbm;
            pn = tile / nbm;
        } else {
            tile = (int)blockIdx.x;
            kb = 0;
            nk = nk_all;
            ue = 0;
            tile_order(tile, nbm, nbn, 4, pm, pn);
        }
        // every wave is done with the previous segment's ring and scale blocks before the refill
        if (!first_seg) __syncthreads();
        first_seg = false;
        const int m0 = pm * BM, n0 = pn * BN;

        // ---- ring loads (scalar base + 32-bit lane offsets); rows past M / N clamp to the last row
        uint32_t xo[XDMA], wo[WDMA];
#pragma unroll
        for (int j = 0; j < XDMA; j++) {
            const int b = j * NWAVE + wave, r = 8 * b + (lane >> 3);
            const int c = (lane & 7) ^ xsw(r);
            xo[j] = (uint32_t)(min(r, M - 1 - m0) * ldx * 2 + c * 16);
        }
#pragma unroll
        for (int j = 0; j < WDMA; j++) {
            const int b = j * NWAVE + wave;
            const int per = 1024 / RB;                          // rows per load (32 / 16)
            const int r = per * b + lane / (64 / per);
            wo[j] = (uint32_t)(min(r, N - 1 - n0) * wld + (((lane % (64 / per)) ^ wsw<WK>(r)) << 4));
        }
        const int scol = min(n0 + 64 * (wave & 3) + lane, N - 1);   // scale (waves 0-3) / zero (4-7) column of this lane
        const unsigned spg = WK == W_UINT4 ? (unsigned)(wa.gs / BK) : 1u;   // stages per group
        // Scale / zero blocks (uint4, groups per row a multiple of SZG, 16-byte aligned tables): a
        // block of SZG groups is loaded once, with the first stage of the block (or of the workgroup's
        // K range), instead of a 2-byte scattered load per stage.  Otherwise the per-stage loads.
        // (stages per group a power of two, so that a stage's group and block are shifts and masks:
        // the per-stage bookkeeping sits between the MFMAs)
        const bool szblk = WK == W_UINT4 && G % SZG == 0 && (spg & (spg - 1)) == 0 && ((uintptr_t)wa.scale16 % 16) == 0 &&
                           ((uintptr_t)wa.zero16 % 16) == 0;
        const int spg_sh = spg ? __builtin_ctz(spg) : 0;          // log2 stages per group (szblk)
        static_assert(SZG == 8, "scale blocks of 8 groups");
        const unsigned spb_mask = (spg << 3) - 1;                 // stages per scale block - 1
        uint8_t *const szbuf = smem + NSTAGE * SLOT;
        const uint8_t *xb = (const uint8_t *)(x + (int64_t)m0 * ldx);
        const uint8_t *wb = wa.wq + (int64_t)n0 * wld;
        // The tile's activation and weight rows as buffer descriptors: a load is the descriptor, the
        // stage's k offset as scalar offset and the lane's row offset as vector offset (no per-load
        // address arithmetic).
        const __amdgpu_buffer_rsrc_t rsx = raw_rsrc(xb), rsw = raw_rsrc(wb);
        // load q of a stage (q < 8: activation block q; then weight blocks; then, for uint4, the
        // stage's scale and zero words of the wave's 64 columns)
        auto issue_one = [&](int slot, int kt, auto qc) {
            constexpr int q = decltype(qc)::value;
            uint8_t *sl = smem + slot * SLOT;
            if constexpr (q < XDMA) {
                constexpr int b8 = q * NWAVE;
                buffer_load_lds16(rsx, (lds_ptr)(sl + 1024 * (b8 + wave)), xo[q], kt * BK * 2);
            } else if constexpr (q < XDMA + WDMA) {
                constexpr int j = q - XDMA;
                buffer_load_lds16(rsw, (lds_ptr)(sl + XBYTES + 1024 * (j * NWAVE + wave)), wo[j], kt * RB);
            } else if constexpr (WK == W_UINT4) {
                const bool zero = wave >= 4;
                if (szblk) {
                    // the block of the stage's group, with the block's first stage (or the range's)
                    if (kt == kb || ((unsigned)kt & spb_mask) == 0) {
                        const unsigned blk = (unsigned)kt >> (spg_sh + 3);
                        const int64_t gi = (int64_t)scol * G + SZG * blk;
                        __builtin_amdgcn_global_load_lds((glb_ptr)((zero ? wa.zero16 : wa.scale16) + gi),
                                                         (lds_ptr)(szbuf + (blk & 1) * SZB_BYTES + 1024 * wave), 16, 0, 0);
                    }
                } else {
                    const int64_t gi = (int64_t)scol * G + (int)((unsigned)kt / spg);   // the stage's group
                    __builtin_amdgcn_global_load_lds((glb_ptr)((zero ? wa.zero16 : wa.scale16) + gi),
                                                     (lds_ptr)(sl + XBYTES + BN * RB + 256 * wave), 2, 0, 0);
                }
            }
        };
        auto issue_all = [&](int slot, int kt) {
            [&]<int... Q>(std::integer_sequence<int, Q...>) {
                (issue_one(slot, kt, std::integral_constant<int, Q>{}), ...);
            }(std::make_integer_sequence<int, LPS>{});
        };

        // ---- fragments
        auto read_x = [&](int slot, int t, int i) -> XV {
            const int r = 32 * i + frow, c = 4 * h + t;
            return __builtin_bit_cast(XV, *(const v4i *)(smem + slot * SLOT + r * XROW + ((c ^ xsw(r)) << 4)));
        };
        // the lane's packed weights of a stage (its 32 k of each of its two columns) and, for uint4,
        // the columns' group scale s (held as s 2^24 and s 2^20) and -z s: a weight is
        // round_16(fmaf(q, s, -z s)), one fma_mix per weight (dq_pair_u4)
        struct WRaw { v4i w[TN][RB / 32]; float s[TN], s4[TN], z[TN]; };
        auto read_w = [&](int slot, int kt, WRaw &r) {
            const uint8_t *sl = smem + slot * SLOT + XBYTES;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = WCOLS * wave + 32 * j + frow;
#pragma unroll
                for (int c = 0; c < RB / 32; c++)
                    r.w[j][c] = *(const v4i *)(sl + n * RB + ((((RB / 32) * h + c) ^ wsw<WK>(n)) << 4));
                if constexpr (WK == W_UINT4) {
                    float sv, zv;
                    if (szblk) {
                        const unsigned g = (unsigned)kt >> spg_sh;
                        const uint8_t *zb = szbuf + ((g / SZG) & 1) * SZB_BYTES + 16 * n + 2 * (g % SZG);
                        sv = f16_to_f32(*(const uint16_t *)zb);
                        zv = f16_to_f32(*(const uint16_t *)(zb + BN * 16));
                    } else {
                        sv = f16_to_f32(*(const uint32_t *)(sl + BN * RB + 4 * n));
                        zv = f16_to_f32(*(const uint32_t *)(sl + BN * RB + BN * 4 + 4 * n));
                    }
                    r.s[j] = sv * kTwo24;     // s 2^24 and s 2^20 for the fp16-subnormal nibbles (dq_pair_u4)
                    r.s4[j] = sv * kTwo20;
                    r.z[j] = -(zv * sv);      // -z s
                } else {
                    r.s[j] = r.s4[j] = 1.0f;
                    r.z[j] = 0.0f;
                }
            }
        };
        // pair e (k = 32 h + 8 t + 2e, +1) of column tile j's weights in k-step t, packed
        auto dq_pair = [&](const WRaw &r, int j, int t, int e) -> uint32_t {
            if constexpr (WK == W_UINT4) {
                return dq_pair_u4<XDT>(nib_split((uint32_t)r.w[j][0][t]), e, r.s[j], r.s4[j], r.z[j]);
            } else {
                const uint32_t p = (uint32_t)r.w[j][t >> 1][2 * (t & 1) + (e >> 1)];
                if constexpr (XDT == PSQ_F16) {
                    return i8pair_f16(p, e & 1);
                } else {
                    const int sh = 16 * (e & 1);
                    return pack2<XDT>((float)(int8_t)((p >> sh) & 0xffu), (float)(int8_t)((p >> (sh + 8)) & 0xffu));
                }
            }
        };

        v16f acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
        auto mfma = [&](int i, int j, const XV &wf, const XV &xf) {
            if constexpr (XDT == PSQ_BF16)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf, xf, acc[i][j], 0, 0, 0);
            else
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf, xf, acc[i][j], 0, 0, 0);
        };

        // Stage kt + 1 landed: every load but those of the NSTAGE - 2 younger stages is complete.  With
        // scale blocks a stage issues LPS - 1 loads plus, at a block start, the block's: counting only
        // the LPS - 1 waits for at least the loads it must (the block's is older than the younger
        // stages' loads).
        auto wait_stage = [&] {
            if constexpr (WK == W_UINT4) {
                if (szblk) wait_vmcnt<(NSTAGE - 2) * (LPS - 1)>();
                else wait_vmcnt<(NSTAGE - 2) * LPS>();
            } else {
                wait_vmcnt<(NSTAGE - 2) * LPS>();
            }
        };

        // ---- prologue: stages 0 .. NSTAGE-2 in flight, stage 0 landed, its first fragments ready
#pragma unroll
        for (int st = 0; st < NSTAGE - 1; st++) issue_all(st, kb + min(st, nk - 1));
        wait_stage();
        stage_barrier();
        WRaw wr;
        read_w(0, kb, wr);
        XV xa[TM], xb2[TM], wa0[TN], wb0[TN];
#pragma unroll
        for (int i = 0; i < TM; i++) xa[i] = read_x(0, 0, i);
#pragma unroll
        for (int j = 0; j < TN; j++) {
            uint32_t hw[4];
#pragma unroll
            for (int e = 0; e < 4; e++) hw[e] = dq_pair(wr, j, 0, e);
            wa0[j] = __builtin_bit_cast(XV, v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]});
        }

        // One k-step: the NQ = TM TN MFMAs of step t on (xc, wc); behind MFMA q the activation
        // fragment q / TN of the next step (q % TN == 0), one of the next step's 4 TN weight pairs
        // (every NQ / (4 TN)-th MFMA), and for k-steps 0-2 a third of the stage's refill loads.
        // The instruction order is pinned: sched_barrier after every MFMA.
        auto kstep = [&](auto tnc, auto basec, XV (&xc)[TM], XV (&wc)[TN], XV (&xn)[TM], XV (&wn)[TN], int xslot,
                         const WRaw &wraw, int fill_slot, int fill_kt) {
            constexpr int tn = decltype(tnc)::value, fill_base = decltype(basec)::value;
            uint32_t hw[TN][4];
            [&]<int... Q>(std::integer_sequence<int, Q...>) {
                ([&] {
                    constexpr int q = Q;
                    mfma(q / TN, q % TN, wc[q % TN], xc[q / TN]);
                    if constexpr (q % TN == 0) xn[q / TN] = read_x(xslot, tn, q / TN);
                    // weight pair pi (column tile pi / 4, pair pi % 4), spread evenly over the k-step
                    constexpr int NP = 4 * TN, PSTRIDE = NQ / NP;
                    static_assert(NQ % NP == 0, "pairs per k-step must divide the MFMAs");
                    constexpr int pi = q % PSTRIDE == 0 ? q / PSTRIDE : -1;
                    if constexpr (pi >= 0) hw[pi >> 2][pi & 3] = dq_pair(wraw, pi >> 2, tn, pi & 3);
                    // the refill loads: LPK of them spread over the k-step, the last of each group
                    constexpr int per = NQ / LPK, u = q / per;
                    if constexpr (fill_base >= 0 && q % per == per - 1 && u < LPK && fill_base + u < LPS)
                        issue_one(fill_slot, fill_kt, std::integral_constant<int, fill_base + u>{});
                    __builtin_amdgcn_sched_barrier(0);
                }(), ...);
            }(std::make_integer_sequence<int, NQ>{});
#pragma unroll
            for (int j = 0; j < TN; j++) wn[j] = __builtin_bit_cast(XV, v4i{(int)hw[j][0], (int)hw[j][1], (int)hw[j][2], (int)hw[j][3]});
        };
        int rs = 0;
#pragma clang loop unroll(disable)
        for (int kt = 0; kt < nk; kt++) {
            const int fill = rs == 0 ? NSTAGE - 1 : rs - 1;     // ring slot of stage kt + NSTAGE - 1
            const int kfill = kb + min(kt + NSTAGE - 1, nk - 1); // (past the end: re-load the last stage)
            const int nxt = rs == NSTAGE - 1 ? 0 : rs + 1;
            using I = std::integral_constant<int, 0>;
            kstep(std::integral_constant<int, 1>{}, I{}, xa, wa0, xb2, wb0, rs, wr, fill, kfill);
            kstep(std::integral_constant<int, 2>{}, std::integral_constant<int, LPK>{}, xb2, wb0, xa, wa0, rs, wr, fill, kfill);
            kstep(std::integral_constant<int, 3>{}, std::integral_constant<int, 2 * LPK>{}, xa, wa0, xb2, wb0, rs, wr, fill, kfill);
            // stage kt + 1 landed for every wave; nobody reads stage kt's slot any more
            wait_stage();
            stage_barrier();
            read_w(nxt, kb + kt + 1, wr);
            kstep(I{}, std::integral_constant<int, -1>{}, xb2, wb0, xa, wa0, nxt, wr, 0, 0);
            rs = nxt;
        }
        wait_vmcnt<0>();   // the re-issued tail loads land before the ring is refilled or released

        // ---- part of a tile (stream-K).  Its workgroups, in range order, are lf .. lf + nc - 1, and
        // its sum is fixed as ((p_{nc-1} + p_{nc-2}) + ...) + p_0 over their partial tiles, so the
        // result does not depend on which workgroup finishes last.  Each but the last to finish
        // writes its fp32 partial and then counts itself in cnt[tile]; the one that finds
        // the other nc - 1 counted zeroes the count, adds the tile up and runs the epilogue: into its own registers
        // when it holds the end of the tile (p_{nc-1}, the usual case: ranges run their segments
        // from the last), else from memory, its own partial included.
        if (SKM && (kb != 0 || nk != nk_all)) {
            const int64_t tb = (int64_t)tile * nk_all;
            const int lf = sk_owner(tb, U, SK), nc = sk_owner(tb + nk_all - 1, U, SK) - lf + 1, myc = lw - lf;
            uint32_t *flag = (uint32_t *)(smem + lds_bytes<WK, BM>());
            // A partial tile is kept in the lanes' own order: register group (i, j, g) of wave w at
            // 16 (64 (4 (TN (TM w + i) + j) + g) + lane) bytes, so that each store and load moves 1 KB
            // in whole lines, and the adding workgroup reads exactly what the same lane wrote.  Stores
            // and loads carry sc1 (agent coherence: through, not into, the XCDs' own L2s), so the
            // partials need no L2 write-back or invalidation, only the wait for the stores before the
            // count.
            const uint32_t lofs = (uint32_t)(wave * (TM * TN * 4 * 1024) + lane * 16);
            constexpr int SC1 = 16;    // cache-policy bit sc1 of the buffer intrinsics
            auto slot_rsrc = [&](int l) {
                const int sl = __builtin_amdgcn_readfirstlane(sk_slot(l, tile, U, SK, nk_all));
                return raw_rsrc(wa.part + (int64_t)sl * (BM * BN));
            };
            // every other workgroup finished: no count to take
            if (tid == 0) *flag = __hip_atomic_load(wa.cnt + tile, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            // (through readfirstlane: a value the compiler knows is uniform, so that what depends
            // on it stays in scalar registers)
            bool last = __builtin_amdgcn_readfirstlane(*flag) == nc - 1;
            if (!last || myc != nc - 1) {   // the partial, for the others or to be read back below
                const __amdgpu_buffer_rsrc_t rs = slot_rsrc(lw);
                static_for<TM>([&](auto ic) {
                    static_for<TN>([&](auto jc) {
                        static_for<4>([&](auto gc) {
                            constexpr int i = decltype(ic)::value, j = decltype(jc)::value, g = decltype(gc)::value;
                            const v4i v{agpr_read_for_store(acc[i][j][4 * g]), agpr_read_for_store(acc[i][j][4 * g + 1]),
                                        agpr_read_for_store(acc[i][j][4 * g + 2]), agpr_read_for_store(acc[i][j][4 * g + 3])};
                            __builtin_amdgcn_raw_buffer_store_b128(v, rs, lofs + ((i * TN + j) * 4 + g) * 1024, 0, SC1);
                        });
                    });
                });
            }
            if (!last) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the partial is written before the count
                __syncthreads();
                if (tid == 0) *flag = atomicAdd(wa.cnt + tile, 1u);
                __syncthreads();
                if (__builtin_amdgcn_readfirstlane(*flag) != nc - 1) continue;
            }
            // every other workgroup of the tile has counted itself and touches the counter no more:
            // zero it again, for the next launch on this workspace
            if (tid == 0) __hip_atomic_store(wa.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");       // (its own partial, when it wrote one)
            // add p_c into the registers (or, first, load it), 16 words a lane in flight
            auto add = [&](int c, bool first) {
                const __amdgpu_buffer_rsrc_t rs = slot_rsrc(lf + c);
                constexpr int CH = TM < 4 ? TM : 4;   // row tiles per chunk
                static_for<TM / CH>([&](auto chc) {
                    constexpr int ch = decltype(chc)::value;
                    v4i v[CH][TN][4];
                    static_for<CH>([&](auto ic) {
                        static_for<TN>([&](auto jc) {
                            static_for<4>([&](auto gc) {
                                constexpr int i = decltype(ic)::value, j = decltype(jc)::value, g = decltype(gc)::value;
                                v[i][j][g] = __builtin_amdgcn_raw_buffer_load_b128(
                                    rs, lofs + (((CH * ch + i) * TN + j) * 4 + g) * 1024, 0, SC1);
                            });
                        });
                    });
                    static_for<CH>([&](auto ic) {
                        static_for<TN>([&](auto jc) {
                            static_for<16>([&](auto rc) {
                                constexpr int i = decltype(ic)::value, j = decltype(jc)::value, r = decltype(rc)::value;
                                constexpr int ia = CH * ch + i;
                                const float pv = __int_as_float(v[i][j][r >> 2][r & 3]);
                                acc[ia][j][r] = first ? pv : __int_as_float(agpr_read(acc[ia][j][r])) + pv;
                            });
                        });
                    });
                    __builtin_amdgcn_sched_barrier(0);
                });
            };
            if (myc != nc - 1) add(nc - 1, true);
#pragma clang loop unroll(disable)
            for (int c = nc - 2; c >= 0; c--) add(c, false);
        }

        // ---- epilogue: acc[i][j] is the transposed 32 x 32 tile, lane (l & 31) holds output row
        // m = m0 + 32 i + (l & 31), register 4g + c column n = n0 + WCOLS wave + 32 j + 8 g + 4 h + c.
        //   y = round_out(fmaf(acc, s[n], bias[n]))   (s = 1 for uint4)
        const int nl0 = WCOLS * wave + 4 * h;                    // the lane's first column in the tile
        const int esz = wa.y_dtype == PSQ_F32 ? 4 : 2;
        uint8_t *rowp[TM];
        bool live[TM];
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int m = m0 + 32 * i + frow;
            live[i] = m < M;
            rowp[i] = (uint8_t *)wa.y + ((int64_t)min(m, M - 1) * wa.ldy + n0 + nl0) * esz;
        }
        // operands of the lane's 4 columns n0 + nl0 + nc .. + 3: the row scale (int8) and the bias
        auto operands = [&](int nc, float (&cs)[4], float (&bs)[4]) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int n = min(n0 + nl0 + nc + c, N - 1);
                cs[c] = (WK == W_INT8) ? wa.scale32[n] : 1.0f;
                bs[c] = wa.bias ? load_elem(wa.bias, n, wa.bias_dtype) : 0.0f;
            }
        };
        auto value = [&](int i, int j, int r, float c, float b) {
            return __builtin_fmaf(__int_as_float(agpr_read(acc[i][j][r])), c, b);
        };
        const bool fast = wa.y_dtype != PSQ_F32 && n0 + BN <= N && ((uintptr_t)wa.y & 15) == 0 && (wa.ldy * 2) % 16 == 0;
        if (fast) {
            // lanes l and l + 32 hold the same row: one v_permlane32_swap per word gives lane l columns
            // 16 pr + 0..7 and lane l + 32 columns 16 pr + 8..15 of the column pair pr, one 16-byte store
            const bool bf = wa.y_dtype == PSQ_BF16;
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int pr = 0; pr < 2; pr++) {
                    const int nc = 32 * j + 16 * pr;
                    float cs[2][4], bs[2][4];
                    operands(nc, cs[0], bs[0]);
                    operands(nc + 8, cs[1], bs[1]);
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        uint32_t x0[2], x1[2];
#pragma unroll
                        for (int hh = 0; hh < 2; hh++) {
                            uint32_t *o = hh == 0 ? x0 : x1;
                            const int r = 8 * pr + 4 * hh;
                            const float v0 = value(i, j, r, cs[hh][0], bs[hh][0]), v1 = value(i, j, r + 1, cs[hh][1], bs[hh][1]);
                            const float v2 = value(i, j, r + 2, cs[hh][2], bs[hh][2]), v3 = value(i, j, r + 3, cs[hh][3], bs[hh][3]);
                            o[0] = bf ? pack_half2<PSQ_BF16>(v0, v1) : pack_half2<PSQ_F16>(v0, v1);
                            o[1] = bf ? pack_half2<PSQ_BF16>(v2, v3) : pack_half2<PSQ_F16>(v2, v3);
                        }
                        uint32_t lo[2], hi[2];
#pragma unroll
                        for (int d = 0; d < 2; d++) {
                            const auto sw = __builtin_amdgcn_permlane32_swap(x0[d], x1[d], false, false);
                            lo[d] = sw[0];
                            hi[d] = sw[1];
                        }
                        uint8_t *p = rowp[i] + (nc + 4 * h) * 2;
                        if (live[i]) *(v4i *)p = v4i{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
        } else {
            const int n_left0 = N - (n0 + nl0);
            static_for<TN>([&](auto jc) {
                static_for<4>([&](auto gc) {
                    constexpr int j = decltype(jc)::value, g = decltype(gc)::value, nc = 32 * j + 8 * g;
                    float cs[4], bs[4];
                    operands(nc, cs, bs);
                    static_for<TM>([&](auto ic) {
                        constexpr int i = decltype(ic)::value;
                        static_for<4>([&](auto cc) {
                            constexpr int c = decltype(cc)::value;
                            const float v = value(i, j, 4 * g + c, cs[c], bs[c]);
                            if (live[i] && c < n_left0 - nc) store_elem(rowp[i], nc + c, wa.y_dtype, v);
                        });
                    });
                    __builtin_amdgcn_sched_barrier(0);
                });
            });
        }
    }
}

// ------------------------------------------------------ uint4 streaming kernel (M <= 64)
// The weight-streaming shapes of W4A16 (a few tokens to a short prompt against the whole weight)
// with groups of a multiple of 128 and K a multiple of 256.  A workgroup of 8 waves owns 128
// weight rows (output columns) over the whole K, so every weight byte is read once and the
// activations once per workgroup.
//  * Waves: column group cg = w & 3 (32 weight rows, two 16-column MFMA tiles) and block parity
//    p = w >> 2.  K runs in ring steps of 256: 128-k block 2s of each step goes to the parity-0
//    waves, block 2s + 1 to the parity-1 waves, and the two partial sums are added once at the end
//    (parity 0 + parity 1, a fixed order).  Each activation fragment read from LDS feeds two MFMAs
//    (the wave's two column tiles), so the 4 waves of a parity read the activations of their block
//    once each -- half the LDS reads of 16 columns per wave -- and 256 k of a weight row is one
//    whole 128-byte line per load.
//  * Loads: per step the workgroup's 128 rows x 128 bytes of nibbles, the two blocks' group scales
//    and zeros and the 16 MT rows x 512 bytes of activations go global->LDS into a ring of NSLOT
//    steps, NSLOT - 1 steps ahead of the one computed; one barrier per step.  Nothing is loaded into
//    registers ahead of time, so the compiler's own load tracking adds no waits across the loop.
//  * Swizzles: ds_read_b128 on gfx950 does not serve 16 consecutive lanes per LDS cycle (an
//    in-bounds probe of twelve address patterns rules that out), so the 16-byte chunks are placed
//    with bit shuffles of the row that keep every fragment read conflict free under each lane
//    grouping consistent with the probe: activation chunk c of row r at c ^ xsw(r) (512-byte rows),
//    weight chunk c of row r at c ^ wsw(r) (128-byte rows).
//  * The lane dequantizes its 64 weights per step (two rows x 32 k), w = round_16(fmaf(q, s, -z s))
//    (dq_pair_u4: 17 VALU ops per 8 weights): one fma where the dequantize kernel computes
//    (q - z) s, so a weight can differ from it by one 16-bit ulp (about 2^-16 of the weights), far
//    inside the fp32-accumulation bar.
//  * MFMA 16x16x32 with the activations as the A operand: lane (n = l & 15, h = l >> 4) holds output
//    column n of each column tile and rows 4 h .. 4 h + 3 of each 16-row tile; lane group h carries
//    k = 32 h + 8 t .. + 7 of the block in k-step t for both operands.
namespace ws {
constexpr int ROWS = 128;                                   // weight rows per workgroup
constexpr int NW = 8;                                       // waves: 4 column groups x 2 parities
constexpr int STEP = 256;                                   // k per ring step (two 128-k blocks)
template <int MT> constexpr int XSLOT() { return MT * 16 * STEP * 2; }   // activations of a step
constexpr int WSLOT = ROWS * STEP / 2;                       // nibbles of a step (16 KB)
constexpr int SZSLOT = 2 * 2 * ROWS * 4;                     // [scale | zero][parity][row], 32-bit slots
// Scale / zero loads, by mode SZM:
//  * SZ_TABLE: the workgroup's whole scale and zero tables (ROWS rows x G groups x 2 bytes each,
//    contiguous in memory) go to LDS once, ahead of the ring, when they fit SZT_MAX bytes (G a
//    multiple of 8 up to 40, MT <= 3);
//  * SZ_BLOCK: blocks of 8 groups (one 16-byte load per row and array: 4 loads per block, issued
//    with the block's first step into one of two 4 KB buffers past the ring), G a multiple of 8;
//  * SZ_STEP: each step loads its blocks' values (one 2-byte value per row and array and block),
//    any G.
// On gfx950 a global->LDS load costs about the cache lines it touches, and the per-step form reads
// 64 rows of the [N, G] tables per 256 bytes (~64 lines): at G = 40 about 2/3 of the lines of a
// step; the block form cuts that eightfold and the table form to nothing.
enum { SZ_STEP = 0, SZ_TABLE = 1, SZ_BLOCK = 2 };
constexpr int SZT_MAX = 2 * ROWS * 40 * 2;                   // 20 KB: G <= 40 (K = 5120 at g = 128)
constexpr int SZB_BYTES = 2 * ROWS * 16;                      // one block of 8 groups, both arrays
template <int SZM> constexpr int sz_extra() { return SZM == SZ_TABLE ? SZT_MAX : SZM == SZ_BLOCK ? 2 * SZB_BYTES : 0; }
template <int MT, int SZM> constexpr int SLOT() { return XSLOT<MT>() + WSLOT + (SZM == SZ_STEP ? SZSLOT : 0); }
template <int MT, int SZM> constexpr int NSLOT() { return (163840 - sz_extra<SZM>()) / SLOT<MT, SZM>(); }
template <int MT, int SZM> constexpr int lds_bytes() { return NSLOT<MT, SZM>() * SLOT<MT, SZM>() + sz_extra<SZM>(); }
// the table form keeps a ring of at least three steps (MT <= 3)
template <int MT> constexpr bool szt_fits() { return NSLOT<MT, SZ_TABLE>() >= 3; }
// chunk swizzles (see above): row bits (0, 3, 1, 2) -> chunk bits (0, 1, 2, 3), and for the 128-byte
// weight rows row bits (1, 3, 2) -> chunk bits (0, 1, 2)
__device__ __forceinline__ int xsw(int r) { return (r & 1) | ((r >> 2) & 2) | ((r << 1) & 4) | ((r << 1) & 8); }
__device__ __forceinline__ int wsw(int r) { return ((r >> 1) & 1) | ((r >> 2) & 2) | (r & 4); }
}  // namespace ws

template <int XDT, int MT, int SZM>
__global__ void __launch_bounds__(ws::NW * 64)
gemm_w4_stream(const uint16_t *__restrict__ x, int64_t ldx, int M, int N, int K, WArgs wa)
{
    using namespace ws;
    constexpr int NX = NSLOT<MT, SZM>(), DD = NX - 1;        // ring slots; steps in flight
    constexpr int XS = XSLOT<MT>(), SL = SLOT<MT, SZM>();
    constexpr bool SZT = SZM == SZ_TABLE;
    static_assert(DD >= 2, "ring too shallow");
    // a block of scales is read last by step 4 hg (b + 1) - 1 and its buffer refilled with step
    // 4 hg (b + 2): after the barrier of step 4 hg (b + 2) + 1 - NX, safe while NX <= 4 hg + 2
    static_assert(SZM != SZ_BLOCK || NX <= 6, "scale blocks need a ring of at most 6 steps");
    using XV = typename std::conditional<XDT == PSQ_BF16, v8bf, v8h>::type;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nr = lane & 15, h = lane >> 4;
    const int cg = wave & 3, par = wave >> 2;
    const int ns = K / STEP;
    const int G = K / wa.gs, hg = wa.gs / 128;               // groups per row; 128-k blocks per group
    const int64_t wld = K / 2;
    const int wg_row0 = blockIdx.x * ROWS;
    // the weights from the workgroup's first row: lane offsets stay below 128 rows (32 bits)
    const uint8_t *const wq = wa.wq + (int64_t)wg_row0 * wld;

    // ---- ring loads of a step (all global->LDS; rows past N clamp to the last row)
    // weights: 16 loads of 1 KB = 8 rows x 128 bytes; wave w issues loads 2 w and 2 w + 1.  Lane L
    // of load d fills row 8 d + L / 8, physical chunk L % 8, holding logical chunk pc ^ wsw(row).
    uint32_t wo[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = 8 * (2 * wave + i) + (lane >> 3), pc = lane & 7;
        wo[i] = (uint32_t)((min(wg_row0 + r, N - 1) - wg_row0) * wld + ((pc ^ wsw(r)) << 4));
    }
    // scales and zeros: wave w fetches array w & 1 (scale, zero) of block parity (w >> 1) & 1 for
    // rows 64 (w >> 2) + L, one 16-bit value per lane into its 32-bit slot.  The group of block
    // 2 s + bp is kept as a running quotient and remainder by hg on the scalar unit.
    const int sz_arr = wave & 1, sz_par = (wave >> 1) & 1, sz_row = 64 * (wave >> 2) + lane;
    const uint16_t *const szrow = (sz_arr ? wa.zero16 : wa.scale16) + (int64_t)min(wg_row0 + sz_row, N - 1) * G;
    const int sz_dst = ((2 * sz_arr + sz_par) * ROWS + 64 * (wave >> 2)) * 4;
    int gq = sz_par / hg, gr = sz_par % hg;                 // block sz_par + 2 s of the next step issued
    // activations: 8 MT loads of 1 KB = 2 rows x 512 bytes; wave w issues loads w, w + 8, .. whose
    // rows start below M (xd of them, a wave-uniform count that picks its vmcnt waits).  Lane L fills
    // row 2 j + L / 32, physical chunk L % 32, holding logical chunk pc ^ xsw(row).  Rows past M feed
    // output rows that are never stored.
    constexpr int XDMAX = (8 * MT + NW - 1) / NW;            // MT
    const int nxl = (M + 1) / 2;
    const int xd = wave < nxl ? min(XDMAX, (nxl - wave + NW - 1) / NW) : 0;
    uint32_t xo[XDMAX];
#pragma unroll
    for (int i = 0; i < XDMAX; i++) {
        const int row = 2 * (wave + NW * i) + (lane >> 5), pc = lane & 31;
        xo[i] = (uint32_t)(min(row, M - 1) * ldx * 2 + ((pc ^ xsw(row)) << 4));
    }
    // scale blocks (SZ_BLOCK): waves 0-3 load, per block, array w & 1 for rows 64 (w >> 1) + L, the
    // 16 bytes of groups 8 b .. 8 b + 7 of the row; buffer (b & 1), [array][row][8 groups]
    uint8_t *const szb = smem + NX * SL;
    const uint16_t *const szblk_src = (wave & 1 ? wa.zero16 : wa.scale16) +
                                      (int64_t)min(wg_row0 + 64 * ((wave >> 1) & 1) + lane, N - 1) * G;
    const int szblk_dst = ((wave & 1) * ROWS + 64 * ((wave >> 1) & 1)) * 16;
    // whether this wave issues a scale block with step st (the block's first step)
    auto sz_extra_at = [&](int st) { return SZM == SZ_BLOCK && wave < 4 && st < ns && st % (4 * hg) == 0; };
    // steps are issued in order, once each (past the end: the last step again, into a slot nobody
    // reads any more)
    auto issue = [&](int st, int slot) {
        const int sc = min(st, ns - 1);
        uint8_t *const sl = smem + slot * SL;
        const uint8_t *const wb = wq + (int64_t)sc * (STEP / 2);
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_global_load_lds((glb_ptr)(wb + wo[i]), (lds_ptr)(sl + XS + 1024 * (2 * wave + i)), 16, 0, 0);
        if constexpr (SZM == SZ_STEP) {
            __builtin_amdgcn_global_load_lds((glb_ptr)(szrow + min(gq, G - 1)), (lds_ptr)(sl + XS + WSLOT + sz_dst), 2, 0, 0);
            gr += 2;
            if (gr >= hg) { gr -= hg; gq++; }
            if (gr >= hg) { gr -= hg; gq++; }
        } else if constexpr (SZM == SZ_BLOCK) {
            if (sz_extra_at(st)) {
                const int b = st / (4 * hg);
                __builtin_amdgcn_global_load_lds((glb_ptr)(szblk_src + b * 8),
                                                 (lds_ptr)(szb + (b & 1) * SZB_BYTES + szblk_dst), 16, 0, 0);
            }
        }
        const uint8_t *const xb = (const uint8_t *)x + (int64_t)sc * STEP * 2;
#pragma unroll
        for (int i = 0; i < XDMAX; i++)
            if (i < xd) __builtin_amdgcn_global_load_lds((glb_ptr)(xb + xo[i]), (lds_ptr)(sl + 1024 * (wave + NW * i)), 16, 0, 0);
    };

    // The next step's weights, scales and -z s go into registers ahead (Ops); the activation
    // fragments are read from the step's own slot inside compute, one k-step ahead of their MFMAs
    // (only two k-steps of fragments are live, which keeps MT = 4 within the 256 registers of two
    // waves per SIMD; the slot is refilled only after the barrier of the next step).
    struct Ops { v4i wv[2]; float sc[2], sc4[2], zs[2]; };
    auto read_x = [&](int slot, int t, XV (&xf)[MT]) {
        const uint8_t *const sl = smem + slot * SL;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int row = 16 * mt + nr, c = 16 * par + 4 * h + t;
            xf[mt] = __builtin_bit_cast(XV, *(const v4i *)(sl + row * (STEP * 2) + ((c ^ xsw(row)) << 4)));
        }
    };
    // the group of this wave's block of step s (2 s + par), as a running quotient and remainder by
    // hg (table form; steps are read in order)
    int tq = par / hg, tr = par % hg;
    const uint16_t *const szt = (const uint16_t *)(smem + NX * SL);     // [scale | zero][row][G]
    auto read_w = [&](int slot, Ops &o) {
        const uint8_t *const sl = smem + slot * SL;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int row = 32 * cg + 16 * j + nr, c = 4 * par + h;
            o.wv[j] = *(const v4i *)(sl + XS + row * (STEP / 2) + ((c ^ wsw(row)) << 4));
            float sv, zv;
            if constexpr (SZT) {
                sv = f16_to_f32(szt[row * G + tq]);
                zv = f16_to_f32(szt[(ROWS + row) * G + tq]);
            } else if constexpr (SZM == SZ_BLOCK) {
                const uint16_t *bb = (const uint16_t *)(szb + ((tq >> 3) & 1) * SZB_BYTES) + (tq & 7);
                sv = f16_to_f32(bb[row * 8]);
                zv = f16_to_f32(bb[(ROWS + row) * 8]);
            } else {
                const uint32_t *sz = (const uint32_t *)(sl + XS + WSLOT);
                sv = f16_to_f32(sz[par * ROWS + row]);
                zv = f16_to_f32(sz[(2 + par) * ROWS + row]);
            }
            o.zs[j] = -(zv * sv);
            o.sc[j] = sv * kTwo24;             // s 2^24 and s 2^20 (dq_pair_u4)
            o.sc4[j] = sv * kTwo20;
        }
        if constexpr (SZM != SZ_STEP) {
            tr += 2;
            if (tr >= hg) { tr -= hg; tq++; }
            if (tr >= hg) { tr -= hg; tq++; }
        }
    };
    v4f acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[mt][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // Step in `slot` with weights `o`: the first k-step's fragments are issued, then all the
    // step's weight fragments dequantized (the MFMAs then read registers no VALU op still writes; a
    // fragment register rewritten behind its MFMA costs a wait per k-step), then per k-step the
    // next k-step's fragments and this one's MFMAs.
    auto compute = [&](int slot, const Ops &o) {
        XV xf[2][MT];
        read_x(slot, 0, xf[0]);
        XV wfs[2][4];
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const Nib4 v = nib_split((uint32_t)o.wv[j][t]);
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; e++) w[e] = dq_pair_u4<XDT>(v, e, o.sc[j], o.sc4[j], o.zs[j]);
                wfs[j][t] = __builtin_bit_cast(XV, v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
            }
        static_for<4>([&](auto tc) {
            constexpr int t = decltype(tc)::value;
            if constexpr (t + 1 < 4) read_x(slot, t + 1, xf[(t + 1) & 1]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    if constexpr (XDT == PSQ_BF16)
                        acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[t & 1][mt], wfs[j][t], acc[mt][j], 0, 0, 0);
                    else
                        acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[t & 1][mt], wfs[j][t], acc[mt][j], 0, 0, 0);
                }
        });
    };
    // step s landed for every wave: this wave's loads per step are 2 + xd (+ 1 per step, SZ_STEP; + 1
    // with the first step of a scale block, waves 0-3, SZ_BLOCK: at most one such step among the
    // `younger` steps issued after s, which are fewer than 4 hg), then the barrier
    auto wait_step = [&](auto youngerc, int s) {
        constexpr int younger = decltype(youngerc)::value, L = SZM == SZ_STEP ? 3 : 2;
        int extra = 0;
        if constexpr (SZM == SZ_BLOCK) {
#pragma unroll
            for (int q = 1; q <= younger; q++) extra += sz_extra_at(s + q) ? 1 : 0;
        }
        const int sel = xd + (extra ? 5 : 0);
        switch (sel) {
        case 0: wait_vmcnt<younger * L>(); break;
        case 1: wait_vmcnt<younger * (L + 1)>(); break;
        case 2: wait_vmcnt<younger * (L + 2)>(); break;
        case 3: wait_vmcnt<younger * (L + 3)>(); break;
        case 4: wait_vmcnt<younger * (L + 4)>(); break;
        case 5: wait_vmcnt<younger * L + 1>(); break;
        case 6: wait_vmcnt<younger * (L + 1) + 1>(); break;
        case 7: wait_vmcnt<younger * (L + 2) + 1>(); break;
        case 8: wait_vmcnt<younger * (L + 3) + 1>(); break;
        default: wait_vmcnt<younger * (L + 4) + 1>(); break;
        }
        stage_barrier();
    };

    // Software pipeline: step s + 1 is waited for (and its weights read) before step s computes, so
    // the LDS reads overlap step s's work.  A step's activation fragments are read while it
    // computes, so the slot of step s - 1 is refilled (with step s - 1 + NX) only after the barrier
    // of step s, which every wave reaches after finishing step s - 1; the last step has no barrier
    // and refills nothing.  Past the end the refills load the last step again (the vmcnt waits count
    // a constant number of younger steps).
    if constexpr (SZT) {
        // the tables: ROWS G halves per array, contiguous from the workgroup's first row, in 1 KB
        // loads spread over the waves; lanes past the last row read the last 16 bytes instead (their
        // columns are never stored).  Issued before step 0, so step 0's wait covers them (loads
        // complete in order).
        const int tb = ROWS * G * 2, nl = (tb + 1023) / 1024;
        const int64_t valid = (int64_t)min(ROWS, N - wg_row0) * G * 2;
        for (int i = wave; i < 2 * nl; i += NW) {
            const int arr = i >= nl, off = (i - arr * nl) * 1024 + 16 * lane;
            const uint8_t *src = (const uint8_t *)((arr ? wa.zero16 : wa.scale16) + (int64_t)wg_row0 * G);
            if (off < tb)
                __builtin_amdgcn_global_load_lds((glb_ptr)(src + min((int64_t)off, valid - 16)),
                                                 (lds_ptr)(smem + NX * SL + arr * tb + (i - arr * nl) * 1024), 16, 0, 0);
        }
    }
#pragma unroll
    for (int st = 0; st < DD; st++) issue(st, st);
    Ops oa, ob;
    wait_step(std::integral_constant<int, DD - 1>{}, 0);
    read_w(0, oa);
    int cslot = 0, fslot = DD;                               // slot of step s, slot to refill
    auto step = [&](int st, const Ops &cur, Ops &nxt) {
        const int nslot = cslot == NX - 1 ? 0 : cslot + 1;
        if (st + 1 < ns) {
            wait_step(std::integral_constant<int, DD - 2>{}, st + 1);
            read_w(nslot, nxt);
            issue(st - 1 + NX, fslot);
            fslot = fslot == NX - 1 ? 0 : fslot + 1;
        }
        compute(cslot, cur);
        cslot = nslot;
    };
    for (int st = 0; st < ns; st += 2) {
        step(st, oa, ob);
        if (st + 1 < ns) step(st + 1, ob, oa);
    }
    // the two parities' partial sums: parity 1 writes, parity 0 adds (fixed order), once every load
    // has landed and every wave is done with the ring
    wait_vmcnt<0>();
    __syncthreads();
    float *const red = (float *)smem + cg * (MT * 2 * 4 * 64);
    if (par == 1) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int v = 0; v < 4; v++) red[((mt * 2 + j) * 4 + v) * 64 + lane] = acc[mt][j][v];
    }
    __syncthreads();
    if (par == 1) return;
    // y[m][n] = round_out((acc_0 + acc_1) + bias[n]); lane: n = column tile j's row nr, m = 16 mt + 4 h + v
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int n = wg_row0 + 32 * cg + 16 * j + nr;
        if (n >= N) continue;
        const float bb = wa.bias ? load_elem(wa.bias, n, wa.bias_dtype) : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = 16 * mt + 4 * h + v;
                if (m < M)
                    store_elem(wa.y, (int64_t)m * wa.ldy + n, wa.y_dtype,
                               (acc[mt][j][v] + red[((mt * 2 + j) * 4 + v) * 64 + lane]) + bb);
            }
    }
}

// ------------------------------------------------------ uint4 decode kernel (M <= 8)
// Decode shapes (a few tokens against the whole weight).  Work items are (16-column unit, 256-k
// block) pairs, unit after unit.  One workgroup per CU (8 waves) takes a contiguous range of units
// (U / G of them, G = min(CUs, units)), loads the activations (M rows, at most 80 KB at K = 5120)
// into LDS once behind one barrier, and its waves split the range's items into 8 equal contiguous
// runs.  After that the waves never meet until the end: each streams its run through a private LDS
// ring of D blocks that it alone fills and reads, so a block is ready when the wave's own load
// counter says so (no barrier per block).
//  * The balance: N = 25600 is 1600 units; in 128-column workgroups of one unit per wave that left 56
//    of 256 CUs idle, with every wave 20 blocks long.  Here every CU works, a wave runs at most 18
//    blocks, and a unit split between waves of one CU is added up through LDS after the loop, by the
//    wave holding the unit's last block, over the waves' partial sums in the fixed order
//    ((p_{n-1} + p_{n-2}) + ..) + p_0 -- no global traffic (units split across CUs, with their
//    partials through memory and atomic counts, measured slower: at ~20 us a launch, each of their
//    end-of-run round trips cost 1-3 us).
//  * Scales and zeros: with G a multiple of 8 up to 40 and at most 8 units per CU, the CU's rows of
//    both tables (contiguous in memory) go to LDS once with the activations (SZT); else each block
//    loads its 16 rows' values into the ring (2-byte loads: ~16 cache lines each, as many as the
//    block's weights).
//  * The ring starts with two blocks and grows by one extra block per step up to D: issuing all D
//    blocks before the first compute took ~12K cycles.  The two waves of a SIMD take turns at the
//    higher issue priority: left to age order the older one ran ahead and the younger one finished
//    alone.
// The arithmetic is the streaming kernel's (w = round_16(fmaf(q, s, -z s)), 16x16x32 MFMA with the
// activations as the A operand, lane group h carrying k = 64 h + 8 t of the block in k-step t).
namespace wd {
constexpr int NW = 8;                                 // waves per workgroup
constexpr int B = 256;                                // k per block
constexpr int WBYTES = 16 * B / 2;                    // a wave's nibbles per block (2 KB)
constexpr int SZW = 256;                              // a block's scale / zero words (no table)
constexpr int MAXM = 8;
constexpr int TROWS = 128;                            // rows of the scale / zero table
constexpr int SZT_MAX = 2 * TROWS * 40 * 2;           // 20 KB: G <= 40
__host__ __device__ inline int64_t xrow(int64_t K) { return 2 * K + 16; } // padded activation row in LDS (bytes)
constexpr int MAXU = 32;                              // units per workgroup
constexpr int BIASB = MAXU * 16 * 4;                  // the workgroup's bias values, one word each
inline int64_t lds_bytes(int64_t M, int64_t K, int D, bool szt)
{
    return M * xrow(K) + (int64_t)NW * D * (WBYTES + (szt ? 0 : SZW)) + (szt ? SZT_MAX : 0) + BIASB;
}
// The wave's 16 weight rows are 128 bytes each, lane (n, h) reading chunks 2 h and 2 h + 1 of row n:
// chunk c of row r sits at c ^ dsw(r), row bits (3, 1, 2) -> chunk bits (0, 1, 2), a placement free of
// bank conflicts for gfx950's ds_read_b128 lane groups (the earlier c ^ ((r >> 1) & 7) conflicted
// two ways).
__device__ __forceinline__ int dsw(int r) { return ((r >> 3) & 1) | (r & 6); }
// run g of W over T items is [run_start(g), run_start(g + 1)); run_owner(t) is the run holding item t
__host__ __device__ inline int64_t run_start(int64_t g, int64_t T, int64_t W) { return g * T / W; }
__host__ __device__ inline int64_t run_owner(int64_t t, int64_t T, int64_t W) { return ((t + 1) * W + T - 1) / T - 1; }
}  // namespace wd

template <int XDT, int D, bool SZT>
__global__ void __launch_bounds__(wd::NW * 64)
gemm_w4_decode(const uint16_t *__restrict__ x, int64_t ldx, int M, int N, int K, WArgs wa)
{
    using namespace wd;
    using XV = typename std::conditional<XDT == PSQ_BF16, v8bf, v8h>::type;
    constexpr int WS = WBYTES + (SZT ? 0 : SZW);          // ring slot bytes
    constexpr int LOADS = SZT ? 2 : 3;                   // ring loads per block
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nr = lane & 15, h = lane >> 4;
    const int nb = K / B, G = K / wa.gs, hg = wa.gs / 128;
    const int64_t wld = K / 2, xr = xrow(K);
    // the workgroup's units [ua, ub) (G = gridDim.x workgroups over the units), their I items, this
    // wave's run [t0, t1) of them (absolute item numbers)
    // (the runs of one workgroup in 32-bit arithmetic: I < 2^28 / NW, checked by the host)
    const int64_t units = (N + 15) / 16;
    const int64_t ua = run_start(blockIdx.x, units, gridDim.x), ub = run_start(blockIdx.x + 1, units, gridDim.x);
    const int I = (int)((ub - ua) * nb);
    auto wrun = [&](int w) { return w * I / NW; };                     // run start of wave w (relative)
    auto wowner = [&](int t) { return ((t + 1) * NW + I - 1) / I - 1; };  // the wave holding relative item t
    const int64_t t0 = ua * nb + wrun(wave), t1 = ua * nb + wrun(wave + 1);
    uint8_t *const tab = smem + (int64_t)M * xr;                                  // [scale | zero][row][G]
    uint8_t *const bl = tab + (SZT ? SZT_MAX : 0);                                // bias, word per column
    uint8_t *const ring0 = bl + BIASB;
    uint8_t *const ring = ring0 + (int64_t)wave * D * WS;
    const int64_t trow0 = 16 * ua;                     // the table's first row

    // the bias of the workgroup's columns, column i of the range in word i (global->LDS: a register
    // load at a unit's end made the compiler drain the wave's ring before the store)
    if (wa.bias && 64 * wave < 16 * (ub - ua)) {
        const int64_t n = min(16 * ua + 64 * wave + lane, (int64_t)N - 1);
        if (wa.bias_dtype == PSQ_F32)
            __builtin_amdgcn_global_load_lds((glb_ptr)((const float *)wa.bias + n), (lds_ptr)(bl + 256 * wave), 4, 0, 0);
        else
            __builtin_amdgcn_global_load_lds((glb_ptr)((const uint16_t *)wa.bias + n), (lds_ptr)(bl + 256 * wave), 2, 0, 0);
    }

    // the activations: row m at m * xr, 1 KB per wave load (K % 512 == 0: whole loads per row)
    const int per_row = (int)(2 * (int64_t)K / 1024), nx = M * per_row;
    for (int j = wave; j < nx; j += NW) {
        const int m = j / per_row, c = j - m * per_row;
        __builtin_amdgcn_global_load_lds((glb_ptr)((const uint8_t *)x + (int64_t)m * ldx * 2 + c * 1024 + lane * 16),
                                         (lds_ptr)(smem + (int64_t)m * xr + c * 1024), 16, 0, 0);
    }
    if constexpr (SZT) {
        // TROWS G halves per array from row trow0, in 1 KB loads; lanes past the last row read the
        // last 16 bytes instead (their columns are never stored; G % 8 == 0 keeps every load aligned)
        const int tb = TROWS * G * 2, nl = (tb + 1023) / 1024;
        const int64_t valid = min((int64_t)TROWS, (int64_t)N - trow0) * G * 2;
        for (int i = wave; i < 2 * nl; i += NW) {
            const int arr = i >= nl, j = i - arr * nl, off = j * 1024 + 16 * lane;
            const uint8_t *src = (const uint8_t *)((arr ? wa.zero16 : wa.scale16) + trow0 * G);
            if (off < tb)
                __builtin_amdgcn_global_load_lds((glb_ptr)(src + min((int64_t)off, valid - 16)),
                                                 (lds_ptr)(tab + arr * tb + j * 1024), 16, 0, 0);
        }
    }
    // a block's ring loads: item t (past the end of the run: its last item again, into a slot nobody
    // reads).  Weights: rows 8 d + L / 8 (d = 0, 1) of the unit, physical chunk L % 8, holding
    // logical chunk pc ^ dsw(row); rows past N clamp to the last row.  Without the table, lane L also
    // fetches array L >> 5 (scale, zero), row (L >> 1) & 15 and 128-k half L & 1 into word L.
    // the next item to issue, as unit ic and block ikb (running: no division per block); past the end
    // of the run the last item is issued again
    int64_t ti = t0;
    int64_t ic = t0 / nb;
    int ikb = (int)(t0 - ic * nb);
    int igq = 0, igr = 0;                              // (2 ikb) / hg and (2 ikb) % hg (no table)
    if constexpr (!SZT) { igq = (2 * ikb) / hg; igr = (2 * ikb) % hg; }
    // weights of unit ic: the unit's first row as the base, the lanes' row offsets (rows past N
    // clamped) set again only when the unit changes
    const uint8_t *ubase = nullptr;
    uint32_t wo[2];
    auto set_unit = [&] {
        ubase = wa.wq + (16 * ic) * wld;
#pragma unroll
        for (int d = 0; d < 2; d++) {
            const int r = 8 * d + (lane >> 3);
            wo[d] = (uint32_t)((min(16 * ic + r, (int64_t)N - 1) - 16 * ic) * wld + (((lane & 7) ^ dsw(r)) << 4));
        }
    };
    if (t0 < t1) set_unit();
    auto issue = [&](int slot) {
        uint8_t *const sl = ring + slot * WS;
        const uint8_t *const wb = ubase + ikb * (B / 2);
#pragma unroll
        for (int d = 0; d < 2; d++)
            __builtin_amdgcn_global_load_lds((glb_ptr)(wb + wo[d]), (lds_ptr)(sl + 1024 * d), 16, 0, 0);
        if constexpr (!SZT) {
            const int64_t row = min(16 * ic + ((lane >> 1) & 15), (int64_t)N - 1);
            const int g = min(igq + ((lane & 1) && igr + 1 >= hg ? 1 : 0), G - 1);
            __builtin_amdgcn_global_load_lds((glb_ptr)((lane < 32 ? wa.scale16 : wa.zero16) + row * G + g),
                                             (lds_ptr)(sl + WBYTES), 2, 0, 0);
        }
        if (++ti < t1) {
            if (++ikb == nb) {
                ikb = 0;
                ic++;
                igq = igr = 0;
                set_unit();
            } else if constexpr (!SZT) {
                igr += 2;
                if (igr >= hg) { igr -= hg; igq++; }
                if (igr >= hg) { igr -= hg; igq++; }
            }
        }
    };
    // The ring starts with two blocks and grows by one extra block per step until D are in flight:
    // issuing all D blocks before the first compute took ~12K cycles (~160 global->LDS loads per CU).
    // Block b goes to slot b % D; before the wait of step j (for block j + 1) min(2 + 2 j, j + D) blocks
    // are issued, min(j, D - 2) of them younger than block j + 1.
    // (a wave with an empty run -- fewer items than waves -- loads no ring blocks at all)
    const bool active = t0 < t1;
    int nissued = 0;
    auto issue_next = [&] { issue(nissued % D); nissued++; };
    if (active) {
        issue_next();
        issue_next();
        wait_vmcnt<LOADS * 2>();        // this wave's activation and table loads (issued first) landed
    } else {
        wait_vmcnt<0>();
    }
    stage_barrier();                    // ... and every other wave's

    struct Ops { XV xf[8]; v4i wv[2]; float sc, sc4, zs; };
    const uint8_t *const xrow_p = smem + (int64_t)min(nr, M - 1) * xr;
    // the next item to read, as unit rc and block rkb, and the table group of its 128-k half 0
    // (running, as for the issues)
    int64_t rc = t0 / nb;
    int rkb = (int)(t0 - rc * nb);
    int rgq = (2 * rkb) / hg, rgr = (2 * rkb) % hg;
    auto read = [&](int slot, bool advance, Ops &o) {
        const uint8_t *const sl = ring + slot * WS;
#pragma unroll
        for (int s = 0; s < 8; s++)
            o.xf[s] = __builtin_bit_cast(XV, *(const v4i *)(xrow_p + ((int64_t)rkb * B + 64 * h + 8 * s) * 2));
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int cc = 2 * h + i;
            o.wv[i] = *(const v4i *)(sl + nr * (B / 2) + ((cc ^ dsw(nr)) << 4));
        }
        float sv, zv;
        if constexpr (SZT) {
            const int row = (int)(16 * rc - trow0) + nr, g = rgq + ((h >> 1) && rgr + 1 >= hg ? 1 : 0);
            const uint16_t *tb16 = (const uint16_t *)tab;
            sv = f16_to_f32(tb16[row * G + g]);
            zv = f16_to_f32(tb16[(TROWS + row) * G + g]);
        } else {
            const int si = (nr << 1) | (h >> 1);
            const uint32_t *sz = (const uint32_t *)(sl + WBYTES);
            sv = f16_to_f32(sz[si]);
            zv = f16_to_f32(sz[32 + si]);
        }
        o.zs = -(zv * sv);
        o.sc = sv * kTwo24;                 // s 2^24 and s 2^20 (dq_pair_u4)
        o.sc4 = sv * kTwo20;
        if (advance) {
            if (++rkb == nb) {
                rkb = 0;
                rc++;
                rgq = rgr = 0;
            } else {
                rgr += 2;
                if (rgr >= hg) { rgr -= hg; rgq++; }
                if (rgr >= hg) { rgr -= hg; rgq++; }
            }
        }
    };
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const Ops &o) {
        XV wfs[8];
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const Nib4 v = nib_split((uint32_t)o.wv[s >> 2][s & 3]);
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; e++) w[e] = dq_pair_u4<XDT>(v, e, o.sc, o.sc4, o.zs);
            wfs[s] = __builtin_bit_cast(XV, v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            if constexpr (XDT == PSQ_BF16) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(o.xf[s], wfs[s], acc, 0, 0, 0);
            else acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.xf[s], wfs[s], acc, 0, 0, 0);
        }
    };
    // y[m][n] = round_out(v + bias[n]) for unit c; lane: n = 16 c + nr, m = 4 h + r
    auto store = [&](int64_t c, v4f v) {
        const int64_t n = 16 * c + nr;
        if (n >= N) return;
        float bb = 0.0f;
        if (wa.bias) {
            const uint32_t bw = ((const uint32_t *)bl)[16 * (c - ua) + nr];
            bb = wa.bias_dtype == PSQ_F32 ? __uint_as_float(bw) : wa.bias_dtype == PSQ_BF16 ? bf16_to_f32(bw & 0xffffu)
                                                                                             : f16_to_f32(bw);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 4 * h + r;
            if (m < M) store_elem(wa.y, (int64_t)m * wa.ldy + n, wa.y_dtype, v[r] + bb);
        }
    };

    // Pipeline: block t + 1 is read while block t computes; block t's slot is refilled once its
    // registers have been used (after compute).  Block t + 1 has landed when at most D - 2 younger
    // blocks of this wave are in flight.  At the end of a unit (or of the run) the segment's sum is
    // stored (a whole unit), kept (a partial first segment) or left in acc (a partial last one).
    Ops oa, ob;
    int slot = 0;
    v4f acc0 = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    bool first_partial = false, last_partial = false;
    if (t0 < t1) {
        wait_vmcnt<LOADS * 1>();
        read(0, true, oa);
    }
    // this wave's loads of block j + 1 landed: min(j, D - 2) younger blocks may be in flight
    auto wait_next = [&](int j) {
        switch (min(j, D - 2)) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<LOADS * 1>(); break;
        case 2: wait_vmcnt<LOADS * 2>(); break;
        case 3: wait_vmcnt<LOADS * 3>(); break;
        case 4: wait_vmcnt<LOADS * 4>(); break;
        case 5: wait_vmcnt<LOADS * 5>(); break;
        default: wait_vmcnt<LOADS * 6>(); break;
        }
    };
    // the item computed, as unit cc and block ckb; whether the current segment began at a unit's start
    int64_t cc = t0 / nb;
    int ckb = (int)(t0 - cc * nb);
    bool seg_whole_start = ckb == 0;
    auto step = [&](int64_t t, const Ops &cur, Ops &nxt) {
        const int nslot = slot == D - 1 ? 0 : slot + 1;
        const int j = (int)(t - t0);
        // the two waves of a SIMD (w, w + 4) take turns at the higher issue priority, two blocks each:
        // left to age order the older wave ran ahead and the younger one finished alone
        if (((j >> 1) ^ (wave >> 2)) & 1) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
        wait_next(j);
        read(nslot, t + 2 < t1, nxt);                  // item t + 1 (past the end: read again, unused)
        compute(cur);
        issue_next();                                  // block j + D at the latest: slot j % D is free
        if (nissued <= j + D) issue_next();            // the ramp
        slot = nslot;
        const bool unit_end = ckb == nb - 1;
        if (t == t1 - 1 || unit_end) {
            if (seg_whole_start && unit_end) {
                store(cc, acc);
                acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            } else if (t != t1 - 1) {                  // a partial segment that ends before the run: the first
                acc0 = acc;
                first_partial = true;
                acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            } else {
                last_partial = true;                   // the run's last segment (or its only one)
            }
            seg_whole_start = true;
        }
        if (++ckb == nb) {
            ckb = 0;
            cc++;
        }
    };
    for (int64_t t = t0; t < t1; t += 2) {
        step(t, oa, ob);
        if (t + 1 < t1) step(t + 1, ob, oa);
    }
    __builtin_amdgcn_s_setprio(0);
    wait_vmcnt<0>();                                    // the re-issued tail loads, before any partial traffic

    // ---- units split between this CU's waves: each wave's partial first segment (unit t0 / nb) and
    // partial last one (unit (t1 - 1) / nb) go to LDS slot 2 w + (0: the run's first unit, 1: else),
    // 1 KB in the lanes' order, once every wave is done with its ring; the wave holding a unit's last
    // block then adds the unit up in wave order (its own partial from registers) and stores it.
    __syncthreads();
    float *const red = (float *)ring0;
    // units relative to ua (int): the run's first and last, and the first unit of wave w's run
    const int rf = wrun(wave) / nb, rl = t0 < t1 ? (wrun(wave + 1) - 1) / nb : rf;
    auto slot_of = [&](int w, int c) { return 2 * w + (wrun(w) / nb == c ? 0 : 1); };
    auto put = [&](int c, v4f v) { *(v4f *)(red + (slot_of(wave, c) * 64 + lane) * 4) = v; };
    if (first_partial) put(rf, acc0);
    if (last_partial) put(rl, acc);
    __syncthreads();
    auto addup = [&](int c, v4f v) {
        const int lf = wowner(c * nb), ll = wowner(c * nb + nb - 1);
        v4f sum = v;                                   // this wave holds the unit's last block: p_{n-1}
        for (int w = ll - 1; w >= lf; w--)             // (waves with empty runs hold no partial)
            if (wrun(w + 1) > wrun(w)) sum = sum + *(const v4f *)(red + (slot_of(w, c) * 64 + lane) * 4);
        store(ua + c, sum);
    };
    // a partial segment ending at its unit's last block: the first one (always), or the only one
    if (first_partial) addup(rf, acc0);
    if (last_partial && wrun(wave + 1) % nb == 0) addup(rl, acc);
}

// The decode kernel's ring depth for M rows of K (0: the shape does not fit).
int decode_depth(int64_t M, int64_t K, bool szt)
{
    for (int d : {8, 6, 4, 3})
        if (wd::lds_bytes(M, K, d, szt) <= 163840) return d;
    return 0;
}

// Launch plan of the decode kernel: G workgroups (one per CU while there are units) and the scale /
// zero form (the table when G is a multiple of 8 up to 40, the tables are 16-byte aligned and a
// workgroup's units are at most TROWS / 16).
struct DecodePlan {
    int64_t G = 0;              // workgroups
    bool szt = false;
    int depth = 0;
};
DecodePlan plan_decode(int64_t M, int64_t N, int64_t K, int gs, const void *scale, const void *zero, int cus)
{
    DecodePlan p;
    const int64_t units = (N + 15) / 16, G = K / gs;
    p.G = std::min<int64_t>(units, cus);
    const int64_t upw = (units + p.G - 1) / p.G;                 // units per workgroup, at most
    if (upw * (K / wd::B) * wd::NW >= (1LL << 31)) p.G = 0;      // a workgroup's runs need 32-bit item numbers
    if (upw > wd::MAXU) p.G = 0;                                  // its bias words in LDS
    p.szt = G % 8 == 0 && G <= 40 && upw <= wd::TROWS / 16 && ((uintptr_t)scale & 15) == 0 &&
            ((uintptr_t)zero & 15) == 0;
    p.depth = decode_depth(M, K, p.szt);
    if (p.depth == 0 && p.szt) {
        p.szt = false;
        p.depth = decode_depth(M, K, false);
    }
    return p;
}

template <int XDT, int D, bool SZT>
int launch_decode_d(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa, hipStream_t st,
                    const char *name)
{
    auto kern = gemm_w4_decode<XDT, D, SZT>;
    const int lds = (int)wd::lds_bytes(M, K, D, SZT);
    if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 163840) != hipSuccess)
        return set_error(PSQ_E_DEVICE, "%s: cannot reserve LDS", name);
    const dim3 grid((unsigned)wa.sk), block(wd::NW * 64);
    kern<<<grid, block, lds, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
    return check_launch(name);
}

template <int XDT>
int launch_decode(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, WArgs wa, const DecodePlan &p,
                  hipStream_t st, const char *name)
{
    wa.sk = (int)p.G;
    auto go = [&](auto szc) {
        constexpr bool S = decltype(szc)::value;
        switch (p.depth) {
        case 8: return launch_decode_d<XDT, 8, S>(x, ldx, M, N, K, wa, st, name);
        case 6: return launch_decode_d<XDT, 6, S>(x, ldx, M, N, K, wa, st, name);
        case 4: return launch_decode_d<XDT, 4, S>(x, ldx, M, N, K, wa, st, name);
        default: return launch_decode_d<XDT, 3, S>(x, ldx, M, N, K, wa, st, name);
        }
    };
    return p.szt ? go(std::true_type{}) : go(std::false_type{});
}

// ------------------------------------------------------ uint4 decode kernel, K split over the waves
// One or two tokens (M <= 2) with 1024 <= K <= 6144.  One workgroup per CU takes a contiguous range
// of 16-column units (as the kernel above); its 8 waves split K instead of the items: wave w owns
// the 128-k half blocks [w H / 8, (w + 1) H / 8) of every unit (H = K / 128, at most XMAX), so it
// loads its activation fragments into registers once, from global memory, and its loop reads only
// weights (and scales) from LDS.  Each wave streams its (unit, half block) items, unit after unit,
// through a private ring of D 1 KB slots (16 rows x 64 bytes: one global->LDS load each), all D in
// flight from the start.  At the end of a unit the waves' partial sums meet in LDS behind one
// barrier, and one wave adds them in wave order and stores the unit.  The arithmetic per weight is
// the kernel above's (w = round_16(fmaf(q, s, -z s)), 16x16x32 MFMA, activations as the A operand).
// Measured at N = 25600, K = 5120 on one host, alternating launches: M = 1 21.4 us against 23.8 us
// of the kernel above, M = 2 21.9 / 22.7 us; at M = 4 it was even and at M = 8 slower (24.1 /
// 22.3 us), so those stay with the kernel above.  Ring depths 4 / 6 / 8 gave 21.4 / 22.0 / 22.1 us.
namespace wx {
constexpr int NW = 8;                          // waves per workgroup
constexpr int HB = 128;                        // k per item (half block)
constexpr int XMAX = 6;                        // half blocks per wave: K <= NW * XMAX * HB = 6144
constexpr int MAXM = 2;                        // rows
constexpr int WB = 16 * HB / 2;                // an item's nibbles (1 KB)
constexpr int SZW = 256;                       // an item's scale / zero words (no table)
constexpr int RED = 2 * NW * 1024;             // two sets of the waves' partial sums
constexpr int BIASB = wd::BIASB;               // the workgroup's bias values (at most wd::MAXU units)
constexpr int D = 4;                           // ring depth
inline int lds_bytes(bool szt) { return (szt ? wd::SZT_MAX : 0) + RED + BIASB + NW * D * (WB + (szt ? 0 : SZW)); }
// chunk c (16 bytes) of row r of an item sits at position c ^ psw(r): the 16 lanes (r, c) of one
// ds_read_b128 lane group then cover the 64 banks once
__device__ __forceinline__ int psw(int r) { return (r >> 2) & 3; }
}  // namespace wx

template <int XDT, bool SZT>
__global__ void __launch_bounds__(wx::NW * 64)
gemm_w4_decode_ks(const uint16_t *__restrict__ x, int64_t ldx, int M, int N, int K, WArgs wa)
{
    using namespace wx;
    using XV = typename std::conditional<XDT == PSQ_BF16, v8bf, v8h>::type;
    constexpr int WS = WB + (SZT ? 0 : SZW);
    constexpr int LOADS = SZT ? 1 : 2;                 // ring loads per item
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nr = lane & 15, h = lane >> 4;
    const int G = K / wa.gs, hg = wa.gs / HB, H = K / HB;
    const int64_t wld = K / 2;
    const int64_t units = (N + 15) / 16;
    const int64_t ua = wd::run_start(blockIdx.x, units, gridDim.x), ub = wd::run_start(blockIdx.x + 1, units, gridDim.x);
    const int h0 = wave * H / NW, cnt = (wave + 1) * H / NW - h0;    // K >= 1024: cnt >= 1
    const int I = (int)(ub - ua) * cnt;                              // this wave's items
    uint8_t *const tab = smem;                                       // [scale | zero][row][G] (SZT)
    float *const red = (float *)(smem + (SZT ? wd::SZT_MAX : 0));
    uint8_t *const bl = smem + (SZT ? wd::SZT_MAX : 0) + RED;
    uint8_t *const ring = bl + BIASB + wave * D * WS;
    const int64_t trow0 = 16 * ua;

    // the bias of the workgroup's columns, column i of the range in word i (global->LDS: a register
    // load would make the compiler drain the ring before the first store that uses it)
    if (wa.bias && 64 * wave < 16 * (ub - ua)) {
        const int64_t n = min(16 * ua + 64 * wave + lane, (int64_t)N - 1);
        if (wa.bias_dtype == PSQ_F32)
            __builtin_amdgcn_global_load_lds((glb_ptr)((const float *)wa.bias + n), (lds_ptr)(bl + 256 * wave), 4, 0, 0);
        else
            __builtin_amdgcn_global_load_lds((glb_ptr)((const uint16_t *)wa.bias + n), (lds_ptr)(bl + 256 * wave), 2, 0, 0);
    }
    // the scale and zero rows of the workgroup's units (as the kernel above)
    if constexpr (SZT) {
        const int tb = wd::TROWS * G * 2, nl = (tb + 1023) / 1024;
        const int64_t valid = min((int64_t)wd::TROWS, (int64_t)N - trow0) * G * 2;
        for (int i = wave; i < 2 * nl; i += NW) {
            const int arr = i >= nl, j = i - arr * nl, off = j * 1024 + 16 * lane;
            const uint8_t *src = (const uint8_t *)((arr ? wa.zero16 : wa.scale16) + trow0 * G);
            if (off < tb)
                __builtin_amdgcn_global_load_lds((glb_ptr)(src + min((int64_t)off, valid - 16)),
                                                 (lds_ptr)(tab + arr * tb + j * 1024), 16, 0, 0);
        }
    }
    // the activation fragments: lane (n, h) of k-step t of half block j carries k = 128 (h0 + j) +
    // 32 h + 8 t .. + 7 of row min(n, M - 1); entries past the wave's last half block repeat it
    // (loaded, never used).  Loaded before the ring, so the wait below covers them.
    XV xf[XMAX][4];
    {
        const uint16_t *xr = x + (int64_t)min(nr, M - 1) * ldx + 32 * h;
#pragma unroll
        for (int j = 0; j < XMAX; j++)
#pragma unroll
            for (int t = 0; t < 4; t++)
                xf[j][t] = __builtin_bit_cast(XV, *(const v4i *)(xr + (h0 + min(j, cnt - 1)) * HB + 8 * t));
    }
    // the ring: item ti = (unit iu, half block h0 + ij); past the last item the last again (into a
    // slot nobody reads).  The unit's row addresses (rows past N clamped) are set when it changes.
    int ti = 0, ij = 0;
    int64_t iu = ua;
    const int lr = lane >> 2, lc = (lane & 3) ^ psw(lane >> 2);
    const uint8_t *wrow = nullptr;
    const uint16_t *srow = nullptr;
    auto set_unit = [&] {
        wrow = wa.wq + min(16 * iu + lr, (int64_t)N - 1) * wld + h0 * (HB / 2) + 16 * lc;
        if constexpr (!SZT) srow = (h & 1 ? wa.zero16 : wa.scale16) + min(16 * iu + nr, (int64_t)N - 1) * G;
    };
    set_unit();
    auto issue = [&](int slot) {
        uint8_t *const sl = ring + slot * WS;
        __builtin_amdgcn_global_load_lds((glb_ptr)(wrow + ij * (HB / 2)), (lds_ptr)sl, 16, 0, 0);
        if constexpr (!SZT)     // lane 16 a + n: array a & 1 (scale, zero) of row n, into word lane
            __builtin_amdgcn_global_load_lds((glb_ptr)(srow + (h0 + ij) / hg), (lds_ptr)(sl + WB), 2, 0, 0);
        if (ti + 1 < I) {
            ti++;
            if (++ij == cnt) {
                ij = 0;
                iu++;
                set_unit();
            }
        }
    };
    __builtin_amdgcn_sched_barrier(0);       // the ring loads after the activation loads (the wait counts on it)
    for (int s = 0; s < D; s++) issue(s);
    wait_vmcnt<LOADS * D>();                 // this wave's bias, table and activation loads landed
    stage_barrier();                         // ... and every other wave's

    auto store = [&](int64_t c, v4f v) {
        const int64_t n = 16 * c + nr;
        if (n >= N) return;
        float bb = 0.0f;
        if (wa.bias) {
            const uint32_t bw = ((const uint32_t *)bl)[16 * (c - ua) + nr];
            bb = wa.bias_dtype == PSQ_F32 ? __uint_as_float(bw) : wa.bias_dtype == PSQ_BF16 ? bf16_to_f32(bw & 0xffffu)
                                                                                             : f16_to_f32(bw);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 4 * h + r;
            if (m < M) store_elem(wa.y, (int64_t)m * wa.ldy + n, wa.y_dtype, v[r] + bb);
        }
    };
    const int wpos = 16 * (h ^ psw(nr));
    int slot = 0;
    for (int64_t u = ua; u < ub; u++) {
        v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < XMAX; j++) {
            if (j < cnt) {
                wait_vmcnt<LOADS * (D - 1)>();   // this item's loads landed
                const uint8_t *const sl = ring + slot * WS;
                const v4i wv = *(const v4i *)(sl + nr * 64 + wpos);
                float sv, zv;
                if constexpr (SZT) {
                    const uint16_t *tb16 = (const uint16_t *)tab;
                    const int row = (int)(16 * (u - ua)) + nr, g = (h0 + j) / hg;
                    sv = f16_to_f32(tb16[row * G + g]);
                    zv = f16_to_f32(tb16[(wd::TROWS + row) * G + g]);
                } else {
                    const uint32_t *sz = (const uint32_t *)(sl + WB);
                    sv = f16_to_f32(sz[nr]);
                    zv = f16_to_f32(sz[16 + nr]);
                }
                const float zs = -(zv * sv), s24 = sv * kTwo24, s20 = sv * kTwo20;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const Nib4 v = nib_split((uint32_t)wv[t]);
                    uint32_t w[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) w[e] = dq_pair_u4<XDT>(v, e, s24, s20, zs);
                    const XV wf = __builtin_bit_cast(XV, v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]});
                    if constexpr (XDT == PSQ_BF16) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xf[j][t], wf, acc, 0, 0, 0);
                    else acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j][t], wf, acc, 0, 0, 0);
                }
                // the slot's data are used; the refill may not move above that (lifted above the
                // compute, the load into LDS overtook the read of the same slot)
                __builtin_amdgcn_sched_barrier(0);
                issue(slot);
                slot = slot == D - 1 ? 0 : slot + 1;
            }
        }
        // the unit's partial sums, set (u - ua) % 2, wave after wave; one wave adds them in wave order
        float *const rb = red + ((u - ua) & 1) * NW * 256;
        *(v4f *)(rb + (wave * 64 + lane) * 4) = acc;
        stage_barrier();
        if (wave == (int)((u - ua) % NW)) {
            v4f s = *(const v4f *)(rb + lane * 4);
#pragma unroll
            for (int w = 1; w < NW; w++) s = s + *(const v4f *)(rb + (w * 64 + lane) * 4);
            store(u, s);
        }
    }
    wait_vmcnt<0>();                         // the re-issued tail loads, before the workgroup ends
}

// Whether the K-split decode kernel takes a decode shape (planned as for the kernel above): at most
// MAXM rows and half blocks that split over the waves within XMAX each.
bool decode_ks_fits(int64_t M, int64_t K, const DecodePlan &p)
{
    return p.G > 0 && M <= wx::MAXM && K % wx::HB == 0 && K >= wx::HB * wx::NW && K <= wx::HB * wx::NW * wx::XMAX;
}

template <int XDT, bool SZT>
int launch_decode_ks_s(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa, int64_t G,
                       hipStream_t st, const char *name)
{
    auto kern = gemm_w4_decode_ks<XDT, SZT>;
    const int lds = wx::lds_bytes(SZT);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(PSQ_E_DEVICE, "%s: no device", name);
    static bool attr_set[64] = {};
    if (dev < 64 && !attr_set[dev]) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
            return set_error(PSQ_E_DEVICE, "%s: cannot reserve %d bytes of LDS", name, lds);
        attr_set[dev] = true;
    }
    kern<<<dim3((unsigned)G), dim3(wx::NW * 64), lds, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
    return check_launch(name);
}

template <int XDT>
int launch_decode_ks(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa,
                     const DecodePlan &p, hipStream_t st, const char *name)
{
    return p.szt ? launch_decode_ks_s<XDT, true>(x, ldx, M, N, K, wa, p.G, st, name)
                 : launch_decode_ks_s<XDT, false>(x, ldx, M, N, K, wa, p.G, st, name);
}

template <int XDT, int MT, int SZM>
int launch_stream_mt(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa, hipStream_t st,
                     const char *name)
{
    auto kern = gemm_w4_stream<XDT, MT, SZM>;
    constexpr int lds = ws::lds_bytes<MT, SZM>();
    static_assert(lds <= 163840, "LDS of the streaming kernel");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(PSQ_E_DEVICE, "%s: no device", name);
    static bool attr_set[64] = {};
    if (dev < 64 && !attr_set[dev]) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
            return set_error(PSQ_E_DEVICE, "%s: cannot reserve %d bytes of LDS", name, lds);
        attr_set[dev] = true;
    }
    const dim3 grid((unsigned)((N + ws::ROWS - 1) / ws::ROWS)), block(ws::NW * 64);
    kern<<<grid, block, lds, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
    return check_launch(name);
}

// The scale / zero form: the table when the workgroup's tables fit beside a ring of three steps, the
// 8-group blocks otherwise; both need 16-byte-aligned tables whose rows are whole 16-byte chunks (G a
// multiple of 8; the clamped loads of the last workgroup then stay aligned and inside its rows).
template <int XDT, int MT>
int launch_stream_m(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa, hipStream_t st,
                    const char *name)
{
    const int64_t G = K / wa.gs;
    const bool dense = G % 8 == 0 && ((uintptr_t)wa.scale16 & 15) == 0 && ((uintptr_t)wa.zero16 & 15) == 0;
    if constexpr (ws::szt_fits<MT>())
        if (dense && 2 * ws::ROWS * G * 2 <= ws::SZT_MAX) return launch_stream_mt<XDT, MT, ws::SZ_TABLE>(x, ldx, M, N, K, wa, st, name);
    if (dense) return launch_stream_mt<XDT, MT, ws::SZ_BLOCK>(x, ldx, M, N, K, wa, st, name);
    return launch_stream_mt<XDT, MT, ws::SZ_STEP>(x, ldx, M, N, K, wa, st, name);
}

template <int XDT>
int launch_stream(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa, hipStream_t st,
                  const char *name)
{
    const int mt = (int)((M + 15) / 16);
    if (mt == 1) return launch_stream_m<XDT, 1>(x, ldx, M, N, K, wa, st, name);
    if (mt == 2) return launch_stream_m<XDT, 2>(x, ldx, M, N, K, wa, st, name);
    if (mt == 3) return launch_stream_m<XDT, 3>(x, ldx, M, N, K, wa, st, name);
    return launch_stream_m<XDT, 4>(x, ldx, M, N, K, wa, st, name);
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

constexpr int64_t SKINNY_MAX_M = 64;   // largest M of the streaming and skinny kernels

template <int XDT, int WK, int BM, bool SKM>
int launch_tiled_bm(const uint16_t *x, int64_t ldx, int64_t M, int64_t N, int64_t K, const WArgs &wa, hipStream_t st,
                    const char *name)
{
    auto kern = gemm_wonly_tiled<XDT, WK, BM, SKM>;
    constexpr int lds = wt::lds_bytes<WK, BM>() + (SKM ? 16 : 0);   // + the word that broadcasts a stream-K count
    static_assert(lds <= 163840, "LDS of the tiled kernel");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(PSQ_E_DEVICE, "%s: no device", name);
    static bool attr_set[64] = {};   // per device; the attribute is idempotent
    if (dev < 64 && !attr_set[dev]) {
        if (hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
            return set_error(PSQ_E_DEVICE, "%s: cannot reserve %d bytes of LDS", name, lds);
        attr_set[dev] = true;
    }
    const int64_t tiles = ((M + BM - 1) / BM) * ((N + wt::BN - 1) / wt::BN);
    kern<<<dim3((unsigned)(SKM ? wa.sk : tiles)), dim3(wt::THREADS), lds, st>>>(x, ldx, (int)M, (int)N, (int)K, wa);
    return check_launch(name);
}

// Launch plan of the tiled kernel, in units of one 128-row tile's K stage on a lightly loaded GPU.
//  * Data-parallel (one tile per workgroup): ceil(tiles / CUs) rounds of nk stages; a 256-row
//    tile's stage costs about kBm256Cost of a 128-row one (the dequantization serves twice the
//    rows: at N=25600 x K=5120, 126 us for a 256-row tile against 78 for a 128-row one).
//  * Stream-K, 128-row tiles only (the 256-row kernel has no registers to spare for it), over G
//    workgroups: ceil(tiles nk / G) stages each.  With G a multiple s of the tiles, each workgroup
//    takes one K range of one tile (one partial, written or added up); otherwise up to two
//    segments (a second ring prologue, two partials).  Each partial costs about kSkPartCost.
//  * The kernel is power-limited: with more than about 78% of the CUs busy the clock drops, a
//    stage taking about 1 + 0.6 (busy fraction - 0.78) times as long (M=128 x N=25600: 1.13 us a
//    stage on 200 CUs, 1.2-1.37 on 256).
// Stream-K is taken when it beats data-parallel by more than kSkMargin, and needs a workspace:
// the tiles' arrival counters (kSkCntBytes, room for kSkMaxTiles) and two fp32 partial tiles per
// workgroup.  Without stream-K, 128-row tiles while they fit one round of workgroups.
constexpr int kSkMinUnits = 8;                              // K stages per workgroup at least
constexpr double kSkPartCost = 3.0, kSkRestartCost = 2.0, kSkMargin = 0.9;
constexpr double kBm256Cost = 1.4;
constexpr int64_t kSkMaxTiles = 16384;
constexpr int64_t kSkCntBytes = kSkMaxTiles * 4;
constexpr int64_t kSkSlotBytes = 128LL * wt::BN * 4;        // one 128-row fp32 partial tile
constexpr int kSkMaxGroups = 256;
constexpr int64_t kMaxWsBytes = kSkCntBytes + 2 * kSkMaxGroups * kSkSlotBytes;   // 64 MB + 64 KB

inline double clock_factor(int64_t busy, int cus)
{
    const double f = (double)busy / cus - 0.78;
    return f > 0 ? 1.0 + 0.6 * f : 1.0;
}

struct TiledPlan {
    int bm = 128;
    int64_t tiles = 0;
    int sk = 0;                 // stream-K workgroups (0: data-parallel)
    int64_t ws_bytes = 0;
};

TiledPlan plan_tiled(int64_t M, int64_t N, int64_t K, int cus, bool allow_sk)
{
    TiledPlan p;
    const int64_t nbn = (N + wt::BN - 1) / wt::BN, nk = K / wt::BK;
    p.bm = ((M + 127) / 128) * nbn <= cus ? 128 : 256;
    p.tiles = ((M + p.bm - 1) / p.bm) * nbn;
    if (!allow_sk) return p;
    const double t_dp = (double)((p.tiles + cus - 1) / cus * nk) * (p.bm == 256 ? kBm256Cost : 1.0) *
                        clock_factor(std::min<int64_t>(p.tiles, cus), cus);
    const int64_t t128 = ((M + 127) / 128) * nbn, units = t128 * nk;
    if (t128 > kSkMaxTiles) return p;
    double best = kSkMargin * t_dp;
    int64_t best_g = 0;
    auto consider = [&](int64_t g, bool aligned) {
        if (g < 1 || g > cus || g > kSkMaxGroups || units / g < kSkMinUnits) return;
        const double t = (double)((units + g - 1) / g) * clock_factor(g, cus) +
                         (aligned ? kSkPartCost : 2 * kSkPartCost + kSkRestartCost);
        if (t < best) {
            best = t;
            best_g = g;
        }
    };
    for (int64_t sp = 2; t128 * sp <= cus; sp++) consider(t128 * sp, true);   // one K range of one tile each
    consider(cus, false);
    if (best_g) {
        p.bm = 128;
        p.tiles = t128;
        p.sk = (int)best_g;
        p.ws_bytes = kSkCntBytes + 2 * best_g * kSkSlotBytes;
    }
    return p;
}

// The weight-streaming kernel takes the uint4 shapes with M <= SKINNY_MAX_M and groups of a
// multiple of 128; the skinny kernel takes M <= SKINNY_MAX_M when K is a whole number of
// 128-element blocks (and, for uint4, the groups hold whole 32-element lane runs); the tiled
// kernel takes the rest.  One exception with a split-K workspace (`ws`): a streaming grid of at
// most half the CUs (N up to 64 x 128 columns on 256 CUs) over a long K (>= 8192) goes to the tiled
// kernel's stream-K, which spreads the K range over every CU (64 x 5120 x 13824: 103.8 -> 51.9 us;
// 64 x 5120 x 25600: 150.9 -> 62.5 us).  At K = 5120 the streaming kernel stays ahead (33.8 against
// 37.0 us at 64 x 5120), and without a workspace the tiled kernel could not split.
enum class Path { Decode, Stream, Skinny, Tiled };

Path choose_path(int wk, int64_t ldx, int64_t M, int64_t N, int64_t K, int gs, bool ws, int cus)
{
    if (wk == W_UINT4 && M <= wd::MAXM && gs % 128 == 0 && K % 512 == 0 && decode_depth(M, K, false) > 0 &&
        ldx <= (1LL << 22))
        return Path::Decode;
    if (wk == W_UINT4 && M <= SKINNY_MAX_M && gs % 128 == 0 && K % ws::STEP == 0 && ldx <= (1LL << 22)) {
        if (ws && cus > 0 && 2 * ((N + ws::ROWS - 1) / ws::ROWS) <= cus && K >= 8192 && K <= (1LL << 22) &&
            plan_tiled(M, N, K, cus, true).sk > 0)
            return Path::Tiled;
        return Path::Stream;
    }
    if (M <= SKINNY_MAX_M && K % SK_BLOCK == 0 && (wk != W_UINT4 || gs % 32 == 0)) return Path::Skinny;
    return Path::Tiled;
}

// Workspace bytes of a call (0: no split); the split needs a device, else 0.
int64_t workspace_bytes(int wk, int64_t ldx, int64_t M, int64_t N, int64_t K, int gs)
{
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const int cus = cu_count(dev);
    const Path path = choose_path(wk, ldx, M, N, K, gs, true, cus);
    if (path != Path::Tiled) return 0;
    return plan_tiled(M, N, K, cus, true).ws_bytes;
}

// workspace: NULL = data-parallel tiles only; else at least workspace_bytes(), its counter words
// (the first kSkCntBytes) zero when first passed: every launch leaves them zero, and writes every
// partial it reads.
template <int WK>
int launch(const void *x, int x_dtype, int64_t ldx, int64_t M, int64_t N, int64_t K, WArgs wa,
           void *workspace, int64_t ws_bytes, hipStream_t st, const char *name)
{
    const uint16_t *xp = (const uint16_t *)x;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(PSQ_E_DEVICE, "%s: no device", name);
    Path path = choose_path(WK, ldx, M, N, K, wa.gs, workspace != nullptr, cu_count(dev));
    if (path == Path::Decode) {
        const DecodePlan plan = plan_decode(M, N, K, wa.gs, wa.scale16, wa.zero16, cu_count(dev));
        if (decode_ks_fits(M, K, plan))
            return x_dtype == PSQ_BF16 ? launch_decode_ks<PSQ_BF16>(xp, ldx, M, N, K, wa, plan, st, name)
                                       : launch_decode_ks<PSQ_F16>(xp, ldx, M, N, K, wa, plan, st, name);
        if (plan.G > 0)
            return x_dtype == PSQ_BF16 ? launch_decode<PSQ_BF16>(xp, ldx, M, N, K, wa, plan, st, name)
                                       : launch_decode<PSQ_F16>(xp, ldx, M, N, K, wa, plan, st, name);
        path = Path::Stream;   // too many items per workgroup for 32-bit runs: the streaming kernel takes it
    }
    if (path == Path::Stream)
        return x_dtype == PSQ_BF16 ? launch_stream<PSQ_BF16>(xp, ldx, M, N, K, wa, st, name)
                                   : launch_stream<PSQ_F16>(xp, ldx, M, N, K, wa, st, name);
    if (path == Path::Skinny) {
        if (x_dtype == PSQ_BF16) launch_skinny<PSQ_BF16, WK>(xp, ldx, M, N, K, wa, st);
        else launch_skinny<PSQ_F16, WK>(xp, ldx, M, N, K, wa, st);
        return check_launch(name);
    }
    if (ldx > (1LL << 22)) return set_error(PSQ_E_SHAPE, "%s: ldx above 2^22", name);   // 32-bit row offsets
    if (K > (1LL << 22)) return set_error(PSQ_E_SHAPE, "%s: K above 2^22", name);       // (of the weights too)
    const TiledPlan plan = plan_tiled(M, N, K, cu_count(dev), workspace != nullptr);
    wa.sk = 0;
    if (plan.sk) {
        if (ws_bytes < plan.ws_bytes)
            return set_error(PSQ_E_ARG, "%s: workspace of %lld bytes, %lld needed", name, (long long)ws_bytes,
                             (long long)plan.ws_bytes);
        if ((uintptr_t)workspace & 255) return set_error(PSQ_E_ARG, "%s: workspace must be 256-byte aligned", name);
        wa.sk = plan.sk;
        wa.cnt = (uint32_t *)workspace;
        wa.part = (float *)((uint8_t *)workspace + kSkCntBytes);
    }
    auto go = [&](auto xc) {
        constexpr int XDT = decltype(xc)::value;
        if (plan.sk) return launch_tiled_bm<XDT, WK, 128, true>(xp, ldx, M, N, K, wa, st, name);
        return plan.bm == 128 ? launch_tiled_bm<XDT, WK, 128, false>(xp, ldx, M, N, K, wa, st, name)
                              : launch_tiled_bm<XDT, WK, 256, false>(xp, ldx, M, N, K, wa, st, name);
    };
    return x_dtype == PSQ_BF16 ? go(std::integral_constant<int, PSQ_BF16>{}) : go(std::integral_constant<int, PSQ_F16>{});
}

int check_common(const char *name, const void *x, int x_dtype, int64_t ldx, const void *wq, const void *y, int y_dtype,
                 int64_t ldy, const void *bias, int bias_dtype, int64_t M, int64_t N, int64_t K)
{
    if (M < 0 || N < 0 || K < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    // an empty problem touches nothing: empty tensors may come with null data pointers
    if (M > 0 && N > 0 && (!x || !wq || !y)) return set_error(PSQ_E_ARG, "%s: null pointer", name);
    if (x_dtype != PSQ_BF16 && x_dtype != PSQ_F16) return set_error(PSQ_E_ARG, "%s: activations must be bf16/f16", name);
    if (!valid_dtype(y_dtype) || (bias && !valid_dtype(bias_dtype))) return set_error(PSQ_E_ARG, "%s: bad dtype", name);
    if (K == 0 || K % KSTAGE) return set_error(PSQ_E_SHAPE, "%s: K=%lld must be a positive multiple of %d", name, (long long)K, KSTAGE);
    if (ldx < K || ldx % 8 || ((uintptr_t)x & 15)) return set_error(PSQ_E_SHAPE, "%s: x rows must be 16-byte aligned", name);
    if (((uintptr_t)wq & 15)) return set_error(PSQ_E_SHAPE, "%s: weights must be 16-byte aligned", name);
    if (ldy < N) return set_error(PSQ_E_SHAPE, "%s: ldy < N", name);
    if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 30)) return set_error(PSQ_E_SHAPE, "%s: size too large", name);
    return PSQ_OK;
}

// One weight-only GEMM call (the checks of every entry point, then the launch).
int gemm_w4a16(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq, const uint16_t *w_scale,
               const uint16_t *w_zero, int group_size, const void *bias, int bias_dtype, void *y, int y_dtype,
               int64_t ldy, int64_t M, int64_t N, int64_t K, void *workspace, int64_t ws_bytes, void *stream,
               const char *name)
{
    if (int e = check_common(name, x, x_dtype, ldx, wq, y, y_dtype, ldy, bias, bias_dtype, M, N, K)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!w_scale || !w_zero) return set_error(PSQ_E_ARG, "%s: null scale/zero", name);
    if (group_size <= 0 || group_size % KSTAGE || K % group_size)
        return set_error(PSQ_E_SHAPE, "%s: group size %d must be a multiple of %d dividing K", name, group_size, KSTAGE);
    if (int e = require_device()) return e;
    WArgs wa{wq, w_scale, w_zero, nullptr, group_size, bias, bias_dtype, y, y_dtype, ldy};
    return launch<W_UINT4>(x, x_dtype, ldx, M, N, K, wa, workspace, ws_bytes, (hipStream_t)stream, name);
}

int gemm_w8a16(const void *x, int x_dtype, int64_t ldx, const int8_t *wq, const float *w_scale, const void *bias,
               int bias_dtype, void *y, int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *workspace,
               int64_t ws_bytes, void *stream, const char *name)
{
    if (int e = check_common(name, x, x_dtype, ldx, wq, y, y_dtype, ldy, bias, bias_dtype, M, N, K)) return e;
    if (M == 0 || N == 0) return PSQ_OK;
    if (!w_scale) return set_error(PSQ_E_ARG, "%s: null scale", name);
    if (int e = require_device()) return e;
    WArgs wa{(const uint8_t *)wq, nullptr, nullptr, w_scale, 0, bias, bias_dtype, y, y_dtype, ldy};
    return launch<W_INT8>(x, x_dtype, ldx, M, N, K, wa, workspace, ws_bytes, (hipStream_t)stream, name);
}

// ------------------------------------------------------------------ allocation-free variant
// psq_gemm_w4a16_noalloc keeps its stream-K counters and partial tiles in `scratch`, a file-scope
// device array of the largest workspace any plan asks for (kMaxWsBytes = 64 MB + 64 KB), held by
// every GPU the library runs on until the process ends.  In host code `scratch` names a host-side
// stand-in, not a device address: its address on a device comes from hipGetSymbolAddress, taken
// once per device with that device current, and only that address is passed to the kernels.
// A `static __device__` array starts zeroed, and every launch leaves its counters zero (the last
// workgroup of a tile resets the tile's) and writes every partial it reads: nothing needs clearing.
// Calls that overlap on one GPU share it and race.
static __device__ __align__(256) uint8_t scratch[kMaxWsBytes];

constexpr int kMaxDev = 64;
std::once_flag g_scratch_once[kMaxDev];
void *g_scratch_ptr[kMaxDev];
hipError_t g_scratch_status[kMaxDev];

int scratch_on_device(void **ptr)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev)
        return set_error(PSQ_E_DEVICE, "gemm_w4a16_noalloc: no current HIP device");
    std::call_once(g_scratch_once[dev], [dev] {
        void *p = nullptr;
        g_scratch_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = p;
    });
    if (g_scratch_status[dev] != hipSuccess || !g_scratch_ptr[dev])
        return set_error(PSQ_E_DEVICE, "gemm_w4a16_noalloc: no scratch address on device %d: %s", dev,
                         hipGetErrorString(g_scratch_status[dev]));
    *ptr = g_scratch_ptr[dev];
    return PSQ_OK;
}

}  // namespace
}  // namespace psq

extern "C" {

int psq_gemm_w4a16(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq, const uint16_t *w_scale,
                   const uint16_t *w_zero, int group_size, const void *bias, int bias_dtype, void *y, int y_dtype,
                   int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    return psq::gemm_w4a16(x, x_dtype, ldx, wq, w_scale, w_zero, group_size, bias, bias_dtype, y, y_dtype, ldy, M, N,
                           K, nullptr, 0, stream, "gemm_w4a16");
}

int psq_gemm_w4a16_ws(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq, const uint16_t *w_scale,
                      const uint16_t *w_zero, int group_size, const void *bias, int bias_dtype, void *y, int y_dtype,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, void *workspace, int64_t workspace_bytes,
                      void *stream)
{
    return psq::gemm_w4a16(x, x_dtype, ldx, wq, w_scale, w_zero, group_size, bias, bias_dtype, y, y_dtype, ldy, M, N,
                           K, workspace, workspace_bytes, stream, "gemm_w4a16");
}

int psq_gemm_w8a16(const void *x, int x_dtype, int64_t ldx, const int8_t *wq, const float *w_scale, const void *bias,
                   int bias_dtype, void *y, int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    return psq::gemm_w8a16(x, x_dtype, ldx, wq, w_scale, bias, bias_dtype, y, y_dtype, ldy, M, N, K, nullptr, 0,
                           stream, "gemm_w8a16");
}

int psq_gemm_w8a16_ws(const void *x, int x_dtype, int64_t ldx, const int8_t *wq, const float *w_scale,
                      const void *bias, int bias_dtype, void *y, int y_dtype, int64_t ldy, int64_t M, int64_t N,
                      int64_t K, void *workspace, int64_t workspace_bytes, void *stream)
{
    return psq::gemm_w8a16(x, x_dtype, ldx, wq, w_scale, bias, bias_dtype, y, y_dtype, ldy, M, N, K, workspace,
                           workspace_bytes, stream, "gemm_w8a16");
}

int psq_gemm_w4a16_noalloc(const void *x, int x_dtype, int64_t ldx, const uint8_t *wq, const uint16_t *w_scale,
                           const uint16_t *w_zero, int group_size, const void *bias, int bias_dtype, void *y,
                           int y_dtype, int64_t ldy, int64_t M, int64_t N, int64_t K, void *stream)
{
    using namespace psq;
    if (M > 0 && N > 0 && K > 0) {
        if (int e = require_device()) return e;
        const int64_t need = workspace_bytes(W_UINT4, ldx, M, N, K, group_size);
        if (need > kMaxWsBytes)
            return set_error(PSQ_E_SHAPE, "gemm_w4a16_noalloc: %lld bytes of stream-K scratch needed, %lld available",
                             (long long)need, (long long)kMaxWsBytes);
    }
    void *ptr = nullptr;
    if (int e = scratch_on_device(&ptr)) return e;
    return gemm_w4a16(x, x_dtype, ldx, wq, w_scale, w_zero, group_size, bias, bias_dtype, y, y_dtype, ldy, M, N, K,
                      ptr, kMaxWsBytes, stream, "gemm_w4a16_noalloc");
}

int64_t psq_gemm_wonly_workspace_bytes(int weight_kind, int64_t ldx, int64_t M, int64_t N, int64_t K, int group_size)
{
    if (weight_kind != PSQ_W_UINT4 && weight_kind != PSQ_W_INT8) return 0;
    return psq::workspace_bytes(weight_kind == PSQ_W_UINT4 ? psq::W_UINT4 : psq::W_INT8, ldx, M, N, K, group_size);
}

}  // extern "C"
