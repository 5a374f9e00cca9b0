// gemm_q8.hip -- W8A8 int8 and fp8-e4m3 GEMMs on gfx950 MFMA with a fused dequant epilogue.
//
// Replaces comfy-kitchen int8_linear and torch._scaled_mm behind
// F.linear(QuantizedTensor, QuantizedTensor, bias) (powershard/quant_linear.py:230-242).
//   y[m][n] = round_out(fmaf((float)acc[m][n], a_scale[m] * w_scale[n], bias[n]))
//   int8: acc = sum_k a[m][k] w[n][k] in int32 (v_mfma_i32_32x32x32_i8, exact)
//   fp8 : acc = the same in fp32 (v_mfma_f32_32x32x64_f8f6f4, e4m3 x e4m3)
//
// Tiling (MI355X-first): a 256 x 256 output tile per workgroup of 4 waves, one per SIMD (2 x 2,
// each wave 128 x 128 = 4 x 4 MFMA tiles of 32 x 32, accumulators in the AGPR half of the
// register file).  K runs in stages of 64 bytes through a 4-deep LDS ring (4 x 32 KB) filled by
// direct global->LDS loads (global_load_lds_dwordx4: no staging registers, no LDS write
// instructions), three stages in flight.  Fragments are double-buffered in registers so the
// LDS reads of the next k-step overlap the MFMAs of the current one; one barrier per stage.  Workgroups are renumbered so each XCD owns a contiguous, L2-friendly
// group of tiles.  MFMA-bound: 2 M N K ops per launch.
#include "psq_common.hpp"

namespace psq {
namespace {

// Tuning knobs (compile-time): ring depth and the int8 LDS swizzle.
#ifndef PSQ_Q8_NSTAGE
#define PSQ_Q8_NSTAGE 4
#endif
#ifndef PSQ_Q8_SWZ
#define PSQ_Q8_SWZ 1
#endif
#ifndef PSQ_Q8_GROUP_M
#define PSQ_Q8_GROUP_M 8
#endif

constexpr int BM = 256, BN = 256, BK = 64;    // BK in bytes (= elements for int8/fp8)
constexpr int NSTAGE = PSQ_Q8_NSTAGE;          // LDS ring depth: NSTAGE - 1 stages in flight
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

// Store 4 consecutive outputs (RNE to bf16 / f16, or fp32); `n_left` bounds a partial group.
template <int OUT>
__device__ __forceinline__ void store4(void *y, int64_t off, const float (&v)[4], bool vec, int n_left)
{
    if constexpr (OUT == OUT_F32) {
        float *p = (float *)y + off;
        if (vec) {
            *(v4f *)p = v4f{v[0], v[1], v[2], v[3]};
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (c < n_left) p[c] = v[c];
        }
    } else {
        uint16_t *p = (uint16_t *)y + off;
        uint32_t h[4];
#pragma unroll
        for (int c = 0; c < 4; c++) h[c] = f32_to_half<OUT>(v[c]);
        if (vec) {
            *(v2i *)p = v2i{(int)(h[0] | (h[1] << 16)), (int)(h[2] | (h[3] << 16))};
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (c < n_left) p[c] = (uint16_t)h[c];
        }
    }
}

// LDS: the K-loop ring, reused by the epilogue as four 32 KB per-wave staging areas, then the
// tile's row scales, column scales and biases.
constexpr size_t kRingBytes = (NSTAGE * 2 * STAGE_BYTES) > 131072 ? (NSTAGE * 2 * STAGE_BYTES) : 131072;

typedef __attribute__((address_space(3))) uint8_t *lds_ptr;
typedef const __attribute__((address_space(1))) void *glb_ptr;

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

// Scheduling hints (masks: 0x008 MFMA, 0x020 VMEM read, 0x100 DS read).  With one wave per
// SIMD every issue slot not spent on an MFMA idles the matrix core, so the global->LDS loads of a
// refill and the LDS fragment reads of the next k-step are each slotted behind an MFMA: the loads
// first (they follow only reads the first MFMA already waited for), then the reads.
template <int N_VMEM, int N_DS, int N_MFMA>
__device__ __forceinline__ void interleave_with_mfma()
{
    static_assert(N_VMEM + N_DS <= N_MFMA, "one memory instruction per MFMA at most");
#pragma unroll
    for (int i = 0; i < N_VMEM; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
#pragma unroll
    for (int i = 0; i < N_DS; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, (N_MFMA - N_VMEM) / N_DS, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
}

template <bool FP8> struct Frag;
template <> struct Frag<false> { typedef v4i T; static constexpr int KSTEP = 32; };   // 32x32x32 i8
template <> struct Frag<true> { typedef v8i T; static constexpr int KSTEP = 64; };    // 32x32x64 f8f6f4

template <bool FP8, int OUT>
__global__ void __launch_bounds__(NTHREADS, 1)
gemm_q8_kernel(const uint8_t *__restrict__ A, int64_t lda, const uint8_t *__restrict__ W, int64_t ldw,
               int M, int N, int K, Epi ep)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];   // [NSTAGE][A | W]
    using Acc = typename std::conditional<FP8, v16f, v16i>::type;
    using FT = typename Frag<FP8>::T;
    constexpr int KSTEP = Frag<FP8>::KSTEP;
    constexpr int KS = BK / KSTEP;                 // MFMA k-steps per stage (2 for int8, 1 for fp8)
    constexpr int LPS = 2 * LOADS;                 // DMA instructions per wave per stage

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nbm = (M + BM - 1) / BM, nbn = (N + BN - 1) / BN;
    int pm, pn;
    tile_order(blockIdx.x, nbm, nbn, GROUP_M, pm, pn);
    const int m0 = pm * BM, n0 = pn * BN;

    // The tile's epilogue operands (256 row scales, 256 column scales, 256 biases) go to LDS past
    // the ring before the loads of the K loop, so the epilogue reads them without memory latency.
    float *s_as = (float *)(smem + kRingBytes), *s_ws = s_as + BM, *s_b = s_ws + BN;
    if constexpr (OUT != OUT_I32) {
        s_as[tid] = ep.a_scale[min(m0 + tid, M - 1)];
        const int nc = min(n0 + tid, N - 1);
        s_ws[tid] = ep.w_scale[ep.w_per_row ? nc : 0];
        s_b[tid] = ep.bias ? load_elem(ep.bias, nc, ep.bias_dtype) : 0.0f;
    }

    // global -> LDS: a wave load moves 1 KB = 16 rows x 4 chunks; lane L fills physical slot L of
    // the block (row 16 b + L / 4, physical chunk L % 4) and reads the logical chunk stored there.
    const uint8_t *pa[LOADS];
    const uint8_t *pw[LOADS];
#pragma unroll
    for (int j = 0; j < LOADS; j++) {
        const int b = j * (NTHREADS / 64) + wave;
        const int r = 16 * b + (lane >> 2);
        const int c = (lane & 3) ^ (FP8 ? (((r >> 1) & 1) << 1) : swz_i8(r));
        pa[j] = A + (int64_t)min(m0 + r, M - 1) * lda + c * 16;
        pw[j] = W + (int64_t)min(n0 + r, N - 1) * ldw + c * 16;
    }
    auto issue_stage = [&](int kt, int slot) {
        const int64_t koff = (int64_t)kt * BK;
        lds_ptr dA = (lds_ptr)(smem + slot * 2 * STAGE_BYTES);
#pragma unroll
        for (int j = 0; j < LOADS; j++) {
            const int b = j * (NTHREADS / 64) + wave;
            __builtin_amdgcn_global_load_lds((glb_ptr)(pa[j] + koff), dA + 1024 * b, 16, 0, 0);
            __builtin_amdgcn_global_load_lds((glb_ptr)(pw[j] + koff), dA + STAGE_BYTES + 1024 * b, 16, 0, 0);
        }
    };

    // MFMA operand layout (32 x 32 tiles): lane holds row (lane & 31) of A / of W and the k-slice
    // (lane >> 5) of the instruction's K; A and W use the same slice, so the dot products are
    // complete whatever order the hardware sums a slice in.
    const int frow = lane & 31, fk = lane >> 5;
    auto read_frags = [&](int kt, int ks, FT (&fa)[TM], FT (&fw)[TN]) {
        const uint8_t *sA = smem + (kt % NSTAGE) * 2 * STAGE_BYTES;
        const uint8_t *sW = sA + STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int r = wm * WAVE_M + i * 32 + frow;
            if constexpr (FP8) fa[i] = *(const v8i *)(sA + swz<true>(r, 2 * fk));
            else fa[i] = *(const v4i *)(sA + swz<false>(r, 2 * ks + fk));
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int r = wn * WAVE_N + j * 32 + frow;
            if constexpr (FP8) fw[j] = *(const v8i *)(sW + swz<true>(r, 2 * fk));
            else fw[j] = *(const v4i *)(sW + swz<false>(r, 2 * ks + fk));
        }
    };
    auto mfma = [&](Acc (&acc)[TM][TN], const FT (&fa)[TM], const FT (&fw)[TN]) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (FP8)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fw[j], acc[i][j], 0, 0, 0, 127,
                                                                               0, 127);
                else
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fw[j], acc[i][j], 0, 0, 0);
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
    // Prologue: stages 0 .. NSTAGE-2 in flight.  Every step below issues exactly one stage (clamped
    // to the last one, re-loading it into a ring slot nobody reads again), so the number of loads
    // younger than the stage being waited for is always (NSTAGE - 2) LPS: the waits carry no branches.
#pragma unroll
    for (int s = 0; s < NSTAGE - 1; s++) issue_stage(min(s, nk - 1), s);
    wait_vmcnt<(NSTAGE - 2) * LPS>();
    stage_barrier();

    // One MFMA k-step g = KS * kt + ks: at the first k-step of stage kt refill the ring slot last
    // read in stage kt - 1 (every wave passed the barrier that ended it); prefetch the fragments of
    // step g + 1 into `nxt` -- after the stage's barrier when g + 1 opens a new stage -- then run
    // the MFMAs of step g on `cur`.  Steps alternate between two register buffers in pairs, so the
    // buffer roles are static.
    auto kstep = [&](int g, FT (&ca)[TM], FT (&cw)[TN], FT (&na)[TM], FT (&nw)[TN]) {
        const int kt = g / KS, ks = g - kt * KS;
        if (ks == 0) issue_stage(min(kt + NSTAGE - 1, nk - 1), (kt + NSTAGE - 1) % NSTAGE);
        if (ks + 1 < KS) {
            read_frags(kt, ks + 1, na, nw);
        } else {
            wait_vmcnt<(NSTAGE - 2) * LPS>();   // stage kt + 1 landed for this wave ...
            stage_barrier();         // ... and for every wave
            read_frags(min(kt + 1, nk - 1), 0, na, nw);
        }
        mfma(acc, ca, cw);
        if (ks == 0) interleave_with_mfma<LPS, TM + TN, TM * TN>();
        else interleave_with_mfma<0, TM + TN, TM * TN>();
    };
    FT fa0[TM], fw0[TN], fa1[TM], fw1[TN];
    if constexpr (FP8) {
        // fp8 fragments are 32 bytes: one register set (the allocator cannot double-buffer them
        // beside 256 accumulators); a stage's reads still overlap its MFMAs in issue order.
#pragma clang loop unroll(disable)
        for (int kt = 0; kt < nk; kt++) {
            issue_stage(min(kt + NSTAGE - 1, nk - 1), (kt + NSTAGE - 1) % NSTAGE);
            read_frags(kt, 0, fa0, fw0);
            mfma(acc, fa0, fw0);
            // reads first (the MFMAs consume them in issue order), then one refill load per MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
#pragma unroll
            for (int i = 0; i < LPS; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - LPS, 0);
            wait_vmcnt<(NSTAGE - 2) * LPS>();
            stage_barrier();
        }
    } else {
        read_frags(0, 0, fa0, fw0);
        const int steps = nk * KS;
#pragma clang loop unroll(disable)
        for (int g = 0; g < steps; g += 2) {
            kstep(g, fa0, fw0, fa1, fw1);
            if (g + 1 < steps) kstep(g + 1, fa1, fw1, fa0, fw0);
        }
    }

    // ---------------------------------------------------------------- epilogue
    // Each wave stages its 128 x 128 accumulators through its own 32 KB of the (now idle) LDS
    // ring, 64 rows at a time, in row-major order; a lane then owns 4 consecutive columns of a
    // row: y = round_out(fmaf(acc, a_scale[m] * w_scale[n], bias[n])), stored as full row segments.
    // MFMA layout of a 32 x 32 tile: lane holds column (lane & 31) and, for register r, row
    // 8 (r / 4) + 4 (lane / 32) + (r % 4).
    wait_vmcnt<0>();   // the last (redundant) ring loads must land before the ring is reused
    __syncthreads();   // every wave is done reading the ring
    float *stage = (float *)(smem + wave * (32 * 1024));
    const int col4 = (lane & 31) * 4;                 // the lane's 4 columns within the wave tile
    const int nb = n0 + wn * WAVE_N + col4;           // first global column of the lane
    float ws[4], bs[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        ws[c] = (OUT == OUT_I32) ? 1.0f : s_ws[wn * WAVE_N + col4 + c];
        bs[c] = (OUT == OUT_I32) ? 0.0f : s_b[wn * WAVE_N + col4 + c];
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int il = 0; il < 2; il++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = il * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const Acc &a = acc[2 * h + il][j];
                    float v;
                    if constexpr (OUT == OUT_I32 || !FP8) v = __int_as_float((int)a[r]);
                    else v = a[r];
                    stage[row * 128 + j * 32 + (lane & 31)] = v;
                }
#pragma unroll 4
        for (int st = 0; st < 32; st++) {
            const int row = 2 * st + (lane >> 5);
            const v4f raw = *(const v4f *)(stage + row * 128 + col4);
            // whole-vector reinterpretation only: hipcc mis-lowers __builtin_bit_cast applied to a
            // single ext_vector element (it reads element 0)
            const v4i rawi = __builtin_bit_cast(v4i, raw);
            const int m = m0 + wm * WAVE_M + h * 64 + row;
            if (m >= M) continue;
            if constexpr (OUT == OUT_I32) {
                int32_t *C = (int32_t *)ep.y + (int64_t)m * ep.ldy + nb;
                if (ep.vec && nb + 3 < N) {
                    *(v4i *)C = rawi;
                } else {
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        if (nb + c < N) C[c] = rawi[c];
                }
            } else {
                const float as = s_as[wm * WAVE_M + h * 64 + row];
                float y[4];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float accv = FP8 ? raw[c] : (float)rawi[c];
                    y[c] = __builtin_fmaf(accv, as * ws[c], bs[c]);
                }
                store4<OUT>(ep.y, (int64_t)m * ep.ldy + nb, y, ep.vec && nb + 3 < N, N - nb);
            }
        }
    }
}

constexpr size_t kSmemBytes = kRingBytes + 3 * 256 * sizeof(float);   // ring (>= the 128 KB epilogue stage) + scales

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
    const int64_t nblk = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    kern<<<dim3((unsigned)nblk), dim3(NTHREADS), kSmemBytes, st>>>(a, lda, w, ldw, (int)M, (int)N, (int)K, ep);
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
