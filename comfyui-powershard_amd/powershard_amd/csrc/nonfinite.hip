// nonfinite.hip -- one pass over a bf16 / f16 / f32 tensor that reports whether any element is NaN
// or +-Inf, by raising a device flag to the caller's ticket.
//
// The check that closes Int8Linear.forward (powershard/operations.py:130-131,
// `not torch.isfinite(out).all()`: raise FloatingPointError) costs two torch kernels over the
// output (a bool tensor, then its reduction).  Here the test is done on the raw bits, 16 bytes per
// thread and step, and only a thread that finds a non-finite element writes: atomicMax(flag,
// ticket).  The flag is never cleared: callers keep one per stream and pass increasing tickets, so
// a call's elements were all finite exactly when the flag after it is below its ticket, and no
// clearing launch (or hipMemsetAsync, which does not replay correctly in a captured graph) is
// needed.
#include "psq_common.hpp"

#include <algorithm>

namespace psq {
namespace {

// 1 when the word (one fp32, or two 16-bit elements) holds an element with all exponent bits set:
// an Inf or a NaN
__device__ __forceinline__ int word_nonfinite(uint32_t w, int dtype)
{
    if (dtype == PSQ_F32) return (w & 0x7f800000u) == 0x7f800000u;
    const uint32_t m = dtype == PSQ_F16 ? 0x7c007c00u : 0x7f807f80u;
    const uint32_t t = (w & m) ^ m;   // a half whose exponent bits are all set becomes zero there
    return ((t & 0xffffu) == 0) | ((t >> 16) == 0);
}

__global__ void __launch_bounds__(256)
nonfinite_kernel(const uint8_t *__restrict__ p, int64_t nvec, const uint8_t *__restrict__ tail, int tail_elems,
                 int dtype, unsigned long long *flag, unsigned long long ticket)
{
    int bad = 0;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += stride) {
        const v4i v = *(const v4i *)(p + i * 16);
        bad |= word_nonfinite((uint32_t)v[0], dtype) | word_nonfinite((uint32_t)v[1], dtype) |
               word_nonfinite((uint32_t)v[2], dtype) | word_nonfinite((uint32_t)v[3], dtype);
    }
    // the elements past the last whole 16 bytes (fewer than 8), one per thread of block 0
    if (blockIdx.x == 0 && (int)threadIdx.x < tail_elems) {
        if (dtype == PSQ_F32) {
            bad |= word_nonfinite(((const uint32_t *)tail)[threadIdx.x], dtype);
        } else {
            const uint32_t h = ((const uint16_t *)tail)[threadIdx.x];
            bad |= word_nonfinite(h | (h << 16), dtype);
        }
    }
    if (bad) atomicMax(flag, ticket);
}

}  // namespace
}  // namespace psq

extern "C" int psq_flag_nonfinite(const void *x, int dtype, int64_t n, unsigned long long *flag,
                                  unsigned long long ticket, void *stream)
{
    using namespace psq;
    const char *name = "flag_nonfinite";
    if (n < 0) return set_error(PSQ_E_ARG, "%s: negative size", name);
    if (!valid_dtype(dtype)) return set_error(PSQ_E_ARG, "%s: bad dtype", name);
    if (!flag || ((uintptr_t)flag & 7)) return set_error(PSQ_E_ARG, "%s: flag must be an aligned 8-byte word", name);
    if (ticket == 0) return set_error(PSQ_E_ARG, "%s: tickets start at 1", name);
    if (n == 0) return PSQ_OK;
    if (!x) return set_error(PSQ_E_ARG, "%s: null pointer", name);
    const int esz = dtype == PSQ_F32 ? 4 : 2;
    if ((uintptr_t)x % esz) return set_error(PSQ_E_ARG, "%s: misaligned elements", name);
    if (int e = require_device()) return e;
    // the 16-byte body from the first 16-byte boundary; the elements before it and after it
    // (fewer than 8 on each side) are checked by block 0
    const uint8_t *b = (const uint8_t *)x;
    const int64_t nbytes = n * esz;
    const int64_t lead = std::min<int64_t>(nbytes, (16 - (int64_t)((uintptr_t)b & 15)) & 15);
    const int64_t nvec = (nbytes - lead) / 16;
    const int64_t rest = nbytes - lead - nvec * 16;
    hipStream_t st = (hipStream_t)stream;
    constexpr int64_t kMaxGrid = 2048;   // 8 waves per CU; a larger tensor is walked grid-stride
    const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>((nvec + 255) / 256, kMaxGrid));
    if (lead) {
        nonfinite_kernel<<<1, 256, 0, st>>>(nullptr, 0, b, (int)(lead / esz), dtype, flag, ticket);
        if (int e = check_launch(name)) return e;
    }
    nonfinite_kernel<<<grid, 256, 0, st>>>(b + lead, nvec, b + lead + nvec * 16, (int)(rest / esz), dtype, flag,
                                           ticket);
    return check_launch(name);
}
