// psq_runtime.hip -- version, error reporting and device capability of libpsquant.
//
// Follows the reference's native-library idiom (powershard/ats_allocator.cpp:14-52): plain
// extern "C" entry points over raw pointers, failures reported by return value, lazily
// initialised state.  The device probe replaces native_support()'s compute-capability and
// comfy-kitchen capability checks (powershard/quant_linear.py:245-265).
#include "psq_common.hpp"

#include <mutex>
#include <stdio.h>
#include <string.h>

namespace psq {

static thread_local char g_err[512] = "";

int set_error(int code, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(PSQ_E_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return PSQ_OK;
}

static constexpr int kMaxDevices = 64;
static std::once_flag g_once[kMaxDevices];
static int g_supported[kMaxDevices];

static int probe(int dev)
{
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int require_device()
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return set_error(PSQ_E_DEVICE, "no current HIP device");
    std::call_once(g_once[dev], [dev] { g_supported[dev] = probe(dev); });
    if (!g_supported[dev]) return set_error(PSQ_E_DEVICE, "device %d is not gfx950", dev);
    return PSQ_OK;
}

// CUs of each device (persistent grid sizes, wave-fill decisions), cached per device; the value
// written by concurrent first calls is the same.
int cu_count(int dev)
{
    static int cus[kMaxDevices] = {};
    if (dev < 0 || dev >= kMaxDevices) return 256;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

}  // namespace psq

extern "C" {

int psq_abi_version(void) { return PSQ_ABI_VERSION; }

const char *psq_last_error(void) { return psq::g_err; }

int psq_device_supported(int device)
{
    if (device < 0 || device >= psq::kMaxDevices) return 0;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device >= count) return 0;
    std::call_once(psq::g_once[device], [device] { psq::g_supported[device] = psq::probe(device); });
    return psq::g_supported[device];
}

}  // extern "C"
