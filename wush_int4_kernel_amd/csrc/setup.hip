// setup.hip -- wush_init() and the per-device one-time set-up behind it.
//
// The reference sets its only launch attribute lazily behind a static flag
// on the first call (csrc/gemm_cutlass_int4.cu:62-67, :111-119) and warns
// that attribute calls are illegal during graph capture.  Here the set-up is
// an explicit entry point that the torch module calls at import, guarded per
// device by std::call_once, so no launch inside a capture has to run it.
#include <mutex>

#include "setup.h"
#include "../../include/wush_int4.h"

namespace wush {
namespace {

std::once_flag g_once[kMaxDevices];
int g_status[kMaxDevices];

// Split-K scratch of wush_gemm_s4_noalloc: every device holds its own copy
// from the library's load until the process ends.  Host code never uses the
// array's name as an address (on the host it is a stand-in symbol): the
// device address comes from hipGetSymbolAddress, once per device, below.
static __device__ __align__(256) float scratch[WUSH_GEMM_SCRATCH_BYTES / sizeof(float)];
void* g_scratch[kMaxDevices];
int g_cus[kMaxDevices];

}  // namespace

int device_setup(int* dev) {
    int d = 0;
    const hipError_t e = hipGetDevice(&d);
    if (e != hipSuccess) return (int)e;
    if (d < 0 || d >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::call_once(g_once[d], [d] {
        int cus = 0;
        g_cus[d] = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, d) == hipSuccess && cus > 0
                       ? cus
                       : 256;
        int st = gemm_h16_init_device();
        if (st == 0) st = gemv_init_device(d);
        if (st == 0) {
            void* p = nullptr;
            st = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (st == 0 && p == nullptr) st = (int)hipErrorInvalidSymbol;
            g_scratch[d] = st == 0 ? p : nullptr;
        }
        g_status[d] = st;
    });
    *dev = d;
    return g_status[d];
}

int device_cus(int dev) { return dev >= 0 && dev < kMaxDevices && g_cus[dev] > 0 ? g_cus[dev] : 256; }

void* scratch_address(int dev) { return dev >= 0 && dev < kMaxDevices ? g_scratch[dev] : nullptr; }

}  // namespace wush

extern "C" int wush_init(void) {
    int n = 0, cur = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return (int)e;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return (int)e;
    int first = 0;
    for (int d = 0; d < n && d < wush::kMaxDevices; ++d) {
        int st = (int)hipSetDevice(d);
        int dd = 0;
        if (st == 0) st = wush::device_setup(&dd);
        if (st != 0 && first == 0) first = st;
    }
    e = hipSetDevice(cur);
    if (first == 0 && e != hipSuccess) first = (int)e;
    return first;
}
