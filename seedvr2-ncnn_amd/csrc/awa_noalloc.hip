// awa_forward_noalloc: the fused AWA layer without device allocation.
//
// The only device memory awa_forward allocates while it runs is the plan's
// workspace (the per-window text rows [nwin][T_x][H][d], averaged
// afterwards, or a split layer's key segments, combined afterwards) and, on
// the first call with a head count, the work lists. Here the workspace is a
// file-scope device array, one copy per GPU, and the work lists must already
// be on the device (awa_plan_upload builds them when the plan desc names the
// head count).
//
// In host code the array's name is only a host-side stand-in: its device
// address on each GPU comes from hipGetSymbolAddress, taken once per device
// with that device current (by awa_runtime_init, or by the first no-alloc
// call on a device that was not set up through it), and only that address
// is handed to kernels. Resolving the symbol loads the array's code object,
// which is when the runtime reserves the array's memory on that device.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "awa_internal.h"
#include "seedvr2_awa.h"

namespace
{

static __device__ __align__(256) unsigned char scratch[AWA_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array (resolved once per
// device); null with awa_last_error() set on failure.
void* device_scratch()
{
    int device = -1;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices)
    {
        awa::set_error("no current HIP device for the no-alloc scratch buffer");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device])
    {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
        {
            awa::set_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}

} // namespace

namespace awa
{

int noalloc_setup()
{
    return device_scratch() ? AWA_OK : AWA_ERR_DEVICE;
}

} // namespace awa

extern "C" int awa_forward_noalloc(const awa_plan* plan, const awa_blob* video_qkv, const awa_blob* text_qkv,
                                   const awa_blob* video_out, const awa_blob* text_out, int compute, void* stream)
{
    void* ptr = device_scratch();
    if (!ptr)
        return AWA_ERR_DEVICE;
    const awa::Scratch s{ptr, AWA_NOALLOC_SCRATCH_BYTES};
    return awa::forward_fused(plan, video_qkv, text_qkv, nullptr, video_out, text_out, compute,
                              static_cast<hipStream_t>(stream), nullptr, &s);
}
