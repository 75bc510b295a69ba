/*
 * attn_scratch.hip - the partials of janas_attn_run_dev_noalloc: one fixed
 * device array per GPU, held from the library's first janas_attn_create on
 * that GPU until the process ends, so that those calls allocate nothing.
 *
 * In host code `scratch` names a host-side stand-in, not device memory:
 * its device address is looked up once per device (scratch_init, with the
 * device current) and only that address is handed to kernels.
 */
#include <mutex>

#include <hip/hip_runtime.h>

#include "../../include/janas_attn.h"
#include "attn_kernels.h"

namespace janas {
namespace {

__device__ __align__(256) char scratch[JANAS_ATTN_NOALLOC_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices];
bool g_tried[kMaxDevices];

}  // namespace

int scratch_init(int dev)
{
    if (dev < 0 || dev >= kMaxDevices)
        return JANAS_ATTN_EDEVICE;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_tried[dev]) {
        g_tried[dev] = true;
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess && p)
            g_ptr[dev] = p;
        else
            (void)hipGetLastError();
    }
    return g_ptr[dev] ? JANAS_ATTN_OK : JANAS_ATTN_EDEVICE;
}

void *scratch_ptr(int dev)
{
    if (dev < 0 || dev >= kMaxDevices)
        return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    return g_ptr[dev];
}

}  // namespace janas
