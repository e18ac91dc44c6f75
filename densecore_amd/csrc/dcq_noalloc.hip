// dcq_noalloc.hip — the device-resident workspace behind dcq_mul_mat_noalloc.
//
// dcq_mul_mat needs a workspace for the quantized activations whenever the product does not
// run in one fused decode kernel (M > 8, or shapes outside the fused kernels). A caller that
// cannot allocate (code under stream capture, a serving loop that forbids hipMalloc) gets it
// from `scratch`, a static device array that every GPU the library runs on holds from the
// module's load until the process ends: DCQ_NOALLOC_SCRATCH_BYTES for the quantized activation
// and 16 MiB after it for split-K partial sums, the room dcq_mul_mat_workspace_size gives at most
// (so the kernels split K exactly as dcq_mul_mat with a workspace of that size does).
//
// In host code `scratch` names a host-side stand-in, not the device array: the device address
// is looked up once per device with hipGetSymbolAddress (with that device current) and kept;
// only that address is handed to kernels. Each GPU has its own copy at its own address.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/dcq.h"
#include "dcq_kernels.h"

constexpr size_t kSplitRoom = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[DCQ_NOALLOC_SCRATCH_BYTES + kSplitRoom];

namespace dcq {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

int noalloc_scratch(void** ptr, size_t* bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return DCQ_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return DCQ_ERR_HIP;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    *bytes = DCQ_NOALLOC_SCRATCH_BYTES + kSplitRoom;
    return DCQ_OK;
}

}  // namespace dcq
