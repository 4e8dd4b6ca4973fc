// Decode without device allocation (ssq_decode_noalloc): the split partials that ssq_decode keeps
// in a caller-provided workspace live in a library-owned, per-device scratch array instead, so a
// caller that cannot allocate device memory (code under HIP graph capture, a serving loop that
// forbids hipMalloc) needs to pass only the inputs and outputs.
//
// Every call on one device shares that device's array: calls that overlap on one device (two
// streams, two threads) race on it and must be serialised by the caller.  The array holds only
// split partials, which each call writes before it reads them, so nothing in it has to start at
// zero and no call clears it.
#include "ssq_common.h"

#include <mutex>

namespace {
constexpr size_t kScratchBytes = SSQ_NOALLOC_SCRATCH_BYTES;  // per device, held until the process ends
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device, resolved once per device

// The array's device address on the current device.  In host code `scratch` names a host-side
// stand-in, not device memory: kernels receive this address, never the symbol.
int scratch_on_current_device(void** out) {
    int dev = 0;
    int rc = ssq_check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    SSQ_REQUIRE(dev >= 0 && dev < kMaxDevices, "device ordinal %d outside [0, %d)", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        rc = ssq_check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (rc) return rc;
        SSQ_REQUIRE(p != nullptr, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return SSQ_OK;
}
}  // namespace

extern "C" int ssq_decode_noalloc(const ssq_decode_args* a, void* stream) {
    if (!a) return ssq_fail(SSQ_ERR_INVALID, "args is NULL");
    void* ws = nullptr;
    int rc = scratch_on_current_device(&ws);
    if (rc) return rc;
    // 0 for a problem that runs one split per unit, and for invalid arguments (ssq_decode reports them)
    const size_t need = ssq_decode_workspace_size(a);
    if (need > kScratchBytes)
        return ssq_fail(SSQ_ERR_UNSUPPORTED,
                        "ssq_decode_noalloc: this problem needs %zu bytes of split workspace, more than the "
                        "library's %zu-byte scratch; call ssq_decode with a workspace instead",
                        need, kScratchBytes);
    return ssq_decode(a, need ? ws : nullptr, need, stream);
}
