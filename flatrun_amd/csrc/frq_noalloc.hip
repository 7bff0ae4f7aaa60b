// frq_dev_gemv_noalloc: frq_dev_gemv for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). The scratch that frq_dev_gemv takes from a per-stream
// registry (grown with hipMalloc on first use) lives here in one file-scope
// device array of fixed size instead:
//   [0, kSlotBytes)            per-row exchange slots of the matrix-core
//                              Q4_K GEMV when its rows are split over two
//                              workgroups: 8 bytes per output row, zero
//                              before every launch (cleared on the first
//                              call on a device; every launch leaves them 0);
//   [kSlotBytes, kScratchBytes) split-K partial sums (rows longer than one
//                              workgroup): n x slices x 4 bytes.
// Each device holds its own copy of the array for the life of the process.
// Every call on a device shares it, so calls that overlap on one device (two
// streams, two threads) race; calls issued in order on one stream do not.
#include <hip/hip_runtime.h>

#include <mutex>

#include "frq.h"
#include "frq_kernels.h"

namespace {

constexpr size_t kScratchBytes = (size_t)FRQ_NOALLOC_SCRATCH_BYTES;
constexpr size_t kSlotBytes = (size_t)1 << 20;
static_assert(kScratchBytes > kSlotBytes && kSlotBytes % 256 == 0, "scratch layout");

// In host code this name is a stand-in, not a device address: host code
// uses only the per-device pointers from hipGetSymbolAddress below.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
uint8_t* g_ptr[kMaxDevices] = {};   // device address of `scratch` on each device, once resolved

// The array's address on the current device; on the first call on a device
// it is looked up and its slot region cleared (by a kernel on `stream`, so
// the call stays capturable and ordered before the launch that reads it).
int scratch_ptr(hipStream_t stream, uint8_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return frq::fail_hip(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return frq::fail_unsupported("noalloc gemv: device index beyond 63");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return frq::fail_hip(e, "hipGetSymbolAddress(scratch)");
        e = frq::launch_fill(static_cast<float*>(p), 0.0f, (int64_t)(kSlotBytes / 4), stream);
        if (e != hipSuccess) return frq::fail_hip(e, "clearing the noalloc slots");
        g_ptr[dev] = static_cast<uint8_t*>(p);
    }
    *out = g_ptr[dev];
    return FRQ_OK;
}

}  // namespace

extern "C" int frq_dev_gemv_noalloc(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n,
                                    int64_t k, int64_t batch, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t* base = nullptr;
    if (int rc = scratch_ptr(s, &base)) return rc;
    frq::FixedScratch fx;
    fx.slots = reinterpret_cast<uint64_t*>(base);
    fx.slot_bytes = kSlotBytes;
    fx.part = reinterpret_cast<float*>(base + kSlotBytes);
    fx.part_bytes = kScratchBytes - kSlotBytes;
    return frq::dev_gemv_fixed(qtype, w, w_bytes, x, y, n, k, batch, stream, fx);
}
