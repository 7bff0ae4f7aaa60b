// C-ABI layer of libfrq_hip.so (declared in include/frq.h).
//
// Validation mirrors the reference's pybind11 module (src/flatrun_native/
// _C.cpp): the same checks in the same order with the same messages, so a
// caller that maps FRQ_ERR_SHAPE / FRQ_ERR_SIZE to RuntimeError sees the
// errors the reference raises. Host-buffer calls stage through one
// grow-only device workspace per device, serialised by a mutex (the
// reference holds the GIL for the whole call, so it is serial too).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "frq.h"
#include "frq_kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(FRQ_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// A tuned launch: the launchers refuse a geometry they do not take with
// hipErrorInvalidValue / hipErrorInvalidConfiguration before launching
// anything, which is the caller's argument, not a device failure.
int tuned_fail(hipError_t e, const char* what) {
    if (e == hipErrorInvalidValue || e == hipErrorInvalidConfiguration)
        return fail(FRQ_ERR_UNSUPPORTED, "%s: launch geometry not accepted (%s)", what, hipGetErrorString(e));
    return hip_fail(e, what);
}

#define FRQ_HIP(call)                                   \
    do {                                                \
        hipError_t e_ = (call);                         \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

struct Fmt {
    const char* name;
    int64_t bbytes, belems;
};

bool fmt_of(int qtype, Fmt* f) {
    switch (qtype) {
        case FRQ_Q8_0: *f = {"Q8_0", 34, 32}; return true;
        case FRQ_Q4_K: *f = {"Q4_K", 144, 256}; return true;
        case FRQ_Q5_K: *f = {"Q5_K", 176, 256}; return true;
        case FRQ_Q6_K: *f = {"Q6_K", 210, 256}; return true;
        case FRQ_Q1_0: *f = {"Q1_0", 18, 128}; return true;
        case FRQ_Q4_0: *f = {"Q4_0", 18, 32}; return true;
        case FRQ_Q5_0: *f = {"Q5_0", 22, 32}; return true;
        case FRQ_Q5_1: *f = {"Q5_1", 24, 32}; return true;
        default: return false;
    }
}

int have_device() {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return fail(FRQ_ERR_NO_DEVICE, "no HIP device available");
    }
    return FRQ_OK;
}

// Grow-only staging buffer on the current device.
struct Workspace {
    std::mutex mu;
    std::vector<void*> ptr;
    std::vector<size_t> cap;
};
Workspace g_ws;

// Returns a device buffer of >= bytes on the current device; caller holds g_ws.mu.
int workspace(size_t bytes, void** out) {
    int dev = 0;
    FRQ_HIP(hipGetDevice(&dev));
    if ((size_t)dev >= g_ws.ptr.size()) {
        g_ws.ptr.resize(dev + 1, nullptr);
        g_ws.cap.resize(dev + 1, 0);
    }
    if (g_ws.cap[dev] < bytes) {
        if (g_ws.ptr[dev]) FRQ_HIP(hipFree(g_ws.ptr[dev]));
        g_ws.ptr[dev] = nullptr;
        g_ws.cap[dev] = 0;
        size_t want = bytes < (size_t)1 << 20 ? (size_t)1 << 20 : bytes;
        FRQ_HIP(hipMalloc(&g_ws.ptr[dev], want));
        g_ws.cap[dev] = want;
    }
    *out = g_ws.ptr[dev];
    return FRQ_OK;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Split-K scratch, one per (device, stream): launches on one stream are
// ordered, so they can share it; launches on different streams get their own.
// Counters and partial sums live in separate allocations: the counters must
// be zero before every launch (zeroed once when allocated, left zero by every
// launch), so nothing else may ever write their memory.
//
// A buffer is never freed while something may still use it. Growing replaces
// the buffer with a larger one and keeps the old one in `retired` until the
// stream is destroyed (frq_stream_destroy), because a graph captured earlier
// on that stream still launches kernels on the old address; the counters of
// a retired buffer stay zero, since every launch leaves them so. The registry
// lock is held from the lookup through the launch, so one thread cannot
// retire a buffer another is about to launch with. Capacities grow at least
// twofold, so a stream retires O(log size) buffers.
struct SkScratch {
    void* part = nullptr;
    size_t part_cap = 0;
    void* cnt = nullptr;
    size_t cnt_cap = 0;
    std::vector<void*> retired;
};
std::mutex g_sk_mu;
std::map<std::pair<int, hipStream_t>, SkScratch> g_sk;

int grow(void** ptr, size_t* cap, size_t bytes, bool zero, std::vector<void*>* retired, hipStream_t stream) {
    if (*cap >= bytes) return FRQ_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    FRQ_HIP(hipStreamIsCapturing(stream, &cs));
    if (cs != hipStreamCaptureStatusNone)
        return fail(FRQ_ERR_UNSUPPORTED, "scratch for this shape must exist before graph capture: run the call once "
                                         "on the stream before capturing it");
    size_t want = bytes < ((size_t)1 << 16) ? ((size_t)1 << 16) : bytes;
    if (want < 2 * *cap) want = 2 * *cap;
    void* p = nullptr;
    FRQ_HIP(hipMalloc(&p, want));
    if (zero) {   // on the launch stream: ordered before the kernel that first reads it
        const hipError_t e = hipMemsetAsync(p, 0, want, stream);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return hip_fail(e, "hipMemsetAsync(scratch)");
        }
    }
    if (*ptr) retired->push_back(*ptr);
    *ptr = p;
    *cap = want;
    return FRQ_OK;
}

// Scratch for one launch on `stream`; the caller holds g_sk_mu (see above)
// until the launch has been enqueued.
int sk_scratch_locked(hipStream_t stream, size_t part_bytes, size_t cnt_bytes, float** part, uint32_t** cnt) {
    *part = nullptr;
    *cnt = nullptr;
    if (part_bytes == 0 && cnt_bytes == 0) return FRQ_OK;
    int dev = 0;
    FRQ_HIP(hipGetDevice(&dev));
    SkScratch& sc = g_sk[{dev, stream}];
    if (int rc = grow(&sc.part, &sc.part_cap, part_bytes, false, &sc.retired, stream)) return rc;
    if (int rc = grow(&sc.cnt, &sc.cnt_cap, cnt_bytes, true, &sc.retired, stream)) return rc;
    *part = static_cast<float*>(sc.part);
    *cnt = static_cast<uint32_t*>(sc.cnt);
    return FRQ_OK;
}

// Frees the scratch of every device's entry for `stream` (the stream's work
// has finished: the caller synchronised it).
void sk_release_stream(hipStream_t stream) {
    std::lock_guard<std::mutex> lk(g_sk_mu);
    for (auto it = g_sk.begin(); it != g_sk.end();) {
        if (it->first.second != stream) {
            ++it;
            continue;
        }
        SkScratch& sc = it->second;
        int cur = 0;
        (void)hipGetDevice(&cur);
        (void)hipSetDevice(it->first.first);
        if (sc.part) (void)hipFree(sc.part);
        if (sc.cnt) (void)hipFree(sc.cnt);
        for (void* p : sc.retired) (void)hipFree(p);
        (void)hipSetDevice(cur);
        it = g_sk.erase(it);
    }
}

// One GEMV on device buffers: the matrix-core Q4_K kernel where it is the
// faster one (gemv_mx_default), else the whole-row kernel when a row fits one
// workgroup, else split-K.
// Scratch (the matrix-core kernel's per-row exchange slots when rows are
// split over two workgroups, the split-K partials) comes from the stream's
// registry, or from `fixed` when given (nothing is allocated then; a shape
// that needs more than `fixed` holds is refused before anything launches).
int gemv_device(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, hipStream_t s,
                const frq::FixedScratch* fixed = nullptr) {
    if (frq::gemv_mx_default(qtype, w, x, n, k)) {
        frq::MxPlan mp;
        frq::plan_gemv_mx(n, k, &mp);
        const size_t need = frq::gemv_mx_slot_bytes(mp, n);
        if (fixed) {
            if (need > fixed->slot_bytes)
                return fail(FRQ_ERR_UNSUPPORTED, "gemv: %zu bytes of row slots needed, the fixed scratch holds %zu",
                            need, fixed->slot_bytes);
            FRQ_HIP(frq::launch_gemv_mx(w, x, y, n, k, mp, fixed->slots, s));
            return FRQ_OK;
        }
        float* part = nullptr;
        uint32_t* cnt = nullptr;
        std::lock_guard<std::mutex> lk(g_sk_mu);
        if (int rc = sk_scratch_locked(s, 0, need, &part, &cnt)) return rc;
        FRQ_HIP(frq::launch_gemv_mx(w, x, y, n, k, mp, reinterpret_cast<uint64_t*>(cnt), s));
        return FRQ_OK;
    }
    if (frq::gemv_supported(qtype, n, k)) {   // whole-row kernel, one slice: no scratch
        FRQ_HIP(frq::launch_gemv(qtype, w, x, y, n, k, nullptr, s));
        return FRQ_OK;
    }
    frq::SplitKPlan sp;
    if (!frq::plan_gemv_sk(qtype, n, k, &sp))
        return fail(FRQ_ERR_UNSUPPORTED, "gemv: k=%lld has no kernel plan for this format", (long long)k);
    size_t pb = 0, cb = 0;
    frq::gemv_sk_scratch(sp, n, &pb, &cb);
    if (fixed) {
        if (pb > fixed->part_bytes || cb > 0)
            return fail(FRQ_ERR_UNSUPPORTED, "gemv: %zu bytes of split-K partials needed, the fixed scratch holds %zu",
                        pb, fixed->part_bytes);
        FRQ_HIP(frq::launch_gemv_sk(qtype, w, x, y, n, k, sp, fixed->part, nullptr, s));
        return FRQ_OK;
    }
    float* part = nullptr;
    uint32_t* cnt = nullptr;
    std::lock_guard<std::mutex> lk(g_sk_mu);
    if (int rc = sk_scratch_locked(s, pb, cb, &part, &cnt)) return rc;
    FRQ_HIP(frq::launch_gemv_sk(qtype, w, x, y, n, k, sp, part, cnt, s));
    return FRQ_OK;
}

// Scratch a GEMV of this shape needs (0 for both when none), for callers
// that bring their own: slot bytes must be zero before the launch.
void gemv_scratch_need(int qtype, const uint8_t* w, const float* x, int64_t n, int64_t k, size_t* slot_bytes,
                       size_t* part_bytes) {
    *slot_bytes = *part_bytes = 0;
    if (frq::gemv_mx_default(qtype, w, x, n, k)) {
        frq::MxPlan mp;
        frq::plan_gemv_mx(n, k, &mp);
        *slot_bytes = frq::gemv_mx_slot_bytes(mp, n);
        return;
    }
    if (frq::gemv_supported(qtype, n, k)) return;
    frq::SplitKPlan sp;
    if (!frq::plan_gemv_sk(qtype, n, k, &sp)) return;
    size_t cb = 0;
    frq::gemv_sk_scratch(sp, n, part_bytes, &cb);
}

// Rows of x that the fp32-contract matrix-core GEMM (W read once per tile of
// x rows) can take: Q4_K, Q6_K and Q8_0 with two or more rows.
bool batched_gemm(int qtype, const uint8_t* w, const float* x, int64_t batch, int64_t n, int64_t k) {
    if (batch < 2 || !frq::gemm_f32_supported(qtype, batch, n, k)) return false;
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    return !(reinterpret_cast<uintptr_t>(x) & 15) && !(qtype == FRQ_Q4_K ? (wa & 15) : (wa & 1));
}

// Up to this many rows of x (two or more), a matrix that the small-M kernel
// takes (gemv_mr_ok) runs it, one launch per chunk of two or three rows,
// each reading W once, rather than the GEMM (latency-bound at few rows, one
// K-step of loads in flight per workgroup). Measured (graph-replayed, us):
//   Q4_K 3584 x 18944: 2 / 3 / 6 rows 17.0 / 20.1 / 38-41; GEMM 46 from 4 rows
//   Q6_K 4096 x 14336: 2 / 3 / 6 / 10 rows 16.0 / 18.3 / 34.1 / 64; GEMM 70
//   Q8_0 4096 x 4096: 2 / 3 / 6 / 8 rows 7.8 / 9.3 / 16.9 / 22.9; GEMM 20.7
int64_t mr_rows_before_gemm(int qtype) {
    return qtype == FRQ_Q6_K ? 10 : 6;
}

// Q4_K batches the fp32 matrix-core kernel takes in one launch: four rows of
// x (k <= 24576), or five to eight where k <= 8192. Two and three rows take
// the small-M element-wise kernel, longer batches chunks of it or the GEMM.
// Measured (us, graph-replayed): Q4_K 3584 x 18944, matrix cores 2 / 3 / 4
// rows 24.7 / 26.2 / 27.6, element-wise small-M 17.1 / 20.4 / 34 (2 + 2),
// 5 / 6 rows 35.5 / 39.6 (3 + 2, 3 + 3), GEMM 42.7 at 7; Q4_K 4096 x 4096,
// matrix cores 4 / 5 / 6 rows 8.7 / 11.1 / 12.0, GEMM 18.3 at 7.
bool mb_takes(int qtype, const uint8_t* w, const float* x, int64_t batch, int64_t n, int64_t k) {
    frq::MbPlan p;
    return qtype == FRQ_Q4_K && batch >= 4 && batch <= frq::kGemvMbMax && frq::gemv_mb_ok(w, x, k) &&
           frq::plan_gemv_mb(n, k, (int)batch, &p);
}

// Up to this many rows of x, a matrix that the small-M kernel does not take
// (its alignment, block count or k) runs one GEMV per row rather than the
// GEMM: each GEMV reads the weights again, but at a few rows its time per
// row stays below the GEMM's (Q4_K 3584 x 18944: 12.6 us per row against 46;
// Q6_K 4096 x 14336: 13.3 against 70; Q8_0 4096 x 4096: 5.4 against 20.7).
constexpr int64_t kRowsBeforeGemm = 3;

// Which kernels a batch of x rows takes: the small-M kernel for two to
// mr_rows_before_gemm rows, else one GEMV per row up to kRowsBeforeGemm
// rows, else the GEMM where batched_gemm allows, else one GEMV per row.
enum class BatchRoute { SmallM, Gemm, Rows };
BatchRoute batch_route(int qtype, const uint8_t* w, const float* x, int64_t batch, int64_t n, int64_t k) {
    if (mb_takes(qtype, w, x, batch, n, k) ||
        (batch >= 2 && batch <= mr_rows_before_gemm(qtype) && frq::gemv_mr_ok(qtype, w, x, k)))
        return BatchRoute::SmallM;
    if (batch > kRowsBeforeGemm && batched_gemm(qtype, w, x, batch, n, k)) return BatchRoute::Gemm;
    return BatchRoute::Rows;
}

// y[b * ldy + i] = (W x_b)[i] for b < batch, by batch_route. Scratch as
// gemv_device (the small-M kernel uses none).
int gemv_batched(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int64_t batch,
                 int64_t ldy, hipStream_t s, const frq::FixedScratch* fixed = nullptr) {
    const BatchRoute route = batch_route(qtype, w, x, batch, n, k);
    if (route == BatchRoute::SmallM && mb_takes(qtype, w, x, batch, n, k)) {
        frq::MbPlan p;
        frq::plan_gemv_mb(n, k, (int)batch, &p);
        FRQ_HIP(frq::launch_gemv_mb(w, x, y, n, k, (int)batch, ldy, p, s));
        return FRQ_OK;
    }
    if (route == BatchRoute::SmallM) {
        for (int64_t b = 0; b < batch;) {   // chunks of 2 or 3 rows: 4 = 2 + 2, 5 = 3 + 2, 7 = 3 + 2 + 2
            const int64_t rem = batch - b, m = rem == 4 ? 2 : (rem < 3 ? rem : 3);
            FRQ_HIP(frq::launch_gemv_mr(qtype, w, x + b * k, y + b * ldy, n, k, (int)m, ldy, s));
            b += m;
        }
        return FRQ_OK;
    }
    if (route == BatchRoute::Gemm) {
        if (fixed) {   // as many K-splits as the fixed partial region holds
            FRQ_HIP(frq::launch_gemm_f32(qtype, w, x, y, batch, n, k, ldy, s, fixed->part, fixed->part_bytes));
            return FRQ_OK;
        }
        const size_t pb = frq::gemm_f32_scratch(qtype, batch, n, k);
        float* part = nullptr;
        uint32_t* cnt = nullptr;
        std::lock_guard<std::mutex> lk(g_sk_mu);
        if (int rc = sk_scratch_locked(s, pb, 0, &part, &cnt)) return rc;
        FRQ_HIP(frq::launch_gemm_f32(qtype, w, x, y, batch, n, k, ldy, s, part, pb));
        return FRQ_OK;
    }
    for (int64_t b = 0; b < batch; ++b)
        if (int rc = gemv_device(qtype, w, x + b * k, y + b * ldy, n, k, s, fixed)) return rc;
    return FRQ_OK;
}

// Host dequant: stage weight, decode (fp32, or fp16 bits), copy back.
// n_elems may be ragged.
template <typename T>
int host_dequant_t(int qtype, const uint8_t* weight, size_t weight_bytes, int64_t n_elems, T* out) {
    if (n_elems == 0) return FRQ_OK;
    if (int rc = have_device()) return rc;
    std::lock_guard<std::mutex> lk(g_ws.mu);
    const size_t wb = align256(weight_bytes), yb = align256((size_t)n_elems * sizeof(T));
    void* base = nullptr;
    if (int rc = workspace(wb + yb, &base)) return rc;
    uint8_t* dw = static_cast<uint8_t*>(base);
    T* dy = reinterpret_cast<T*>(dw + wb);
    FRQ_HIP(hipMemcpy(dw, weight, weight_bytes, hipMemcpyHostToDevice));
    if constexpr (sizeof(T) == 2)
        FRQ_HIP(frq::launch_dequant_f16(qtype, dw, dy, n_elems, nullptr));
    else
        FRQ_HIP(frq::launch_dequant(qtype, dw, dy, n_elems, nullptr));
    FRQ_HIP(hipMemcpy(out, dy, (size_t)n_elems * sizeof(T), hipMemcpyDeviceToHost));
    return FRQ_OK;
}

int host_dequant(int qtype, const uint8_t* weight, size_t weight_bytes, int64_t n_elems, float* out) {
    return host_dequant_t(qtype, weight, weight_bytes, n_elems, out);
}

// Host matmul over seq rows of x (already validated).
int host_matmul(int qtype, const float* x, size_t seq, const uint8_t* weight, size_t weight_bytes, size_t n,
                size_t k, float* out) {
    if (seq == 0 || n == 0) return FRQ_OK;
    if (k == 0) {   // empty dot products: the reference's accumulators stay 0
        std::memset(out, 0, seq * n * sizeof(float));
        return FRQ_OK;
    }
    if (int rc = have_device()) return rc;
    if (!frq::gemv_sk_supported(qtype) && !frq::gemv_supported(qtype, (int64_t)n, (int64_t)k))
        return fail(FRQ_ERR_UNSUPPORTED, "matmul: k=%zu is beyond the single-workgroup row limit of this library", k);
    std::lock_guard<std::mutex> lk(g_ws.mu);
    const size_t wb = align256(weight_bytes), xb = align256(seq * k * 4), yb = align256(seq * n * 4);
    void* base = nullptr;
    if (int rc = workspace(wb + xb + yb, &base)) return rc;
    uint8_t* dw = static_cast<uint8_t*>(base);
    float* dx = reinterpret_cast<float*>(dw + wb);
    float* dy = reinterpret_cast<float*>(dw + wb + xb);
    FRQ_HIP(hipMemcpy(dw, weight, weight_bytes, hipMemcpyHostToDevice));
    FRQ_HIP(hipMemcpy(dx, x, seq * k * 4, hipMemcpyHostToDevice));
    if (int rc = gemv_batched(qtype, dw, dx, dy, (int64_t)n, (int64_t)k, (int64_t)seq, (int64_t)n, nullptr)) return rc;
    FRQ_HIP(hipMemcpy(out, dy, seq * n * 4, hipMemcpyDeviceToHost));
    return FRQ_OK;
}

// _C.cpp dequant_<q>_py checks (e.g. :54-67).
int check_dequant_2d(const Fmt& f, size_t weight_bytes, int64_t out_dim, int64_t in_dim) {
    if (out_dim < 0 || in_dim < 0) return fail(FRQ_ERR_SHAPE, "%s: negative shape", f.name);
    const int64_t total = out_dim * in_dim;
    if (total % f.belems != 0)
        return fail(FRQ_ERR_SHAPE, "%s tensor element count must be a multiple of %lld", f.name, (long long)f.belems);
    const int64_t nblk = total / f.belems;
    if ((int64_t)weight_bytes != nblk * f.bbytes)
        return fail(FRQ_ERR_SIZE, "%s weight byte size mismatch: expected %lld bytes, got %zu", f.name,
                    (long long)(nblk * f.bbytes), weight_bytes);
    return FRQ_OK;
}

// _C.cpp matmul_<q>_py checks (e.g. :105-120).
int check_matmul(const Fmt& f, size_t x_len, size_t weight_bytes, size_t n, size_t k) {
    if (k % (size_t)f.belems != 0)
        return fail(FRQ_ERR_SHAPE, "%s matmul: in_features must be a multiple of %lld", f.name, (long long)f.belems);
    if (x_len != k) return fail(FRQ_ERR_SHAPE, "%s matmul: x.size() != k", f.name);
    if (weight_bytes != n * (k / (size_t)f.belems) * (size_t)f.bbytes)
        return fail(FRQ_ERR_SIZE, "%s matmul: weight byte size mismatch", f.name);
    return FRQ_OK;
}

// _C.cpp matmul_<q>_batched_py checks (e.g. :160-182).
int check_batched(const Fmt& f, int x_ndim, size_t x_cols, size_t weight_bytes, size_t n, size_t k) {
    if (k % (size_t)f.belems != 0)
        return fail(FRQ_ERR_SHAPE, "%s matmul (batched): in_features must be a multiple of %lld", f.name,
                    (long long)f.belems);
    if (x_ndim != 2) return fail(FRQ_ERR_SHAPE, "%s matmul (batched): x must be 2-D (seq, k)", f.name);
    if (x_cols != k) return fail(FRQ_ERR_SHAPE, "%s matmul (batched): x.shape[1] != k", f.name);
    if (weight_bytes != n * (k / (size_t)f.belems) * (size_t)f.bbytes)
        return fail(FRQ_ERR_SIZE, "%s matmul (batched): weight byte size mismatch", f.name);
    return FRQ_OK;
}

int dequant_2d(int qtype, const uint8_t* weight, size_t weight_bytes, int64_t out_dim, int64_t in_dim, float* out) {
    Fmt f;
    fmt_of(qtype, &f);
    if (int rc = check_dequant_2d(f, weight_bytes, out_dim, in_dim)) return rc;
    if ((!weight && weight_bytes) || (!out && out_dim * in_dim)) return fail(FRQ_ERR_INVALID, "null buffer");
    return host_dequant(qtype, weight, weight_bytes, out_dim * in_dim, out);
}

int matmul_1d(int qtype, const float* x, size_t x_len, const uint8_t* weight, size_t weight_bytes, size_t n, size_t k,
              float* out) {
    Fmt f;
    fmt_of(qtype, &f);
    if (int rc = check_matmul(f, x_len, weight_bytes, n, k)) return rc;
    if ((!x && k) || (!weight && weight_bytes) || (!out && n)) return fail(FRQ_ERR_INVALID, "null buffer");
    return host_matmul(qtype, x, 1, weight, weight_bytes, n, k, out);
}

int matmul_2d(int qtype, const float* x, int x_ndim, size_t seq, size_t x_cols, const uint8_t* weight,
              size_t weight_bytes, size_t n, size_t k, float* out) {
    Fmt f;
    fmt_of(qtype, &f);
    if (int rc = check_batched(f, x_ndim, x_cols, weight_bytes, n, k)) return rc;
    if ((!x && seq * k) || (!weight && weight_bytes) || (!out && seq * n)) return fail(FRQ_ERR_INVALID, "null buffer");
    return host_matmul(qtype, x, seq, weight, weight_bytes, n, k, out);
}

// Format, element count and byte size of a dequant call (the NumPy
// decoders' ceil-div block rule, gguf.py:61-73), and non-null buffers.
int dequant_checks(int qtype, const void* w, size_t w_bytes, int64_t n_elems, const void* y) {
    Fmt f;
    if (!fmt_of(qtype, &f)) return fail(FRQ_ERR_INVALID, "unknown quant type %d", qtype);
    if (n_elems < 0) return fail(FRQ_ERR_SHAPE, "%s: negative element count", f.name);
    const int64_t nblk = (n_elems + f.belems - 1) / f.belems;
    if ((int64_t)w_bytes != nblk * f.bbytes)
        return fail(FRQ_ERR_SIZE, "%s weight byte size mismatch: expected %lld bytes, got %zu", f.name,
                    (long long)(nblk * f.bbytes), w_bytes);
    if ((!w && w_bytes) || (!y && n_elems)) return fail(FRQ_ERR_INVALID, "null buffer");
    return FRQ_OK;
}

int check_dev_ptrs(int qtype, const void* w, const float* x, const float* y) {
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    const bool k_quant16 = qtype == FRQ_Q4_K || qtype == FRQ_Q5_K;
    if (k_quant16 ? (wa & 15) : (wa & 1)) return fail(FRQ_ERR_ALIGN, "weight pointer misaligned for its format");
    if (x && (reinterpret_cast<uintptr_t>(x) & 15)) return fail(FRQ_ERR_ALIGN, "x must be 16-byte aligned");
    if (y && (reinterpret_cast<uintptr_t>(y) & 3)) return fail(FRQ_ERR_ALIGN, "y must be 4-byte aligned");
    return FRQ_OK;
}

}  // namespace

extern "C" {

const char* frq_version(void) { return "flatrun_amd 0.2.0 (gfx950 HIP: Q8_0, Q4_K, Q5_K, Q6_K, Q1_0; dequant Q4_0, Q5_0, Q5_1)"; }
int frq_is_neon(void) { return 0; }
const char* frq_last_error(void) { return g_err.c_str(); }

int frq_device_count(int* count) {
    if (!count) return fail(FRQ_ERR_INVALID, "null count");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        n = 0;
    }
    *count = n;
    return FRQ_OK;
}

int frq_block_info(int qtype, int64_t* block_bytes, int64_t* block_elems) {
    Fmt f;
    if (!fmt_of(qtype, &f)) return fail(FRQ_ERR_INVALID, "unknown quant type %d", qtype);
    if (block_bytes) *block_bytes = f.bbytes;
    if (block_elems) *block_elems = f.belems;
    return FRQ_OK;
}

int frq_dequant_q4_k(const uint8_t* w, size_t wb, int64_t o, int64_t i, float* out) { return dequant_2d(FRQ_Q4_K, w, wb, o, i, out); }
int frq_dequant_q8_0(const uint8_t* w, size_t wb, int64_t o, int64_t i, float* out) { return dequant_2d(FRQ_Q8_0, w, wb, o, i, out); }
int frq_dequant_q6_k(const uint8_t* w, size_t wb, int64_t o, int64_t i, float* out) { return dequant_2d(FRQ_Q6_K, w, wb, o, i, out); }

int frq_dequant(int qtype, const uint8_t* weight, size_t weight_bytes, int64_t n_elems, float* out) {
    if (int rc = dequant_checks(qtype, weight, weight_bytes, n_elems, out)) return rc;
    return host_dequant(qtype, weight, weight_bytes, n_elems, out);
}

int frq_dequant_f16(int qtype, const uint8_t* weight, size_t weight_bytes, int64_t n_elems, uint16_t* out) {
    if (int rc = dequant_checks(qtype, weight, weight_bytes, n_elems, out)) return rc;
    return host_dequant_t(qtype, weight, weight_bytes, n_elems, out);
}

int frq_matmul_q4_k(const float* x, size_t xl, const uint8_t* w, size_t wb, size_t n, size_t k, float* out) { return matmul_1d(FRQ_Q4_K, x, xl, w, wb, n, k, out); }
int frq_matmul_q8_0(const float* x, size_t xl, const uint8_t* w, size_t wb, size_t n, size_t k, float* out) { return matmul_1d(FRQ_Q8_0, x, xl, w, wb, n, k, out); }
int frq_matmul_q6_k(const float* x, size_t xl, const uint8_t* w, size_t wb, size_t n, size_t k, float* out) { return matmul_1d(FRQ_Q6_K, x, xl, w, wb, n, k, out); }

int frq_matmul_q4_k_batched(const float* x, int nd, size_t seq, size_t xc, const uint8_t* w, size_t wb, size_t n, size_t k, float* out) {
    return matmul_2d(FRQ_Q4_K, x, nd, seq, xc, w, wb, n, k, out);
}
int frq_matmul_q8_0_batched(const float* x, int nd, size_t seq, size_t xc, const uint8_t* w, size_t wb, size_t n, size_t k, float* out) {
    return matmul_2d(FRQ_Q8_0, x, nd, seq, xc, w, wb, n, k, out);
}
int frq_matmul_q6_k_batched(const float* x, int nd, size_t seq, size_t xc, const uint8_t* w, size_t wb, size_t n, size_t k, float* out) {
    return matmul_2d(FRQ_Q6_K, x, nd, seq, xc, w, wb, n, k, out);
}

int frq_matmul(int qtype, const float* x, size_t seq, const uint8_t* weight, size_t weight_bytes, size_t n, size_t k,
               float* out) {
    Fmt f;
    if (!fmt_of(qtype, &f)) return fail(FRQ_ERR_INVALID, "unknown quant type %d", qtype);
    return matmul_2d(qtype, x, 2, seq, k, weight, weight_bytes, n, k, out);
}

int frq_dev_dequant(int qtype, const void* w, size_t w_bytes, int64_t n_elems, float* y, void* stream) {
    if (int rc = dequant_checks(qtype, w, w_bytes, n_elems, y)) return rc;
    if (n_elems == 0) return FRQ_OK;
    if (int rc = check_dev_ptrs(qtype, w, nullptr, y)) return rc;
    FRQ_HIP(frq::launch_dequant(qtype, static_cast<const uint8_t*>(w), y, n_elems, static_cast<hipStream_t>(stream)));
    return FRQ_OK;
}

int frq_dev_dequant_f16(int qtype, const void* w, size_t w_bytes, int64_t n_elems, uint16_t* y, void* stream) {
    if (int rc = dequant_checks(qtype, w, w_bytes, n_elems, y)) return rc;
    if (n_elems == 0) return FRQ_OK;
    if (int rc = check_dev_ptrs(qtype, w, nullptr, nullptr)) return rc;
    if (reinterpret_cast<uintptr_t>(y) & 1) return fail(FRQ_ERR_ALIGN, "y must be 2-byte aligned");
    FRQ_HIP(frq::launch_dequant_f16(qtype, static_cast<const uint8_t*>(w), y, n_elems,
                                    static_cast<hipStream_t>(stream)));
    return FRQ_OK;
}

static int dev_gemv_checks(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                           int64_t batch, Fmt* f) {
    if (!fmt_of(qtype, f)) return fail(FRQ_ERR_INVALID, "unknown quant type %d", qtype);
    if (n < 0 || k < 0 || batch < 0) return fail(FRQ_ERR_SHAPE, "%s: negative shape", f->name);
    if (k % f->belems) return fail(FRQ_ERR_SHAPE, "%s matmul: in_features must be a multiple of %lld", f->name, (long long)f->belems);
    if ((int64_t)w_bytes != n * (k / f->belems) * f->bbytes)
        return fail(FRQ_ERR_SIZE, "%s matmul: weight byte size mismatch", f->name);
    if (n == 0 || batch == 0) return FRQ_OK;
    if (!w || !x || !y) return fail(FRQ_ERR_INVALID, "null buffer");
    if (int rc = check_dev_ptrs(qtype, w, x, y)) return rc;
    if (k > 0 && !frq::gemv_sk_supported(qtype) && !frq::gemv_supported(qtype, n, k))
        return fail(FRQ_ERR_UNSUPPORTED, "%s matmul: k=%lld is beyond the single-workgroup row limit of this library",
                    f->name, (long long)k);
    return FRQ_OK;
}

static int dev_gemv(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                    int64_t batch, void* stream, const frq::FixedScratch* fixed) {
    Fmt f;
    if (int rc = dev_gemv_checks(qtype, w, w_bytes, x, y, n, k, batch, &f)) return rc;
    if (n == 0 || batch == 0) return FRQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (k == 0) {   // empty dot products are 0; a kernel fill keeps the call graph-capturable
        FRQ_HIP(frq::launch_fill(y, 0.0f, batch * n, s));
        return FRQ_OK;
    }
    const uint8_t* wp = static_cast<const uint8_t*>(w);
    if (fixed) {   // refuse an oversized shape before any row is launched
        size_t sb = 0, pb = 0;
        // the small-M kernel needs no scratch and the batched GEMM splits K
        // within what is there; rows that run one GEMV each need theirs
        if (batch_route(qtype, wp, x, batch, n, k) == BatchRoute::Rows) gemv_scratch_need(qtype, wp, x, n, k, &sb, &pb);
        if (sb > fixed->slot_bytes || pb > fixed->part_bytes)
            return fail(FRQ_ERR_UNSUPPORTED,
                        "%s gemv n=%lld k=%lld needs %zu slot + %zu partial bytes of scratch; the fixed scratch "
                        "holds %zu + %zu", f.name, (long long)n, (long long)k, sb, pb, fixed->slot_bytes,
                        fixed->part_bytes);
    }
    return gemv_batched(qtype, wp, x, y, n, k, batch, n, s, fixed);
}

int frq_dev_gemv(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                 int64_t batch, void* stream) {
    return dev_gemv(qtype, w, w_bytes, x, y, n, k, batch, stream, nullptr);
}

int frq_gemv_group_fusable(int count, const int* qtypes, const void* const* w, int64_t k) {
    if (count < 1 || count > frq::kGemvGroupMax || !qtypes || !w) return 0;
    return frq::gemv_group_fusable(count, qtypes, reinterpret_cast<const uint8_t* const*>(w), k) ? 1 : 0;
}

int frq_dev_gemv_group(int count, const int* qtypes, const void* const* w, const size_t* w_bytes, const int64_t* n,
                       const float* x, int64_t k, float* const* y, int64_t batch, int64_t y_stride, void* stream) {
    if (count < 1 || count > frq::kGemvGroupMax)
        return fail(FRQ_ERR_INVALID, "gemv group: count %d outside [1, %d]", count, frq::kGemvGroupMax);
    if (!qtypes || !w || !w_bytes || !n || !y) return fail(FRQ_ERR_INVALID, "gemv group: null argument array");
    if (y_stride < 0) return fail(FRQ_ERR_SHAPE, "gemv group: negative y_stride");
    Fmt f;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        if (int rc = dev_gemv_checks(qtypes[i], w[i], w_bytes[i], x, y[i], n[i], k, batch, &f)) return rc;
        total += n[i];
    }
    if (total == 0 || batch == 0) return FRQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* wp[frq::kGemvGroupMax];
    float* yb[frq::kGemvGroupMax];
    for (int i = 0; i < count; ++i) wp[i] = static_cast<const uint8_t*>(w[i]);
    const bool fused = k > 0 && frq::gemv_group_fusable(count, qtypes, wp, k);
    if (k > 0 && batch >= 2) {   // prefill-shaped: each matrix once, its rows of x together
        for (int i = 0; i < count; ++i)
            if (n[i])
                if (int rc = gemv_batched(qtypes[i], wp[i], x, y[i], n[i], k, batch, y_stride ? y_stride : n[i], s))
                    return rc;
        return FRQ_OK;
    }
    for (int64_t b = 0; b < batch; ++b) {
        for (int i = 0; i < count; ++i) yb[i] = y[i] + b * (y_stride ? y_stride : n[i]);
        if (k == 0) {   // empty dot products are 0 (kernel fill: graph-capturable)
            for (int i = 0; i < count; ++i)
                if (n[i]) FRQ_HIP(frq::launch_fill(yb[i], 0.0f, n[i], s));
        } else if (fused) {
            FRQ_HIP(frq::launch_gemv_group(count, qtypes, wp, n, yb, x + b * k, k, s));
        } else {
            for (int i = 0; i < count; ++i)
                if (n[i])
                    if (int rc = gemv_device(qtypes[i], wp[i], x + b * k, yb[i], n[i], k, s)) return rc;
        }
    }
    return FRQ_OK;
}

int frq_dev_gemv_tuned(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                       frq_gemv_config* cfg, void* stream) {
    Fmt f;
    if (!cfg) return fail(FRQ_ERR_INVALID, "null config");
    if (int rc = dev_gemv_checks(qtype, w, w_bytes, x, y, n, k, 1, &f)) return rc;
    if (n == 0 || k == 0) return fail(FRQ_ERR_SHAPE, "tuned gemv needs n > 0 and k > 0");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* wp = static_cast<const uint8_t*>(w);
    if (cfg->kernel != FRQ_GEMV_AUTO && cfg->kernel != FRQ_GEMV_SPLITK && cfg->kernel != FRQ_GEMV_ROWS &&
        cfg->kernel != FRQ_GEMV_MX && cfg->kernel != FRQ_GEMV_MB)
        return fail(FRQ_ERR_INVALID, "tuned gemv: unknown kernel %d", cfg->kernel);
    if (cfg->kernel == FRQ_GEMV_MB) {
        if (qtype != FRQ_Q4_K) return fail(FRQ_ERR_UNSUPPORTED, "the fp32 matrix-core GEMV takes Q4_K");
        if (!frq::gemv_mb_ok(wp, x, k))
            return fail(FRQ_ERR_ALIGN, "the fp32 matrix-core GEMV needs 16-byte aligned weights and x");
        frq::MbPlan mp;
        mp.rows = cfg->rows;
        mp.nbp = cfg->unroll;
        if (!frq::plan_gemv_mb(n, k, 1, &mp))
            return fail(FRQ_ERR_UNSUPPORTED, "fp32 matrix-core GEMV: no plan for n=%lld k=%lld rows=%d pairs=%d",
                        (long long)n, (long long)k, cfg->rows, cfg->unroll);
        hipError_t e = frq::launch_gemv_mb(wp, x, y, n, k, 1, n, mp, s);
        if (e != hipSuccess) return tuned_fail(e, "launch_gemv_mb");
        cfg->cpl = 1;
        cfg->rows = mp.rows;
        cfg->unroll = mp.nbp;
        cfg->slices = 1;
        cfg->waves_per_wg = mp.waves;
        cfg->items = mp.grid;
        return FRQ_OK;
    }
    if (cfg->kernel == FRQ_GEMV_MX || (cfg->kernel == FRQ_GEMV_AUTO && frq::gemv_mx_default(qtype, wp, x, n, k))) {
        if (qtype != FRQ_Q4_K) return fail(FRQ_ERR_UNSUPPORTED, "the matrix-core GEMV takes Q4_K");
        if ((reinterpret_cast<uintptr_t>(wp) | reinterpret_cast<uintptr_t>(x)) & 15)
            return fail(FRQ_ERR_ALIGN, "the matrix-core GEMV needs 16-byte aligned weights and x");
        frq::MxPlan mp;
        mp.rows = cfg->rows;
        mp.tiles = cfg->cpl;
        mp.ksplit = cfg->slices;
        mp.depth = cfg->unroll;
        if (!frq::plan_gemv_mx(n, k, &mp))
            return fail(FRQ_ERR_UNSUPPORTED,
                        "matrix-core GEMV: no plan for n=%lld k=%lld rows=%d tiles=%d ksplit=%d depth=%d",
                        (long long)n, (long long)k, cfg->rows, cfg->cpl, cfg->slices, cfg->unroll);
        float* part = nullptr;
        uint32_t* cnt = nullptr;
        std::lock_guard<std::mutex> lk(g_sk_mu);
        if (int rc = sk_scratch_locked(s, 0, frq::gemv_mx_slot_bytes(mp, n), &part, &cnt)) return rc;
        hipError_t e = frq::launch_gemv_mx(wp, x, y, n, k, mp, reinterpret_cast<uint64_t*>(cnt), s);
        if (e != hipSuccess) return tuned_fail(e, "launch_gemv_mx");
        cfg->kernel = FRQ_GEMV_MX;
        cfg->cpl = mp.tiles;
        cfg->rows = mp.rows;
        cfg->unroll = mp.depth;
        cfg->slices = mp.ksplit;
        cfg->waves_per_wg = mp.waves;
        cfg->items = mp.grid;
        return FRQ_OK;
    }
    if (cfg->kernel == FRQ_GEMV_SPLITK ||
        (cfg->kernel == FRQ_GEMV_AUTO && !frq::gemv_supported(qtype, n, k) && frq::gemv_sk_supported(qtype))) {
        frq::SplitKPlan p;
        p.cpl = cfg->cpl;
        p.rows = cfg->rows;
        p.unroll = cfg->unroll;
        if (!frq::plan_gemv_sk(qtype, n, k, &p)) return fail(FRQ_ERR_UNSUPPORTED, "split-K plan rejected");
        size_t pb = 0, cb = 0;
        frq::gemv_sk_scratch(p, n, &pb, &cb);
        float* part = nullptr;
        uint32_t* cnt = nullptr;
        std::lock_guard<std::mutex> lk(g_sk_mu);
        if (int rc = sk_scratch_locked(s, pb, cb, &part, &cnt)) return rc;
        hipError_t e = frq::launch_gemv_sk(qtype, wp, x, y, n, k, p, part, cnt, s);
        if (e != hipSuccess) return tuned_fail(e, "launch_gemv_sk");
        cfg->kernel = FRQ_GEMV_SPLITK;
        cfg->cpl = p.cpl;
        cfg->rows = p.rows;
        cfg->unroll = p.unroll;
        cfg->slices = p.slices;
        cfg->waves_per_wg = p.items >= 4 ? 4 : (int)p.items;
        cfg->items = p.items;
        return FRQ_OK;
    }
    frq::GemvPlan p;
    p.cpl = cfg->cpl;
    p.rows_per_wg = cfg->rows;
    p.unroll = cfg->unroll;
    p.slices = cfg->slices;
    hipError_t e = frq::launch_gemv(qtype, wp, x, y, n, k, &p, s);
    if (e != hipSuccess) return tuned_fail(e, "launch_gemv");
    cfg->kernel = FRQ_GEMV_ROWS;
    cfg->cpl = p.cpl;
    cfg->rows = p.rows_per_wg;
    cfg->unroll = p.unroll;
    cfg->slices = p.slices > 0 ? p.slices : 1;
    cfg->waves_per_wg = p.waves;
    cfg->items = p.grid;
    return FRQ_OK;
}

static int gemm_checks(int qtype, size_t w_bytes, int64_t m, int64_t n, int64_t k, Fmt* f) {
    if (qtype != FRQ_Q4_K && qtype != FRQ_Q6_K && qtype != FRQ_Q8_0)
        return fail(FRQ_ERR_UNSUPPORTED, "gemm: quant type %d has no matrix-core GEMM (Q4_K, Q6_K, Q8_0)", qtype);
    fmt_of(qtype, f);
    const int64_t kq = qtype == FRQ_Q8_0 ? 128 : 256;
    if (m < 0 || n < 0 || k < 0) return fail(FRQ_ERR_SHAPE, "%s gemm: negative shape", f->name);
    if (k % kq) return fail(FRQ_ERR_SHAPE, "%s gemm: in_features must be a multiple of %lld", f->name, (long long)kq);
    if ((int64_t)w_bytes != n * (k / f->belems) * f->bbytes)
        return fail(FRQ_ERR_SIZE, "%s gemm: weight byte size mismatch", f->name);
    if (m > 0 && n > 0 && k > 0 && !frq::gemm_bf16_supported(qtype, m, n, k))
        return fail(FRQ_ERR_UNSUPPORTED, "%s gemm: shape beyond this library's limits", f->name);
    return FRQ_OK;
}

int frq_dev_gemm_bf16(int qtype, const void* w, size_t w_bytes, const uint16_t* x, float* y, int64_t m, int64_t n,
                      int64_t k, void* stream) {
    Fmt f;
    if (int rc = gemm_checks(qtype, w_bytes, m, n, k, &f)) return rc;
    if (m == 0 || n == 0) return FRQ_OK;
    if (!y) return fail(FRQ_ERR_INVALID, "null buffer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (k == 0) {
        FRQ_HIP(frq::launch_fill(y, 0.0f, m * n, s));
        return FRQ_OK;
    }
    if (!w || !x) return fail(FRQ_ERR_INVALID, "null buffer");
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    if ((qtype == FRQ_Q4_K ? (wa & 15) : (wa & 1)) || (reinterpret_cast<uintptr_t>(x) & 15))
        return fail(FRQ_ERR_ALIGN, "%s gemm: weight or x misaligned", f.name);
    if (reinterpret_cast<uintptr_t>(y) & 3) return fail(FRQ_ERR_ALIGN, "y must be 4-byte aligned");
    float* part = nullptr;
    uint32_t* cnt = nullptr;
    std::lock_guard<std::mutex> lk(g_sk_mu);
    if (int rc = sk_scratch_locked(s, frq::gemm_bf16_scratch(m, n, k), 0, &part, &cnt)) return rc;   // split-K partials
    FRQ_HIP(frq::launch_gemm_bf16(qtype, static_cast<const uint8_t*>(w), x, y, m, n, k, s, part));
    return FRQ_OK;
}

int frq_dev_gemm_bf16_group(int count, const int* qtypes, const void* const* w, const size_t* w_bytes,
                            const int64_t* n, const uint16_t* x, int64_t m, int64_t k, float* const* y,
                            int64_t y_stride, void* stream) {
    if (count < 1 || count > frq::kGemmGroupMax)
        return fail(FRQ_ERR_INVALID, "gemm group: count %d outside [1, %d]", count, frq::kGemmGroupMax);
    if (!qtypes || !w || !w_bytes || !n || !y) return fail(FRQ_ERR_INVALID, "gemm group: null argument array");
    if (y_stride < 0 || y_stride > 0x7FFFFFFF) return fail(FRQ_ERR_SHAPE, "gemm group: y_stride outside [0, 2^31)");
    Fmt f;
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        if (int rc = gemm_checks(qtypes[i], w_bytes[i], m, n[i], k, &f)) return rc;
        if (y_stride && y_stride < n[i]) return fail(FRQ_ERR_SHAPE, "gemm group: y_stride below a matrix's rows");
        total += n[i];
    }
    if (m == 0 || total == 0) return FRQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < count; ++i)
        if (n[i] && !y[i]) return fail(FRQ_ERR_INVALID, "null buffer");
    if (k == 0) {   // empty dot products are 0 (kernel fills: graph-capturable)
        for (int i = 0; i < count; ++i) {
            if (!n[i]) continue;
            if (!y_stride || y_stride == n[i]) {
                FRQ_HIP(frq::launch_fill(y[i], 0.0f, m * n[i], s));
            } else {
                for (int64_t r = 0; r < m; ++r) FRQ_HIP(frq::launch_fill(y[i] + r * y_stride, 0.0f, n[i], s));
            }
        }
        return FRQ_OK;
    }
    if (!x || (reinterpret_cast<uintptr_t>(x) & 15)) return fail(FRQ_ERR_ALIGN, "gemm group: x null or misaligned");
    // segments with rows: one launch for all of them (or a single matrix's own GEMM)
    int qt[frq::kGemmGroupMax], c = 0;
    const uint8_t* wp[frq::kGemmGroupMax];
    int64_t nn[frq::kGemmGroupMax], ld[frq::kGemmGroupMax];
    size_t wb[frq::kGemmGroupMax];
    float* yy[frq::kGemmGroupMax];
    for (int i = 0; i < count; ++i) {
        if (!n[i]) continue;
        const uintptr_t wa = reinterpret_cast<uintptr_t>(w[i]);
        if (!w[i] || (qtypes[i] == FRQ_Q4_K ? (wa & 15) : (wa & 1)))
            return fail(FRQ_ERR_ALIGN, "gemm group: weight %d null or misaligned", i);
        if (reinterpret_cast<uintptr_t>(y[i]) & 3) return fail(FRQ_ERR_ALIGN, "y must be 4-byte aligned");
        qt[c] = qtypes[i];
        wp[c] = static_cast<const uint8_t*>(w[i]);
        wb[c] = w_bytes[i];
        nn[c] = n[i];
        ld[c] = y_stride ? y_stride : n[i];
        yy[c] = y[i];
        ++c;
    }
    if (c == 1 && ld[0] == nn[0]) return frq_dev_gemm_bf16(qt[0], wp[0], wb[0], x, yy[0], m, nn[0], k, stream);
    float* part = nullptr;
    uint32_t* cnt = nullptr;
    std::lock_guard<std::mutex> lk(g_sk_mu);
    if (int rc = sk_scratch_locked(s, frq::gemm_bf16_group_scratch(c, nn, m, k), 0, &part, &cnt)) return rc;
    FRQ_HIP(frq::launch_gemm_bf16_group(c, qt, wp, nn, yy, ld, x, m, k, s, part));
    return FRQ_OK;
}

int frq_gemm_bf16(int qtype, const uint16_t* x, const uint8_t* w, size_t w_bytes, int64_t m, int64_t n, int64_t k,
                  float* y) {
    Fmt f;
    if (int rc = gemm_checks(qtype, w_bytes, m, n, k, &f)) return rc;
    if (m == 0 || n == 0) return FRQ_OK;
    if (!y || (k > 0 && (!x || !w))) return fail(FRQ_ERR_INVALID, "null buffer");
    if (k == 0) {
        std::memset(y, 0, (size_t)(m * n) * sizeof(float));
        return FRQ_OK;
    }
    if (int rc = have_device()) return rc;
    std::lock_guard<std::mutex> lk(g_ws.mu);
    const size_t wb = align256(w_bytes), xb = align256((size_t)(m * k) * 2), yb = align256((size_t)(m * n) * 4);
    void* base = nullptr;
    if (int rc = workspace(wb + xb + yb, &base)) return rc;
    uint8_t* dw = static_cast<uint8_t*>(base);
    uint16_t* dx = reinterpret_cast<uint16_t*>(dw + wb);
    float* dy = reinterpret_cast<float*>(dw + wb + xb);
    FRQ_HIP(hipMemcpy(dw, w, w_bytes, hipMemcpyHostToDevice));
    FRQ_HIP(hipMemcpy(dx, x, (size_t)(m * k) * 2, hipMemcpyHostToDevice));
    // the device entry point: same kernel plan (split-K scratch included) as resident weights
    if (int rc = frq_dev_gemm_bf16(qtype, dw, w_bytes, dx, dy, m, n, k, nullptr)) return rc;
    FRQ_HIP(hipMemcpy(y, dy, (size_t)(m * n) * 4, hipMemcpyDeviceToHost));
    return FRQ_OK;
}

int frq_dev_gemm_q4_k_bf16(const void* w, size_t w_bytes, const uint16_t* x, float* y, int64_t m, int64_t n,
                           int64_t k, void* stream) {
    return frq_dev_gemm_bf16(FRQ_Q4_K, w, w_bytes, x, y, m, n, k, stream);
}

int frq_gemm_q4_k_bf16(const uint16_t* x, const uint8_t* w, size_t w_bytes, int64_t m, int64_t n, int64_t k,
                       float* y) {
    return frq_gemm_bf16(FRQ_Q4_K, x, w, w_bytes, m, n, k, y);
}

int frq_dev_copy(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes % 16) return fail(FRQ_ERR_INVALID, "copy size must be a multiple of 16 bytes");
    if (((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15) != 0)
        return fail(FRQ_ERR_ALIGN, "copy buffers must be 16-byte aligned");
    if (bytes == 0) return FRQ_OK;
    if (!dst || !src) return fail(FRQ_ERR_INVALID, "null buffer");
    FRQ_HIP(frq::launch_copy(dst, src, (int64_t)bytes, static_cast<hipStream_t>(stream)));
    return FRQ_OK;
}

int frq_dev_read_xor(const void* src, size_t bytes, uint32_t* out, void* stream) {
    static_assert(FRQ_READ_XOR_WORDS == frq::kReadXorWords, "read_xor word count");
    if (bytes % 16) return fail(FRQ_ERR_INVALID, "read size must be a multiple of 16 bytes");
    if ((reinterpret_cast<uintptr_t>(src) & 15) != 0) return fail(FRQ_ERR_ALIGN, "read buffer must be 16-byte aligned");
    if (!out || (reinterpret_cast<uintptr_t>(out) & 3) != 0) return fail(FRQ_ERR_INVALID, "null or unaligned output words");
    if (bytes != 0 && !src) return fail(FRQ_ERR_INVALID, "null buffer");
    FRQ_HIP(frq::launch_read_xor(src, (int64_t)bytes, out, static_cast<hipStream_t>(stream)));
    return FRQ_OK;
}

int frq_dev_silu_mul(const float* gateup, int64_t ld_in, float* out, int64_t ld_out, int64_t rows, int64_t inter,
                     void* stream) {
    if (rows < 0 || inter < 0) return fail(FRQ_ERR_INVALID, "silu_mul: negative rows or inter");
    if (rows == 0 || inter == 0) return FRQ_OK;
    if (ld_in < 2 * inter || ld_out < inter)
        return fail(FRQ_ERR_INVALID, "silu_mul: ld_in must be >= 2 inter and ld_out >= inter");
    if (!gateup || !out) return fail(FRQ_ERR_INVALID, "silu_mul: null buffer");
    if (((reinterpret_cast<uintptr_t>(gateup) | reinterpret_cast<uintptr_t>(out)) & 3) != 0)
        return fail(FRQ_ERR_ALIGN, "silu_mul: buffers must be 4-byte aligned");
    FRQ_HIP(frq::launch_silu_mul(gateup, ld_in, out, ld_out, rows, inter, static_cast<hipStream_t>(stream)));
    return FRQ_OK;
}

int frq_dev_gemv_swiglu(int qtype_gate, const void* w_gate, size_t gate_bytes, int qtype_up, const void* w_up,
                        size_t up_bytes, int64_t inter, const float* x, int64_t k, float* gateup, float* act,
                        int64_t batch, void* stream) {
    if (inter < 0) return fail(FRQ_ERR_SHAPE, "gemv swiglu: negative inter");
    if (!act) return fail(FRQ_ERR_INVALID, "gemv swiglu: null act");
    if (reinterpret_cast<uintptr_t>(act) & 3) return fail(FRQ_ERR_ALIGN, "gemv swiglu: act must be 4-byte aligned");
    Fmt f;
    if (int rc = dev_gemv_checks(qtype_gate, w_gate, gate_bytes, x, gateup, inter, k, batch, &f)) return rc;
    if (int rc = dev_gemv_checks(qtype_up, w_up, up_bytes, x, gateup, inter, k, batch, &f)) return rc;
    if (inter == 0 || batch == 0) return FRQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint8_t* wg = static_cast<const uint8_t*>(w_gate);
    const uint8_t* wu = static_cast<const uint8_t*>(w_up);
    if (batch == 1 && frq::gemv_swiglu_fusable(qtype_gate, wg, qtype_up, wu, k)) {
        FRQ_HIP(frq::launch_gemv_swiglu(wg, wu, x, gateup, act, inter, k, s));
        return FRQ_OK;
    }
    const int qt[2] = {qtype_gate, qtype_up};
    const void* wp[2] = {w_gate, w_up};
    const size_t wb[2] = {gate_bytes, up_bytes};
    const int64_t nn[2] = {inter, inter};
    float* yy[2] = {gateup, gateup + inter};
    if (int rc = frq_dev_gemv_group(2, qt, wp, wb, nn, x, k, yy, batch, 2 * inter, stream)) return rc;
    FRQ_HIP(frq::launch_silu_mul(gateup, 2 * inter, act, inter, batch, inter, s));
    return FRQ_OK;
}

int frq_gemv_swiglu_fusable(int qtype_gate, const void* w_gate, int qtype_up, const void* w_up, int64_t k) {
    return frq::gemv_swiglu_fusable(qtype_gate, static_cast<const uint8_t*>(w_gate), qtype_up,
                                    static_cast<const uint8_t*>(w_up), k)
               ? 1
               : 0;
}

int frq_set_device(int device) { FRQ_HIP(hipSetDevice(device)); return FRQ_OK; }
int frq_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(FRQ_ERR_INVALID, "null ptr");
    FRQ_HIP(hipMalloc(ptr, bytes ? bytes : 1));
    return FRQ_OK;
}
int frq_free(void* ptr) { FRQ_HIP(hipFree(ptr)); return FRQ_OK; }
int frq_host_alloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(FRQ_ERR_INVALID, "null ptr");
    FRQ_HIP(hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault));
    return FRQ_OK;
}
int frq_host_free(void* ptr) { FRQ_HIP(hipHostFree(ptr)); return FRQ_OK; }
int frq_memcpy_h2d(void* d, const void* s, size_t b) { FRQ_HIP(hipMemcpy(d, s, b, hipMemcpyHostToDevice)); return FRQ_OK; }
int frq_memcpy_d2h(void* d, const void* s, size_t b) { FRQ_HIP(hipMemcpy(d, s, b, hipMemcpyDeviceToHost)); return FRQ_OK; }
int frq_memcpy_h2d_async(void* d, const void* s, size_t b, void* st) {
    FRQ_HIP(hipMemcpyAsync(d, s, b, hipMemcpyHostToDevice, static_cast<hipStream_t>(st)));
    return FRQ_OK;
}
int frq_memcpy_d2h_async(void* d, const void* s, size_t b, void* st) {
    FRQ_HIP(hipMemcpyAsync(d, s, b, hipMemcpyDeviceToHost, static_cast<hipStream_t>(st)));
    return FRQ_OK;
}
int frq_memset_async(void* d, int v, size_t b, void* st) {
    FRQ_HIP(hipMemsetAsync(d, v, b, static_cast<hipStream_t>(st)));
    return FRQ_OK;
}
int frq_stream_create(void** s) {
    if (!s) return fail(FRQ_ERR_INVALID, "null stream");
    hipStream_t st = nullptr;
    FRQ_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = st;
    return FRQ_OK;
}
int frq_stream_destroy(void* s) {
    hipStream_t st = static_cast<hipStream_t>(s);
    if (st) {   // the stream's scratch can go once its work is done (the null stream's stays)
        FRQ_HIP(hipStreamSynchronize(st));
        sk_release_stream(st);
    }
    FRQ_HIP(hipStreamDestroy(st));
    return FRQ_OK;
}
int frq_stream_synchronize(void* s) { FRQ_HIP(hipStreamSynchronize(static_cast<hipStream_t>(s))); return FRQ_OK; }
int frq_stream_wait_event(void* s, void* e) {
    FRQ_HIP(hipStreamWaitEvent(static_cast<hipStream_t>(s), static_cast<hipEvent_t>(e), 0));
    return FRQ_OK;
}
int frq_event_create(void** e) {
    if (!e) return fail(FRQ_ERR_INVALID, "null event");
    hipEvent_t ev = nullptr;
    FRQ_HIP(hipEventCreate(&ev));
    *e = ev;
    return FRQ_OK;
}
int frq_event_destroy(void* e) { FRQ_HIP(hipEventDestroy(static_cast<hipEvent_t>(e))); return FRQ_OK; }
int frq_event_record(void* e, void* s) {
    FRQ_HIP(hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(s)));
    return FRQ_OK;
}
int frq_event_synchronize(void* e) { FRQ_HIP(hipEventSynchronize(static_cast<hipEvent_t>(e))); return FRQ_OK; }
int frq_event_elapsed_ms(float* ms, void* a, void* b) {
    if (!ms) return fail(FRQ_ERR_INVALID, "null ms");
    FRQ_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b)));
    return FRQ_OK;
}
int frq_device_synchronize(void) { FRQ_HIP(hipDeviceSynchronize()); return FRQ_OK; }

int frq_stream_begin_capture(void* s) {
    if (!s) return fail(FRQ_ERR_INVALID, "graph capture needs a created stream, not the null stream");
    FRQ_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(s), hipStreamCaptureModeThreadLocal));
    return FRQ_OK;
}
int frq_stream_end_capture(void* s, void** graph_exec) {
    if (!s || !graph_exec) return fail(FRQ_ERR_INVALID, "null stream or graph handle");
    hipGraph_t g = nullptr;
    FRQ_HIP(hipStreamEndCapture(static_cast<hipStream_t>(s), &g));
    hipGraphExec_t ex = nullptr;
    const hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph_exec = ex;
    return FRQ_OK;
}
int frq_graph_launch(void* ex, void* s) {
    if (!ex) return fail(FRQ_ERR_INVALID, "null graph");
    FRQ_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(ex), static_cast<hipStream_t>(s)));
    return FRQ_OK;
}
int frq_graph_destroy(void* ex) {
    if (ex) FRQ_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(ex)));
    return FRQ_OK;
}

}  // extern "C"

namespace frq {
// frq_dev_gemv with its scratch in `fixed` (frq_noalloc.hip).
int dev_gemv_fixed(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                   int64_t batch, void* stream, const FixedScratch& fixed) {
    return dev_gemv(qtype, w, w_bytes, x, y, n, k, batch, stream, &fixed);
}
int fail_unsupported(const char* msg) { return fail(FRQ_ERR_UNSUPPORTED, "%s", msg); }
int fail_hip(hipError_t e, const char* what) { return hip_fail(e, what); }
}  // namespace frq
