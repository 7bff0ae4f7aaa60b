// Matvec of a few rows of x at once: Y[r, i] = sum_j W[i, j] X[r, j] for
// r < M (M = 2, 3), the reference's batched entry points (matmul_<q>_batched,
// _C.cpp:154-283) at small seq, reading W once for the M rows. Q4_K, Q6_K
// and Q8_0.
//
// Mapping (every format). A workgroup owns R output rows and all of k; lane
// (block b, part p) holds one fixed slice of block b (Q4_K and Q6_K: 32
// elements, 8 lanes per block; Q8_0: 16 elements, 2 lanes per block) and its
// x for those elements and M rows in registers. The weights of U rows are in
// flight while the previous U are summed. Per (row, x row) the lane sums go
// through a 16-lane DPP tree and LDS, and one thread per output adds the
// 4 * waves partial sums in a fixed order, so the result of a row of x
// depends neither on the other rows in the launch nor on M.
//
// Arithmetic per format:
//   Q4_K: per weight, as the single-row element-wise GEMV: with s = d*sc and
//     t = dmin*m of the weight's sub-block (both exact fp32 products: an fp16
//     times a 6-bit integer), w = fma(s, q, -t) is the dequant's fp32 value
//     (s*q is exact, so the one rounding is the reference's), and each row
//     adds fma(w, x[r, j], acc_r) in fp32. Every product is formed per
//     weight, so cancelling weights (s*q = t under a large x) keep the bound
//     c * 2^-24 * sum_j |w_j x_j| per output.
//   Q6_K, Q8_0: the single-row ring kernels' per-lane sums (Q6RingLane,
//     Q8RingLane in frq_ringrow.h) for each row of x, and the same reduction
//     order, so every row has the bits of a single-row ring-kernel call.
#include <type_traits>
#include "frq_common.h"
#include "frq_kernels.h"
#include "frq_ringrow.h"

namespace frq {
namespace {

// Q4_K lane: part p = 0..7 holds qs bytes 16p .. 16p+15 of its block, i.e.
// group g = p / 2 (bytes 32g .. 32g+31: sub-block 2g in the low, 2g + 1 in
// the high nibbles) and its half hf = p % 2, so low nibbles (plane A) are
// elements 64g + 16hf + t and high nibbles (plane B) 64g + 32 + 16hf + t
// (t < 16). Lane hf decodes the (sc, m) pair of sub-block 2g + hf only and
// reads the other one's (s, t) from its DPP neighbour (lane ^ 1). Codes
// enter as q * u (fp8 conversion, two per instruction; the scale carries
// 1 / u), as in the single-row element-wise kernel.
struct Q4KMrLane {
    static constexpr int kLanes = 8, kBytes = kQ4KBytes, kElems = kQKElems;
    using X = float[2][16];                             // x of plane A, plane B
    struct Row {
        uint4 hd, qv;
    };
    uint32_t off_h, off_q;
    float u_inv;
    int g, hf;
    PairDecode pdec;

    __device__ __forceinline__ Q4KMrLane(int blk, int p) : pdec(p) {
        g = p >> 1;
        hf = p & 1;
        u_inv = 1.0f / fp8_unit();
        off_h = (uint32_t)blk * kQ4KBytes;
        off_q = off_h + 16 + 32 * g + 16 * hf;
    }
    __device__ __forceinline__ void load_x(const float* __restrict__ xrow, int blk, X& xv) const {
        const float* xb = xrow + (int64_t)blk * kQKElems + 64 * g + 16 * hf;
        const float* xa = xb;
        const float* xo = xb + 32;
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(xa + i);
            const float4 c = *reinterpret_cast<const float4*>(xo + i);
            xv[0][i] = a.x; xv[0][i + 1] = a.y; xv[0][i + 2] = a.z; xv[0][i + 3] = a.w;
            xv[1][i] = c.x; xv[1][i + 1] = c.y; xv[1][i + 2] = c.z; xv[1][i + 3] = c.w;
        }
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, Row& t) const {
        t.hd = bload_b128(rs, row_off + off_h);
        t.qv = bload_b128(rs, row_off + off_q);
    }
    template <int M>
    __device__ __forceinline__ void dot(const Row& t, const X (&xv)[M], float (&pu)[M]) const {
        uint32_t sc0, m0;
        pdec(t.hd.y, t.hd.z, t.hd.w, sc0, m0);
        const float d = f16_bits_to_f32(t.hd.x), dm = f16_bits_to_f32(t.hd.x >> 16);
        const float so = (d * u_inv) * (float)sc0, to = dm * (float)m0;  // exact
        const float sn = dpp_mov<0xB1>(so), tn = dpp_mov<0xB1>(to);     // quad_perm [1,0,3,2]
        const float sa = hf ? sn : so, ta = hf ? tn : to;               // plane A: sub-block 2g
        const float sb = hf ? so : sn, tb = hf ? to : tn;               // plane B: 2g + 1
        float a[M], b[M];
#pragma unroll
        for (int r = 0; r < M; ++r) a[r] = b[r] = 0.0f;
        const uint32_t qw[4] = {t.qv.x, t.qv.y, t.qv.z, t.qv.w};
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            float f[8];
            nibbles8_fp8(qw[wd], f);                    // f[0..3] plane A, f[4..7] plane B
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float wl = __builtin_fmaf(sa, f[c], -ta);
                const float wh = __builtin_fmaf(sb, f[4 + c], -tb);
#pragma unroll
                for (int r = 0; r < M; ++r) {
                    a[r] = __builtin_fmaf(wl, xv[r][0][4 * wd + c], a[r]);
                    b[r] = __builtin_fmaf(wh, xv[r][1][4 * wd + c], b[r]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < M; ++r) pu[r] = a[r] + b[r];
    }
};

struct Q6KMrLane : Q6RingLane {
    static constexpr int kLanes = 8, kBytes = kQ6KBytes, kElems = kQKElems;
    using X = float[4][8];
    using Row = Q6RingRow;
    __device__ __forceinline__ Q6KMrLane(int blk, int p) : Q6RingLane(blk, p) {}
};

struct Q80MrLane : Q8RingLane {
    static constexpr int kLanes = 2, kBytes = kQ80Bytes, kElems = kQ80Elems;
    using X = float[16];
    using Row = Q8RingRow;
    __device__ __forceinline__ Q80MrLane(int blk, int p) : Q8RingLane(blk, p) {}
};

// Threads per workgroup at most: x of M rows sits beside two load batches
// in the registers. Q8_0 holds 16 x values per row and lane, the others 32.
template <class F>
constexpr int mr_threads() {
    return F::kLanes == 2 ? 1024 : 768;
}
// Rows per load batch: two, one for Q4_K / Q6_K at M = 3 (registers).
template <class F>
constexpr int mr_batch(int m) {
    return (F::kLanes == 8 && m == 3) ? 1 : 2;
}

// U rows of W per load batch, two batches in flight; at most T threads.
template <class F, int M, int U, int T>
__global__ void __launch_bounds__(T) gemv_mr_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                    float* __restrict__ y, int64_t n, int nb, int R, int64_t ldy) {
    extern __shared__ float red[];                      // [R][M][4 * waves]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk_raw = tid / F::kLanes;
    const bool active = blk_raw < nb;
    const int blk = active ? blk_raw : 0;              // inactive lanes re-read block 0; their sums are dropped
    const F ln(blk, tid % F::kLanes);
    const int64_t k = (int64_t)nb * F::kElems;

    // Row priorities (row_priority, here by quarter of the row range, set
    // with uniform branches since the loop is not unrolled): Q4_K 3584 x
    // 18944 at 2 / 3 rows 16.9 -> 16.0 / 20.4 -> 18.9 us, 14336 x 4096 at 2
    // rows 13.7 -> 12.9; Q6_K and Q8_0 gained nothing and stay without.
    constexpr bool kPrio = std::is_same<F, Q4KMrLane>::value;
    typename F::X xv[M];
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(3);
#pragma unroll
    for (int r = 0; r < M; ++r) ln.load_x(x + r * k, blk, xv[r]);

    const int64_t row0 = (int64_t)blockIdx.x * R;
    const int nrows = (int)(n - row0 < R ? n - row0 : R);
    const uint32_t row_bytes = (uint32_t)nb * F::kBytes;
    const auto rs = buffer_rsrc(w + row0 * (int64_t)row_bytes, (uint32_t)nrows * row_bytes);
    const int red_stride = 4 * nwaves;

    typename F::Row rows[2][U];
    auto load = [&](int set, int rr) {
#pragma unroll
        for (int uu = 0; uu < U; ++uu) {
            const int row = rr + uu < nrows ? rr + uu : nrows - 1;
            ln.load(rs, (uint32_t)row * row_bytes, rows[set][uu]);
        }
    };
    auto compute = [&](int set, int rr) {
#pragma unroll
        for (int uu = 0; uu < U; ++uu) {
            float pu[M];
            ln.template dot<M>(rows[set][uu], xv, pu);
            if (rr + uu < nrows) {
#pragma unroll
                for (int r = 0; r < M; ++r) {
                    const float v = row16_sum(active ? pu[r] : 0.0f);
                    if ((lane & 15) == 15) red[((rr + uu) * M + r) * red_stride + 4 * wave + (lane >> 4)] = v;
                }
            }
        }
    };

    // No branch around the second half: loads past the last row re-read it
    // and compute() stores nothing for such rows, which keeps the load
    // counters the same on every path through the loop. The scheduling
    // barriers keep each batch's loads issued before the wait for the
    // previous batch.
    load(0, 0);
    for (int rr = 0; rr < nrows; rr += 2 * U) {
        if constexpr (kPrio) {
            const int q = (4 * rr) / nrows;
            if (q <= 0) __builtin_amdgcn_s_setprio(3);
            else if (q == 1) __builtin_amdgcn_s_setprio(2);
            else if (q == 2) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
        load(1, rr + U);
        __builtin_amdgcn_sched_barrier(0);
        compute(0, rr);
        load(0, rr + 2 * U);
        __builtin_amdgcn_sched_barrier(0);
        compute(1, rr + U);
    }
    __syncthreads();
    for (int idx = tid; idx < nrows * M; idx += blockDim.x) {
        const int row = idx / M, r = idx - row * M;
        const float* rp = red + (row * M + r) * red_stride;
        float s = 0.0f;
        for (int w2 = 0; w2 < red_stride; ++w2) s += rp[w2];
        y[r * ldy + row0 + row] = s;
    }
}

template <class F>
hipError_t mr_go(const uint8_t* w, const float* x, float* y, int64_t n, int nb, int m, int64_t ldy, hipStream_t s) {
    constexpr int T = mr_threads<F>();
    const int waves = (nb * F::kLanes + 63) / 64;
    // Rows per workgroup: as many workgroups as the registers let 256 CUs
    // hold at once (Q4_K / Q6_K: 12 waves per CU at M = 2, 3; Q8_0: 24),
    // but at least 4 rows (or one round of 256 workgroups, if fewer), since
    // every workgroup reads all of x for its rows; at most 16.
    const int per_cu = ((F::kLanes == 2 ? 24 : 12) / waves) > 1 ? (F::kLanes == 2 ? 24 : 12) / waves : 1;
    const int64_t r_round = (n + 255) / 256;
    int64_t R = (n + 256 * per_cu - 1) / (256 * per_cu);
    if (R < (r_round < 4 ? r_round : 4)) R = r_round < 4 ? r_round : 4;
    if (R < 1) R = 1;
    if (R > 16) R = 16;
    const int64_t grid = (n + R - 1) / R;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    const size_t lds = sizeof(float) * (size_t)R * m * 4 * waves;
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * waves));
    switch (m) {
        case 2: gemv_mr_kernel<F, 2, mr_batch<F>(2), T><<<gd, bd, lds, s>>>(w, x, y, n, nb, (int)R, ldy); break;
        case 3: gemv_mr_kernel<F, 3, mr_batch<F>(3), T><<<gd, bd, lds, s>>>(w, x, y, n, nb, (int)R, ldy); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool gemv_mr_ok(int qtype, const uint8_t* w, const float* x, int64_t k) {
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w), xa = reinterpret_cast<uintptr_t>(x);
    if (k <= 0 || (xa & 15)) return false;
    switch (qtype) {
        case kTypeQ4K:   // 16-byte loads of the blocks
            return k % kQKElems == 0 && (k / kQKElems) * 8 <= mr_threads<Q4KMrLane>() && (wa & 15) == 0;
        case kTypeQ6K:   // aligned windows: 4-byte rows (even block count), each block's neighbour present
            return k % kQKElems == 0 && (k / kQKElems) % 2 == 0 &&
                   (k / kQKElems) * 8 <= mr_threads<Q6KMrLane>() && (wa & 3) == 0;
        case kTypeQ80:
            return k % kQ80Elems == 0 && (k / kQ80Elems) % 2 == 0 &&
                   (k / kQ80Elems) * 2 <= mr_threads<Q80MrLane>() && (wa & 3) == 0;
        default:
            return false;
    }
}

hipError_t launch_gemv_mr(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int m,
                          int64_t ldy, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (m < 2 || m > kGemvMrMax || ldy < n || !gemv_mr_ok(qtype, w, x, k)) return hipErrorInvalidValue;
    switch (qtype) {
        case kTypeQ4K: return mr_go<Q4KMrLane>(w, x, y, n, (int)(k / kQKElems), m, ldy, stream);
        case kTypeQ6K: return mr_go<Q6KMrLane>(w, x, y, n, (int)(k / kQKElems), m, ldy, stream);
        case kTypeQ80: return mr_go<Q80MrLane>(w, x, y, n, (int)(k / kQ80Elems), m, ldy, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace frq
