// Split-K, software-pipelined GEMV kernels (gfx950): y[n] = W[n, k] . x[k].
//
// Work decomposition. Every wavefront is an independent work item
// (row block rb of R rows) x (K-slice s of at most 64 work units), so the
// four SIMDs of a CU stay evenly loaded whatever k is, and any k is covered.
//   * A lane owns one work unit of its slice and keeps that unit's slice of x
//     in VGPRs for all R rows of the item (x is read once per item, from L2).
//   * Rows go in batches of U; the loads of batch b+1 are issued before batch
//     b is computed (two register sets, unrolled), so HBM reads overlap the
//     dequant arithmetic inside every wave.
//   * Each row's lane partials are summed with DPP. With one slice the sum
//     is y[row]; with S > 1 slices it goes to a partial buffer, and a second
//     kernel sums the S partials of every row in slice order -- a
//     deterministic result, with the kernel boundary making the partials of
//     waves on other XCDs visible (no cache flushes inside the kernel).
//
// Q4_K work unit (CPL=2): one 32-byte qs group g of a block: 64 elements,
// sub-blocks 2g (low nibbles) and 2g+1 (high nibbles); CPL=1: half a group
// (16 qs bytes, 32 elements). Element order as in gguf.py:209-219.
#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {

namespace {

// y[r] = part[0][r] + part[1][r] + ... + part[S-1][r], in slice order (the
// same bits however the slices were scheduled). Runs after the split-K
// kernel, whose boundary makes every slice's partials visible.
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                            int64_t n, int S) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= n) return;
    y[r] = sum_planes<float>([&](int s) { return part[(int64_t)s * n + r]; }, S);
}

}  // namespace

template <int CPL, int U>
__global__ void __launch_bounds__(256) gemv_q4_k_sk_kernel(const uint8_t* __restrict__ w,
                                                           const float* __restrict__ x, float* __restrict__ y,
                                                           float* __restrict__ part,
                                                           int64_t n, int nb, int S, int ubase, int urem, int R,
                                                           int64_t items) {
    constexpr int UPB = 8 / CPL;   // work units per block
    constexpr int NE = 16 * CPL;   // low (and high) nibbles per lane
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (item >= items) return;
    const int64_t rblk = item / S;
    const int s = (int)(item - rblk * S);
    const int u0 = s * ubase + (s < urem ? s : urem);
    const int ulen = ubase + (s < urem ? 1 : 0);
    const bool active = lane < ulen;
    const int unit = u0 + (active ? lane : 0);
    const int blk = unit / UPB, sub = unit % UPB;
    const int g = (CPL == 2) ? sub : (sub >> 1);
    const int hh = (CPL == 2) ? 0 : (sub & 1);
    const ScaleDecode dec(g);

    const int64_t r0 = rblk * R;
    const int64_t r1 = r0 + R < n ? r0 + R : n;
    const int64_t row_bytes = (int64_t)nb * kQ4KBytes;
    const uint8_t* wb = w + (int64_t)blk * kQ4KBytes;
    const int qoff = 16 + 32 * g + 16 * hh;

    auto load = [&](Q4KRow<CPL>(&t)[U], int64_t rfirst) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (active && rfirst + u < r1) {
                const uint8_t* p = wb + (rfirst + u) * row_bytes;
                t[u].hd = *reinterpret_cast<const uint4*>(p);
#pragma unroll
                for (int c = 0; c < CPL; ++c) t[u].q[c] = *reinterpret_cast<const uint4*>(p + qoff + 16 * c);
            } else {
                t[u].hd = make_uint4(0, 0, 0, 0);
#pragma unroll
                for (int c = 0; c < CPL; ++c) t[u].q[c] = make_uint4(0, 0, 0, 0);
            }
        }
    };

    // first batch in flight before x is fetched
    Q4KRow<CPL> A[U], B[U];
    load(A, r0);

    float xl[NE], xh[NE];
    {
        const float* xb = x + (int64_t)blk * kQKElems + 64 * g + 16 * hh;
#pragma unroll
        for (int i = 0; i < NE; i += 4) {
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f), c = a;
            if (active) {
                a = *reinterpret_cast<const float4*>(xb + i);
                c = *reinterpret_cast<const float4*>(xb + 32 + i);
            }
            xl[i] = a.x; xl[i + 1] = a.y; xl[i + 2] = a.z; xl[i + 3] = a.w;
            xh[i] = c.x; xh[i + 1] = c.y; xh[i + 2] = c.z; xh[i + 3] = c.w;
        }
    }

    auto compute = [&](const Q4KRow<CPL>(&t)[U], int64_t rfirst) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint32_t sc0, m0, sc1, m1;
            dec(t[u].hd.y, t[u].hd.z, t[u].hd.w, sc0, m0, sc1, m1);
            const float d = f16_bits_to_f32(t[u].hd.x), dm = f16_bits_to_f32(t[u].hd.x >> 16);
            // per weight: w = fma(s, f, -t) (f = q, or 16 q with s pre-divided by 16)
            const float s0 = d * (float)sc0, t0 = dm * (float)m0;
            const float s1 = (d * 0.0625f) * (float)sc1, t1 = dm * (float)m1;
            float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const uint32_t qw[4] = {t[u].q[c].x, t[u].q[c].y, t[u].q[c].z, t[u].q[c].w};
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    const uint32_t lo = vand(qw[wd], 0x0F0F0F0Fu);
                    const uint32_t hi = vand(qw[wd], 0xF0F0F0F0u);   // 16 * high nibble
                    const int e = 16 * c + 4 * wd;
                    a0 = __builtin_fmaf(__builtin_fmaf(s0, byte_f(lo, 0), -t0), xl[e + 0], a0);
                    a1 = __builtin_fmaf(__builtin_fmaf(s0, byte_f(lo, 1), -t0), xl[e + 1], a1);
                    a0 = __builtin_fmaf(__builtin_fmaf(s0, byte_f(lo, 2), -t0), xl[e + 2], a0);
                    a1 = __builtin_fmaf(__builtin_fmaf(s0, byte_f(lo, 3), -t0), xl[e + 3], a1);
                    b0 = __builtin_fmaf(__builtin_fmaf(s1, byte_f(hi, 0), -t1), xh[e + 0], b0);
                    b1 = __builtin_fmaf(__builtin_fmaf(s1, byte_f(hi, 1), -t1), xh[e + 1], b1);
                    b0 = __builtin_fmaf(__builtin_fmaf(s1, byte_f(hi, 2), -t1), xh[e + 2], b0);
                    b1 = __builtin_fmaf(__builtin_fmaf(s1, byte_f(hi, 3), -t1), xh[e + 3], b1);
                }
            }
            const float pu = (a0 + a1) + (b0 + b1);
            const float v = wave_sum(pu);
            if (lane == 0 && rfirst + u < r1) {
                if (S == 1) y[rfirst + u] = v;
                else part[(int64_t)s * n + rfirst + u] = v;
            }
        }
    };

    for (int64_t r = r0; r < r1; r += 2 * U) {
        load(B, r + U);
        compute(A, r);
        load(A, r + 2 * U);
        compute(B, r + U);
    }
}

// ------------------------------------------------------------------ planner

namespace {

int sk_units_per_block(int qtype, int cpl) {
    switch (qtype) {
        case kTypeQ4K: return 8 / cpl;
        default: return 0;
    }
}

bool sk_cpl_valid(int qtype, int cpl) {
    switch (qtype) {
        case kTypeQ4K: return cpl == 1 || cpl == 2;
        default: return false;
    }
}

int sk_block_elems(int qtype) { return qtype == kTypeQ80 ? kQ80Elems : qtype == kTypeQ10 ? kQ10Elems : kQKElems; }

}  // namespace

bool gemv_sk_supported(int qtype) { return qtype == kTypeQ4K; }

bool plan_gemv_sk(int qtype, int64_t n, int64_t k, SplitKPlan* p) {
    if (!gemv_sk_supported(qtype) || n <= 0 || k <= 0 || k % sk_block_elems(qtype)) return false;
    const int64_t nb = k / sk_block_elems(qtype);
    if (p->cpl <= 0) {
        // fewest idle lanes over all slices; prefer the larger unit on ties
        double best = 2.0;
        for (int cpl = 2; cpl >= 1; --cpl) {
            const int64_t units = nb * sk_units_per_block(qtype, cpl);
            const int64_t S = (units + 63) / 64;
            const double idle = 1.0 - (double)units / (double)(S * 64);
            if (idle < best - 1e-9) {
                best = idle;
                p->cpl = cpl;
            }
        }
    }
    if (!sk_cpl_valid(qtype, p->cpl)) return false;
    const int64_t units = nb * sk_units_per_block(qtype, p->cpl);
    p->slices = (int)((units + 63) / 64);
    p->unit_base = (int)(units / p->slices);
    p->unit_rem = (int)(units % p->slices);
    if (p->unroll != 2 && p->unroll != 4) p->unroll = 4;
    if (p->rows <= 0) {
        // ~10 waves per CU over 256 CUs, at least 4 rows per item to amortise the x load
        const int64_t target = 2560;
        int64_t r = (n * p->slices + target - 1) / target;
        p->rows = (int)(r < 4 ? 4 : r > 64 ? 64 : r);
    }
    if (p->rows > 64) return false;
    p->row_blocks = (n + p->rows - 1) / p->rows;
    p->items = p->row_blocks * p->slices;
    return true;
}

void gemv_sk_scratch(const SplitKPlan& p, int64_t n, size_t* partial_bytes, size_t* counter_bytes) {
    *partial_bytes = p.slices > 1 ? (size_t)n * p.slices * 4 : 0;
    *counter_bytes = 0;
}

hipError_t launch_gemv_sk(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k,
                          const SplitKPlan& p, float* part, uint32_t* cnt, hipStream_t stream) {
    if (p.items <= 0) return hipSuccess;
    if (p.slices > 1 && !part) return hipErrorInvalidValue;
    (void)cnt;
    const int nb = (int)(k / sk_block_elems(qtype));
    const int wpg = p.items >= 4 ? 4 : (int)p.items;      // independent waves per workgroup
    const dim3 bd(64 * wpg), gd((unsigned)((p.items + wpg - 1) / wpg));
#define FRQ_SK_ARGS w, x, y, part, n, nb, p.slices, p.unit_base, p.unit_rem, p.rows, p.items
    switch (qtype) {
        case kTypeQ4K:
            if (p.cpl == 2) {
                if (p.unroll == 2) gemv_q4_k_sk_kernel<2, 2><<<gd, bd, 0, stream>>>(FRQ_SK_ARGS);
                else gemv_q4_k_sk_kernel<2, 4><<<gd, bd, 0, stream>>>(FRQ_SK_ARGS);
            } else {
                if (p.unroll == 2) gemv_q4_k_sk_kernel<1, 2><<<gd, bd, 0, stream>>>(FRQ_SK_ARGS);
                else gemv_q4_k_sk_kernel<1, 4><<<gd, bd, 0, stream>>>(FRQ_SK_ARGS);
            }
            break;
        default: return hipErrorInvalidValue;
    }
#undef FRQ_SK_ARGS
    if (p.slices > 1)
        splitk_reduce_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(part, y, n, p.slices);
    return hipGetLastError();
}

}  // namespace frq
