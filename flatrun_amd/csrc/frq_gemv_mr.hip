// Q4_K matvec of a few rows of x at once: Y[r, i] = sum_j W[i, j] X[r, j]
// for r < M (M <= 3), the reference's batched entry (matmul_q4_k_batched,
// _C.cpp:154-197) at small seq, reading W once for the M rows.
//
// Arithmetic, per weight, as the single-row element-wise GEMV: with
// s = d*sc and t = dmin*m of the weight's sub-block (both exact fp32
// products: an fp16 times a 6-bit integer), w = fma(s, q, -t) is the
// dequant's fp32 value (s*q is exact, so the one rounding is the
// reference's), and each row adds fma(w, x[r, j], acc_r) in fp32. Every
// product is formed per weight, so cancelling weights (s*q = t under a large
// x) keep the bound c * 2^-24 * sum_j |w_j x_j| per output.
//
// Mapping. A workgroup owns R output rows and all of k; lane (block b,
// part p = tid % 8) holds qs bytes 16p .. 16p+15 of block b, i.e. group
// g = p / 2 (bytes 32g .. 32g+31: sub-block 2g in the low, 2g + 1 in the
// high nibbles) and its half hf = p % 2, so low nibbles are elements
// 64g + 16hf + t and high nibbles 64g + 32 + 16hf + t (t < 16). Its x for
// those 32 elements and M rows stays in registers; the weights of U rows
// are in flight while the previous U are summed. Per (row, x row) the lane
// sums go through a 16-lane DPP tree and LDS, and one thread per output adds
// the 4 * waves partial sums in a fixed order, so the result of a row of x
// depends neither on the other rows in the launch nor on M.
#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {
namespace {

// U rows of W per load batch, two batches in flight.
template <int M, int U>
__global__ void __launch_bounds__(768) gemv_q4_k_mr_kernel(const uint8_t* __restrict__ w,
                                                           const float* __restrict__ x, float* __restrict__ y,
                                                           int64_t n, int nb, int R, int64_t ldy) {
    extern __shared__ float red[];                      // [R][M][4 * waves]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk_raw = tid >> 3, p = tid & 7;
    const bool active = blk_raw < nb;
    const int blk = active ? blk_raw : 0;              // inactive lanes re-read block 0; their sums are dropped
    const int g = p >> 1, hf = p & 1;
    const int64_t k = (int64_t)nb * kQKElems;

    // Plane ownership: lane hf owns scale pair 2g + hf, whose weights are
    // its plane A (low nibbles for hf = 0, high for hf = 1, as 16 q with the
    // scale pre-divided by 16); plane B is the other nibble plane, whose pair
    // the DPP neighbour (lane ^ 1) owns. Each lane decodes one pair and reads
    // the neighbour's (s, t) with one DPP move each.
    const bool own_hi = hf != 0;
    const float hfac = own_hi ? 0.0625f : 1.0f;
    const uint32_t mask_a = own_hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu, mask_b = ~mask_a;
    float xl[M][16], xh[M][16];                         // x of plane A, plane B
#pragma unroll
    for (int r = 0; r < M; ++r) {
        const float* xb = x + r * k + (int64_t)blk * kQKElems + 64 * g + 16 * hf;
        const float* xa = xb + (own_hi ? 32 : 0);
        const float* xo = xb + (own_hi ? 0 : 32);
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(xa + i);
            const float4 c = *reinterpret_cast<const float4*>(xo + i);
            xl[r][i] = a.x; xl[r][i + 1] = a.y; xl[r][i + 2] = a.z; xl[r][i + 3] = a.w;
            xh[r][i] = c.x; xh[r][i + 1] = c.y; xh[r][i + 2] = c.z; xh[r][i + 3] = c.w;
        }
    }

    const int64_t row0 = (int64_t)blockIdx.x * R;
    const int nrows = (int)(n - row0 < R ? n - row0 : R);
    const uint32_t row_bytes = (uint32_t)nb * kQ4KBytes;
    const auto rs = buffer_rsrc(w + row0 * (int64_t)row_bytes, (uint32_t)nrows * row_bytes);
    const uint32_t off_h = (uint32_t)blk * kQ4KBytes, off_q = off_h + 16 + 32 * g + 16 * hf;
    const int red_stride = 4 * nwaves;
    const PairDecode pdec(p);

    uint4 hd[2][U], qv[2][U];
    auto load = [&](int set, int rr) {
#pragma unroll
        for (int uu = 0; uu < U; ++uu) {
            const int row = rr + uu < nrows ? rr + uu : nrows - 1;
            hd[set][uu] = bload_b128(rs, (uint32_t)row * row_bytes + off_h);
            qv[set][uu] = bload_b128(rs, (uint32_t)row * row_bytes + off_q);
        }
    };
    auto compute = [&](int set, int rr) {
#pragma unroll
        for (int uu = 0; uu < U; ++uu) {
            const uint4 h = hd[set][uu];
            uint32_t sc0, m0;
            pdec(h.y, h.z, h.w, sc0, m0);
            const float d = f16_bits_to_f32(h.x), dm = f16_bits_to_f32(h.x >> 16);
            const float sa = (d * hfac) * (float)sc0, ta = dm * (float)m0;    // exact
            const float sb = dpp_mov<0xB1>(sa), tb = dpp_mov<0xB1>(ta);     // quad_perm [1,0,3,2]
            float a[M], b[M];
#pragma unroll
            for (int r = 0; r < M; ++r) a[r] = b[r] = 0.0f;
            const uint32_t qw[4] = {qv[set][uu].x, qv[set][uu].y, qv[set][uu].z, qv[set][uu].w};
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                float f[8];
                nibbles8(qw[wd], f, mask_a, mask_b);    // f[0..3] plane A, f[4..7] plane B
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float wl = __builtin_fmaf(sa, f[c], -ta);
                    const float wh = __builtin_fmaf(sb, f[4 + c], -tb);
#pragma unroll
                    for (int r = 0; r < M; ++r) {
                        a[r] = __builtin_fmaf(wl, xl[r][4 * wd + c], a[r]);
                        b[r] = __builtin_fmaf(wh, xh[r][4 * wd + c], b[r]);
                    }
                }
            }
            if (rr + uu < nrows) {
#pragma unroll
                for (int r = 0; r < M; ++r) {
                    const float v = row16_sum(active ? a[r] + b[r] : 0.0f);
                    if ((lane & 15) == 15) red[((rr + uu) * M + r) * red_stride + 4 * wave + (lane >> 4)] = v;
                }
            }
        }
    };

    // No branch around the second half: loads past the last row re-read it
    // and compute() stores nothing for such rows, which keeps the load
    // counters the same on every path through the loop.
    // The scheduling barriers keep each batch's loads issued before the
    // wait for the previous batch.
    load(0, 0);
    for (int rr = 0; rr < nrows; rr += 2 * U) {
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

}  // namespace

bool gemv_q4k_mr_ok(const uint8_t* w, const float* x, int64_t k) {
    if (k <= 0 || k % kQKElems) return false;
    const int64_t nb = k / kQKElems;
    if (nb * 8 > 768) return false;                     // one lane per 16 qs bytes, at most 12 waves
    return ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15) == 0;
}

hipError_t launch_gemv_q4k_mr(const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int m, int64_t ldy,
                              hipStream_t stream) {
    if (n <= 0 || m <= 0) return hipSuccess;
    if (m > kGemvMrMax || ldy < n || !gemv_q4k_mr_ok(w, x, k)) return hipErrorInvalidValue;
    const int nb = (int)(k / kQKElems);
    const int waves = (nb * 8 + 63) / 64;
    // one round of 256 workgroups while rows allow, at most 16 rows each
    int64_t R = (n + 255) / 256;
    if (R < 1) R = 1;
    if (R > 16) R = 16;
    const int64_t grid = (n + R - 1) / R;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    const size_t lds = sizeof(float) * (size_t)R * m * 4 * waves;
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * waves));
    switch (m) {
        case 1: gemv_q4_k_mr_kernel<1, 2><<<gd, bd, lds, stream>>>(w, x, y, n, nb, (int)R, ldy); break;
        case 2: gemv_q4_k_mr_kernel<2, 2><<<gd, bd, lds, stream>>>(w, x, y, n, nb, (int)R, ldy); break;
        case 3: gemv_q4_k_mr_kernel<3, 1><<<gd, bd, lds, stream>>>(w, x, y, n, nb, (int)R, ldy); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace frq
