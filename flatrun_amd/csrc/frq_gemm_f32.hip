// Batched matvec with the fp32 contract on the gfx950 matrix cores:
//   Y[M, N] (fp32) = X[M, K] (fp32) . W[N, K]^T, W = raw Q4_K, Q6_K or Q8_0 blocks.
//
// The reference's batched entry points (matmul_<q>_batched, _C.cpp:154-283)
// run one fp32 matvec per row of X and dequantize W again for every row. Here
// W is read once per tile of X rows, and the products run on
// v_mfma_f32_32x32x16_bf16 without giving up the fp32 contract:
//   * W enters as integer codes, which bf16 holds exactly: Q4_K q - c in
//     -15..15 (c the sub-block's code nearest t / s, below), Q6_K q - 32 in
//     -32..31, Q8_0 q in -128..127;
//   * X enters as three bf16 pieces, x = x1 + x2 + x3 with x1 = bf16(x),
//     x2 = bf16(x - x1), x3 = bf16(x - x1 - x2) (round to nearest; every
//     subtraction is exact), which carry all 24 bits of an fp32 x whose
//     pieces stay normal (|x| >= 2^-110);
//   * every product code * piece is exact in fp32, and the matrix cores sum
//     them in fp32 over one sub-block (Q4_K 32 elements, Q6_K 16, Q8_0 32);
//   * the sub-block's scale is applied in fp32 per (row, sub-block):
//     y += s * S - (t - s c) * sum(x) (Q4_K, s = d*sc, t = dmin*m),
//     y += d*sc * S (Q6_K), y += d * S (Q8_0), with sum(x) of the sub-block
//     in fp32.
// The codes make every term of S and sum(x) within 3 |w_j x_j| (Q4_K, see
// CFmt<Q4_K>::codes) or equal to it, so every row's error is bounded like
// the matvec kernels':  |y - y_exact| <= c * 2^-24 * sum_j |w_j x_j|,
// c a small multiple of the summation depth (tested at 1e-5 against fp64).
// That holds for x in {0} U [2^-100, 2^100], where all three pieces are
// normal bf16 and no product or sum overflows. Every value of x is checked:
// the workgroups of one tile of x rows stage the same values, so the one
// whose column tile is the step index modulo the column-tile count checks
// that step. A row of x with any value outside (tiny, subnormal, huge, inf,
// NaN) is flagged in a word per row, tagged with a per-launch number (no
// clearing between launches), and a second kernel computes its outputs
// again weight by weight in fp64 (w the exact dequantized fp32 value,
// products exact, one rounding to fp32 at the end; inf and NaN propagate as
// IEEE arithmetic has them): the split-adding kernel when K is split, else
// a per-row kernel that returns at once for rows without the flag.
//
// Tiling: a workgroup of 4 waves owns a BM x BN tile of Y (WM x WN waves of
// 32 x 64, two 32 x 32 MFMA tiles each) and walks K in steps of 32. Each
// step stages X's three bf16 pieces and sum(x) (BM rows) and W's codes and
// per-row scales (BN rows) into LDS, double-buffered, the next step's global
// loads in flight during this step's MFMAs. Few output tiles (few X rows)
// split K over S workgroups whose fp32 partial planes a second kernel adds
// in split order (deterministic).
// MFMA operand layouts (32x32x16, 8 bf16 per lane): A lane l holds row l%32,
// k = 8*(l/32) .. +7 of the 16-k slice; B lane l holds column l%32, same k;
// D register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "frq_common.h"
#include "frq_kernels.h"

#include <atomic>

namespace frq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kCK = 32;              // K per step
constexpr int kCRow = kCK + 8;       // bf16 per LDS row (rows padded to 80 bytes)

__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));   // round to nearest even
}
__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// Codes of one step for one W row: `cnt` (8, 16 or 32) consecutive elements of
// the step starting at element `k0` of the step, as bf16, plus the row's
// scales for the step (written by the thread with k0 == 0).
template <int QT>
struct CFmt;

// Q4_K: step j of a block is sub-block j (32 elements): qs bytes
// 32 (j >> 1) + i, low nibbles for even j, high for odd (gguf.py:209-219).
template <>
struct CFmt<kTypeQ4K> {
    static constexpr int kBytes = kQ4KBytes, kElems = kQKElems;
    template <int CNT>
    struct Raw {
        u32x4 h;
        uint32_t q[CNT / 4];
    };
    template <int CNT>
    __device__ static void load(Raw<CNT>& r, const uint8_t* wrow, int step, int k0) {
        const uint8_t* bp = wrow + (int64_t)(step >> 3) * kQ4KBytes;
        const int j = step & 7;
        r.h = *reinterpret_cast<const u32x4*>(bp);
        const uint8_t* qp = bp + 16 + 32 * (j >> 1) + k0;
        if constexpr (CNT == 8) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(qp);
            r.q[0] = v[0];
            r.q[1] = v[1];
        } else {
#pragma unroll
            for (int c = 0; c < CNT / 16; ++c) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(qp + 16 * c);
#pragma unroll
                for (int i = 0; i < 4; ++i) r.q[4 * c + i] = v[i];
            }
        }
    }
    // Centred codes: w = s q - t = s (q - c) - (t - s c) with c = round(t / s)
    // clamped to 0 .. 15, so the code q - c (-15 .. 15, exact in bf16) is 0 on
    // the weight nearest zero and |s (q - c)| + |t - s c| <= 3 |w| for every
    // q (|t - s c| <= |s| / 2 unless clamped, and then both terms have the
    // sign of w). The sub-block sum s * S - t' * sum(x) then keeps the bound
    // sum |w x| even for an outlier x on a weight where s q = t.
    template <int CNT>
    __device__ static void codes(const Raw<CNT>& r, int step, uint32_t* out, float* scl, bool first) {
        const int j = step & 7;
        const uint32_t sh = (j & 1) ? 4u : 0u;
        uint32_t sc, mn;
        k4_scale_min(r.h[1], r.h[2], r.h[3], j, sc, mn);
        const float s = f16_bits_to_f32(r.h[0]) * (float)sc;          // exact
        const float t = f16_bits_to_f32(r.h[0] >> 16) * (float)mn;    // exact
        // s = 0 or non-finite: fmaxf drops a NaN, so c lands in 0 .. 15 anyway
        const float cf = fminf(fmaxf(__builtin_rintf(t * __builtin_amdgcn_rcpf(s)), 0.0f), 15.0f);
        const int ci = (int)cf;
#pragma unroll
        for (int i = 0; i < CNT / 4; ++i) {
            const uint32_t v = (r.q[i] >> sh) & 0x0F0F0F0Fu;
            out[2 * i] = bf16_pair((float)((int)(v & 15u) - ci), (float)((int)((v >> 8) & 15u) - ci));
            out[2 * i + 1] = bf16_pair((float)((int)((v >> 16) & 15u) - ci), (float)((int)(v >> 24) - ci));
        }
        if (first) {
            scl[0] = s;
            scl[1] = __builtin_fmaf(-s, cf, t);                       // t - s c, one rounding
        }
    }
};

// Q8_0: a step is one block [d f16][q int8 x 32] (34 bytes, 2-byte aligned).
template <>
struct CFmt<kTypeQ80> {
    static constexpr int kBytes = kQ80Bytes, kElems = kQ80Elems;
    template <int CNT>
    struct Raw {
        uint32_t d;
        uint32_t q[CNT / 4];
    };
    template <int CNT>
    __device__ static void load(Raw<CNT>& r, const uint8_t* wrow, int step, int k0) {
        const uint8_t* bp = wrow + (int64_t)step * kQ80Bytes;
        r.d = ld_u16(bp);
#pragma unroll
        for (int i = 0; i < CNT / 4; ++i) r.q[i] = ld_u32_a2(bp + 2 + k0 + 4 * i);
    }
    template <int CNT>
    __device__ static void codes(const Raw<CNT>& r, int step, uint32_t* out, float* scl, bool first) {
        (void)step;
#pragma unroll
        for (int i = 0; i < CNT / 4; ++i) {
            const uint32_t v = r.q[i];
            out[2 * i] = bf16_pair((float)(int)(int8_t)(v & 0xFFu), (float)(int)(int8_t)((v >> 8) & 0xFFu));
            out[2 * i + 1] = bf16_pair((float)(int)(int8_t)((v >> 16) & 0xFFu), (float)(int)(int8_t)(v >> 24));
        }
        if (first) {
            scl[0] = f16_bits_to_f32(r.d);
            scl[1] = 0.0f;
        }
    }
};

// Q6_K: step j of a block covers elements 32j .. 32j+31 = 128h + 32ks + l
// (h = j >> 2, ks = j & 3, l < 32): q = nibble of ql[64h + 32 (ks & 1) + l]
// (high nibble for ks >= 2) | bits 2ks, 2ks+1 of qh[32h + l] << 4, code
// q - 32, scale sc[8h + l / 16 + 2ks] (gguf.py:401-419): two 16-element
// sub-blocks per step. Fields are 2-byte aligned (210-byte blocks).
template <>
struct CFmt<kTypeQ6K> {
    static constexpr int kBytes = kQ6KBytes, kElems = kQKElems;
    template <int CNT>
    struct Raw {
        uint32_t ql[CNT / 4], qh[CNT / 4];
        uint32_t sc, d;
    };
    template <int CNT>
    __device__ static void load(Raw<CNT>& r, const uint8_t* wrow, int step, int k0) {
        const uint8_t* bp = wrow + (int64_t)(step >> 3) * kQ6KBytes;
        const int j = step & 7, h = j >> 2, ks = j & 3;
#pragma unroll
        for (int i = 0; i < CNT / 4; ++i) {
            r.ql[i] = ld_u32_a2(bp + 64 * h + 32 * (ks & 1) + k0 + 4 * i);
            r.qh[i] = ld_u32_a2(bp + 128 + 32 * h + k0 + 4 * i);
        }
        r.sc = ld_u16(bp + 192 + 8 * h + 2 * ks);   // sc[8h + 2ks], sc[8h + 2ks + 1]
        r.d = ld_u16(bp + 208);
    }
    template <int CNT>
    __device__ static void codes(const Raw<CNT>& r, int step, uint32_t* out, float* scl, bool first) {
        const int ks = step & 3;
        const uint32_t nsh = ks >= 2 ? 4u : 0u, hsh = 2u * (uint32_t)ks;
#pragma unroll
        for (int i = 0; i < CNT / 4; ++i) {
            const uint32_t q = ((r.ql[i] >> nsh) & 0x0F0F0F0Fu) | (((r.qh[i] >> hsh) & 0x03030303u) << 4);
            out[2 * i] = bf16_pair((float)((int)(q & 63u) - 32), (float)((int)((q >> 8) & 63u) - 32));
            out[2 * i + 1] = bf16_pair((float)((int)((q >> 16) & 63u) - 32), (float)((int)(q >> 24) - 32));
        }
        if (first) {
            const float d = f16_bits_to_f32(r.d);
            scl[0] = d * (float)(int)(int8_t)(r.sc & 0xFFu);
            scl[1] = d * (float)(int)(int8_t)((r.sc >> 8) & 0xFFu);
        }
    }
};

// Element j of a W row as the dequantizer gives it (fp32, gguf.py op order):
// Q4_K fl(d sc q) - fl(dmin m), Q6_K d sc (q - 32), Q8_0 d q.
template <int QT>
__device__ float weight_at(const uint8_t* __restrict__ wrow, int j) {
    if constexpr (QT == kTypeQ4K) {
        const uint8_t* bp = wrow + (int64_t)(j >> 8) * kQ4KBytes;
        const int e = j & 255, sb = e >> 5, l = e & 31;
        const uint4 h = *reinterpret_cast<const uint4*>(bp);
        uint32_t sc, mn;
        k4_scale_min(h.y, h.z, h.w, sb, sc, mn);
        const uint32_t q = (bp[16 + 32 * (sb >> 1) + l] >> (4 * (sb & 1))) & 15u;
        return f16_bits_to_f32(h.x) * (float)sc * (float)q - f16_bits_to_f32(h.x >> 16) * (float)mn;
    } else if constexpr (QT == kTypeQ6K) {
        const uint8_t* bp = wrow + (int64_t)(j >> 8) * kQ6KBytes;
        const int e = j & 255, hh = e >> 7, ks = (e >> 5) & 3, l = e & 31;
        const uint32_t ql = (bp[64 * hh + 32 * (ks & 1) + l] >> (ks >= 2 ? 4 : 0)) & 15u;
        const uint32_t qh = (bp[128 + 32 * hh + l] >> (2 * ks)) & 3u;
        const float sc = (float)(int)(int8_t)bp[192 + 8 * hh + (l >> 4) + 2 * ks];
        return f16_bits_to_f32(ld_u16(bp + 208)) * sc * (float)((int)(ql | (qh << 4)) - 32);
    } else {
        const uint8_t* bp = wrow + (int64_t)(j >> 5) * kQ80Bytes;
        return f16_bits_to_f32(ld_u16(bp)) * (float)(int)(int8_t)bp[2 + (j & 31)];
    }
}

// sum_j w[j] x[j] in fp64 (products of fp32 values exact), rounded to fp32 once.
template <int QT>
__device__ float row_dot_exact(const uint8_t* __restrict__ wrow, const float* __restrict__ xrow, int K) {
    double acc = 0.0;
    for (int j = 0; j < K; ++j) acc = __builtin_fma((double)weight_at<QT>(wrow, j), (double)xrow[j], acc);
    return (float)acc;
}

template <int QT, int WM, int WN, int MI>
__global__ void __launch_bounds__(64 * WM * WN) gemm_f32c_kernel(const uint8_t* __restrict__ w,
                                                                 const float* __restrict__ x, float* __restrict__ y,
                                                                 int M, int N, int K, int64_t ldy, int S,
                                                                 float* __restrict__ part,
                                                                 uint32_t* __restrict__ flags, uint32_t epoch) {
    static_assert(WM * WN == 4 || WM * WN == 8, "four or eight waves");
    constexpr int NT = 64 * WM * WN;                  // threads
    constexpr int BM = 32 * MI * WM, BN = 64 * WN;    // a wave owns 32 MI x 64 of the tile
    constexpr int XT = NT / BM, XV = kCK / XT;       // X staging: threads per row, values per thread
    constexpr int WT = NT / BN, WV = kCK / WT;       // W staging: threads per row, codes per thread
    static_assert((XV == 4 || XV == 8) && (WV == 8 || WV == 16 || WV == 32), "staging shapes");
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][3][BM * kCRow];
    __shared__ __attribute__((aligned(16))) uint16_t ws[2][BN * kCRow];
    __shared__ __attribute__((aligned(16))) float xsum[2][BM];
    __shared__ __attribute__((aligned(16))) float wsc[2][BN][2];
    using F = CFmt<QT>;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int mtiles = (M + BM - 1) / BM;
    const int mt = (int)(blockIdx.x % mtiles), rest = (int)(blockIdx.x / mtiles);
    const int split = rest % S, nt = rest / S;
    const int m0 = mt * BM, n0 = nt * BN;
    const int64_t row_bytes = (int64_t)(K / F::kElems) * F::kBytes;
    const int total = K / kCK;                          // K-split `split` covers steps [sbase, sbase + steps)
    const int sbase = (int)((int64_t)split * total / S);
    const int steps = (int)((int64_t)(split + 1) * total / S) - sbase;

    const int xr = tid / XT, xk = (tid % XT) * XV;    // X staging: row xr, elements xk .. xk + XV - 1
    // over the steps this workgroup checks (its row xr is the same in all):
    // |x| without its sign as bits << 1, the exponent in the top byte (inf
    // and NaN above every finite value): the largest, and the smallest
    // nonzero as (bits << 1) - 1, where 0 wraps to the top and drops out
    uint32_t xr_max = 0, xr_min1 = 0xFFFFFFFFu;
    const int ntiles = (N + BN - 1) / BN;
    const float* xrow = x + (int64_t)(m0 + xr < M ? m0 + xr : M - 1) * K;
    const int wr = tid / WT, wk = (tid % WT) * WV;    // W staging: row wr, codes wk .. wk + WV - 1
    const uint8_t* wrow = w + (int64_t)(n0 + wr < N ? n0 + wr : N - 1) * row_bytes;

    struct Stage {
        f32x4 xv[XV / 4];
        typename F::template Raw<WV> wr;
    };
    Stage stg[2];
    auto load_step = [&](Stage& st, int s) __attribute__((always_inline)) {
        const int kb = (sbase + s) * kCK;
#pragma unroll
        for (int i = 0; i < XV / 4; ++i) st.xv[i] = *reinterpret_cast<const f32x4*>(xrow + kb + xk + 4 * i);
        F::template load<WV>(st.wr, wrow, sbase + s, wk);
    };
    auto stage_step = [&](const Stage& st, int buf, int s) __attribute__((always_inline)) {
        // X: three bf16 pieces per value and the row's sum over the step
        uint32_t p1[XV / 2], p2[XV / 2], p3[XV / 2];
        float sx = 0.0f;
        if ((sbase + s) % ntiles == nt % ntiles) {        // workgroup-uniform
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                const uint32_t u = __float_as_uint(st.xv[i >> 2][i & 3]) << 1;
                xr_max = max(xr_max, u);
                xr_min1 = min(xr_min1, u - 1u);
            }
        }
#pragma unroll
        for (int i = 0; i < XV / 2; ++i) {
            const float a = st.xv[i >> 1][2 * (i & 1)], b = st.xv[i >> 1][2 * (i & 1) + 1];
            sx += a + b;
            p1[i] = bf16_pair(a, b);
            const float ra = a - bf16_lo(p1[i]), rb = b - bf16_hi(p1[i]);
            p2[i] = bf16_pair(ra, rb);
            p3[i] = bf16_pair(ra - bf16_lo(p2[i]), rb - bf16_hi(p2[i]));
        }
        const int xo = xr * kCRow + xk;
        if constexpr (XV == 8) {
            *reinterpret_cast<u32x4*>(&xs[buf][0][xo]) = u32x4{p1[0], p1[1], p1[2], p1[3]};
            *reinterpret_cast<u32x4*>(&xs[buf][1][xo]) = u32x4{p2[0], p2[1], p2[2], p2[3]};
            *reinterpret_cast<u32x4*>(&xs[buf][2][xo]) = u32x4{p3[0], p3[1], p3[2], p3[3]};
        } else {
            *reinterpret_cast<u32x2*>(&xs[buf][0][xo]) = u32x2{p1[0], p1[1]};
            *reinterpret_cast<u32x2*>(&xs[buf][1][xo]) = u32x2{p2[0], p2[1]};
            *reinterpret_cast<u32x2*>(&xs[buf][2][xo]) = u32x2{p3[0], p3[1]};
        }
        if constexpr (XV == 4) {   // 8 values per row-quad lane group: sum over the XT lanes of the row
            static_assert(XT == 8, "layout");
            sx += dpp_mov<0xB1>(sx);
            sx += dpp_mov<0x4E>(sx);
            sx += dpp_mov<0x141>(sx);
        } else {
            static_assert(XT == 4, "layout");
            sx += dpp_mov<0xB1>(sx);
            sx += dpp_mov<0x4E>(sx);
        }
        if (tid % XT == 0) xsum[buf][xr] = sx;
        // W: codes and per-row scales
        uint32_t cw[WV / 2];
        float scl[2];
        F::template codes<WV>(st.wr, sbase + s, cw, scl, wk == 0);
#pragma unroll
        for (int i = 0; i < WV / 8; ++i)
            *reinterpret_cast<u32x4*>(&ws[buf][wr * kCRow + wk + 8 * i]) = u32x4{cw[4 * i], cw[4 * i + 1], cw[4 * i + 2],
                                                                                cw[4 * i + 3]};
        static_assert(WV % 8 == 0, "whole 16-byte code chunks");
        if (wk == 0) {
            wsc[buf][wr][0] = scl[0];
            wsc[buf][wr][1] = scl[1];
        }
    };

    f32x16 acc[MI][2];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

    const int mbase = 32 * MI * wm, kh = 8 * (lane >> 5);
    // Per step: the B fragments (both 16-k halves, both column tiles) once;
    // then each 32-row sub-tile mi in turn with its own A fragments and two
    // sub-block sums live (cs), scaled into acc when its sub-block ends.
    auto compute = [&](int buf) __attribute__((always_inline)) {
        bf16x8 b[2][2];                                  // [ks][ni]
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                b[ks][ni] = *reinterpret_cast<const bf16x8*>(
                    &ws[buf][(64 * wn + 32 * ni + (lane & 31)) * kCRow + 16 * ks + kh]);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
            const int row = mbase + 32 * mi + (lane & 31);
            bf16x8 a[2][3];                              // [ks][piece]
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int p = 0; p < 3; ++p)
                    a[ks][p] = *reinterpret_cast<const bf16x8*>(&xs[buf][p][row * kCRow + 16 * ks + kh]);
            // sum(x) of the lane's 16 rows (Q4_K min term): rows 32 mi + 8 i + 4 (l / 32) + j
            f32x4 sxr[4];
            if constexpr (QT == kTypeQ4K) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    sxr[i] = *reinterpret_cast<const f32x4*>(&xsum[buf][mbase + 32 * mi + 8 * i + 4 * (lane >> 5)]);
            }
            f32x16 cs[2];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    // a new sub-block starts from a zero C operand (no register clears)
                    const f32x16 zero = {};
                    cs[ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks][0], b[ks][ni],
                                                                     (QT == kTypeQ6K || ks == 0) ? zero : cs[ni], 0, 0, 0);
#pragma unroll
                    for (int p = 1; p < 3; ++p)
                        cs[ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks][p], b[ks][ni], cs[ni], 0, 0, 0);
                }
                if (QT == kTypeQ6K || ks == 1) {   // one sub-block done: scale it into the accumulators
#pragma unroll
                    for (int ni = 0; ni < 2; ++ni) {
                        const int nl = 64 * wn + 32 * ni + (lane & 31);
                        const float sc = wsc[buf][nl][QT == kTypeQ6K ? ks : 0];
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[mi][ni][r] = __builtin_fmaf(sc, cs[ni][r], acc[mi][ni][r]);
                        if constexpr (QT == kTypeQ4K) {
                            const float t = wsc[buf][nl][1];
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                acc[mi][ni][r] = __builtin_fmaf(-t, sxr[r >> 2][r & 3], acc[mi][ni][r]);
                        }
                    }
                }
            }
        }
    };

    // Global loads run two steps ahead of the products (32-row wave tiles):
    // step s + 2 is loaded into staging set s % 2 while step s is computed, and staged
    // into LDS (buffer (s + 1) % 2) after step s + 1's loads have had a whole
    // step to arrive. The loop is unrolled by two so each staging set is a
    // compile-time choice, and loads and stages are unconditional (past the
    // last step they repeat it into a buffer nothing reads again), so the
    // compiler's wait before a stage covers one staging set only. An odd
    // last step is computed after the loop from buffer 0.
    const int last = steps - 1;
    if constexpr (MI == 1) {
        load_step(stg[0], 0);
        load_step(stg[1], last < 1 ? last : 1);
        stage_step(stg[0], 0, 0);
        __syncthreads();
        int s0 = 0;
        for (; s0 + 1 < steps; s0 += 2) {
            static_for<0, 2>([&](auto jc) {
                constexpr int j = decltype(jc)::value;  // s % 2: LDS buffer and staging set of step s
                const int s = s0 + j;
                load_step(stg[j], s + 2 < last ? s + 2 : last);
                compute(j);
                stage_step(stg[j ^ 1], j ^ 1, s + 1 < last ? s + 1 : last);
                __syncthreads();
            });
        }
        if (s0 < steps) compute(0);
    } else {
        // 64-row wave tiles do twice the products per step, which covers the
        // load latency with one staging set (the registers of a second do
        // not fit beside the accumulators)
        load_step(stg[0], 0);
        stage_step(stg[0], 0, 0);
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            const int buf = s & 1;
            load_step(stg[0], s + 1 < last ? s + 1 : last);
            compute(buf);
            stage_step(stg[0], buf ^ 1, s + 1 < last ? s + 1 : last);
            __syncthreads();
        }
    }

    // every value checked here 0 or in [2^-100, 2^100] (exponent fields
    // 27 .. 227; inf and NaN have 255), else flag the row (rare)
    if ((xr_max > (227u << 24) || xr_min1 < (27u << 24) - 1u) && m0 + xr < M) flags[m0 + xr] = epoch;
    // S > 1: this split's partial tile goes to plane `split` (rows of N)
    float* out = S == 1 ? y : part + (int64_t)split * M * N;
    const int64_t ld = S == 1 ? ldy : N;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int n = n0 + 64 * wn + 32 * ni + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + mbase + 32 * mi + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M && n < N) out[(int64_t)m * ld + n] = acc[mi][ni][r];
            }
        }
}

// Unsplit launches: the rows flagged for this launch, weight by weight in
// fp64 (one workgroup per row of x; the others return at once).
template <int QT>
__global__ void __launch_bounds__(256) gemm_f32_fixup_kernel(float* __restrict__ y, int N, int64_t ldy,
                                                             const uint32_t* __restrict__ flags, uint32_t epoch,
                                                             const uint8_t* __restrict__ w,
                                                             const float* __restrict__ x, int K) {
    const int m = (int)blockIdx.x;
    if (flags[m] != epoch) return;
    const int64_t row_bytes = (int64_t)(K / CFmt<QT>::kElems) * CFmt<QT>::kBytes;
    for (int n = threadIdx.x; n < N; n += blockDim.x)
        y[(int64_t)m * ldy + n] = row_dot_exact<QT>(w + (int64_t)n * row_bytes, x + (int64_t)m * K, K);
}

// Split-K sums: y = the planes added in split order, except rows flagged
// for this launch (x outside the pieces' range), which are computed weight
// by weight in fp64. Row blockIdx.x, four columns per thread.
template <int QT>
__global__ void __launch_bounds__(256) gemm_f32_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                              int S, int M, int N, int64_t ldy,
                                                              const uint32_t* __restrict__ flags, uint32_t epoch,
                                                              const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x, int K) {
    const int m = (int)blockIdx.x;
    const int n0 = 4 * ((int)blockIdx.y * (int)blockDim.x + (int)threadIdx.x);
    if (n0 >= N) return;
    const int64_t count = (int64_t)M * N, base = (int64_t)m * N;
    float* yr = y + (int64_t)m * ldy;
    if (flags[m] == epoch) {                             // workgroup-uniform
        const int64_t row_bytes = (int64_t)(K / CFmt<QT>::kElems) * CFmt<QT>::kBytes;
        for (int n = n0; n < n0 + 4 && n < N; ++n)
            yr[n] = row_dot_exact<QT>(w + (int64_t)n * row_bytes, x + (int64_t)m * K, K);
        return;
    }
    if (n0 + 4 <= N && ((N | ldy) & 3) == 0 && !(reinterpret_cast<uintptr_t>(y) & 15)) {
        const f32x4 v = sum_planes<f32x4>(
            [&](int q) { return *reinterpret_cast<const f32x4*>(part + q * count + base + n0); }, S);
        *reinterpret_cast<f32x4*>(yr + n0) = v;
    } else {
        for (int n = n0; n < n0 + 4 && n < N; ++n)
            yr[n] = sum_planes<float>([&](int q) { return part[q * count + base + n]; }, S);
    }
}

template <int QT>
void f32c_go(int bm, int bn, dim3 g, hipStream_t s, const uint8_t* w, const float* x, float* y, int M, int N, int K,
             int64_t ldy, int S, float* part, uint32_t* flags, uint32_t epoch) {
    if (bm == 32)
        gemm_f32c_kernel<QT, 1, 4, 1><<<g, dim3(256), 0, s>>>(w, x, y, M, N, K, ldy, S, part, flags, epoch);
    else if (bm == 64)
        gemm_f32c_kernel<QT, 2, 2, 1><<<g, dim3(256), 0, s>>>(w, x, y, M, N, K, ldy, S, part, flags, epoch);
    else if (bn == 128)
        gemm_f32c_kernel<QT, 4, 2, 1><<<g, dim3(512), 0, s>>>(w, x, y, M, N, K, ldy, S, part, flags, epoch);
    else
        gemm_f32c_kernel<QT, 2, 4, 2><<<g, dim3(512), 0, s>>>(w, x, y, M, N, K, ldy, S, part, flags, epoch);
    if (S > 1) {
        gemm_f32_reduce_kernel<QT><<<dim3((unsigned)M, (unsigned)((N + 1023) / 1024)), dim3(256), 0, s>>>(
            part, y, S, M, N, ldy, flags, epoch, w, x, K);
    } else {
        gemm_f32_fixup_kernel<QT><<<dim3((unsigned)M), dim3(256), 0, s>>>(y, N, ldy, flags, epoch, w, x, K);
    }
}

// One flag word per row of x, after the partial planes of a K-split launch
// (at the start of the scratch when K is not split).
size_t flag_bytes(int64_t m) { return ((size_t)m * sizeof(uint32_t) + 255) & ~(size_t)255; }

// Tile shape: BM x BN = 32 x 256 for up to 32 rows of X, 64 x 128 up to
// kF32cMidRows rows, else eight waves on 128 rows: 128 x 256 for Q4_K (waves
// of 64 x 64: each staged x piece serves 256 columns, each W code 128 rows),
// 128 x 128 for Q6_K and Q8_0 (waves of 32 x 64, loads two steps ahead).
// Measured at 512 rows: Q4_K 3584 x 18944 303 vs 324 us; Q6_K 4096 x 14336
// 245 vs 282 us; Q8_0 4096 x 4096 66 vs 72 us (128 x 128 vs 128 x 256).
constexpr int64_t kF32cMidRows = 64;
void f32c_tile(int qtype, int64_t m, int* bm, int* bn) {
    *bm = m <= 32 ? 32 : m <= kF32cMidRows ? 64 : 128;
    *bn = m <= 32 ? 256 : m <= kF32cMidRows ? 128 : qtype == kTypeQ4K ? 256 : 128;
}

}  // namespace

bool gemm_f32_supported(int qtype, int64_t m, int64_t n, int64_t k) {
    const int64_t kq = qtype == kTypeQ80 ? kQ80Elems : (qtype == kTypeQ4K || qtype == kTypeQ6K) ? kQKElems : 0;
    if (kq == 0 || m <= 0 || n <= 0 || k <= 0 || k % kq || m > 0x7FFFFFFF || n > 0x7FFFFFFF || k > 0x7FFFFFFF)
        return false;
    int bm, bn;
    f32c_tile(qtype, m, &bm, &bn);
    return ((m + bm - 1) / bm) * ((n + bn - 1) / bn) <= 0x7FFFFFFF;
}

// K-splits: the largest S in {1, 2, 4, ..., 64} that leaves every split >= 8
// steps (splits differ by at most one step), keeps the grid within one round
// of workgroups (per_round) and its partial planes within `part_cap` bytes;
// shapes that fill the GPU are not split.
int gemm_f32_splits(int qtype, int64_t m, int64_t n, int64_t k, size_t part_cap) {
    int bm, bn;
    f32c_tile(qtype, m, &bm, &bn);
    const int64_t tiles = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    const int64_t steps = k / kCK;
    const double plane = (double)m * (double)n * sizeof(float), flagb = (double)flag_bytes(m);
    // one round of workgroups: two 4-wave workgroups per CU, or one 8-wave
    // 128-row workgroup (85 or 105 KB of LDS)
    const int64_t per_round = bm == 128 ? 256 : 512;
    int best = 1;
    for (int sp = 2; sp <= 64; sp *= 2) {
        if (steps / sp < 8 || tiles * sp > per_round || sp * plane + flagb > (double)part_cap) break;
        best = sp;
    }
    return best;
}

size_t gemm_f32_scratch(int qtype, int64_t m, int64_t n, int64_t k, size_t part_cap) {
    const int sp = gemm_f32_splits(qtype, m, n, k, part_cap);
    return (sp > 1 ? (size_t)sp * (size_t)m * (size_t)n * sizeof(float) : 0) + flag_bytes(m);
}

hipError_t launch_gemm_f32(int qtype, const uint8_t* w, const float* x, float* y, int64_t m, int64_t n, int64_t k,
                           int64_t ldy, hipStream_t stream, float* part, size_t part_cap) {
    if (ldy < n) return hipErrorInvalidValue;
    if (!gemm_f32_supported(qtype, m, n, k)) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(x) & 15) return hipErrorInvalidValue;
    if (qtype == kTypeQ4K && (reinterpret_cast<uintptr_t>(w) & 15)) return hipErrorInvalidValue;
    if (qtype != kTypeQ4K && (reinterpret_cast<uintptr_t>(w) & 1)) return hipErrorInvalidValue;
    const int sp = gemm_f32_splits(qtype, m, n, k, part ? part_cap : 0);
    int bm, bn;
    f32c_tile(qtype, m, &bm, &bn);
    const int64_t tiles = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    if (tiles * sp > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 g((unsigned)(tiles * sp));
    // per-launch tag of the row flags (never 0, the value of fresh scratch)
    static std::atomic<uint32_t> launches{0};
    uint32_t epoch = ++launches;
    if (epoch == 0) epoch = ++launches;
    if (!part || part_cap < gemm_f32_scratch(qtype, m, n, k, part_cap)) return hipErrorInvalidValue;
    uint32_t* flags = reinterpret_cast<uint32_t*>(part + (sp > 1 ? (size_t)sp * (size_t)m * (size_t)n : 0));
    switch (qtype) {
        case kTypeQ4K:
            f32c_go<kTypeQ4K>(bm, bn, g, stream, w, x, y, (int)m, (int)n, (int)k, ldy, sp, part, flags, epoch);
            break;
        case kTypeQ6K:
            f32c_go<kTypeQ6K>(bm, bn, g, stream, w, x, y, (int)m, (int)n, (int)k, ldy, sp, part, flags, epoch);
            break;
        case kTypeQ80:
            f32c_go<kTypeQ80>(bm, bn, g, stream, w, x, y, (int)m, (int)n, (int)k, ldy, sp, part, flags, epoch);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace frq
