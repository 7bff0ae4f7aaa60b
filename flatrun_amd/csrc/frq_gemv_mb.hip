// Q4_K matvec of up to eight rows of x at once with the products on the
// matrix cores in fp32 (v_mfma_f32_4x4x1_16b_f32): Y[r, i] = sum_j W[i, j]
// X[r, j] for r < m, the reference's matmul_q4_k / matmul_q4_k_batched
// (q4_k.h:427-449, _C.cpp:154-197) with W read once for the m rows.
//
// Arithmetic. Every weight is dequantized on its own, w = fma(s, q, -t) with
// s = d*sc and t = dmin*m of its sub-block (both exact fp32 products, s*q
// exact), i.e. the dequant's fp32 bits, and every product w * x enters an
// fp32 sum through one fused multiply-add: the instruction computes
// D[b][i][j] = A[b][i] * B[b][j] + C[b][i][j] for 16 independent 4 x 4 outer
// products b with one rounding per element and keeps fp32 denormals, so each
// output is a sequence of fp32 fmas over its weights followed by fp32 sums
// of the partials, and |y - y_exact| <= c * 2^-24 * sum_j |w_j x_j| holds for
// every finite x, cancelling weights included (the element-wise kernel's
// bound).
//
// Operand roles. Lane l = 4 kb + c: as A it supplies the weight of W row c
// (of the wave's current group of four rows) at a k it owns, as B the x of
// x row c (of the current column group) at the same k; output lane 4 kb + j,
// register i receives row i, x row j. The 16 k slots kb are 16-byte parts of
// a pair of blocks: slot kb = 8 p + h takes qs bytes 16 h .. 16 h + 15 of
// block p of the pair, i.e. group g = h / 2 (sub-block 2g in the low, 2g + 1
// in the high nibbles) and half hh = h % 2: low nibble of byte e is element
// 64 g + 16 hh + e, high nibble element 64 g + 32 + 16 hh + e. 32 MFMAs per
// pair and row group, one per nibble; a lane's k slot and x stay fixed while
// the wave sweeps its row groups.
//
// Codes to float: a byte holding q < 16 converts as an fp8 (e4m3) code to
// q * u exactly, u = the value of code 1, two bytes per instruction; the
// scale carries 1 / u (a power of two, so s / u * (q u) = s q exactly).
//
// Work mapping. A workgroup owns R <= 4 G rows (G groups of four, rows past
// the end re-read the last row and are not stored) and all of k: wave w owns
// block pairs [w NBP, w NBP + NBP). Per pair the wave loads x of its pair
// (the next pair's x right after the last products of the current one, into
// the same registers: a second x buffer took the kernel past 128 VGPRs and
// into scratch, 22.8 us against 21.0-21.4 for 4 rows of 3584 x 18944), then
// for each row group the
// two 16-byte loads per lane (block header, the lane's qs bytes) that a ring
// of two slots keeps one step ahead. Accumulators persist per row group over
// the pairs; at the end each row group's four k slots per 16-lane row are
// summed with DPP, and the four rows' partials of every wave meet in LDS,
// added in a fixed order. The last wavefront skips the pairs past the row's
// end (a wave-uniform branch). A row's result depends on its own x only: not
// on m, on the other rows of x, or on which column it takes.
#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// x of one pair for one lane: [column group][plane][e]
template <int CG>
struct MbX {
    float v[CG][2][16];
};

// x of the lane's k slot in one pair, per column group: rows of x past m,
// and blocks past the row's end, read as zeros (offsets beyond the buffer).
// No branch: every value is written on every path.
template <int CG>
__device__ __forceinline__ void mb_load_x(__amdgpu_buffer_rsrc_t xs, int64_t k, int c, bool valid, int blk, int g,
                                          int hh, MbX<CG>& xv) {
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
        const int64_t e0 = (int64_t)(4 * cg + c) * k + (int64_t)blk * kQKElems + 64 * g + 16 * hh;
        const uint32_t off = valid ? (uint32_t)(4 * e0) : 0x80000000u;
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            const uint4 a = bload_b128(xs, off + 4 * e), o = bload_b128(xs, off + 128 + 4 * e);
            xv.v[cg][0][e] = __uint_as_float(a.x); xv.v[cg][0][e + 1] = __uint_as_float(a.y);
            xv.v[cg][0][e + 2] = __uint_as_float(a.z); xv.v[cg][0][e + 3] = __uint_as_float(a.w);
            xv.v[cg][1][e] = __uint_as_float(o.x); xv.v[cg][1][e + 1] = __uint_as_float(o.y);
            xv.v[cg][1][e + 2] = __uint_as_float(o.z); xv.v[cg][1][e + 3] = __uint_as_float(o.w);
        }
    }
}

// Sum over the four k slots of a 16-lane row (lanes 4 kb + j, kb in
// 4q .. 4q + 3): lane 16q + j (j < 4) ends with it, the same order for
// every j.
__device__ __forceinline__ float mb_row_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
    return v;
}

template <int NBP, int G, int CG>
__global__ void __launch_bounds__(1024) gemv_q4_k_mb_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                           float* __restrict__ y, int64_t n, int nb, int m, int R,
                                                           int64_t ldy) {
    extern __shared__ float red[];                      // [4 G rows][4 CG x rows][waves][4 DPP rows]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
    const int c = lane & 3, kb = lane >> 2, p = kb >> 3, h = kb & 7, g = h >> 1, hh = h & 1;
    const int64_t k = (int64_t)nb * kQKElems;
    const int npairs = (nb + 1) >> 1;
    const int64_t row0 = (int64_t)blockIdx.x * R;
    const int nrows = (int)(n - row0 < R ? n - row0 : R);
    const uint32_t row_bytes = (uint32_t)nb * kQ4KBytes;
    const auto rs = buffer_rsrc(w + row0 * (int64_t)row_bytes, (uint32_t)nrows * row_bytes);
    const auto xs = buffer_rsrc(x, (uint32_t)((int64_t)m * k * 4));   // x rows past m read as 0
    const float u_inv = 1.0f / fp8_unit();
    const ScaleDecode dec(g);

    // block of pair jp for this lane; invalid past the row's end (x = 0, s = t = 0).
    // The last wavefront may own fewer pairs: it skips the others (uniform).
    auto blk_of = [&](int jp) { return 2 * (wave * NBP + jp) + p; };
    auto valid_of = [&](int jp) { return wave * NBP + jp < npairs && blk_of(jp) < nb; };
    const int own = npairs - wave * NBP < NBP ? npairs - wave * NBP : NBP;   // >= 1

    struct Slot {
        uint4 hd, qv;
    };
    Slot ring[2];
    auto load = [&](int step, Slot& s) {
        const int jp = step / G, rg = step % G;
        const int r = 4 * rg + c < nrows ? 4 * rg + c : nrows - 1;
        const int blk = valid_of(jp) ? blk_of(jp) : 0;
        const uint32_t off = (uint32_t)r * row_bytes + (uint32_t)blk * kQ4KBytes;
        s.hd = bload_b128(rs, off);
        s.qv = bload_b128(rs, off + 16 + 16 * h);
    };

    f32x4 acc[CG][G];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int rg = 0; rg < G; ++rg) acc[cg][rg] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Row priorities (row_priority): with three pairs per wavefront (13+
    // wavefronts, one workgroup per CU) they let the wavefronts that are
    // behind issue first (4 rows of 3584 x 18944: 23.6 -> 22.9 us); with one
    // or two pairs they cost (4096 x 14336: 20.3 -> 20.8, 14336 x 4096: 20.8
    // -> 24.0), same process.
    constexpr bool kPrio = NBP == 3;
    MbX<CG> xb;
    row_priority<kPrio, NBP * G, 0>();
    mb_load_x<CG>(xs, k, c, valid_of(0), blk_of(0), g, hh, xb);
    __builtin_amdgcn_sched_barrier(0);
    load(0, ring[0]);
    if constexpr (NBP * G > 1) {
        if ((1 / G) < own) load(1, ring[1]);
    }
    __builtin_amdgcn_sched_barrier(0);

    static_for<0, NBP * G>([&](auto sc) {
        constexpr int step = decltype(sc)::value;
        constexpr int jp = step / G, rg = step % G;
        if (jp >= own) return;                          // wave-uniform: a pair past the row's end
        row_priority<kPrio, NBP * G, step>();
        const MbX<CG>& xv = xb;
        Slot& t = ring[step & 1];
        const bool valid = valid_of(jp);
        const float d = valid ? f16_bits_to_f32(t.hd.x) : 0.0f, dm = valid ? f16_bits_to_f32(t.hd.x >> 16) : 0.0f;
        uint32_t sc0, m0, sc1, m1;
        dec(t.hd.y, t.hd.z, t.hd.w, sc0, m0, sc1, m1);
        const float du = d * u_inv;
        const float s_lo = du * (float)sc0, t_lo = dm * (float)m0;   // exact
        const float s_hi = du * (float)sc1, t_hi = dm * (float)m1;
        const uint32_t qw[4] = {t.qv.x, t.qv.y, t.qv.z, t.qv.w};
        if constexpr (step + 2 < NBP * G) {
            // everything this step reads from the slot is in registers now:
            // refill it with the step two ahead before the products
            __builtin_amdgcn_sched_barrier(0);
            if ((step + 2) / G < own) load(step + 2, t);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            float f[8];
            nibbles8_fp8(qw[wd], f);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a = __builtin_fmaf(s_lo, f[e], -t_lo);
#pragma unroll
                for (int cg = 0; cg < CG; ++cg)
                    acc[cg][rg] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, xv.v[cg][0][4 * wd + e], acc[cg][rg], 0, 0, 0);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float a = __builtin_fmaf(s_hi, f[4 + e], -t_hi);
#pragma unroll
                for (int cg = 0; cg < CG; ++cg)
                    acc[cg][rg] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, xv.v[cg][1][4 * wd + e], acc[cg][rg], 0, 0, 0);
            }
        }
        if constexpr (rg == G - 1 && jp + 1 < NBP) {    // the pair's x is used up: the next pair's
            if (jp + 1 < own) mb_load_x<CG>(xs, k, c, valid_of(jp + 1), blk_of(jp + 1), g, hh, xb);
        }
    });

    // acc[cg][rg][i] at lane 4 kb + j: row 4 rg + i, x row 4 cg + j, k slot kb
#pragma unroll
    for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int rg = 0; rg < G; ++rg)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float v = mb_row_sum(acc[cg][rg][i]);
                if ((lane & 15) < 4)
                    red[(((4 * rg + i) * 4 * CG + 4 * cg + (lane & 3)) * nw + wave) * 4 + (lane >> 4)] = v;
            }
    __syncthreads();
    for (int idx = tid; idx < nrows * m; idx += blockDim.x) {
        const int row = idx / m, r = idx - row * m;
        const float* rp = red + (row * 4 * CG + r) * nw * 4;
        float s = 0.0f;
        for (int w2 = 0; w2 < 4 * nw; ++w2) s += rp[w2];
        y[r * ldy + row0 + row] = s;
    }
}

template <int NBP, int CG>
hipError_t mb_go(int G, dim3 gd, dim3 bd, size_t lds, hipStream_t s, const uint8_t* w, const float* x, float* y,
                 int64_t n, int nb, int m, int R, int64_t ldy) {
    switch (G) {
        case 1: gemv_q4_k_mb_kernel<NBP, 1, CG><<<gd, bd, lds, s>>>(w, x, y, n, nb, m, R, ldy); break;
        case 2: gemv_q4_k_mb_kernel<NBP, 2, CG><<<gd, bd, lds, s>>>(w, x, y, n, nb, m, R, ldy); break;
        case 3: gemv_q4_k_mb_kernel<NBP, 3, CG><<<gd, bd, lds, s>>>(w, x, y, n, nb, m, R, ldy); break;
        case 4: gemv_q4_k_mb_kernel<NBP, 4, CG><<<gd, bd, lds, s>>>(w, x, y, n, nb, m, R, ldy); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool plan_gemv_mb(int64_t n, int64_t k, int m, MbPlan* p) {
    if (n <= 0 || k <= 0 || k % kQKElems != 0 || m < 1 || m > kGemvMbMax) return false;
    const int64_t nb = k / kQKElems, npairs = (nb + 1) / 2;
    MbPlan q = *p;
    q.cg = m > 4 ? 2 : 1;
    if (q.nbp <= 0) q.nbp = (int)((npairs + 15) / 16);
    if (q.nbp < 1 || q.nbp > (q.cg == 2 ? 1 : 3)) return false;
    q.waves = (int)((npairs + q.nbp - 1) / q.nbp);
    if (q.waves > 16) return false;
    if (q.rows <= 0) {
        // one round of workgroups where the rows allow: as many per CU as fit
        // (<= 16 waves per CU, i.e. one workgroup of more than 8 waves)
        const int64_t per_cu = q.waves > 8 ? 1 : 16 / q.waves;
        int64_t r = (n + 256 * per_cu - 1) / (256 * per_cu);
        q.rows = (int)(r < 1 ? 1 : r > 16 ? 16 : r);
    }
    if (q.rows < 1 || q.rows > 16) return false;
    q.groups = (q.rows + 3) / 4;
    q.grid = (n + q.rows - 1) / q.rows;
    if (q.grid > 0x7FFFFFFF) return false;
    *p = q;
    return true;
}

bool gemv_mb_ok(const uint8_t* w, const float* x, int64_t k) {
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w), xa = reinterpret_cast<uintptr_t>(x);
    return k > 0 && k % kQKElems == 0 && k <= (int64_t)1 << 24 && (wa & 15) == 0 && (xa & 15) == 0;
}

hipError_t launch_gemv_mb(const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int m, int64_t ldy,
                          const MbPlan& p, hipStream_t stream) {
    if (n <= 0 || m <= 0) return hipSuccess;
    if (m > 4 * p.cg || ldy < n || !gemv_mb_ok(w, x, k)) return hipErrorInvalidValue;
    const int nb = (int)(k / kQKElems);
    if ((int64_t)p.waves * p.nbp * 2 < nb || p.groups * 4 < p.rows) return hipErrorInvalidValue;
    const dim3 gd((unsigned)p.grid), bd((unsigned)(64 * p.waves));
    const size_t lds = sizeof(float) * 16 * 4 * p.cg * p.waves * 4;
    if (p.cg == 2) {
        if (p.nbp != 1) return hipErrorInvalidValue;
        return mb_go<1, 2>(p.groups, gd, bd, lds, stream, w, x, y, n, nb, m, p.rows, ldy);
    }
    switch (p.nbp) {
        case 1: return mb_go<1, 1>(p.groups, gd, bd, lds, stream, w, x, y, n, nb, m, p.rows, ldy);
        case 2: return mb_go<2, 1>(p.groups, gd, bd, lds, stream, w, x, y, n, nb, m, p.rows, ldy);
        case 3: return mb_go<3, 1>(p.groups, gd, bd, lds, stream, w, x, y, n, nb, m, p.rows, ldy);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace frq
