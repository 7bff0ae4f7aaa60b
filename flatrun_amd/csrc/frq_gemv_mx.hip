// Q4_K GEMV, batch 1, with the products on the matrix cores
// (v_mfma_i32_16x16x64_i8): y[i] = sum_j w[i, j] x[j], the reference's
// matmul_q4_k (q4_k.h:427-449) over rows of 256-element blocks
// [d f16][dmin f16][scales 12][qs 128] (gguf.py:192-219).
//
// Arithmetic. Within a 32-element sub-block s of a block, w = d*sc_s*q - dmin*m_s
// with q in 0..15, so a row's block contributes
//     d*sc_s * sum(q x) - dmin*m_s * sum(x)
// per sub-block. x is written once per sub-block as a 60-bit fixed-point
// number relative to the sub-block's largest magnitude: with max |x| < 2^e,
//     x * 2^(30-e) = m1 + m2 * 2^-30 + r,   m1 = trunc(x 2^(30-e)),
//     m2 = trunc(frac * 2^30), |m1|, |m2| < 2^30,
// and m1, m2 each as four balanced base-256 digits (int8). The matrix cores
// form sum(q * digit) exactly in int32 for all eight digits, and sum(digit)
// the same way (the digits against an all-ones B); the epilogue recombines
// each level's four sums exactly in fp64 and forms
//     T = d*sc_s * sum(q m) - dmin*m_s * sum(m)
// in fp64 (d*sc_s and dmin*m_s are exact fp32 values, the sums exact
// integers below 2^39), scales it by 2^(e-30) / 2^(e-60) and adds it to the
// lane's fp64 sum, which is rounded to fp32 once.
//
// Exactness. The split is exact (r = 0) for every x whose lowest set bit is
// at or above 2^(e-60), which holds for every element within 2^36 of its
// sub-block's maximum (24-bit significands). Each lane checks its four
// values (m2 * 2^-30 must reproduce the fraction), and a sub-block with
// max |x| >= 2^30 is never taken. A block of a wave with any inexact value
// (or any inf / NaN) is computed per weight instead, w = fl(fl(d*sc)*q) -
// fl(dmin*m) then fma(w, x, acc) as in q4_k.h:153-185, so every finite x
// keeps the fp32 accumulation bound: for each row,
//     |y - y_exact| <= c * 2^-24 * sum_j |w_j x_j|
// with c a small multiple of the per-row summation depth (fp32 sums of the
// lanes' rounded values). T is formed before any rounding, so the bound
// holds when d*sc_j*q_j and dmin*m_j cancel (a weight at or near zero)
// under a large x_j.
//
// Work mapping. A workgroup owns TR <= 16 RT output rows, as RT tiles of
// TT = ceil(TR / RT) <= 16 rows (the MFMA's 16 columns), and a range of KS
// consecutive halves of the row: KS = 1 all blocks, KS = 2 one half, the two
// halves of a row set in two workgroups. Wave w owns blocks [wL, wL + L) of
// the range, L <= 4. Per wave:
//   1. the x of its blocks is loaded first, then 3 x 16 B of every tile row's
//      block per lane: lane (c = l & 15, g = l >> 4) takes row c's header and
//      qs bytes 16g .. 16g+15 and 64+16g .. 64+16g+15, so each load
//      instruction reads 64 contiguous bytes of each of its 16 rows;
//   2. x -> digits into a wave-private LDS table (lane t splits x[4t..4t+3]
//      of each block; eight lanes share a sub-block's max and sum via DPP);
//   3. per block and tile four MFMAs, one per (load, nibble plane): qs bytes
//      32p .. 32p+31 hold sub-block 2p in their low and 2p+1 in their high
//      nibbles, so k-groups 0, 1 of a load carry one sub-block and k-groups
//      2, 3 the next-but-one. A is block diagonal: rows 8h + d (h = 0, 1)
//      carry digit d of the x of k-groups 2h, 2h+1 and zeros elsewhere, so
//      lane (c, g) of the result receives, for row c, the four digit sums of
//      level g & 1 of sub-block 2(g>>1) + [0, 1, 4, 5][m] for MFMA m. The A
//      operand is read once per block and used by every tile;
//   4. one LDS reduction over waves and k-groups per row, in a fixed order.
//      With KS = 2 the two halves of a row meet through one 64-bit slot per
//      row: each half swaps (1 << 32 | its fp32 bits) into the slot with a
//      relaxed device-scope atomic exchange; the half that receives the other
//      half's value writes y = a + b (fp32 addition commutes, so the bits do
//      not depend on which half finishes first) and returns the slot to 0.
//      The slot carries the value itself, so no other memory is shared and
//      no fence is needed; slots must be 0 before a launch and every launch
//      leaves them 0.
// No barrier separates the waves between the loads and the reduction: the
// only shared LDS data (a zero block that the inactive A lanes read) is
// written and fenced before the first load.
#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kMxMaxL = 4;          // blocks per wave
constexpr int kMxMaxWaves = 16;
constexpr int kTabBlock = 2048;     // digit bytes per block: 4 MFMAs x 4 k-groups x 8 digits x 16
constexpr int kSubTab = 8;          // exponents per block: 2 halves x 4 sub-blocks

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

// Four integers |m| < 2^30 as balanced base-256 digits, transposed: out[i]
// byte j = digit i of m_j, where digit_i = byte_i(m + 0x808080) - 128 for
// i < 3 and digit_3 = byte_3(m + 0x808080) as a signed byte, so that
// m = sum_i digit_i 256^i.
__device__ __forceinline__ void balanced_digits(int m0, int m1, int m2, int m3, uint32_t* out) {
    const uint32_t u0 = (uint32_t)m0 + 0x808080u, u1 = (uint32_t)m1 + 0x808080u;
    const uint32_t u2 = (uint32_t)m2 + 0x808080u, u3 = (uint32_t)m3 + 0x808080u;
    const uint32_t ab_e = perm(u1, u0, 0x06020400u), ab_o = perm(u1, u0, 0x07030501u);
    const uint32_t cd_e = perm(u3, u2, 0x06020400u), cd_o = perm(u3, u2, 0x07030501u);
    out[0] = perm(cd_e, ab_e, 0x05040100u) ^ 0x80808080u;
    out[1] = perm(cd_o, ab_o, 0x05040100u) ^ 0x80808080u;
    out[2] = perm(cd_e, ab_e, 0x07060302u) ^ 0x80808080u;
    out[3] = perm(cd_o, ab_o, 0x07060302u);
}

// float -> int32 toward zero with the hardware's saturation (out-of-range
// values give INT_MIN / INT_MAX, NaN gives 0): |x| 2^(30-e) < 2^30 for every
// finite x, and the exactness test rejects inf and NaN, so the saturated
// cases never reach a result.
__device__ __forceinline__ int cvt_i32_sat(float v) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// x[4t .. 4t+3] of one 256-element block (lane t of a wave): d[0..3] the
// digits of m1, d[4..7] those of m2; eo = e - 30 for the lane's 32-element
// sub-block (max |x| < 2^e); exact = every one of the lane's four values is
// m1 + m2 2^-30 exactly (scaled by 2^(30-e)) and e <= 30.
struct XSplit {
    uint32_t d[8];
    int eo;
    bool exact;
};
__device__ __forceinline__ XSplit x_split(float4 v) {
    XSplit r;
    float ma3, ma4;   // max |x| of the four values (abs source modifiers)
    asm("v_max3_f32 %0, |%1|, |%2|, |%3|" : "=v"(ma3) : "v"(v.x), "v"(v.y), "v"(v.z));
    asm("v_max_f32_e64 %0, |%1|, %2" : "=v"(ma4) : "v"(v.w), "v"(ma3));
    uint32_t mx = __float_as_uint(ma4);   // non-negative fp32 bit patterns order like their values
    mx = max(mx, dpp_u<0xB1>(mx));        // quad_perm [1,0,3,2]
    mx = max(mx, dpp_u<0x4E>(mx));        // quad_perm [2,3,0,1]
    mx = max(mx, dpp_u<0x141>(mx));       // row_half_mirror: max over the 8 lanes
    const int e = __builtin_amdgcn_frexp_expf(__uint_as_float(mx));   // max |x| < 2^e (0 for 0, inf, NaN)
    const int sh = 30 - e;
    const float a[4] = {v.x, v.y, v.z, v.w};
    int m1[4], m2[4];
    bool ok = e <= 30;   // else x 2^(30-e) could lose bits below the smallest subnormal
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float s = __builtin_ldexpf(a[i], sh);
        m1[i] = cvt_i32_sat(s);
        const float f2 = __builtin_ldexpf(s - (float)m1[i], 30);      // exact fraction, times 2^30
        m2[i] = cvt_i32_sat(f2);
        ok = ok && ((float)m2[i] == f2);
    }
    balanced_digits(m1[0], m1[1], m1[2], m1[3], r.d);
    balanced_digits(m2[0], m2[1], m2[2], m2[3], r.d + 4);
    r.eo = e - 30;
    r.exact = ok;
    return r;
}

// sum(q m) from four int32 digit sums: (S3 * 256 + S2) * 65536 + (S1 * 256 + S0).
// 32 elements, q <= 15, |digit| <= 128: |S_i| <= 61440, both halves exact;
// the result (|.| < 2^39) exact in fp64.
__device__ __forceinline__ double digit_sum(i32x4 s) {
    return __builtin_fma((double)((s[3] << 8) + s[2]), 65536.0, (double)((s[1] << 8) + s[0]));
}

// One sub-block and level: T = d*sc * sum(q m) - dmin*m * sum(m) in fp64,
// added to the lane's fp64 sum scaled by the level's 2^eo. d*sc and dmin*m
// are exact (an fp16 times a 6-bit integer), the two sums exact integers,
// so T carries every bit that matters and the lane's sum rounds to fp32 once
// at the end: the error is 2^-24 of the lane's own sum_j (d*sc*q_j - dmin*m) x_j
// (up to 2^-52 of its terms), however close d*sc*q_j comes to dmin*m.
__device__ __forceinline__ double sub_block_add(double acc, double d, double dm, uint32_t sc, uint32_t mn, double dq,
                                                double dx, double pw) {
    const double s = d * (double)sc, t = dm * (double)mn;
    return __builtin_fma(__builtin_fma(s, dq, -(t * dx)), pw, acc);
}

// The per-weight form of one lane's share of a block (used when the split of
// the block's x is not exact): lane (c, g) holds row c's qs bytes 16g .. +15
// (q0) and 64 + 16g .. +15 (q1), i.e. half h = g & 1 of sub-blocks
// [2p, 2p+1, 4+2p, 5+2p] (p = g >> 1): low and high nibbles of q0, low and
// high of q1. w = fl(fl(d*sc)*q) - fl(dmin*m) (dequant op order, gguf.py:209-219).
__device__ __forceinline__ float block_per_weight(uint4 hd, uint4 q0, uint4 q1, const float* __restrict__ xb, int g) {
    // rare path: rolled loops keep its registers few, so the unrolled fast
    // path around it keeps every block's weights in registers
    const int p = g >> 1, h = g & 1;
    const float d = f16_bits_to_f32(hd.x), dm = f16_bits_to_f32(hd.x >> 16);
    float acc = 0.0f;
#pragma unroll 1
    for (int pos = 0; pos < 4; ++pos) {
        const int sb = (pos >> 1) * 4 + 2 * p + (pos & 1);
        uint32_t sc, mn;
        k4_scale_min(hd.y, hd.z, hd.w, sb, sc, mn);
        const float s = d * (float)sc, t = dm * (float)mn;
        const uint4 q = (pos >> 1) ? q1 : q0;
        const uint32_t shr = (pos & 1) ? 4u : 0u;
        const float* xs = xb + 32 * sb + 16 * h;
#pragma unroll 1
        for (int i4 = 0; i4 < 4; ++i4) {
            const float4 xv = *reinterpret_cast<const float4*>(xs + 4 * i4);
            const uint32_t nib = (i4 == 0 ? q.x : i4 == 1 ? q.y : i4 == 2 ? q.z : q.w) >> shr;
            acc = __builtin_fmaf(s * (float)(nib & 15u) - t, xv.x, acc);
            acc = __builtin_fmaf(s * (float)((nib >> 8) & 15u) - t, xv.y, acc);
            acc = __builtin_fmaf(s * (float)((nib >> 16) & 15u) - t, xv.z, acc);
            acc = __builtin_fmaf(s * (float)((nib >> 24) & 15u) - t, xv.w, acc);
        }
    }
    return acc;
}

template <int LMAX, int RT, int KS, int DEPTH>
__global__ void __launch_bounds__(1024) gemv_q4_k_mx_kernel(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            uint64_t* __restrict__ slots, int64_t n, int nb, int L,
                                                            int TR) {
    constexpr int kWaveTab = LMAX * kTabBlock;
    constexpr int kTabAll = kMxMaxWaves * kWaveTab;
    constexpr int kZero = LMAX * kTabBlock;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kTabAll + kZero];
    __shared__ __attribute__((aligned(16))) int etab[kMxMaxWaves * LMAX * kSubTab];
    __shared__ float red[RT * kMxMaxWaves * 64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int64_t wg = blockIdx.x;
    const int half = KS == 2 ? (int)(wg & 1) : 0;
    const int64_t row0 = (KS == 2 ? (wg >> 1) : wg) * TR;
    const int nrows = (int)((n - row0 < TR) ? n - row0 : TR);
    const int TT = (TR + RT - 1) / RT;                  // rows per tile
    const int nbh = KS == 2 ? (nb + 1) / 2 : nb;         // blocks of the first half
    const int kb0 = half ? nbh : 0, nbk = half ? nb - nbh : nbh;
    const int b0 = wave * L;                             // first block of this wave, inside the range
    const int lw = (nbk - b0 < L) ? nbk - b0 : L;        // may be <= 0 for the last waves of a short half
    const int c = lane & 15, g = lane >> 4;
    const uint32_t row_bytes = (uint32_t)nb * kQ4KBytes;
    const auto rs = buffer_rsrc(w + row0 * (int64_t)row_bytes, (uint32_t)nrows * row_bytes);

    // The zero block that the inactive A lanes read is written before any
    // wave reads it. With loads issued one block ahead (DEPTH < LMAX) every
    // wave also issues its x loads before that barrier, so x is requested
    // ahead of the workgroup's weights, and the barrier waits for the LDS
    // writes only (no fence: the x loads stay in flight).
    if constexpr (DEPTH >= LMAX) {
        for (int i = tid; i < kZero / 16; i += blockDim.x)
            reinterpret_cast<uint4*>(lds + kTabAll)[i] = make_uint4(0, 0, 0, 0);
        __syncthreads();
    }

    // x first (small, cache-resident): the digit split then waits for x only,
    // while the weight loads are in flight. Blocks past the wave's slice
    // re-read an earlier block of the row; their sums are dropped.
    float4 xv[LMAX];
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        int blk = kb0 + b0 + (j < lw ? j : lw - 1);
        blk = blk < 0 ? 0 : (blk >= nb ? nb - 1 : blk);
        xv[j] = *reinterpret_cast<const float4*>(x + (int64_t)blk * kQKElems + 4 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DEPTH < LMAX) {
        for (int i = tid; i < kZero / 16; i += blockDim.x)
            reinterpret_cast<uint4*>(lds + kTabAll)[i] = make_uint4(0, 0, 0, 0);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }
    uint4 hd[RT][LMAX], q0[RT][LMAX], q1[RT][LMAX];
    uint32_t roffs[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        int rr = t * TT + (c < TT ? c : TT - 1);         // extra lanes re-read the tile's last row
        rr = rr < nrows ? rr : nrows - 1;
        roffs[t] = (uint32_t)rr * row_bytes;
    }
    // the weight loads of block j for every tile: header, qs 0..63, qs 64..127
    auto issue = [&](auto jc) {
        constexpr int j = decltype(jc)::value;
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            int blk = kb0 + b0 + (j < lw ? j : lw - 1);
            blk = blk < 0 ? 0 : blk;                     // past the row: zeros or a neighbour row, dropped
            const uint32_t off = roffs[t] + (uint32_t)blk * kQ4KBytes;
            hd[t][j] = bload_b128(rs, off);
            q0[t][j] = bload_b128(rs, off + 16 + 16 * g);
            q1[t][j] = bload_b128(rs, off + 80 + 16 * g);
        }
    };
    if constexpr (DEPTH >= LMAX) {
        // every block at once, tile-outer / block-inner (the issue order that measured fastest here)
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int j = 0; j < LMAX; ++j) {
                int blk = kb0 + b0 + (j < lw ? j : lw - 1);
                blk = blk < 0 ? 0 : blk;
                const uint32_t off = roffs[t] + (uint32_t)blk * kQ4KBytes;
                hd[t][j] = bload_b128(rs, off);
                q0[t][j] = bload_b128(rs, off + 16 + 16 * g);
                q1[t][j] = bload_b128(rs, off + 80 + 16 * g);
            }
        }
    } else {
        static_for<0, DEPTH>([&](auto jc) { issue(jc); });
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- x -> digits. Lane t: x[4t .. 4t+3] of the block = sub-block s = t / 8,
    // half h = (t / 4) % 2, bytes 4 (t % 4) .. +3 of the 16-element group.
    // MFMA m = 2 (s / 4) + s % 2 (load s / 4, low or high nibbles) reads the
    // group in k-group kk = 2 ((s / 2) % 2) + h; the 128 bytes of (m, kk) hold
    // its eight digits, digit d in 16-byte slot d ^ (2 kk + m % 2): the 32
    // lanes of a half-wave writing one digit then cover 32 different banks
    // (without the swizzle, 4). The exponent table is ordered [p][position],
    // with p = (s / 2) % 2 and position (s % 2) + 2 (s / 4).
    uint32_t inexact = 0;                                // bit j: block j of this wave is not exact
    {
        const int s = lane >> 3, h = (lane >> 2) & 1;
        const int m = 2 * (s >> 2) + (s & 1), kk = 2 * ((s >> 1) & 1) + h;
        uint8_t* wl = lds + wave * kWaveTab + (m * 4 + kk) * 128 + 4 * (lane & 3);
        const int sw = (2 * kk + (m & 1)) & 7;
        const int pos = (s & 1) + 2 * (s >> 2), pp = (s >> 1) & 1;
        int* we = etab + wave * LMAX * kSubTab + 4 * pp + pos;
#pragma unroll
        for (int j = 0; j < LMAX; ++j) {
            const XSplit dg = x_split(xv[j]);
            uint8_t* p = wl + j * kTabBlock;
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) *reinterpret_cast<uint32_t*>(p + 16 * (dd ^ sw)) = dg.d[dd];
            if ((lane & 7) == 0) we[j * kSubTab] = dg.eo;
            if (__builtin_amdgcn_ballot_w64(!dg.exact) != 0) inexact |= 1u << j;
        }
    }
    // ---- products. Lane (ar = l & 15, akk = l >> 4) of the A operand of
    // MFMA m carries digit ar % 8 of k-group akk when ar / 8 == akk / 2, and
    // zeros otherwise; the digit table and the zero block are read at the
    // same per-MFMA offsets.
    const int ar = lane & 15, akk = lane >> 4;
    // (the digit of row ar sits in slot (ar % 8) ^ (2 akk + m % 2) of (m, akk))
    const bool diag = (ar >> 3) == (akk >> 1);
    const uint8_t* abase_e = diag ? lds + wave * kWaveTab + akk * 128 + ((ar & 7) ^ (2 * akk)) * 16 : lds + kTabAll;
    const uint8_t* abase_o = diag ? lds + wave * kWaveTab + akk * 128 + ((ar & 7) ^ (2 * akk + 1)) * 16
                                  : lds + kTabAll;
    const int p = g >> 1, lev = g & 1;
    const int* eb = etab + wave * LMAX * kSubTab + 4 * p;
    const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    const uint32_t s16 = 16u * (uint32_t)p;
    double acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = 0.0;
    static_for<0, LMAX>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if constexpr (DEPTH < LMAX && j + DEPTH < LMAX) {   // block j + DEPTH's loads before block j's work
            __builtin_amdgcn_sched_barrier(0);
            issue(Int<j + DEPTH>{});
            __builtin_amdgcn_sched_barrier(0);
        }
        if (j >= lw) return;                             // wave-uniform
        if (inexact & (1u << j)) {                       // wave-uniform: per-weight fp32 for this block
            const float* xb = x + (int64_t)(kb0 + b0 + j) * kQKElems;
#pragma unroll
            for (int t = 0; t < RT; ++t) acc[t] += (double)block_per_weight(hd[t][j], q0[t][j], q1[t][j], xb, g);
            return;
        }
        const uint8_t* ab_e = abase_e + j * kTabBlock;
        const uint8_t* ab_o = abase_o + j * kTabBlock;
        const int4 te = *reinterpret_cast<const int4*>(eb + j * kSubTab);          // exponents - 30
        const int el = lev ? -30 : 0;                                              // level 2 carries 2^-30
        double dt[RT], dmt[RT];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            dt[t] = (double)f16_bits_to_f32(hd[t][j].x);
            dmt[t] = (double)f16_bits_to_f32(hd[t][j].x >> 16);
        }
        // MFMA k (0..3): load k / 2, low (k even) or high nibbles; its A operand
        // at ab + 512 k. Lane (c, g) gets, for row c, the four digit sums of
        // level g & 1 of sub-block position k of this lane's group p: sub-blocks
        // [2p, 2p + 1, 4 + 2p, 5 + 2p] (get_scale_min_k4, gguf.py:135-163: with
        // Y, Z, W = bytes 2p, 2p + 1 of scales[0..3], [4..7], [8..11], sc = Y & 63,
        // m = Z & 63 for the first two, sc = (W & 15) | (Y >> 6) << 4,
        // m = (W >> 4) | (Z >> 6) << 4 for the last two).
        static_for<0, 4>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const i32x4 A = *reinterpret_cast<const i32x4*>((k & 1 ? ab_o : ab_e) + 512 * k);
            // sum(m) of this lane's level for the sub-block, exact: the same A
            // against all-ones B (independent of the row, so once per block)
            const i32x4 z = {0, 0, 0, 0};
            const double dx = digit_sum(__builtin_amdgcn_mfma_i32_16x16x64_i8(A, ones, z, 0, 0, 0));
            const int eo = (k == 0 ? te.x : k == 1 ? te.y : k == 2 ? te.z : te.w) + el;
            const double pw = __builtin_ldexp(1.0, eo);
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const uint4 qv = k < 2 ? q0[t][j] : q1[t][j];
                const uint32_t sh = (k & 1) ? 4u : 0u;
                const i32x4 b = {(int)((qv.x >> sh) & 0x0F0F0F0Fu), (int)((qv.y >> sh) & 0x0F0F0F0Fu),
                                 (int)((qv.z >> sh) & 0x0F0F0F0Fu), (int)((qv.w >> sh) & 0x0F0F0F0Fu)};
                const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, b, z, 0, 0, 0);
                const uint4 hdj = hd[t][j];
                uint32_t sc, mn;
                if constexpr (k < 2) {
                    sc = __builtin_amdgcn_ubfe(hdj.y, s16 + 8 * k, 6);
                    mn = __builtin_amdgcn_ubfe(hdj.z, s16 + 8 * k, 6);
                } else {
                    sc = __builtin_amdgcn_ubfe(hdj.w, s16 + 8 * (k - 2), 4) |
                         (__builtin_amdgcn_ubfe(hdj.y, s16 + 8 * (k - 2) + 6, 2) << 4);
                    mn = __builtin_amdgcn_ubfe(hdj.w, s16 + 8 * (k - 2) + 4, 4) |
                         (__builtin_amdgcn_ubfe(hdj.z, s16 + 8 * (k - 2) + 6, 2) << 4);
                }
                acc[t] = sub_block_add(acc[t], dt[t], dmt[t], sc, mn, digit_sum(c), dx, pw);
            }
        });
    });
#pragma unroll
    for (int t = 0; t < RT; ++t) red[(t * kMxMaxWaves + wave) * 64 + lane] = (float)acc[t];
    __syncthreads();
    if (tid < nrows) {
        const int t = tid / TT, cc = tid - t * TT;
        float s = 0.0f;
        for (int wv = 0; wv < nwaves; ++wv) {
            const float* rw = red + (t * kMxMaxWaves + wv) * 64;
            s += (rw[cc] + rw[16 + cc]) + (rw[32 + cc] + rw[48 + cc]);
        }
        if constexpr (KS == 1) {
            y[row0 + tid] = s;
        } else {
            uint64_t* slot = slots + row0 + tid;
            const uint64_t mine = (1ull << 32) | (uint64_t)__float_as_uint(s);
            const uint64_t other = __hip_atomic_exchange(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (other >> 32) {                           // the other half is in: combine and free the slot
                y[row0 + tid] = s + __uint_as_float((uint32_t)other);
                __hip_atomic_store(slot, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// ------------------------------------------------------------------ Q1_0
// Q1_0 GEMV on the matrix cores. A row's block (18 bytes: d f16, 16 bytes of
// sign bits, element e = bit e % 8 of byte e / 8, w = +d if set else -d,
// gguf.py:266-299) contributes d * sum_e (+-x_e). x is written per
// 32-element group of a block as a 30-bit fixed-point number relative to the
// group's largest magnitude (max |x| < 2^e): m = trunc(x 2^(30-e)),
// |m| < 2^30, as four balanced int8 digits. The matrix cores form exactly, in
// int32, for each row, group and digit i,
//     C_i = sum over set bits of digit_i(m)     (sign bits as 0/1 bytes)
//     J_i = sum of digit_i(m)                    (the same A against all-ones B)
// and the lane forms S = sum_i 256^i (2 C_i - J_i) = sum_e (+-m_e) as two
// exact int32 halves whose fp32 sum rounds once, then adds
// ldexp(fl(S * d), e - 30) to its fp32 sum. Truncation loses less than
// 2^(e-30) <= 2^-29 max |x_g| per element, at most 2^-24 max |x_g| over the
// group, and every weight has |w| = |d|, so each group is within 2^-24 of
// its own sum |w_e x_e|; with the fp32 roundings each row keeps
//     |y - y_exact| <= c * 2^-24 * sum_j |w_j x_j|.
// A block whose x holds an inf or a NaN is summed weight by weight in fp32
// (fma(+-d, x_e, acc), the dequant's weights), so those propagate.
//
// Mapping. A workgroup owns TR <= 16 rows (the MFMA's 16 columns) and all of
// k; wave v owns blocks [vL, vL + L). Lane (c, g) (c = l & 15, g = l >> 4)
// loads sign-bit dword g of row c's blocks: elements 32g .. 32g + 31, byte cc
// holding elements 32g + 8cc + j. Its B operand for MFMA h (0, 1) is the four
// dwords (bits >> (4h + jj)) & 0x01010101, jj = 0..3, so byte 4jj + cc is
// element 32g + 8cc + 4h + jj. A is block diagonal: row 4g + i carries digit
// i of the same elements of group g and zeros elsewhere, so lane (c, g) of
// the result receives, for row c, the four digit sums of its own group; it
// keeps its blocks' sum in one register. The digit table is wave-private LDS
// (LDS operations of one wave complete in order, so no barrier is needed
// between a wave's table writes and its reads); one workgroup barrier
// precedes the per-row reduction over waves and groups, in a fixed order.
constexpr int kQ10MxWaves = 16;
constexpr int kQ10MxMaxL = 8;       // blocks per wave
constexpr int kQ10TabBlock = 512;   // digit bytes per block: 2 MFMAs x 4 groups x 4 digits x 16

template <int L>
__global__ void __launch_bounds__(1024) gemv_q1_0_mx_kernel(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int64_t n, int nb, int TR) {
    constexpr int kWaveTab = L * kQ10TabBlock + 16;   // the wave's blocks, then 16 zero bytes
    __shared__ __attribute__((aligned(16))) uint8_t lds[kQ10MxWaves * kWaveTab];
    __shared__ int etab[kQ10MxWaves * L * 4];
    __shared__ float red[kQ10MxWaves * 16];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nwaves = blockDim.x >> 6;
    const int64_t row0 = (int64_t)blockIdx.x * TR;
    const int nrows = (int)((n - row0 < TR) ? n - row0 : TR);
    const int b0 = wave * L;
    const int lw = (nb - b0 < L) ? nb - b0 : L;         // >= 1: nwaves = ceil(nb / L)
    const int c = lane & 15, g = lane >> 4;
    const uint32_t row_bytes = (uint32_t)nb * kQ10Bytes;
    const auto rs = buffer_rsrc(w + row0 * (int64_t)row_bytes, (uint32_t)nrows * row_bytes);
    uint8_t* tab = lds + wave * kWaveTab;

    // x first (small, cache-resident), then every weight load. Set s of the
    // wave (4 elements): block s / 32, group (s / 8) % 4, h = (s / 4) % 2,
    // jj = s % 4, elements 32g + 4h + jj + {0, 8, 16, 24}; lane t owns sets
    // t + 64i (with L = 1 lanes 32..63 repeat lanes 0..31 and write nothing).
    constexpr int kSets = L >= 2 ? L / 2 : 1;
    float xv[kSets][4];
    {
        const auto xs = buffer_rsrc(x, (uint32_t)nb * kQ10Elems * 4u);
#pragma unroll
        for (int i = 0; i < kSets; ++i) {
            const int s = L == 1 ? (lane & 31) : lane + 64 * i;
            const int jb = s >> 5, gg = (s >> 3) & 3, h = (s >> 2) & 1, jj = s & 3;
            const uint32_t blk = (uint32_t)(b0 + (jb < lw ? jb : lw - 1));
            const uint32_t o = 4u * (__umul24(blk, kQ10Elems) + 32 * gg + 4 * h + jj);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                xv[i][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(xs, (int)(o + 32 * q), 0, 0));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t wlo[L], whi[L], wd[L], wsh[L];
    {
        const uint32_t rofs = (uint32_t)(c < nrows ? c : nrows - 1) * row_bytes;   // extra lanes re-read a row
#pragma unroll
        for (int j = 0; j < L; ++j) {
            const uint32_t blk = (uint32_t)(b0 + (j < lw ? j : lw - 1));
            const uint32_t at = __umul24(blk, kQ10Bytes) + 2 + 4 * g;   // this lane's sign-bit dword
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)(rofs + (at & ~3u)), 0, 0);
            wlo[j] = v[0];
            whi[j] = v[1];
            wsh[j] = 8u * (at & 3u);
            wd[j] = bload_u16(rs, rofs + __umul24(blk, kQ10Bytes));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- x -> digits into the wave's table: 64 bytes per (block, h, group),
    // digit d in its 16-byte slot d ^ (2h + group / 2), dword jj of the slot.
    // The swizzle puts the 32 lanes of a half-wave's write (h, group, jj) on
    // 32 different banks; a reader's 16 bytes stay contiguous.
    if (lane < 4) reinterpret_cast<uint32_t*>(tab + L * kQ10TabBlock)[lane] = 0u;
    uint32_t inexact = 0;                                // bit j: block j holds an inf or a NaN
#pragma unroll
    for (int i = 0; i < kSets; ++i) {
        const int s = L == 1 ? (lane & 31) : lane + 64 * i;
        const int jb = s >> 5, gg = (s >> 3) & 3, h = (s >> 2) & 1, jj = s & 3;
        uint32_t mx = 0;                                 // max |x| as bits; >= 0x7F800000 for inf / NaN
#pragma unroll
        for (int q = 0; q < 4; ++q) mx = max(mx, __float_as_uint(xv[i][q]) & 0x7FFFFFFFu);
        mx = max(mx, dpp_u<0xB1>(mx));                   // quad_perm [1,0,3,2]
        mx = max(mx, dpp_u<0x4E>(mx));                   // quad_perm [2,3,0,1]
        mx = max(mx, dpp_u<0x141>(mx));                  // row_half_mirror: the group's 8 lanes
        const bool bad = mx >= 0x7F800000u;
        const int e = bad ? 0 : __builtin_amdgcn_frexp_expf(__uint_as_float(mx));
        int m[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) m[q] = cvt_i32_sat(__builtin_ldexpf(xv[i][q], 30 - e));
        uint32_t dg[4];
        balanced_digits(m[0], m[1], m[2], m[3], dg);
        if (L > 1 || lane < 32) {
            uint8_t* p = tab + ((jb * 2 + h) * 4 + gg) * 64 + 4 * jj;
            const int t = 2 * h + (gg >> 1);
#pragma unroll
            for (int d = 0; d < 4; ++d) *reinterpret_cast<uint32_t*>(p + 16 * (d ^ t)) = dg[d];
            if ((s & 7) == 0) etab[(wave * L + jb) * 4 + gg] = e - 30;
        }
        const uint64_t bl = __builtin_amdgcn_ballot_w64(bad);
        if constexpr (L == 1) {
            if (bl) inexact |= 1u;
        } else {
            if (bl & 0xFFFFFFFFull) inexact |= 1u << (2 * i);
            if (bl >> 32) inexact |= 1u << (2 * i + 1);
        }
    }
    __asm__ volatile("" ::: "memory");                   // table writes stay before the reads

    // ---- products. Lane (ar = l & 15, akk = l >> 4) of A carries digit ar % 4
    // of group akk when ar / 4 == akk, else the zero bytes. Every block's A
    // operands and exponents are read at once, and the blocks run without
    // branches (a block past the wave's range gets d = 0), so their LDS
    // reads, MFMAs and epilogues overlap.
    const int ar = lane & 15, akk = lane >> 4;
    const bool diag = (ar >> 2) == akk;
    const uint8_t* zero = tab + L * kQ10TabBlock;
    const uint8_t* abase0 = diag ? tab + akk * 64 + ((ar & 3) ^ (akk >> 1)) * 16 : zero;
    const uint8_t* abase1 = diag ? tab + 256 + akk * 64 + ((ar & 3) ^ (2 + (akk >> 1))) * 16 : zero;
    const uint32_t astep = diag ? 512u : 0u;            // per block
    float acc = 0.0f;
    if (inexact == 0) {                                  // wave-uniform
        const i32x4 ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
        const i32x4 z = {0, 0, 0, 0};
        constexpr uint32_t M = 0x01010101u;
        i32x4 A[L][2];
        int eo[L];
#pragma unroll
        for (int j = 0; j < L; ++j) {
            A[j][0] = *reinterpret_cast<const i32x4*>(abase0 + j * astep);
            A[j][1] = *reinterpret_cast<const i32x4*>(abase1 + j * astep);
            eo[j] = etab[(wave * L + j) * 4 + g];
        }
#pragma unroll
        for (int j = 0; j < L; ++j) {
            const uint32_t bits = __builtin_amdgcn_alignbit(whi[j], wlo[j], wsh[j]);
            const float d = j < lw ? f16_bits_to_f32(wd[j]) : 0.0f;
            const i32x4 B0 = {(int)(bits & M), (int)((bits >> 1) & M), (int)((bits >> 2) & M),
                              (int)((bits >> 3) & M)};
            const i32x4 B1 = {(int)((bits >> 4) & M), (int)((bits >> 5) & M), (int)((bits >> 6) & M),
                              (int)((bits >> 7) & M)};
            i32x4 C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[j][0], B0, z, 0, 0, 0);
            C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[j][1], B1, C, 0, 0, 0);
            i32x4 J = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[j][0], ones, z, 0, 0, 0);
            J = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[j][1], ones, J, 0, 0, 0);
            // |C_i|, |J_i| <= 32 * 128: both halves below 2^22, exact in fp32
            const int p01 = 2 * ((C[1] << 8) + C[0]) - ((J[1] << 8) + J[0]);
            const int p23 = 2 * ((C[3] << 8) + C[2]) - ((J[3] << 8) + J[2]);
            const float v = __builtin_fmaf((float)p23, 65536.0f, (float)p01);
            acc += __builtin_ldexpf(v * d, eo[j]);
        }
    } else {                                             // an inf or NaN in the wave's x: weight by weight
        for (int j = 0; j < lw; ++j) {
            const uint32_t bits = __builtin_amdgcn_alignbit(whi[j], wlo[j], wsh[j]);
            const float d = f16_bits_to_f32(wd[j]);
            const float* xg = x + (int64_t)(b0 + j) * kQ10Elems + 32 * g;
            float sacc = 0.0f;
#pragma unroll 1
            for (int e = 0; e < 32; ++e) sacc = __builtin_fmaf(((bits >> e) & 1u) ? d : -d, xg[e], sacc);
            acc += sacc;
        }
    }
    // row c: (g0 + g1) + (g2 + g3) in the wave, then the waves in order
    acc += __shfl_xor(acc, 16, 64);
    acc += __shfl_xor(acc, 32, 64);
    if (lane < 16) red[wave * 16 + lane] = acc;
    __syncthreads();
    if (tid < nrows) {
        float s = 0.0f;
        for (int wv = 0; wv < nwaves; ++wv) s += red[wv * 16 + tid];
        y[row0 + tid] = s;
    }
}

template <int LMAX, int RT, int KS>
void mx_go(bool ahead, dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y, uint64_t* slots,
           int64_t n, int nb, int L, int TR) {
    if constexpr (LMAX > 1) {
        if (ahead) {
            gemv_q4_k_mx_kernel<LMAX, RT, KS, 1><<<gd, bd, 0, s>>>(w, x, y, slots, n, nb, L, TR);
            return;
        }
    }
    gemv_q4_k_mx_kernel<LMAX, RT, KS, LMAX><<<gd, bd, 0, s>>>(w, x, y, slots, n, nb, L, TR);
}

template <int RT, int KS>
bool mx_by_l(int L, bool ahead, dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y,
             uint64_t* slots, int64_t n, int nb, int TR) {
    switch (L) {
        case 1: mx_go<1, RT, KS>(ahead, gd, bd, s, w, x, y, slots, n, nb, L, TR); return true;
        case 2: mx_go<2, RT, KS>(ahead, gd, bd, s, w, x, y, slots, n, nb, L, TR); return true;
        case 3: mx_go<3, RT, KS>(ahead, gd, bd, s, w, x, y, slots, n, nb, L, TR); return true;
        case 4:
            if constexpr (RT == 1) {   // two tiles of four blocks do not fit 128 VGPRs (plan_gemv_mx)
                mx_go<4, RT, KS>(ahead, gd, bd, s, w, x, y, slots, n, nb, L, TR);
                return true;
            }
            return false;
        default: return false;
    }
}

}  // namespace

bool plan_gemv_mx(int64_t n, int64_t k, MxPlan* p) {
    if (n <= 0 || k <= 0 || k % kQKElems) return false;
    const int64_t nb = k / kQKElems;
    if (p->ksplit <= 0) p->ksplit = (nb > kMxMaxWaves * kMxMaxL || (n <= 4096 && nb >= 32)) ? 2 : 1;
    if (p->ksplit != 1 && p->ksplit != 2) return false;
    if (p->ksplit == 2 && nb < 2) return false;
    const int64_t nbh = (nb + p->ksplit - 1) / p->ksplit;
    if (nbh > kMxMaxWaves * kMxMaxL) return false;
    p->blocks = (int)((nbh + kMxMaxWaves - 1) / kMxMaxWaves);
    p->waves = (int)((nbh + p->blocks - 1) / p->blocks);
    // two tiles hold 2 x 3 x 16 B of weights per block in registers: at most
    // 3 blocks per wave, so the kernel stays within 128 VGPRs
    if (p->tiles <= 0) p->tiles = ((p->ksplit == 2 || n >= 7168) && p->blocks <= 3) ? 2 : 1;
    if (p->tiles != 1 && (p->tiles != 2 || p->blocks > 3)) return false;
    if (p->rows <= 0) {
        // rows per workgroup: whole rounds of 256 workgroups (one per CU),
        // r rounds of ceil(n / (256 r / KS)) <= 16 RT rows
        const int64_t cap = 16 * p->tiles, per_round = 256 / p->ksplit;
        const int64_t r = (n + cap * per_round - 1) / (cap * per_round);
        p->rows = (int)((n + per_round * r - 1) / (per_round * r));
        if (p->tiles == 2 && p->rows < 2) p->rows = 2;
    }
    if (p->rows < 1 || p->rows > 16 * p->tiles || (p->tiles == 2 && p->rows < 2)) return false;
    // load depth: every block's weight loads issued before the x split, or
    // one block ahead of the products (the x of every wave requested before
    // the workgroup's weights). Graph-replayed, us, all loads / one ahead:
    // 3584 x 18944 12.76 / 12.45, 5120 x 13824 20.8 / 19.0, 3584 x 3584
    // 4.74 / 4.63, 8192 x 11008 14.6 / 15.3: ahead when a wave holds three
    // or more blocks of a half row, or of a one-tile row set.
    if (p->depth <= 0) p->depth = (p->blocks >= 3 && (p->ksplit == 2 || p->tiles == 1)) ? 1 : p->blocks;
    if (p->depth > p->blocks) p->depth = p->blocks;
    if (p->depth != 1 && p->depth != p->blocks) return false;
    p->grid = (n + p->rows - 1) / p->rows * p->ksplit;
    return p->grid <= 0x7FFFFFFF;
}

size_t gemv_mx_slot_bytes(const MxPlan& p, int64_t n) {
    return p.ksplit == 2 ? (size_t)n * sizeof(uint64_t) : 0;
}

bool gemv_mx_eligible(int qtype, const uint8_t* w, const float* x, int64_t n, int64_t k) {
    // Q4_K with enough rows per workgroup to amortise the per-workgroup x
    // split (n > 1280); longer rows than two halves of 64 blocks take the
    // element-wise / split-K kernels.
    if (qtype != kTypeQ4K || n <= 1280 || k <= 0 || k % kQKElems) return false;
    if ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15) return false;
    MxPlan p;
    return plan_gemv_mx(n, k, &p);
}

bool gemv_mx_default(int qtype, const uint8_t* w, const float* x, int64_t n, int64_t k) {
    // The matrix cores against the element-wise fp32 kernel, same process,
    // graph-replayed (us, matrix cores / element-wise): they win by 5 % or
    // more only where every row is whole in one workgroup and one round of
    // at most 256 workgroups covers the rows:
    //   one round, whole rows: 4096x4096 4.91 / 5.18, 8192x4096 6.69 / 7.25,
    //     3584x3584 4.69 / 4.99, 8192x11008 14.29 / 15.98;
    //   several rounds: 14336x4096 9.48 / 9.68, 8960x1536 5.47 / 5.64,
    //     18944x3584 11.73 / 11.43, 5120x13824 18.02 / 16.59;
    //   halves of rows: 3584x18944 12.18 / 12.29, 4096x14336 11.17 / 10.68,
    //     2048x8192 6.38 / 5.33, 1536x8960 7.45 / 6.12.
    // Elsewhere the element-wise kernel is the default.
    if (!gemv_mx_eligible(qtype, w, x, n, k)) return false;
    MxPlan p;
    plan_gemv_mx(n, k, &p);
    return p.ksplit == 1 && p.grid <= 256;
}

hipError_t launch_gemv_mx(const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, const MxPlan& p,
                          uint64_t* slots, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (k <= 0 || k % kQKElems) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15) return hipErrorInvalidValue;
    if (p.ksplit == 2 && !slots) return hipErrorInvalidValue;
    const int nb = (int)(k / kQKElems);
    const dim3 g((unsigned)p.grid), b(64 * p.waves);
    bool ok = false;
    const bool ahead = p.depth < p.blocks;
    if (p.ksplit == 1)
        ok = p.tiles == 1 ? mx_by_l<1, 1>(p.blocks, ahead, g, b, stream, w, x, y, slots, n, nb, p.rows)
                          : mx_by_l<2, 1>(p.blocks, ahead, g, b, stream, w, x, y, slots, n, nb, p.rows);
    else
        ok = p.tiles == 1 ? mx_by_l<1, 2>(p.blocks, ahead, g, b, stream, w, x, y, slots, n, nb, p.rows)
                          : mx_by_l<2, 2>(p.blocks, ahead, g, b, stream, w, x, y, slots, n, nb, p.rows);
    if (!ok) return hipErrorInvalidConfiguration;
    return hipGetLastError();
}

bool gemv_q10_mx_ok(const uint8_t* w, int64_t k) {
    if (k <= 0 || k % kQ10Elems) return false;
    const int64_t nb = k / kQ10Elems;
    // 4-byte aligned sign-bit windows: an aligned base and an even block count
    return (reinterpret_cast<uintptr_t>(w) & 3) == 0 && nb % 2 == 0 && nb <= kQ10MxWaves * kQ10MxMaxL;
}

bool gemv_q10_mx_default(const uint8_t* w, int64_t n, int64_t k) {
    // Measured against the element-wise ring kernel (graph-replayed launches):
    // the matrix cores win while one round of workgroups covers the rows and
    // each workgroup's x split stays short (k <= 4096): 4096 x 4096 4.17 vs
    // 4.76 us, 3072 x 4096 3.94 vs 5.30, 4096 x 1024 2.79 vs 3.64,
    // 6144 x 2048 4.00 vs 4.53. They lose for k = 8192 (4096 x 8192 6.52 vs
    // 6.49, 1024 x 8192 4.89 vs 3.66), below ~1024 rows (512 x 4096 3.42 vs
    // 3.04) and for several rounds at k = 4096 (14336 x 4096 8.6 vs 7.5).
    if (!gemv_q10_mx_ok(w, k) || n < 1024) return false;
    const int64_t nb = k / kQ10Elems;
    return nb <= 32 && (n <= 4096 || (nb <= 16 && n <= 6144));
}

bool plan_gemv_q10_mx(int64_t n, int64_t k, int* L, int* TR) {
    if (n <= 0 || k <= 0 || k % kQ10Elems) return false;
    const int64_t nb = k / kQ10Elems;
    if (*L <= 0) {
        *L = 2;
        while (*L < kQ10MxMaxL && (nb + *L - 1) / *L > 8) *L *= 2;
    }
    if (*L != 1 && *L != 2 && *L != 4 && *L != 8) return false;
    if ((nb + *L - 1) / *L > kQ10MxWaves) return false;
    if (*TR <= 0) {
        const int64_t t = (n + 255) / 256;             // one round of 256 workgroups while rows allow
        *TR = (int)(t > 16 ? 16 : t);
    }
    return *TR >= 1 && *TR <= 16;
}

hipError_t launch_gemv_q10_mx(const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int L, int TR,
                              hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (!gemv_q10_mx_ok(w, k)) return hipErrorInvalidValue;
    if (L <= 0 || TR <= 0 || !plan_gemv_q10_mx(n, k, &L, &TR)) return hipErrorInvalidConfiguration;
    const int nb = (int)(k / kQ10Elems);
    const int64_t grid = (n + TR - 1) / TR;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * ((nb + L - 1) / L)));
    switch (L) {
        case 1: gemv_q1_0_mx_kernel<1><<<gd, bd, 0, stream>>>(w, x, y, n, nb, TR); break;
        case 2: gemv_q1_0_mx_kernel<2><<<gd, bd, 0, stream>>>(w, x, y, n, nb, TR); break;
        case 4: gemv_q1_0_mx_kernel<4><<<gd, bd, 0, stream>>>(w, x, y, n, nb, TR); break;
        case 8: gemv_q1_0_mx_kernel<8><<<gd, bd, 0, stream>>>(w, x, y, n, nb, TR); break;
        default: return hipErrorInvalidConfiguration;
    }
    return hipGetLastError();
}

}  // namespace frq
