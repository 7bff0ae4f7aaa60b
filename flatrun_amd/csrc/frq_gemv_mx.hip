// Q4_K GEMV, batch 1, with the products on the matrix cores
// (v_mfma_i32_16x16x64_i8): y[i] = sum_j w[i, j] x[j], the reference's
// matmul_q4_k (q4_k.h:427-449) over rows of 256-element blocks
// [d f16][dmin f16][scales 12][qs 128] (gguf.py:192-219).
//
// Arithmetic. Within a 32-element sub-block s of a block, w = d*sc_s*q - dmin*m_s
// with q in 0..15, so a row's block contributes
//     d*sc_s * sum(q x) - dmin*m_s * sum(x)
// per sub-block. x is split once per sub-block into an exponent e (the
// sub-block's max |x| < 2^e) and integers m = trunc(x * 2^(30-e)), |m| < 2^30,
// written as four balanced base-256 digits (int8). The matrix cores form
// sum(q * digit) exactly in int32 for each digit; the epilogue recombines the
// four sums (two exact 24-bit halves, one fp32 rounding), scales by 2^(e-30)
// (exact) and d*sc_s, and subtracts dmin*m_s * sum(x) (sum(x) in fp32, fixed
// order). x enters with 30 bits relative to its sub-block maximum; every
// product q*digit is exact, so the result stays within the fp32 accumulation
// tolerance of the element-wise kernels without matching their bits.
//
// Work mapping. A workgroup owns TR <= 16 output rows and the whole row
// length; wave w owns blocks [w L, w L + L) of every row. Per wave:
//   1. the x of its blocks is loaded first, then 3 x 16 B of every row's
//      block per lane: lane (c = l & 15, g = l >> 4) takes row c's header and
//      qs bytes 16g .. 16g+15 and 64+16g .. 64+16g+15, so that each load
//      instruction reads 64 contiguous bytes of each of its 16 rows;
//   2. the x digits go to a wave-private LDS table (lane t splits x[4t..4t+3]
//      of each block; eight lanes share a sub-block's max and sum via DPP);
//   3. four MFMAs per block, chained in pairs: A = the digits, B = the nibbles
//      as int8. qs bytes 32p .. 32p+31 hold sub-block 2p in their low and
//      2p+1 in their high nibbles, so k-groups 0, 1 of the first load carry
//      sub-blocks 0 (low) and 1 (high), k-groups 2, 3 sub-blocks 2 and 3. A
//      row r of A is nonzero only in the two k-groups of sub-block r / 4, so
//      lane (c, g) receives the digit sums of sub-block g (first pair) and
//      4 + g (second pair); the per-row epilogue applies the scales;
//   4. one LDS reduction over waves and k-groups, in a fixed order.
// No barrier separates the waves between the loads and the reduction: the
// only shared LDS data (a zero block that the inactive A lanes read) is
// written and fenced before the first load.
//
// A Q6_K kernel of the same design follows; frq_dev_gemv does not route to it
// (slower than the element-wise Q6_K ring, see gemv_mx_eligible).
#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kMxMaxL = 5;              // Q4_K blocks per wave: k <= 16 waves x 5 blocks x 256
constexpr int kMxMaxLQ6 = 4;            // Q6_K (21 weight VGPRs per block)
constexpr int kMxLimbBlock = 1024;      // digit bytes per block: 256 x 4
constexpr int kMxTabBlock = 16;         // per block: 8 sub-blocks x (exponent, sum x)

__device__ __forceinline__ uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
    return __builtin_amdgcn_perm(s0, s1, sel);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

// x[4t .. 4t+3] of one 256-element block (lane t of a wave) as digits: d[i]
// packs digit i of the four values in element order; eo = e - 30 for the
// lane's 32-element sub-block (max |x| < 2^e); s16 / s32 = sum of x over the
// lane's 16- / 32-element group, the same fp32 bits in every lane of it.
struct XDigits {
    uint32_t d[4];
    int eo;
    float s16, s32;
};
__device__ __forceinline__ XDigits x_digits(float4 v) {
    XDigits r;
    // max |x| of the four values in two instructions (abs source modifiers;
    // 4 masks + 2 integer maxes otherwise: 0.06 us of the 10.85 us launch at
    // 3584 x 18944). Non-negative fp32 bit patterns order like their values.
    float ma3, ma4;
    asm("v_max3_f32 %0, |%1|, |%2|, |%3|" : "=v"(ma3) : "v"(v.x), "v"(v.y), "v"(v.z));
    asm("v_max_f32_e64 %0, |%1|, %2" : "=v"(ma4) : "v"(v.w), "v"(ma3));
    uint32_t mx = __float_as_uint(ma4);
    mx = max(mx, dpp_u<0xB1>(mx));                 // quad_perm [1,0,3,2]
    mx = max(mx, dpp_u<0x4E>(mx));                 // quad_perm [2,3,0,1]
    mx = max(mx, dpp_u<0x141>(mx));                // row_half_mirror: max over the 8 lanes
    float sx = (v.x + v.y) + (v.z + v.w);
    sx += dpp_mov<0xB1>(sx);
    sx += dpp_mov<0x4E>(sx);
    r.s16 = sx;                                    // 4 lanes = 16 elements
    r.s32 = sx + dpp_mov<0x141>(sx);               // 8 lanes = 32 elements
    const int e = __builtin_amdgcn_frexp_expf(__uint_as_float(mx));   // max |x| < 2^e (0 for 0)
    const int sh = 30 - e;
    // |x| 2^(30-e) < 2^30 for finite x; the clamp (one v_med3) only keeps the
    // conversion defined for inf / NaN, whose sums already make y non-finite
    constexpr float kLim = 1073741824.0f;
    auto digit_int = [&](float a) { return (int)__builtin_amdgcn_fmed3f(__builtin_ldexpf(a, sh), -kLim, kLim); };
    const int m0 = digit_int(v.x), m1 = digit_int(v.y), m2 = digit_int(v.z), m3 = digit_int(v.w);
    // m = sum_i digit_i 256^i with digit_i = byte_i(m + 0x808080) - 128
    // (i < 3) and digit_3 = byte_3(m + 0x808080) as a signed byte
    const uint32_t u0 = (uint32_t)m0 + 0x808080u, u1 = (uint32_t)m1 + 0x808080u;
    const uint32_t u2 = (uint32_t)m2 + 0x808080u, u3 = (uint32_t)m3 + 0x808080u;
    const uint32_t ab_e = perm(u1, u0, 0x06020400u), ab_o = perm(u1, u0, 0x07030501u);
    const uint32_t cd_e = perm(u3, u2, 0x06020400u), cd_o = perm(u3, u2, 0x07030501u);
    r.d[0] = perm(cd_e, ab_e, 0x05040100u) ^ 0x80808080u;
    r.d[1] = perm(cd_o, ab_o, 0x05040100u) ^ 0x80808080u;
    r.d[2] = perm(cd_e, ab_e, 0x07060302u) ^ 0x80808080u;
    r.d[3] = perm(cd_o, ab_o, 0x07060302u);
    r.eo = e - 30;
    return r;
}

// sum(q m) from the four int32 digit sums: (S3 * 256 + S2) * 65536 + (S1 * 256 + S0).
// Q4_K (32 elements, q <= 15): |S_i| <= 61440, both halves exact in fp32.
// Q6_K (16 elements, q <= 63): |S_i| <= 129024, |S3| <= 64512, so the high
// half is exact and the low half (< 2^25) rounds at most once, by 2^(e-29)
// in x units: the order of the digit truncation itself.
__device__ __forceinline__ float digit_sum(i32x4 s) {
    return __builtin_fmaf((float)((s[3] << 8) + s[2]), 65536.0f, (float)((s[1] << 8) + s[0]));
}

template <int LMAX>
__global__ void __launch_bounds__(1024) gemv_q4_k_mx_kernel(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int64_t n, int nb, int L, int TR) {
    constexpr int kWaveLimb = LMAX * kMxLimbBlock;
    constexpr int kLimbAll = 16 * kWaveLimb;
    constexpr int kZero = LMAX * kMxLimbBlock;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLimbAll + kZero];
    __shared__ __attribute__((aligned(16))) float tab[16 * LMAX * kMxTabBlock];
    __shared__ float red[16 * 64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int b0 = wave * L;
    const int lw = (nb - b0 < L) ? nb - b0 : L;   // >= 1: the launch gives every wave a block
    const int64_t row0 = (int64_t)blockIdx.x * TR;
    const int nrows = (int)((n - row0 < TR) ? n - row0 : TR);
    const int c = lane & 15, g = lane >> 4;
    const uint32_t row_bytes = (uint32_t)nb * kQ4KBytes;
    const auto rs = buffer_rsrc(w + row0 * (int64_t)row_bytes, (uint32_t)nrows * row_bytes);
    const uint32_t roff = (uint32_t)(c < nrows ? c : nrows - 1) * row_bytes;   // extra lanes re-read the last row

    for (int i = tid; i < kZero / 16; i += blockDim.x)
        reinterpret_cast<uint4*>(lds + kLimbAll)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();

    // x first (small, cache-resident): the digit split then waits for x only,
    // while every weight load is still in flight. Blocks past the wave's
    // slice (last wave only) re-read its last block; their sums are dropped.
    float4 xv[LMAX];
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const int jj = j < lw ? j : lw - 1;
        xv[j] = *reinterpret_cast<const float4*>(x + (int64_t)(b0 + jj) * kQKElems + 4 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 hd[LMAX], q0[LMAX], q1[LMAX];
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const int jj = j < lw ? j : lw - 1;
        const uint32_t off = roff + (uint32_t)(b0 + jj) * kQ4KBytes;
        hd[j] = bload_b128(rs, off);
        q0[j] = bload_b128(rs, off + 16 + 16 * g);
        q1[j] = bload_b128(rs, off + 80 + 16 * g);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- x -> digits. Lane t: x[4t .. 4t+3] of the block = sub-block s = t / 8,
    // half h = (t / 4) % 2, bytes 4 (t % 4) .. +3 of the 16-element group.
    // MFMA m = 2 (s / 4) + s % 2 (load s / 4, low or high nibbles) reads the
    // group in k-group kk = 2 ((s / 2) % 2) + h; table entry (m, kk) holds
    // 4 digits x 16 bytes. The (exponent, sum) table is ordered [s % 4][s / 4].
    {
        const int s = lane >> 3, h = (lane >> 2) & 1;
        const int m = 2 * (s >> 2) + (s & 1), kk = 2 * ((s >> 1) & 1) + h;
        uint8_t* wl = lds + wave * kWaveLimb + (m * 4 + kk) * 64 + 4 * (lane & 3);
        float* wt = tab + wave * LMAX * kMxTabBlock + 4 * (s & 3) + 2 * (s >> 2);
#pragma unroll
        for (int j = 0; j < LMAX; ++j) {
            const XDigits dg = x_digits(xv[j]);
            uint8_t* p = wl + j * kMxLimbBlock;
            *reinterpret_cast<uint32_t*>(p + 0) = dg.d[0];
            *reinterpret_cast<uint32_t*>(p + 16) = dg.d[1];
            *reinterpret_cast<uint32_t*>(p + 32) = dg.d[2];
            *reinterpret_cast<uint32_t*>(p + 48) = dg.d[3];
            *reinterpret_cast<float2*>(wt + j * kMxTabBlock) = make_float2(__int_as_float(dg.eo), dg.s32);
        }
    }

    // ---- products. A lane of the A operand (row r = l & 15 of A, k-group
    // kk = l >> 4) of MFMA m carries digit r % 4 of its k-group when
    // r / 4 == 2 (kk / 2) + m % 2, and zeros otherwise; the digit table and
    // the zero block are read at the same per-MFMA offsets.
    const int ar = lane & 15, akk = lane >> 4;
    const uint8_t* atab = lds + wave * kWaveLimb + akk * 64 + (ar & 3) * 16;
    const uint8_t* abase_lo = ((ar >> 2) == 2 * (akk >> 1)) ? atab : lds + kLimbAll;       // m = 0, 2
    const uint8_t* abase_hi = ((ar >> 2) == 2 * (akk >> 1) + 1) ? atab : lds + kLimbAll;   // m = 1, 3
    const float* tb = tab + wave * LMAX * kMxTabBlock + 4 * g;
    // sub-blocks g and 4 + g (get_scale_min_k4, gguf.py:135-163): with
    // y, z, w = scales[g], scales[4 + g], scales[8 + g],
    // sc_g = y & 63, m_g = z & 63, sc_4+g = (w & 15) | (y >> 6) << 4,
    // m_4+g = (w >> 4) | (z >> 6) << 4
    const uint32_t sh8 = 8u * (uint32_t)g;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const uint8_t* alo = abase_lo + j * kMxLimbBlock;
        const uint8_t* ahi = abase_hi + j * kMxLimbBlock;
        const i32x4 A0 = *reinterpret_cast<const i32x4*>(alo + 0);     // first load, low nibbles
        const i32x4 A1 = *reinterpret_cast<const i32x4*>(ahi + 256);   // first load, high nibbles
        const i32x4 A2 = *reinterpret_cast<const i32x4*>(alo + 512);   // second load, low nibbles
        const i32x4 A3 = *reinterpret_cast<const i32x4*>(ahi + 768);   // second load, high nibbles
        const uint4 a = q0[j], b = q1[j];
        const i32x4 lo0 = {(int)(a.x & 0x0F0F0F0Fu), (int)(a.y & 0x0F0F0F0Fu), (int)(a.z & 0x0F0F0F0Fu),
                           (int)(a.w & 0x0F0F0F0Fu)};
        const i32x4 lo1 = {(int)(b.x & 0x0F0F0F0Fu), (int)(b.y & 0x0F0F0F0Fu), (int)(b.z & 0x0F0F0F0Fu),
                           (int)(b.w & 0x0F0F0F0Fu)};
        const i32x4 hi0 = {(int)((a.x >> 4) & 0x0F0F0F0Fu), (int)((a.y >> 4) & 0x0F0F0F0Fu),
                           (int)((a.z >> 4) & 0x0F0F0F0Fu), (int)((a.w >> 4) & 0x0F0F0F0Fu)};
        const i32x4 hi1 = {(int)((b.x >> 4) & 0x0F0F0F0Fu), (int)((b.y >> 4) & 0x0F0F0F0Fu),
                           (int)((b.z >> 4) & 0x0F0F0F0Fu), (int)((b.w >> 4) & 0x0F0F0F0Fu)};
        const i32x4 z = {0, 0, 0, 0};
        i32x4 sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, lo0, z, 0, 0, 0);
        sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, hi0, sl, 0, 0, 0);    // sub-block g
        i32x4 sh = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, lo1, z, 0, 0, 0);
        sh = __builtin_amdgcn_mfma_i32_16x16x64_i8(A3, hi1, sh, 0, 0, 0);    // sub-block 4 + g

        const uint4 hdj = hd[j];
        const float d = f16_bits_to_f32(hdj.x), dm = f16_bits_to_f32(hdj.x >> 16);
        const uint32_t yb = (hdj.y >> sh8) & 0xFFu, zb = (hdj.z >> sh8) & 0xFFu, wb = (hdj.w >> sh8) & 0xFFu;
        const float sc0 = (float)(yb & 63u), mn0 = (float)(zb & 63u);
        const float sc1 = (float)((wb & 15u) | ((yb >> 6) << 4)), mn1 = (float)((wb >> 4) | ((zb >> 6) << 4));
        const float4 t = *reinterpret_cast<const float4*>(tb + j * kMxTabBlock);   // sub-blocks g, 4+g: (e - 30, sum x)
        const float vl = digit_sum(sl), vh = digit_sum(sh);
        float part = __builtin_ldexpf(vl, __float_as_int(t.x)) * (d * sc0);
        part = __builtin_fmaf(-(dm * mn0), t.y, part);
        part = __builtin_fmaf(__builtin_ldexpf(vh, __float_as_int(t.z)), d * sc1, part);
        part = __builtin_fmaf(-(dm * mn1), t.w, part);
        acc += (j < lw) ? part : 0.0f;
    }
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (tid < nrows) {
        float s = 0.0f;
        for (int wv = 0; wv < nwaves; ++wv)
            s += (red[wv * 64 + tid] + red[wv * 64 + 16 + tid]) + (red[wv * 64 + 32 + tid] + red[wv * 64 + 48 + tid]);
        y[row0 + tid] = s;
    }
}


// Q6_K: blocks [ql 128][qh 64][scales int8 x16][d f16] (210 B, so only 2-byte
// aligned; the buffer loads below are unaligned, which gfx950 serves exactly).
// Element 128h + 32k + l (h < 2, k < 4, l < 32) is
//     q = (ql[64h + 32 (k & 1) + l] >> 4 (k >> 1)) & 15 | ((qh[32h + l] >> 2k) & 3) << 4
// with scale sc[8h + 2k + l / 16] and w = d * sc * (q - 32) (gguf.py:365-420,
// matmul_q6_k q6_k.h). Lane (c, g) takes ql[64h + 16g .. +16) and
// qh[32h + 16 (g & 1) .. +16) of row c for h = 0, 1: the low nibbles are the
// 16-element sub-block 8h + g, the high nibbles 8h + 4 + g, i.e. element
// chunk 4m + g for MFMA m = 2h + (high). One MFMA per sub-block (16 values of
// q in 0..63 as int8), then d * sc * (sum(q x) - 32 sum(x)).
template <int LMAX>
__global__ void __launch_bounds__(1024) gemv_q6_k_mx_kernel(const uint8_t* __restrict__ w,
                                                            const float* __restrict__ x, float* __restrict__ y,
                                                            int64_t n, int nb, int L, int TR) {
    constexpr int kTab = 32;   // per block: 16 chunks x (exponent, sum x), ordered [g][m]
    constexpr int kWaveLimb = LMAX * kMxLimbBlock;
    constexpr int kLimbAll = 16 * kWaveLimb;
    constexpr int kZero = LMAX * kMxLimbBlock;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLimbAll + kZero];
    __shared__ __attribute__((aligned(16))) float tab[16 * LMAX * kTab];
    __shared__ float red[16 * 64];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int b0 = wave * L;
    const int lw = (nb - b0 < L) ? nb - b0 : L;
    const int64_t row0 = (int64_t)blockIdx.x * TR;
    const int nrows = (int)((n - row0 < TR) ? n - row0 : TR);
    const int c = lane & 15, g = lane >> 4;
    const uint32_t row_bytes = (uint32_t)nb * kQ6KBytes;
    const auto rs = buffer_rsrc(w + row0 * (int64_t)row_bytes, (uint32_t)nrows * row_bytes);
    const uint32_t roff = (uint32_t)(c < nrows ? c : nrows - 1) * row_bytes;

    for (int i = tid; i < kZero / 16; i += blockDim.x)
        reinterpret_cast<uint4*>(lds + kLimbAll)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();

    float4 xv[LMAX];
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const int jj = j < lw ? j : lw - 1;
        xv[j] = *reinterpret_cast<const float4*>(x + (int64_t)(b0 + jj) * kQKElems + 4 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 ql0[LMAX], ql1[LMAX], qh0[LMAX], qh1[LMAX], scv[LMAX];
    uint32_t dd[LMAX];
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const int jj = j < lw ? j : lw - 1;
        const uint32_t off = roff + (uint32_t)(b0 + jj) * kQ6KBytes;
        ql0[j] = bload_b128(rs, off + 16 * g);
        ql1[j] = bload_b128(rs, off + 64 + 16 * g);
        qh0[j] = bload_b128(rs, off + 128 + 16 * (g & 1));
        qh1[j] = bload_b128(rs, off + 160 + 16 * (g & 1));
        scv[j] = bload_b128(rs, off + 192);
        dd[j] = bload_u16(rs, off + 208);
    }
    __builtin_amdgcn_sched_barrier(0);

    {   // x -> digits, in element order: lane t owns chunk t / 4, bytes 4 (t % 4) .. +3
        const int ch = lane >> 2;
        uint8_t* wl = lds + wave * kWaveLimb + ch * 64 + 4 * (lane & 3);
        float* wt = tab + wave * LMAX * kTab + 2 * ((ch & 3) * 4 + (ch >> 2));
#pragma unroll
        for (int j = 0; j < LMAX; ++j) {
            const XDigits dg = x_digits(xv[j]);
            uint8_t* p = wl + j * kMxLimbBlock;
            *reinterpret_cast<uint32_t*>(p + 0) = dg.d[0];
            *reinterpret_cast<uint32_t*>(p + 16) = dg.d[1];
            *reinterpret_cast<uint32_t*>(p + 32) = dg.d[2];
            *reinterpret_cast<uint32_t*>(p + 48) = dg.d[3];
            *reinterpret_cast<float2*>(wt + j * kTab) = make_float2(__int_as_float(dg.eo), dg.s16);
        }
    }

    const bool act = ((lane & 15) >> 2) == (lane >> 4);
    const uint8_t* abase = act ? lds + wave * kWaveLimb + (lane >> 4) * 64 + (lane & 3) * 16 : lds + kLimbAll;
    const float* tb = tab + wave * LMAX * kTab + 8 * g;
    // ((qh >> s) & 3) << 4 = rotr(qh, s - 4) & 0x30303030: s = 2 (g >> 1) for the
    // low nibbles (k = g >> 1), 4 + 2 (g >> 1) for the high nibbles (k = 2 + (g >> 1))
    const uint32_t rlo = (28u + 2u * (uint32_t)(g >> 1)) & 31u, rhi = 2u * (uint32_t)(g >> 1);
    const uint32_t scsh = 8u * (uint32_t)g;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
        const uint8_t* ab = abase + j * kMxLimbBlock;
        i32x4 bl[2], bh[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 ql = h ? ql1[j] : ql0[j], qh = h ? qh1[j] : qh0[j];
            const uint32_t qv[4] = {ql.x, ql.y, ql.z, ql.w}, hv[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo_hi = __builtin_amdgcn_alignbit(hv[i], hv[i], rlo) & 0x30303030u;
                const uint32_t hi_hi = __builtin_amdgcn_alignbit(hv[i], hv[i], rhi) & 0x30303030u;
                bl[h][i] = (int)((qv[i] & 0x0F0F0F0Fu) | lo_hi);
                bh[h][i] = (int)(((qv[i] >> 4) & 0x0F0F0F0Fu) | hi_hi);
            }
        }
        const i32x4 z = {0, 0, 0, 0};
        const i32x4 s0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4*>(ab + 0), bl[0], z, 0, 0, 0);
        const i32x4 s1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4*>(ab + 256), bh[0], z, 0, 0, 0);
        const i32x4 s2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4*>(ab + 512), bl[1], z, 0, 0, 0);
        const i32x4 s3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4*>(ab + 768), bh[1], z, 0, 0, 0);

        const float d = f16_bits_to_f32(dd[j]);
        const uint4 sv = scv[j];   // sub-block 4m + g: byte g of dword m
        // signed byte g of each dword (the builtin's result type is unsigned: cast before converting)
        const float sc0 = (float)(int)__builtin_amdgcn_sbfe(sv.x, scsh, 8);
        const float sc1 = (float)(int)__builtin_amdgcn_sbfe(sv.y, scsh, 8);
        const float sc2 = (float)(int)__builtin_amdgcn_sbfe(sv.z, scsh, 8);
        const float sc3 = (float)(int)__builtin_amdgcn_sbfe(sv.w, scsh, 8);
        const float4 ta = *reinterpret_cast<const float4*>(tb + j * kTab);       // m = 0, 1: (e - 30, sum x)
        const float4 tc = *reinterpret_cast<const float4*>(tb + j * kTab + 4);   // m = 2, 3
        float part = (d * sc0) * __builtin_fmaf(-32.0f, ta.y, __builtin_ldexpf(digit_sum(s0), __float_as_int(ta.x)));
        part = __builtin_fmaf(d * sc1, __builtin_fmaf(-32.0f, ta.w, __builtin_ldexpf(digit_sum(s1), __float_as_int(ta.z))), part);
        part = __builtin_fmaf(d * sc2, __builtin_fmaf(-32.0f, tc.y, __builtin_ldexpf(digit_sum(s2), __float_as_int(tc.x))), part);
        part = __builtin_fmaf(d * sc3, __builtin_fmaf(-32.0f, tc.w, __builtin_ldexpf(digit_sum(s3), __float_as_int(tc.z))), part);
        acc += (j < lw) ? part : 0.0f;
    }
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (tid < nrows) {
        float s = 0.0f;
        for (int wv = 0; wv < nwaves; ++wv)
            s += (red[wv * 64 + tid] + red[wv * 64 + 16 + tid]) + (red[wv * 64 + 32 + tid] + red[wv * 64 + 48 + tid]);
        y[row0 + tid] = s;
    }
}

}  // namespace

int mx_max_blocks(int qtype) { return qtype == kTypeQ6K ? kMxMaxLQ6 : kMxMaxL; }

int gemv_mx_rows(int64_t n) {
    // Rows per workgroup: fill the 256 CUs in whole rounds. r rounds of 256
    // workgroups, r = ceil(n / 4096), each of ceil(n / (256 r)) <= 16 rows.
    if (n <= 0) return 0;
    const int64_t r = (n + 4095) / 4096;
    return (int)((n + 256 * r - 1) / (256 * r));
}

bool gemv_mx_eligible(int qtype, const uint8_t* w, const float* x, int64_t n, int64_t k) {
    // Q4_K only: the Q6_K matrix-core kernel measured slower than the
    // element-wise ring on every shape tried (lm_head 152064 x 3584: 166 vs
    // 109 us; 4096 x 14336: 18.3 vs 14.0 us). Its 210-byte blocks make half of
    // its 16-byte loads unaligned, and a lane fetches 82 bytes per block for
    // 52.5 used (qh and scales are shared by several lanes); the ring reads
    // aligned windows once. It stays reachable through the tuned entry.
    if (qtype != kTypeQ4K || n <= 0 || k <= 0 || k % kQKElems) return false;
    if ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15) return false;
    if (k / kQKElems > 16 * mx_max_blocks(qtype)) return false;
    return gemv_mx_rows(n) >= kMxMinRows;
}

hipError_t launch_gemv_mx(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int rows,
                          hipStream_t stream, int* rows_used) {
    if (n <= 0) return hipSuccess;
    if ((qtype != kTypeQ4K && qtype != kTypeQ6K) || k <= 0 || k % kQKElems) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(x) & 15) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(w) & (qtype == kTypeQ4K ? 15 : 1)) return hipErrorInvalidValue;
    const int64_t nb64 = k / kQKElems;
    if (nb64 > 16 * mx_max_blocks(qtype)) return hipErrorInvalidConfiguration;
    const int nb = (int)nb64;
    if (rows <= 0) rows = gemv_mx_rows(n);
    if (rows < 1 || rows > 16) return hipErrorInvalidConfiguration;
    const int L = (nb + 15) / 16;
    const int nw = (nb + L - 1) / L;   // every wave gets >= 1 block: (nw - 1) L < nb
    const int64_t grid = (n + rows - 1) / rows;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    if (rows_used) *rows_used = rows;
    const dim3 g((unsigned)grid), b(64 * nw);
    if (qtype == kTypeQ6K) {
        switch (L) {
            case 1: gemv_q6_k_mx_kernel<1><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
            case 2: gemv_q6_k_mx_kernel<2><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
            case 3: gemv_q6_k_mx_kernel<3><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
            default: gemv_q6_k_mx_kernel<4><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
        }
        return hipGetLastError();
    }
    switch (L) {
        case 1: gemv_q4_k_mx_kernel<1><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
        case 2: gemv_q4_k_mx_kernel<2><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
        case 3: gemv_q4_k_mx_kernel<3><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
        case 4: gemv_q4_k_mx_kernel<4><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
        default: gemv_q4_k_mx_kernel<5><<<g, b, 0, stream>>>(w, x, y, n, nb, L, rows); break;
    }
    return hipGetLastError();
}

}  // namespace frq
