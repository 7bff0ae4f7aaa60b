// One lane's share of one weight row for the Q6_K and Q8_0 register-ring
// kernels, against M rows of x: the loads of a row (aligned windows of a
// 4-byte aligned row, funnel-shifted into place) and the per-lane partial
// sums, one per row of x. The single-row ring kernels (frq_gemv.hip) use
// M = 1 and the small-M kernels (frq_gemv_mr.hip) M = 2, 3, so every row of
// x gets exactly the operations of a single-row call.
#pragma once

#include "frq_common.h"

namespace frq {

// Eight int8 (bytes of a, then of b) as float: one sign-extending
// byte-select convert each.
__device__ __forceinline__ void sbytes8(uint32_t a, uint32_t b, float (&f)[8]) {
    asm("v_cvt_f32_i32_sdwa %0, sext(%8) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f32_i32_sdwa %1, sext(%8) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f32_i32_sdwa %2, sext(%8) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f32_i32_sdwa %3, sext(%8) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3\n\t"
        "v_cvt_f32_i32_sdwa %4, sext(%9) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f32_i32_sdwa %5, sext(%9) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f32_i32_sdwa %6, sext(%9) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f32_i32_sdwa %7, sext(%9) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]), "=&v"(f[6]), "=&v"(f[7])
        : "v"(a), "v"(b));
}

// Q6_K (gguf.py:365-420). Lane (block b, sub = 0..7): half h = sub / 4 of the
// block and l = l0 .. l0 + 7 with l0 = 8 (sub % 4), i.e. the 32 elements
// 128h + 32k + l (k = 0..3). Each 8-byte field (ql, ql + 32, qh, scales) is
// read as the three aligned dwords around it: even blocks read [f, f + 12),
// at most 2 bytes into the next block (which exists when the row's block
// count is even), odd blocks [f - 2, f + 10), whose first 2 bytes are the
// previous block's; v_alignbit by 0 or 16 bits extracts the field, so every
// lane runs the same loads.
struct Q6RingRow {
    uint32_t ql0[3], ql1[3], qh[3], sc[3];
    uint32_t d;
};

struct Q6RingLane {
    uint32_t o_ql0, o_ql1, o_qh, o_sc, o_d, sh;
    int h, l0, s;

    __device__ __forceinline__ Q6RingLane(int blk, int sub) {
        h = sub >> 2;
        l0 = 8 * (sub & 3);
        const int mis = (blk & 1) ? 2 : 0;              // block start mod 4
        sh = 8u * (uint32_t)mis;
        s = (sub & 3) >> 1;                             // l0 / 16
        const uint32_t boff = (uint32_t)(blk * kQ6KBytes);
        o_ql0 = boff + 64 * h + l0 - mis;
        o_ql1 = o_ql0 + 32;
        o_qh = boff + 128 + 32 * h + l0 - mis;
        o_sc = boff + 192 + 8 * h - mis;
        o_d = boff + 208;
    }
    // x[128h + 32k + l0 + i] of one row of x into xv[k][i]
    __device__ __forceinline__ void load_x(const float* __restrict__ xrow, int blk, float (&xv)[4][8]) const {
        const float* xb = xrow + (int64_t)blk * kQKElems + 128 * h + l0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 a = *reinterpret_cast<const float4*>(xb + 32 * k);
            const float4 c = *reinterpret_cast<const float4*>(xb + 32 * k + 4);
            xv[k][0] = a.x; xv[k][1] = a.y; xv[k][2] = a.z; xv[k][3] = a.w;
            xv[k][4] = c.x; xv[k][5] = c.y; xv[k][6] = c.z; xv[k][7] = c.w;
        }
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, Q6RingRow& t) const {
        bload_b96(rs, row_off + o_ql0, t.ql0);
        bload_b96(rs, row_off + o_ql1, t.ql1);
        bload_b96(rs, row_off + o_qh, t.qh);
        bload_b96(rs, row_off + o_sc, t.sc);
        t.d = bload_u16(rs, row_off + o_d);
    }
    // pu[r] = the lane's sum of w * x over its 32 elements for row r of x:
    // per 16-element sub-block k, fp32 sums of code * x (codes 4 (q - 32),
    // exact) then one fma with d * sc / 4 (gguf.py:401-419 values).
    template <int M>
    __device__ __forceinline__ void dot(const Q6RingRow& t, const float (&xv)[M][4][8], float (&pu)[M]) const {
        uint32_t ql0[2], ql1[2], qh[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            ql0[c] = __builtin_amdgcn_alignbit(t.ql0[c + 1], t.ql0[c], sh);
            ql1[c] = __builtin_amdgcn_alignbit(t.ql1[c + 1], t.ql1[c], sh);
            // upper bit of each 2-bit field flipped: the sign of q - 32 (q6_quad_signed)
            qh[c] = __builtin_amdgcn_alignbit(t.qh[c + 1], t.qh[c], sh) ^ 0xAAAAAAAAu;
        }
        const uint32_t sc0 = __builtin_amdgcn_alignbit(t.sc[1], t.sc[0], sh);   // scale bytes 8h .. 8h+3
        const uint32_t sc1 = __builtin_amdgcn_alignbit(t.sc[2], t.sc[1], sh);   // 8h+4 .. 8h+7
        const float d = f16_bits_to_f32(t.d) * 0.25f;     // codes enter as 4 (q - 32)
        // int8 scales sc[8h + s + 2k]: bytes s, s+2 of sc0 (k = 0, 1) and of sc1 (k = 2, 3)
        const float sk[4] = {(float)(int8_t)(sc0 >> (8 * s)), (float)(int8_t)(sc0 >> (8 * s + 16)),
                             (float)(int8_t)(sc1 >> (8 * s)), (float)(int8_t)(sc1 >> (8 * s + 16))};
#pragma unroll
        for (int r = 0; r < M; ++r) pu[r] = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float a0[M], a1[M];
#pragma unroll
            for (int r = 0; r < M; ++r) a0[r] = a1[r] = 0.0f;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t src = (k & 1) ? ql1[c] : ql0[c];
                // bits 2k, 2k+1 of each qh byte -> bits 6, 7; the nibble -> bits 2..5
                const uint32_t hsh = (k == 0) ? (qh[c] << 6) : (k == 1) ? (qh[c] << 4) : (k == 2) ? (qh[c] << 2) : qh[c];
                float f[4];
                q6_quad_signed((k >= 2) ? (src >> 2) : (src << 2), hsh, f);
#pragma unroll
                for (int r = 0; r < M; ++r) {
                    a0[r] = __builtin_fmaf(f[0], xv[r][k][4 * c + 0], a0[r]);
                    a1[r] = __builtin_fmaf(f[1], xv[r][k][4 * c + 1], a1[r]);
                    a0[r] = __builtin_fmaf(f[2], xv[r][k][4 * c + 2], a0[r]);
                    a1[r] = __builtin_fmaf(f[3], xv[r][k][4 * c + 3], a1[r]);
                }
            }
            const float dk = d * sk[k];
#pragma unroll
            for (int r = 0; r < M; ++r) pu[r] = __builtin_fmaf(dk, a0[r] + a1[r], pu[r]);
        }
    }
};

// Q8_0 (gguf.py:112-127, q8_0.h:36-51). Lane (block b, half u = 0, 1) owns
// the 16 int8 at 34b + 2 + 16u. Blocks are 34 bytes, so with a 4-aligned row
// those bytes start at 0 or 2 mod 4: the lane loads the aligned 20-byte
// window and funnel-shifts four dwords out of it.
struct Q8RingRow {
    uint4 q;
    uint32_t q4, d;
};

struct Q8RingLane {
    uint32_t o_win, sh, o_d;
    int u;

    __device__ __forceinline__ Q8RingLane(int blk, int half) {
        u = half;
        const uint32_t at = (uint32_t)(blk * kQ80Bytes + 2 + 16 * u);
        o_win = at & ~3u;
        sh = 8u * (at & 3u);
        o_d = (uint32_t)(blk * kQ80Bytes);
    }
    __device__ __forceinline__ void load_x(const float* __restrict__ xrow, int blk, float (&xv)[16]) const {
        const float* xb = xrow + (int64_t)blk * kQ80Elems + 16 * u;
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(xb + i);
            xv[i] = a.x; xv[i + 1] = a.y; xv[i + 2] = a.z; xv[i + 3] = a.w;
        }
    }
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, uint32_t row_off, Q8RingRow& t) const {
        t.q = bload_b128(rs, row_off + o_win);
        t.q4 = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(row_off + o_win + 16), 0, 0);
        t.d = bload_u16(rs, row_off + o_d);
    }
    // pu[r] = d * (sum of q * x over the lane's 16 elements) for row r of x:
    // four fp32 chains of exact int8 * x products, then the block scale.
    template <int M>
    __device__ __forceinline__ void dot(const Q8RingRow& t, const float (&xv)[M][16], float (&pu)[M]) const {
        const uint32_t w5[5] = {t.q.x, t.q.y, t.q.z, t.q.w, t.q4};
        uint32_t qd[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) qd[c] = __builtin_amdgcn_alignbit(w5[c + 1], w5[c], sh);
        const float d = f16_bits_to_f32(t.d);
        float a0[M], a1[M], a2[M], a3[M];
#pragma unroll
        for (int r = 0; r < M; ++r) a0[r] = a1[r] = a2[r] = a3[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c += 2) {
            float f[8];
            sbytes8(qd[c], qd[c + 1], f);
#pragma unroll
            for (int r = 0; r < M; ++r) {
                a0[r] = __builtin_fmaf(f[0], xv[r][4 * c + 0], a0[r]);
                a1[r] = __builtin_fmaf(f[1], xv[r][4 * c + 1], a1[r]);
                a2[r] = __builtin_fmaf(f[2], xv[r][4 * c + 2], a2[r]);
                a3[r] = __builtin_fmaf(f[3], xv[r][4 * c + 3], a3[r]);
                a0[r] = __builtin_fmaf(f[4], xv[r][4 * c + 4], a0[r]);
                a1[r] = __builtin_fmaf(f[5], xv[r][4 * c + 5], a1[r]);
                a2[r] = __builtin_fmaf(f[6], xv[r][4 * c + 6], a2[r]);
                a3[r] = __builtin_fmaf(f[7], xv[r][4 * c + 7], a3[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < M; ++r) pu[r] = d * ((a0[r] + a1[r]) + (a2[r] + a3[r]));
    }
};

}  // namespace frq
