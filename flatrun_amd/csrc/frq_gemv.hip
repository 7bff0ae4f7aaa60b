// Fused dequant + matvec (GEMV) kernels for gfx950: y[n] = W[n, k] . x[k].
//
// Semantics follow the reference's native matmuls (fp32 in, fp32 out,
// y[i] = sum_j w[i, j] * x[j]): matmul_q4_k q4_k.h:427-449,
// matmul_q6_k q6_k.h:180-201, matmul_q8_0 q8_0.h:187-208; Q5_K and Q1_0
// have no native matmul in the reference and follow its NumPy path
// (dequant @ x, runtime/backend.py:203-213). Accumulation is fp32; the
// order differs from the reference's sequential loop (tolerance contract,
// not bit-exact).
//
// Layout and mapping (all formats):
//   * W is row-major raw GGUF blocks: row i is k/B_elems blocks, contiguous.
//   * A workgroup owns `rows_per_wg` consecutive rows and spans all of k:
//     lane t of the workgroup owns one fixed slice of the k axis (a "work
//     unit" inside block t / LPB) for every row it visits. Its slice of x is
//     loaded once into VGPRs and reused for every row, so x costs no LDS or
//     L1 bandwidth in the row loop; only W streams from HBM.
//   * For each row the lanes of a block read adjacent bytes, so one wave
//     load instruction covers a contiguous span of the row.
//   * Loads for `U` rows are issued before any of them is consumed, to keep
//     enough bytes in flight per wave to cover HBM latency.
//   * Per-row partials are reduced across the wave with DPP, then across the
//     workgroup's waves through LDS in a fixed order (deterministic output).
//   * Every product is w_i x_i with the weight itself: Q4_K / Q5_K form
//     w = fma(s, q, -t) per weight (fl(fl(d*sc)*q - dmin*m): d*sc*q is exact
//     in fp32, so this is the dequantized weight's bits), Q6_K and Q8_0 feed
//     their signed codes (4 (q - 32) and q) and apply the block scale to the
//     sub-block sum. No sum is formed as s * sum(q x) - t * sum(x): with an
//     outlier x_j on a weight where s q_j = t that form cancels two terms of
//     size t |x_j| and loses the bound sum_i |w_i x_i|. Q1_0 sums
//     d * (2 sum_{bit set} x - sum x): its weights are all +-d, so the terms
//     of both sums are within 3 |w_i x_i| and the bound holds.
#include <algorithm>
#include <cstdint>

#include "frq_common.h"
#include "frq_kernels.h"
#include "frq_ringrow.h"

namespace frq {

__device__ __forceinline__ float sbf(uint32_t w, int b) { return (float)(int)(int8_t)((w >> (8 * b)) & 0xFFu); }

// Writes the U row partials of one row batch: wave-reduce each, then either
// store directly (one wave per row) or park the wave's share in LDS.
template <int U>
__device__ __forceinline__ void row_partials_out(const float (&part)[U], int64_t rb, int64_t row0,
                                                 int64_t row_end, float* __restrict__ y,
                                                 float* __restrict__ red, int nwaves, int wave,
                                                 int lane) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const float v = wave_sum(part[u]);
        if (lane == 0 && rb + u < row_end) {
            if (nwaves == 1)
                y[rb + u] = v;
            else
                red[(rb - row0 + u) * nwaves + wave] = v;
        }
    }
}

__device__ __forceinline__ void finish_rows(int64_t row0, int64_t row_end, float* __restrict__ y,
                                            const float* __restrict__ red, int nwaves) {
    if (nwaves == 1) return;
    __syncthreads();
    for (int r = threadIdx.x; r < row_end - row0; r += blockDim.x) {
        float s = 0.0f;
        for (int w = 0; w < nwaves; ++w) s += red[r * nwaves + w];
        y[row0 + r] = s;
    }
}

// ------------------------------------------------------------------ Q4_K
// Work unit: CPL=2 -> one 32-byte qs group g of a block (64 elements,
// 4 lanes per block); CPL=1 -> half a group (16 qs bytes, 32 elements,
// 8 lanes per block). qs byte i of the unit holds element base+i in its low
// nibble and base+32+i in its high nibble (gguf.py:209-219).
//
// Rows stream through a ring of U register slots: each slot is refilled with
// the row U ahead as soon as it has been consumed, so every wave keeps U rows
// of loads in flight (HBM needs ~64 KiB outstanding per CU). The row loop is
// fully unrolled over R rows, so the compiler's s_waitcnt before each slot
// waits for that slot alone (a loop back-edge makes it drain every load).
// There is no per-row guard either:
// every workgroup runs exactly R rows (a skip path would merge a different
// count of outstanding loads into the next row and make its wait drain the
// queue); the last workgroup's rows past n re-read row n-1 and are dropped.
// Each row's lane partials are reduced over 16-lane DPP rows; the four row
// sums per wave collect in LDS and are added in a fixed order when y is
// written once at the end.
//
// Body of one workgroup; `wg` plays the role of blockIdx.x (the grouped
// kernel below passes the index inside its segment). PRIO: row_priority per
// row (wavefronts that are behind issue first). H > 0: two matrices of the
// same shape in one ring of R = 2H rows, rows [wg H, wg H + H) of w (ring
// rows 0 .. H-1, to y) and the same rows of w2 (ring rows H .. 2H-1, to y2),
// so a pair of matrices shares one x load and one unbroken load pipeline;
// thread r then writes both rows r and keeps them in keep[r], keep[H + r].
template <int CPL, int U, int R, bool PRIO = false, int H = 0>
__device__ __forceinline__ void gemv_q4_k_body(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                               float* __restrict__ y, int64_t n, int nb, int64_t wg,
                                               float* keep = nullptr, const uint8_t* __restrict__ w2 = nullptr,
                                               float* __restrict__ y2 = nullptr) {
    static_assert(H == 0 || R == 2 * H, "two matrices: R = 2H");
    static_assert(U <= R, "ring deeper than the row count");
    __shared__ float red[R * 64];                           // [row][wave][DPP row]
    constexpr int LPB = 8 / CPL;
    constexpr int NE = 16 * CPL;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int64_t rb = wg;
    const int blk = tid / LPB, sub = tid % LPB;
    const bool active = blk < nb;
    const int gblk = active ? blk : 0;                      // block index in the row
    const int g = (CPL == 2) ? sub : (sub >> 1);
    const int hh = (CPL == 2) ? 0 : (sub & 1);
    const ScaleDecode dec(g);
    // CPL = 1, scale ownership. The two lanes of group g (hh = 0, 1) are DPP
    // neighbours and read the two halves of the group's 32 qs bytes: plane A
    // (low nibbles) belongs to sub-block 2g, plane B (high nibbles) to 2g + 1.
    // Lane hh decodes only the (sc, m) pair of sub-block 2g + hh and takes
    // the other one's (s, t) from its neighbour with one DPP move each.
    const PairDecode pdec(sub);
    const bool own_hi = CPL == 1 && hh;
    // CPL = 1: codes enter as q * u, u = the value of the fp8 code 1 (a power
    // of two): a nibble below 16 in a byte converts exactly, two per
    // instruction; the scales carry 1 / u so that s' * (q u) = s q exactly.
    const float u_inv = 1.0f / fp8_unit();
    row_priority<PRIO, R, 0>();                             // x and the first rows load at the top priority

    constexpr int RM = H ? H : R;                           // rows per matrix
    const int64_t row0 = rb * RM;
    const int nrows = (int)(n - row0 < RM ? n - row0 : RM);
    const int64_t row_bytes = (int64_t)nb * kQ4KBytes;
    const uint32_t hoff = (uint32_t)gblk * kQ4KBytes;       // lane's block inside a row
    const uint32_t qoff = hoff + 16 + 32 * g + 16 * hh;

    // Loads are unconditional (no control flow around them): rows past the
    // end re-read the last row (cache hits; results not stored), and inactive
    // lanes read block 0 with x zeroed and their partial forced to 0. Each row
    // is one buffer descriptor (wave-uniform, scalar registers) read at the
    // lane's 32-bit offset: no VALU address math per row.
    auto load1 = [&](Q4KRow<CPL>& t, int j) {
        const uint8_t* base = (H && j >= H) ? w2 : w;
        const int jr = (H && j >= H) ? j - H : j;
        const uint8_t* rp = base + (row0 + (jr < nrows ? jr : nrows - 1)) * row_bytes;
        const auto rs = buffer_rsrc(rp, (uint32_t)row_bytes);
        t.hd = bload_b128(rs, hoff);
#pragma unroll
        for (int c = 0; c < CPL; ++c) t.q[c] = bload_b128(rs, qoff + 16 * c);
    };

    float xl[NE], xh[NE];                                   // x of plane A, plane B
    {
        const float* xb = x + (int64_t)gblk * kQKElems + 64 * g + 16 * hh;
        const float* xa = xb + ((CPL == 1) ? 0 : (own_hi ? 32 : 0));
        const float* xo = xb + ((CPL == 1) ? 32 : (own_hi ? 0 : 32));
#pragma unroll
        for (int i = 0; i < NE; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(xa + i);
            const float4 c = *reinterpret_cast<const float4*>(xo + i);
            xl[i] = a.x; xl[i + 1] = a.y; xl[i + 2] = a.z; xl[i + 3] = a.w;
            xh[i] = c.x; xh[i + 1] = c.y; xh[i + 2] = c.z; xh[i + 3] = c.w;
        }
    }
    // x first, then the first U rows: the first use of x waits for x only
    // (in-order vmcnt) and leaves every row load in flight. The barriers keep
    // the scheduler from reordering the phases. Inactive lanes keep block 0's
    // x; their partial is discarded by a select below.
    __builtin_amdgcn_sched_barrier(0);
    Q4KRow<CPL> ring[U];
#pragma unroll
    for (int i = 0; i < U; ++i) load1(ring[i], i);
    __builtin_amdgcn_sched_barrier(0);

    static_for<0, R>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        Q4KRow<CPL>& t = ring[j % U];
        row_priority<PRIO, R, j>();
        // everything read from the slot is read before the slot is refilled
        const float d = f16_bits_to_f32(t.hd.x), dm = f16_bits_to_f32(t.hd.x >> 16);
        // (s, t) of plane A and plane B: w = fma(s, f, -t) per weight (f = q,
        // or 16 q with s pre-divided by 16)
        float sa, ta, sb, tb;
        if constexpr (CPL == 1) {
            uint32_t sc0, m0;
            pdec(t.hd.y, t.hd.z, t.hd.w, sc0, m0);          // this lane's pair 2g + hh
            const float so = (d * u_inv) * (float)sc0, to = dm * (float)m0;
            const float sn = dpp_mov<0xB1>(so), tn = dpp_mov<0xB1>(to);   // the neighbour's pair
            sa = own_hi ? sn : so;                          // plane A: low nibbles, sub-block 2g
            ta = own_hi ? tn : to;
            sb = own_hi ? so : sn;                          // plane B: high nibbles, 2g + 1
            tb = own_hi ? to : tn;
        } else {
            uint32_t sc0, m0, sc1, m1;
            dec(t.hd.y, t.hd.z, t.hd.w, sc0, m0, sc1, m1);
            sa = d * (float)sc0;
            ta = dm * (float)m0;
            sb = (d * 0.0625f) * (float)sc1;
            tb = dm * (float)m1;
        }
        float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t qw[4] = {t.q[c].x, t.q[c].y, t.q[c].z, t.q[c].w};
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                float f[8];                                       // plane A, plane B
                if constexpr (CPL == 1) nibbles8_fp8(qw[wd], f);
                else nibbles8(qw[wd], f);
                const int e = 16 * c + 4 * wd;
                a0 = __builtin_fmaf(__builtin_fmaf(sa, f[0], -ta), xl[e + 0], a0);
                a1 = __builtin_fmaf(__builtin_fmaf(sa, f[1], -ta), xl[e + 1], a1);
                b0 = __builtin_fmaf(__builtin_fmaf(sb, f[4], -tb), xh[e + 0], b0);
                b1 = __builtin_fmaf(__builtin_fmaf(sb, f[5], -tb), xh[e + 1], b1);
                a0 = __builtin_fmaf(__builtin_fmaf(sa, f[2], -ta), xl[e + 2], a0);
                a1 = __builtin_fmaf(__builtin_fmaf(sa, f[3], -ta), xl[e + 3], a1);
                b0 = __builtin_fmaf(__builtin_fmaf(sb, f[6], -tb), xh[e + 2], b0);
                b1 = __builtin_fmaf(__builtin_fmaf(sb, f[7], -tb), xh[e + 3], b1);
            }
        }
        if constexpr (j + U < R) load1(t, j + U);               // refill the slot: row j + U
        const float pu = (a0 + a1) + (b0 + b1);
        // results go to LDS (lgkmcnt): a global store would count in vmcnt
        // and force waits on the in-flight row loads.
        const float v = row16_sum(active ? pu : 0.0f);
        if ((lane & 15) == 15) red[j * 4 * nwaves + 4 * wave + (lane >> 4)] = v;
    });
    __syncthreads();
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        float s = 0.0f;
        for (int w2 = 0; w2 < 4 * nwaves; ++w2) s += red[r * 4 * nwaves + w2];
        y[row0 + r] = s;
        if (keep) keep[r] = s;                              // the caller's LDS copy (fused epilogues)
        if constexpr (H > 0) {                              // the same row of the second matrix
            float s2 = 0.0f;
            for (int w2 = 0; w2 < 4 * nwaves; ++w2) s2 += red[(H + r) * 4 * nwaves + w2];
            y2[row0 + r] = s2;
            if (keep) keep[H + r] = s2;
        }
    }
}

// Row priorities pay from 14 rows per workgroup (3584 x 18944: 12.6 -> 11.9
// us; 28672 x 4096: 16.4 -> 15.8; 4096 x 14336: 10.65 -> 10.2) and cost at
// fewer rows with many workgroups per CU (18944 x 3584 at 8 rows: 12.0 ->
// 12.3; 1024 x 4096 at 4 rows: 3.52 -> 3.58), same process.
template <int CPL, int U, int R>
__global__ void __launch_bounds__(CPL == 1 ? 1024 : 512) __attribute__((amdgpu_waves_per_eu((CPL == 1 && U <= 3) ? 5 : 1)))
gemv_q4_k_kernel(const uint8_t* __restrict__ w, const float* __restrict__ x, float* __restrict__ y, int64_t n, int nb) {
    gemv_q4_k_body<CPL, U, R, (R >= 14)>(w, x, y, n, nb, blockIdx.x);
}

// ------------------------------------------------------------------ Q5_K
// Work unit: one 32-byte qs group g (64 elements, 4 lanes per block). The
// 5th bit of element base+i is bit 2g (low nibble) / 2g+1 (high nibble) of
// qh byte i (gguf.py:252-262).
template <int U>
__global__ void __launch_bounds__(512) gemv_q5_k_kernel(const uint8_t* __restrict__ w,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int64_t n, int nb,
                                                         int rows_per_wg) {
    extern __shared__ float red[];
    constexpr int NE = 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk = tid >> 2, g = tid & 3;
    const bool active = blk < nb;
    const uint32_t rot_lo = (uint32_t)(2 * g + 28) & 31u, rot_hi = (uint32_t)(2 * g + 29) & 31u;

    float xl[NE], xh[NE];
    if (active) {
        const float* xb = x + (int64_t)blk * kQKElems + 64 * g;
#pragma unroll
        for (int i = 0; i < NE; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(xb + i);
            const float4 c = *reinterpret_cast<const float4*>(xb + 32 + i);
            xl[i] = a.x; xl[i + 1] = a.y; xl[i + 2] = a.z; xl[i + 3] = a.w;
            xh[i] = c.x; xh[i + 1] = c.y; xh[i + 2] = c.z; xh[i + 3] = c.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NE; ++i) { xl[i] = 0.0f; xh[i] = 0.0f; }
    }

    const int64_t row0 = (int64_t)blockIdx.x * rows_per_wg;
    const int64_t row_end = row0 + rows_per_wg < n ? row0 + rows_per_wg : n;
    const int64_t row_bytes = (int64_t)nb * kQ5KBytes;
    const uint8_t* wb = w + row0 * row_bytes + (int64_t)blk * kQ5KBytes;

    for (int64_t rb = row0; rb < row_end; rb += U) {
        uint4 hd[U], qh[U][2], qs[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (active && rb + u < row_end) {
                const uint8_t* p = wb + (rb - row0 + u) * row_bytes;
                hd[u] = *reinterpret_cast<const uint4*>(p);
                qh[u][0] = *reinterpret_cast<const uint4*>(p + 16);
                qh[u][1] = *reinterpret_cast<const uint4*>(p + 32);
                qs[u][0] = *reinterpret_cast<const uint4*>(p + 48 + 32 * g);
                qs[u][1] = *reinterpret_cast<const uint4*>(p + 64 + 32 * g);
            } else {
                hd[u] = qh[u][0] = qh[u][1] = qs[u][0] = qs[u][1] = make_uint4(0, 0, 0, 0);
            }
        }
        float part[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint32_t sc0, m0, sc1, m1;
            k4_scale_min(hd[u].y, hd[u].z, hd[u].w, 2 * g, sc0, m0);
            k4_scale_min(hd[u].y, hd[u].z, hd[u].w, 2 * g + 1, sc1, m1);
            const float d = f16_bits_to_f32(hd[u].x), dm = f16_bits_to_f32(hd[u].x >> 16);
            // per weight: w = fma(s, q, -t), q the 5-bit code
            const float s0 = d * (float)sc0, t0 = dm * (float)m0;
            const float s1 = d * (float)sc1, t1 = dm * (float)m1;
            float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t sw[4] = {qs[u][c].x, qs[u][c].y, qs[u][c].z, qs[u][c].w};
                const uint32_t hw[4] = {qh[u][c].x, qh[u][c].y, qh[u][c].z, qh[u][c].w};
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    // 5th bit (bit j of each qh byte) moved to bit 4 of its byte by a
                    // 32-bit rotate right by (j - 4) mod 32: bits that wrap land
                    // outside bit 4 of every byte, so the mask removes them (a plain
                    // shift would push byte 3's high bits out of the dword).
                    const uint32_t hl = __builtin_amdgcn_alignbit(hw[wd], hw[wd], rot_lo);
                    const uint32_t hh = __builtin_amdgcn_alignbit(hw[wd], hw[wd], rot_hi);
                    const uint32_t lo = vand_or(sw[wd], 0x0F0F0F0Fu, vand(hl, 0x10101010u));
                    const uint32_t hi = vand_or(sw[wd] >> 4, 0x0F0F0F0Fu, vand(hh, 0x10101010u));
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
            part[u] = (a0 + a1) + (b0 + b1);
        }
        row_partials_out<U>(part, rb, row0, row_end, y, red, nwaves, wave, lane);
    }
    finish_rows(row0, row_end, y, red, nwaves);
}

// ------------------------------------------------------------------ Q6_K
// Work unit: half h of a block and LQ = 4*CPL consecutive l (l0 = LQ*p),
// which covers elements 128h + 32k + l0 + [0, LQ) for k = 0..3. They need
// ql[64h + l0 ..], ql[64h + 32 + l0 ..], qh[32h + l0 ..] (LQ bytes each) and
// scales sc[8h + l0/16 + 2k] (gguf.py:401-419). Blocks are 210 B, so fields
// are only 2-byte aligned: 4-byte reads go through ld_u32_a2.
template <int CPL, int U>
__global__ void __launch_bounds__(512) gemv_q6_k_kernel(const uint8_t* __restrict__ w,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int64_t n, int nb,
                                                         int rows_per_wg) {
    extern __shared__ float red[];
    constexpr int LQ = 4 * CPL;          // l values per lane
    constexpr int PPH = 32 / LQ;         // lanes per half
    constexpr int LPB = 2 * PPH;         // lanes per block
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk = tid / LPB, sub = tid % LPB;
    const int h = sub / PPH, l0 = LQ * (sub % PPH);
    const bool active = blk < nb;

    float xv[4][LQ];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int i = 0; i < LQ; i += 4) {
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
            if (active) a = *reinterpret_cast<const float4*>(x + (int64_t)blk * kQKElems + 128 * h + 32 * k + l0 + i);
            xv[k][i] = a.x; xv[k][i + 1] = a.y; xv[k][i + 2] = a.z; xv[k][i + 3] = a.w;
        }
    }

    const int64_t row0 = (int64_t)blockIdx.x * rows_per_wg;
    const int64_t row_end = row0 + rows_per_wg < n ? row0 + rows_per_wg : n;
    const int64_t row_bytes = (int64_t)nb * kQ6KBytes;
    const uint8_t* wb = w + row0 * row_bytes + (int64_t)blk * kQ6KBytes;
    const int sidx = l0 >> 4;   // l/16 for this lane's l range

    for (int64_t rb = row0; rb < row_end; rb += U) {
        uint32_t ql0[U][CPL], ql1[U][CPL], qh[U][CPL], sca[U], scb[U], dd[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (active && rb + u < row_end) {
                const uint8_t* p = wb + (rb - row0 + u) * row_bytes;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    ql0[u][c] = ld_u32_a2(p + 64 * h + l0 + 4 * c);
                    ql1[u][c] = ld_u32_a2(p + 64 * h + 32 + l0 + 4 * c);
                    qh[u][c] = ld_u32_a2(p + 128 + 32 * h + l0 + 4 * c);
                }
                sca[u] = ld_u32_a2(p + 192 + 8 * h);
                scb[u] = ld_u32_a2(p + 196 + 8 * h);
                dd[u] = ld_u16(p + 208);
            } else {
#pragma unroll
                for (int c = 0; c < CPL; ++c) ql0[u][c] = ql1[u][c] = qh[u][c] = 0;
                sca[u] = scb[u] = dd[u] = 0;
            }
        }
        float part[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // codes enter as 4 (q - 32) (exact signed bytes): the scale carries 1/4
            const float d = f16_bits_to_f32(dd[u]) * 0.25f;
            const float sk[4] = {sbf(sca[u], sidx), sbf(sca[u], sidx + 2), sbf(scb[u], sidx), sbf(scb[u], sidx + 2)};
            float pu = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    const uint32_t src = (k & 1) ? ql1[u][c] : ql0[u][c];
                    const uint32_t qhx = qh[u][c] ^ 0xAAAAAAAAu;    // upper bit of each 2-bit field flipped
                    // bits 2k, 2k+1 of each qh byte -> bits 6, 7; the nibble -> bits 2..5
                    const uint32_t hsh = (k == 0) ? (qhx << 6) : (k == 1) ? (qhx << 4) : (k == 2) ? (qhx << 2) : qhx;
                    const uint32_t q = vand_or((k >= 2) ? (src >> 2) : (src << 2), 0x3C3C3C3Cu, vand(hsh, 0xC0C0C0C0u));
                    a0 = __builtin_fmaf(sbf(q, 0), xv[k][4 * c + 0], a0);     // 4 (q - 32), signed
                    a1 = __builtin_fmaf(sbf(q, 1), xv[k][4 * c + 1], a1);
                    a0 = __builtin_fmaf(sbf(q, 2), xv[k][4 * c + 2], a0);
                    a1 = __builtin_fmaf(sbf(q, 3), xv[k][4 * c + 3], a1);
                }
                pu = __builtin_fmaf(d * sk[k], a0 + a1, pu);
            }
            part[u] = pu;
        }
        row_partials_out<U>(part, rb, row0, row_end, y, red, nwaves, wave, lane);
    }
    finish_rows(row0, row_end, y, red, nwaves);
}

// Q6_K, register-ring variant (used when the weight base is 4-byte aligned
// and a row has an even number of blocks: every block then starts at 0 or
// 2 mod 4, alternating). Work unit as CPL=2 above: half h of a block and 8
// consecutive l (l0 = 8p), 32 elements; the lane's loads and sums are
// Q6RingLane's (frq_ringrow.h). Rows stream through a ring of U register
// slots, the row loop is unrolled over R rows without guards (as in the Q4_K
// ring kernel), and partials are reduced with DPP into LDS.
template <int U, int R, bool PRIO = false>
__device__ __forceinline__ void gemv_q6_k_ring_body(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                    float* __restrict__ y, int64_t n, int nb, int64_t wg) {
    static_assert(U <= R, "ring deeper than the row count");
    __shared__ float red[R * 64];                           // [row][wave][DPP row]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk_raw = tid >> 3, sub = tid & 7;
    const bool active = blk_raw < nb;
    const int blk = active ? blk_raw : 0;
    const Q6RingLane ln(blk, sub);

    const int64_t row0 = wg * R;
    const int nrows = (int)(n - row0 < R ? n - row0 : R);
    const int64_t row_bytes = (int64_t)nb * kQ6KBytes;

    auto load1 = [&](Q6RingRow& t, int j) {
        const uint8_t* rp = w + (row0 + (j < nrows ? j : nrows - 1)) * row_bytes;
        ln.load(buffer_rsrc(rp, (uint32_t)row_bytes), 0, t);
    };

    float xv[1][4][8];
    row_priority<PRIO, R, 0>();
    ln.load_x(x, blk, xv[0]);
    __builtin_amdgcn_sched_barrier(0);
    Q6RingRow ring[U];
#pragma unroll
    for (int i = 0; i < U; ++i) load1(ring[i], i);
    __builtin_amdgcn_sched_barrier(0);

    static_for<0, R>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        Q6RingRow& t = ring[j % U];
        row_priority<PRIO, R, j>();
        float pu[1];
        ln.dot<1>(t, xv, pu);
        if constexpr (j + U < R) load1(t, j + U);
        __builtin_amdgcn_sched_barrier(0);                  // keep the rows in ring order
        const float v = row16_sum(active ? pu[0] : 0.0f);
        if ((lane & 15) == 15) red[j * 4 * nwaves + 4 * wave + (lane >> 4)] = v;
    });
    __syncthreads();
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        float acc = 0.0f;
        for (int w2 = 0; w2 < 4 * nwaves; ++w2) acc += red[r * 4 * nwaves + w2];
        y[row0 + r] = acc;
    }
}

// PRIO: row priorities, for workgroups of four or more wavefronts (4096 x
// 14336: 13.36 -> 12.83 us); with two-wavefront workgroups, many per CU, they
// cost (lm_head 152064 x 3584: 86.1 -> 93.4 us).
template <int U, int R, bool PRIO>
__global__ void __launch_bounds__(1024) gemv_q6_k_ring_kernel(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, int64_t n, int nb) {
    gemv_q6_k_ring_body<U, R, PRIO>(w, x, y, n, nb, blockIdx.x);
}

// ------------------------------------------------------------------ grouped
// One launch for several weight matrices that multiply the same x (q/k/v,
// gate/up): segment i's rows go to y_i, and segment i owns workgroups
// [wg_begin_i, wg_begin_{i+1}). Every segment has the same k, so one
// workgroup shape (8 lanes per block, all of k) serves both row bodies; the
// segment's format picks the body with a wave-uniform branch. Workgroups of
// a segment do exactly what the single-matrix kernel's workgroups do, so the
// outputs are bit-identical to separate launches (row priorities change the
// order of issue, not the arithmetic).
template <int R>
__global__ void __launch_bounds__(1024) gemv_group_kernel(GemvGroup g, const float* __restrict__ x, int nb) {
    const int64_t b = blockIdx.x;
    int i = 0;
#pragma unroll
    for (int t = 1; t < kGemvGroupMax; ++t)
        if (t < g.count && b >= g.wg_begin[t]) i = t;
    const int64_t wg = b - g.wg_begin[i];
    if (g.qtype[i] == kTypeQ4K)
        gemv_q4_k_body<1, (R < 3 ? R : 3), R, true>(g.w[i], x, g.y[i], g.n[i], nb, wg);
    else
        gemv_q6_k_ring_body<(R < 4 ? R : 4), R, true>(g.w[i], x, g.y[i], g.n[i], nb, wg);
}

// Two Q4_K matrices of the same shape that multiply the same x (gate and up)
// in one launch: workgroup w runs one ring over rows [w R, w R + R) of both
// (gemv_q4_k_body's two-matrix mode), the rows of separate launches bit for
// bit. Against the general grouped kernel, which gives each workgroup rows
// of one matrix, x is loaded once for both.
template <int R>
__global__ void __launch_bounds__(1024) gemv_pair_kernel(const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1,
                                                        const float* __restrict__ x, float* __restrict__ y0,
                                                        float* __restrict__ y1, int64_t n, int nb) {
    gemv_q4_k_body<1, (2 * R < 3 ? 2 * R : 3), 2 * R, (2 * R >= 14), R>(w0, x, y0, n, nb, blockIdx.x, nullptr, w1, y1);
}

// Gate and up of a SwiGLU block in one launch, with the activation:
// workgroup w runs the Q4_K row body once over rows [w R, w R + R) of W_gate
// and the same rows of W_up (one ring of 2R rows, x loaded once), writing both
// to gateup as the grouped launch does (bit-identical rows), and the thread
// that wrote gate and up row r applies act[r] = silu(gate[r]) * up[r] with
// silu_mul's operations. (Two bodies in turn, one per matrix, drained the
// load ring in between and read x twice: 19.3 us against 17.2 for the
// grouped gate|up launch of Llama-3-8B, 14336 x 4096 each.)
template <int R>
__global__ void __launch_bounds__(1024) gemv_swiglu_kernel(const uint8_t* __restrict__ wgate,
                                                          const uint8_t* __restrict__ wup,
                                                          const float* __restrict__ x, float* __restrict__ gateup,
                                                          float* __restrict__ act, int64_t inter, int nb) {
    __shared__ float keep[2 * R];
    const int64_t b = blockIdx.x;
    gemv_q4_k_body<1, (2 * R < 3 ? 2 * R : 3), 2 * R, (2 * R >= 14), R>(wgate, x, gateup, inter, nb, b, keep, wup,
                                                                     gateup + inter);
    const int64_t row0 = b * R;
    const int nrows = (int)(inter - row0 < R ? inter - row0 : R);
    for (int r = threadIdx.x; r < nrows; r += blockDim.x)   // the same thread wrote keep[r] and keep[R + r]
        act[row0 + r] = silu_mul(keep[r], keep[R + r]);
}

// ------------------------------------------------------------------ Q8_0
// Work unit: 8*CPL consecutive int8 of one 34-byte block (32/(8*CPL) lanes
// per block); y = sum_b d_b * sum_i q_i x_i.
template <int CPL, int U>
__global__ void __launch_bounds__(512) gemv_q8_0_kernel(const uint8_t* __restrict__ w,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ y, int64_t n, int nb,
                                                         int rows_per_wg) {
    extern __shared__ float red[];
    constexpr int NE = 8 * CPL;
    constexpr int LPB = 32 / NE;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk = tid / LPB, o = NE * (tid % LPB);
    const bool active = blk < nb;

    float xv[NE];
#pragma unroll
    for (int i = 0; i < NE; i += 4) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        if (active) a = *reinterpret_cast<const float4*>(x + (int64_t)blk * kQ80Elems + o + i);
        xv[i] = a.x; xv[i + 1] = a.y; xv[i + 2] = a.z; xv[i + 3] = a.w;
    }

    const int64_t row0 = (int64_t)blockIdx.x * rows_per_wg;
    const int64_t row_end = row0 + rows_per_wg < n ? row0 + rows_per_wg : n;
    const int64_t row_bytes = (int64_t)nb * kQ80Bytes;
    const uint8_t* wb = w + row0 * row_bytes + (int64_t)blk * kQ80Bytes;

    for (int64_t rb = row0; rb < row_end; rb += U) {
        uint32_t qv[U][NE / 4], dd[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (active && rb + u < row_end) {
                const uint8_t* p = wb + (rb - row0 + u) * row_bytes;
                dd[u] = ld_u16(p);
#pragma unroll
                for (int c = 0; c < NE / 4; ++c) qv[u][c] = ld_u32_a2(p + 2 + o + 4 * c);
            } else {
                dd[u] = 0;
#pragma unroll
                for (int c = 0; c < NE / 4; ++c) qv[u][c] = 0;
            }
        }
        float part[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // int8 q converted signed (no offset to take back out of the sum)
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int c = 0; c < NE / 4; ++c) {
                a0 = __builtin_fmaf(sbf(qv[u][c], 0), xv[4 * c + 0], a0);
                a1 = __builtin_fmaf(sbf(qv[u][c], 1), xv[4 * c + 1], a1);
                a0 = __builtin_fmaf(sbf(qv[u][c], 2), xv[4 * c + 2], a0);
                a1 = __builtin_fmaf(sbf(qv[u][c], 3), xv[4 * c + 3], a1);
            }
            part[u] = f16_bits_to_f32(dd[u]) * (a0 + a1);
        }
        row_partials_out<U>(part, rb, row0, row_end, y, red, nwaves, wave, lane);
    }
    finish_rows(row0, row_end, y, red, nwaves);
}

// Q8_0 register-ring kernel. Lane (block b = t / 2, half u = t % 2) owns
// the 16 int8 at 34b + 2 + 16u (q8_0.h:36-51 element order); its loads and
// sums are Q8RingLane's (frq_ringrow.h). Rows as in the other ring kernels.
template <int U, int R>
__global__ void __launch_bounds__(1024) gemv_q8_0_ring_kernel(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, int64_t n, int nb) {
    static_assert(U <= R, "ring deeper than the row count");
    __shared__ float red[R * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk_raw = tid >> 1;
    const bool active = blk_raw < nb;
    const int blk = active ? blk_raw : 0;
    const Q8RingLane ln(blk, tid & 1);

    const int64_t row0 = (int64_t)blockIdx.x * R;
    const int nrows = (int)(n - row0 < R ? n - row0 : R);
    const int64_t row_bytes = (int64_t)nb * kQ80Bytes;

    auto load1 = [&](Q8RingRow& t, int j) {
        const uint8_t* rp = w + (row0 + (j < nrows ? j : nrows - 1)) * row_bytes;
        ln.load(buffer_rsrc(rp, (uint32_t)row_bytes), 0, t);
    };

    float xv[1][16];
    ln.load_x(x, blk, xv[0]);
    __builtin_amdgcn_sched_barrier(0);
    Q8RingRow ring[U];
#pragma unroll
    for (int i = 0; i < U; ++i) load1(ring[i], i);
    __builtin_amdgcn_sched_barrier(0);

    static_for<0, R>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        Q8RingRow& t = ring[j % U];
        float pu[1];
        ln.dot<1>(t, xv, pu);
        if constexpr (j + U < R) load1(t, j + U);
        __builtin_amdgcn_sched_barrier(0);
        const float v = row16_sum(active ? pu[0] : 0.0f);
        if ((lane & 15) == 15) red[j * 4 * nwaves + 4 * wave + (lane >> 4)] = v;
    });
    __syncthreads();
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        float acc = 0.0f;
        for (int w2 = 0; w2 < 4 * nwaves; ++w2) acc += red[r * 4 * nwaves + w2];
        y[row0 + r] = acc;
    }
}

// ------------------------------------------------------------------ Q1_0
// Work unit: 4*CPL bytes of sign bits (32*CPL elements, 4/CPL lanes per
// block): sum_i (+-d) x_i = d * (2 * sum_{bit set} x_i - sum_i x_i).
template <int CPL, int U>
__global__ void __launch_bounds__(512) gemv_q1_0_kernel(const uint8_t* __restrict__ w,
                                                        const float* __restrict__ x,
                                                        float* __restrict__ y, int64_t n, int nb,
                                                        int rows_per_wg) {
    extern __shared__ float red[];
    constexpr int NE = 32 * CPL;
    constexpr int LPB = 4 / CPL;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk = tid / LPB, o = NE * (tid % LPB);
    const bool active = blk < nb;

    // Element 8b + j of a 4-byte bit word is bit j of byte b. `bits & (0x01010101 << j)`
    // leaves 2^j * bit in byte b, so x is stored pre-scaled by 2^-j (exact
    // power-of-two scaling) and one v_cvt_f32_ubyte<b> + one FMA handles
    // each element.
    float xv[NE];
    float sx = 0.0f;
#pragma unroll
    for (int i = 0; i < NE; i += 4) {
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
        if (active) a = *reinterpret_cast<const float4*>(x + (int64_t)blk * kQ10Elems + o + i);
        xv[i] = a.x; xv[i + 1] = a.y; xv[i + 2] = a.z; xv[i + 3] = a.w;
    }
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        sx += xv[i];
        xv[i] *= 1.0f / (float)(1u << (i & 7));
    }

    const int64_t row0 = (int64_t)blockIdx.x * rows_per_wg;
    const int64_t row_end = row0 + rows_per_wg < n ? row0 + rows_per_wg : n;
    const int64_t row_bytes = (int64_t)nb * kQ10Bytes;
    const uint8_t* wb = w + row0 * row_bytes + (int64_t)blk * kQ10Bytes;

    for (int64_t rb = row0; rb < row_end; rb += U) {
        uint32_t bits[U][CPL], dd[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (active && rb + u < row_end) {
                const uint8_t* p = wb + (rb - row0 + u) * row_bytes;
                dd[u] = ld_u16(p);
#pragma unroll
                for (int c = 0; c < CPL; ++c) bits[u][c] = ld_u32_a2(p + 2 + (o >> 3) + 4 * c);
            } else {
                dd[u] = 0;
#pragma unroll
                for (int c = 0; c < CPL; ++c) bits[u][c] = 0;
            }
        }
        float part[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t t = vand(bits[u][c], 0x01010101u << j);
                    a0 = __builtin_fmaf(byte_f(t, 0), xv[32 * c + j], a0);
                    a1 = __builtin_fmaf(byte_f(t, 1), xv[32 * c + 8 + j], a1);
                    a0 = __builtin_fmaf(byte_f(t, 2), xv[32 * c + 16 + j], a0);
                    a1 = __builtin_fmaf(byte_f(t, 3), xv[32 * c + 24 + j], a1);
                }
            }
            part[u] = f16_bits_to_f32(dd[u]) * __builtin_fmaf(2.0f, a0 + a1, -sx);
        }
        row_partials_out<U>(part, rb, row0, row_end, y, red, nwaves, wave, lane);
    }
    finish_rows(row0, row_end, y, red, nwaves);
}

// Q1_0 register-ring kernel. Lane (block b = t / 4, part u = t % 4) owns the
// 4 sign-bit bytes 18b + 2 + 4u .. +3 (elements 32u .. 32u + 31 of block b;
// element 8c + j is bit j of byte c, LSB first, gguf.py:266-299). Blocks
// are 18 bytes, so with a 4-aligned row those bytes start at 0 or 2 mod 4:
// the lane loads the aligned 8-byte window around them and funnel-shifts.
// `bits & (0x01010101 << j)` leaves 2^j * bit in each byte: x is stored
// pre-scaled by 2^-j (exact), so each element is one v_cvt_f32_ubyteN and
// one FMA, and sum_i (+-d) x_i = d * (2 * sum_{bit set} x_i - sum_i x_i).
// Rows as in the Q4_K / Q6_K ring kernels: fully unrolled over R, clamped
// unconditional buffer loads, U rows in flight, 16-lane row sums in LDS.
template <int U, int R>
__global__ void __launch_bounds__(1024) gemv_q1_0_ring_kernel(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, int64_t n, int nb) {
    static_assert(U <= R, "ring deeper than the row count");
    __shared__ float red[R * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
    const int blk_raw = tid >> 2, u = tid & 3;
    const bool active = blk_raw < nb;
    const int blk = active ? blk_raw : 0;
    const uint32_t at = (uint32_t)(blk * kQ10Bytes + 2 + 4 * u);
    const uint32_t o_win = at & ~3u, sh = 8u * (at & 3u), o_d = (uint32_t)(blk * kQ10Bytes);

    const int64_t row0 = (int64_t)blockIdx.x * R;
    const int nrows = (int)(n - row0 < R ? n - row0 : R);
    const int64_t row_bytes = (int64_t)nb * kQ10Bytes;

    struct Row {
        uint32_t lo, hi, d;
    };
    auto load1 = [&](Row& t, int j) {
        const uint8_t* rp = w + (row0 + (j < nrows ? j : nrows - 1)) * row_bytes;
        const auto rs = buffer_rsrc(rp, (uint32_t)row_bytes);
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)o_win, 0, 0);
        t.lo = v[0];
        t.hi = v[1];
        t.d = bload_u16(rs, o_d);
    };

    float xv[32];
    float sx = 0.0f;
    {
        const float* xb = x + (int64_t)blk * kQ10Elems + 32 * u;
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const float4 a = *reinterpret_cast<const float4*>(xb + i);
            xv[i] = a.x; xv[i + 1] = a.y; xv[i + 2] = a.z; xv[i + 3] = a.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    Row ring[U];
#pragma unroll
    for (int i = 0; i < U; ++i) load1(ring[i], i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        sx += xv[i];
        xv[i] *= 1.0f / (float)(1u << (i & 7));
    }

    static_for<0, R>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        Row& t = ring[j % U];
        const uint32_t bits = __builtin_amdgcn_alignbit(t.hi, t.lo, sh);
        const float d = f16_bits_to_f32(t.d);
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int b = 0; b < 8; b += 2) {
            float f[8];                                             // bit planes b and b + 1
            nibbles8(bits, f, 0x01010101u << b, 0x01010101u << (b + 1));
            a0 = __builtin_fmaf(f[0], xv[b], a0);
            a1 = __builtin_fmaf(f[4], xv[b + 1], a1);
            a0 = __builtin_fmaf(f[1], xv[8 + b], a0);
            a1 = __builtin_fmaf(f[5], xv[8 + b + 1], a1);
            a0 = __builtin_fmaf(f[2], xv[16 + b], a0);
            a1 = __builtin_fmaf(f[6], xv[16 + b + 1], a1);
            a0 = __builtin_fmaf(f[3], xv[24 + b], a0);
            a1 = __builtin_fmaf(f[7], xv[24 + b + 1], a1);
        }
        if constexpr (j + U < R) load1(t, j + U);
        __builtin_amdgcn_sched_barrier(0);
        const float pu = d * __builtin_fmaf(2.0f, a0 + a1, -sx);
        const float v = row16_sum(active ? pu : 0.0f);
        if ((lane & 15) == 15) red[j * 4 * nwaves + 4 * wave + (lane >> 4)] = v;
    });
    __syncthreads();
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        float acc = 0.0f;
        for (int w2 = 0; w2 < 4 * nwaves; ++w2) acc += red[r * 4 * nwaves + w2];
        y[row0 + r] = acc;
    }
}

// ------------------------------------------------------------------ planner

namespace {

struct Fmt {
    int bbytes, belems;
};

Fmt fmt_of(int qtype) {
    switch (qtype) {
        case kTypeQ4K: return {kQ4KBytes, kQKElems};
        case kTypeQ5K: return {kQ5KBytes, kQKElems};
        case kTypeQ6K: return {kQ6KBytes, kQKElems};
        case kTypeQ80: return {kQ80Bytes, kQ80Elems};
        case kTypeQ10: return {kQ10Bytes, kQ10Elems};
        default: return {0, 0};
    }
}

// Lanes one block of this format needs with work unit `cpl`.
int lanes_per_block(int qtype, int cpl) {
    switch (qtype) {
        case kTypeQ4K: return 8 / cpl;
        case kTypeQ5K: return 4;
        case kTypeQ6K: return 16 / cpl;
        case kTypeQ80: return 4 / cpl;
        case kTypeQ10: return 4 / cpl;
        default: return 0;
    }
}

bool cpl_valid(int qtype, int cpl) {
    switch (qtype) {
        case kTypeQ4K: return cpl == 1 || cpl == 2;
        case kTypeQ6K: return cpl == 1 || cpl == 2 || cpl == 4;
        case kTypeQ80: return cpl == 1 || cpl == 2 || cpl == 4;
        case kTypeQ10: return cpl == 1 || cpl == 2;
        case kTypeQ5K: return cpl == 1;
        default: return false;
    }
}

// Workgroup size cap of each kernel (its __launch_bounds__).
int64_t max_lanes(int qtype, int cpl) { return (qtype == kTypeQ4K && cpl == 1) ? 1024 : 512; }

// Work unit: Q4_K always takes the 16-byte unit (8 lanes per block) when the
// row fits a workgroup (twice the waves of the 32-byte unit, which measured
// slower on every shape); the other formats take the smallest-waste unit
// whose row fits in one workgroup.
int pick_cpl(int qtype, int64_t nb) {
    if (qtype == kTypeQ4K) return nb * 8 <= max_lanes(qtype, 1) ? 1 : 0;
    int best = 0;
    double best_waste = 2.0;
    for (int cpl = 1; cpl <= 4; cpl *= 2) {
        if (!cpl_valid(qtype, cpl)) continue;
        const int64_t lanes = nb * lanes_per_block(qtype, cpl);
        if (lanes > max_lanes(qtype, cpl)) continue;
        const int64_t padded = (lanes + 63) / 64 * 64;
        const double waste = (double)(padded - lanes) / (double)padded;
        // prefer larger units on ties: fewer scale decodes per element
        if (waste < best_waste - 1e-9 || (waste <= best_waste + 1e-9 && cpl > best)) {
            best = cpl;
            best_waste = waste;
        }
    }
    return best;
}

// Rows per workgroup: enough rows to amortise the x load into VGPRs, few
// enough that the grid fills 256 CUs evenly.
int pick_rows(int64_t n, int waves) {
    const int64_t kCUs = 256;
    int best_r = 1;
    double best_score = -1.0;
    for (int r = 2; r <= 32; ++r) {
        const int64_t grid = (n + r - 1) / r;
        // waves resident per CU if every workgroup ran at once
        const double per_cu = (double)(grid * waves) / (double)kCUs;
        const double rounds = (double)((grid + kCUs - 1) / kCUs);
        const double balance = (double)grid / (rounds * kCUs);        // 1.0 = even spread
        const double occ = per_cu >= 8.0 ? 1.0 : per_cu / 8.0;       // want >= 8 waves per CU
        const double amort = r >= 8 ? 1.0 : 0.85 + 0.02 * r;         // x reload cost
        const double score = balance * occ * amort;
        if (score > best_score + 1e-9) {
            best_score = score;
            best_r = r;
        }
    }
    return best_r;
}

// Variants whose 8-row batch exceeds the VGPR budget (they would spill to
// scratch) run 4-row batches only.
bool unroll8_ok(int qtype, int cpl) {
    return !((qtype == kTypeQ4K && cpl == 2) || (qtype == kTypeQ6K && cpl == 4) || qtype == kTypeQ5K);
}

// Q4_K: rows per workgroup is a compile-time constant of the kernel, one of
// these; the ring depth is 3 or 5 slots (CPL 2) and 3 (CPL 1: compiled for
// 5 waves per SIMD, <= 96 VGPRs, which measured fastest; deeper rings spill).
constexpr int kQ4KRowSet[] = {1, 2, 4, 7, 8, 14, 16};

bool q4k_rows_ok(int r) {
    for (int v : kQ4KRowSet)
        if (v == r) return true;
    return false;
}

int q4k_ring(int cpl, int want) {
    if (cpl == 2) return want <= 3 ? 3 : 5;
    return want >= 6 ? 6 : want >= 4 ? 4 : 3;
}

// Rows per Q4_K workgroup (measured on MI355X, 256 CUs). Workgroups of 4 or
// more waves run one per CU: take the fewest rows that still cover n with
// at most 256 workgroups (one round, every CU busy). Smaller workgroups
// (short rows) want several resident per CU: 4 rows per workgroup up to
// n = 8192, beyond that the fewest rows that keep <= 2560 workgroups.
int pick_rows_q4k(int64_t n, int waves) {
    const int64_t kCUs = 256;
    if (waves < 4) {
        if (n <= 8192) return 4;
        for (int r : kQ4KRowSet)
            if ((n + r - 1) / r <= 2560) return r;
        return 16;
    }
    for (int r : kQ4KRowSet)
        if ((n + r - 1) / r <= kCUs) return r;
    return 16;
}

template <int CPL, int U, int R>
void q4k_go(dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y, int64_t n, int nb) {
    gemv_q4_k_kernel<CPL, (U < R ? U : R), R><<<gd, bd, 0, s>>>(w, x, y, n, nb);
}

template <int CPL, int U>
bool q4k_rows(int rows, dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y, int64_t n,
              int nb) {
    switch (rows) {
        case 1: q4k_go<CPL, U, 1>(gd, bd, s, w, x, y, n, nb); return true;
        case 2: q4k_go<CPL, U, 2>(gd, bd, s, w, x, y, n, nb); return true;
        case 4: q4k_go<CPL, U, 4>(gd, bd, s, w, x, y, n, nb); return true;
        case 7: q4k_go<CPL, U, 7>(gd, bd, s, w, x, y, n, nb); return true;
        case 8: q4k_go<CPL, U, 8>(gd, bd, s, w, x, y, n, nb); return true;
        case 14: q4k_go<CPL, U, 14>(gd, bd, s, w, x, y, n, nb); return true;
        case 16: q4k_go<CPL, U, 16>(gd, bd, s, w, x, y, n, nb); return true;
        default: return false;
    }
}

hipError_t launch_q4k(int cpl, int ring, int rows, int waves, int64_t grid, const uint8_t* w, const float* x,
                      float* y, int64_t n, int nb, hipStream_t s) {
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * waves));
    bool ok = false;
    if (cpl == 2) {
        ok = ring == 3 ? q4k_rows<2, 3>(rows, gd, bd, s, w, x, y, n, nb)
                       : q4k_rows<2, 5>(rows, gd, bd, s, w, x, y, n, nb);
    } else if (ring == 6) {
        ok = q4k_rows<1, 6>(rows, gd, bd, s, w, x, y, n, nb);
    } else if (ring == 4) {
        ok = q4k_rows<1, 4>(rows, gd, bd, s, w, x, y, n, nb);
    } else {
        ok = q4k_rows<1, 3>(rows, gd, bd, s, w, x, y, n, nb);
    }
    if (!ok) return hipErrorInvalidConfiguration;
    return hipGetLastError();
}

// Q6_K ring kernel: work unit 8 in GemvPlan::cpl (8 lanes per block); needs a
// 4-byte aligned weight base and an even block count per row (see the kernel).
constexpr int kQ6KRingUnit = 8;

bool q6k_ring_ok(const uint8_t* w, int64_t nb) {
    return (reinterpret_cast<uintptr_t>(w) & 3) == 0 && nb % 2 == 0 && nb * 8 <= 1024;
}

// Rows per Q6_K ring workgroup (measured on MI355X): as for Q4_K when a
// workgroup has 4 or more waves; smaller workgroups take the most rows that
// still leave >= 1024 workgroups (lm_head 152064 rows: 16; 4096: 4; 1024: 1).
int pick_rows_q6k(int64_t n, int waves) {
    if (waves >= 4) return pick_rows_q4k(n, waves);
    int best = 1;
    for (int r : kQ4KRowSet)
        if (n / r >= 1024) best = r;
    return best;
}

template <int U, int R, bool P>
void q6k_go(dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y, int64_t n, int nb) {
    gemv_q6_k_ring_kernel<(U < R ? U : R), R, P><<<gd, bd, 0, s>>>(w, x, y, n, nb);
}

template <int U, bool P>
bool q6k_rows(int rows, dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y, int64_t n,
              int nb) {
    switch (rows) {
        case 1: q6k_go<U, 1, P>(gd, bd, s, w, x, y, n, nb); return true;
        case 2: q6k_go<U, 2, P>(gd, bd, s, w, x, y, n, nb); return true;
        case 4: q6k_go<U, 4, P>(gd, bd, s, w, x, y, n, nb); return true;
        case 7: q6k_go<U, 7, P>(gd, bd, s, w, x, y, n, nb); return true;
        case 8: q6k_go<U, 8, P>(gd, bd, s, w, x, y, n, nb); return true;
        case 14: q6k_go<U, 14, P>(gd, bd, s, w, x, y, n, nb); return true;
        case 16: q6k_go<U, 16, P>(gd, bd, s, w, x, y, n, nb); return true;
        default: return false;
    }
}

// Q8_0 ring kernel: work unit 8 in GemvPlan::cpl (2 lanes per block, 16 int8
// each); needs a 4-byte aligned weight base and an even block count.
constexpr int kQ80RingUnit = 8;

bool q80_ring_ok(const uint8_t* w, int64_t nb) {
    return (reinterpret_cast<uintptr_t>(w) & 3) == 0 && nb % 2 == 0 && nb * 2 <= 1024;
}

template <int U, int R>
void q80_go(dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y, int64_t n, int nb) {
    gemv_q8_0_ring_kernel<(U < R ? U : R), R><<<gd, bd, 0, s>>>(w, x, y, n, nb);
}

hipError_t launch_q80_ring(int ring, int rows, int waves, int64_t grid, const uint8_t* w, const float* x, float* y,
                           int64_t n, int nb, hipStream_t s) {
    // ring >= rows: every row's loads in flight at once; else 4 rows at a time
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * waves));
    const bool full = ring >= rows;
    switch (rows) {
        case 1: q80_go<4, 1>(gd, bd, s, w, x, y, n, nb); break;
        case 2: q80_go<4, 2>(gd, bd, s, w, x, y, n, nb); break;
        case 4: q80_go<4, 4>(gd, bd, s, w, x, y, n, nb); break;
        case 7: if (full) q80_go<7, 7>(gd, bd, s, w, x, y, n, nb); else q80_go<4, 7>(gd, bd, s, w, x, y, n, nb); break;
        case 8: if (full) q80_go<8, 8>(gd, bd, s, w, x, y, n, nb); else q80_go<4, 8>(gd, bd, s, w, x, y, n, nb); break;
        case 14: if (full) q80_go<14, 14>(gd, bd, s, w, x, y, n, nb); else q80_go<4, 14>(gd, bd, s, w, x, y, n, nb); break;
        case 16: if (full) q80_go<16, 16>(gd, bd, s, w, x, y, n, nb); else q80_go<4, 16>(gd, bd, s, w, x, y, n, nb); break;
        default: return hipErrorInvalidConfiguration;
    }
    return hipGetLastError();
}

// Q1_0 ring kernel: work unit 8 in GemvPlan::cpl (4 lanes per block, 32
// elements each); needs a 4-byte aligned weight base and an even block count.
constexpr int kQ10RingUnit = 8;
// Q1_0 on the matrix cores (frq_gemv_mx.hip): work unit 16; GemvPlan::unroll
// is the blocks per wavefront, rows_per_wg the rows per workgroup (<= 16).
constexpr int kQ10MxUnit = 16;

bool q10_ring_ok(const uint8_t* w, int64_t nb) {
    return (reinterpret_cast<uintptr_t>(w) & 3) == 0 && nb % 2 == 0 && nb * 4 <= 1024;
}

template <int U, int R>
void q10_go(dim3 gd, dim3 bd, hipStream_t s, const uint8_t* w, const float* x, float* y, int64_t n, int nb) {
    gemv_q1_0_ring_kernel<(U < R ? U : R), R><<<gd, bd, 0, s>>>(w, x, y, n, nb);
}

hipError_t launch_q10_ring(int ring, int rows, int waves, int64_t grid, const uint8_t* w, const float* x, float* y,
                           int64_t n, int nb, hipStream_t s) {
    // ring >= rows: every row's loads in flight at once; else 4 rows at a time
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * waves));
    const bool full = ring >= rows;
    switch (rows) {
        case 1: q10_go<4, 1>(gd, bd, s, w, x, y, n, nb); break;
        case 2: q10_go<4, 2>(gd, bd, s, w, x, y, n, nb); break;
        case 4: q10_go<4, 4>(gd, bd, s, w, x, y, n, nb); break;
        case 7: if (full) q10_go<7, 7>(gd, bd, s, w, x, y, n, nb); else q10_go<4, 7>(gd, bd, s, w, x, y, n, nb); break;
        case 8: if (full) q10_go<8, 8>(gd, bd, s, w, x, y, n, nb); else q10_go<4, 8>(gd, bd, s, w, x, y, n, nb); break;
        case 14: if (full) q10_go<14, 14>(gd, bd, s, w, x, y, n, nb); else q10_go<4, 14>(gd, bd, s, w, x, y, n, nb); break;
        case 16: if (full) q10_go<16, 16>(gd, bd, s, w, x, y, n, nb); else q10_go<4, 16>(gd, bd, s, w, x, y, n, nb); break;
        default: return hipErrorInvalidConfiguration;
    }
    return hipGetLastError();
}

hipError_t launch_q6k_ring(int ring, int rows, int waves, int64_t grid, const uint8_t* w, const float* x, float* y,
                           int64_t n, int nb, hipStream_t s) {
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * waves));
    (void)ring;
    const bool ok = waves >= 4 ? q6k_rows<4, true>(rows, gd, bd, s, w, x, y, n, nb)
                               : q6k_rows<4, false>(rows, gd, bd, s, w, x, y, n, nb);
    if (!ok) return hipErrorInvalidConfiguration;
    return hipGetLastError();
}

template <int U>
hipError_t launch_u(int qtype, int cpl, const uint8_t* w, const float* x, float* y, int64_t n, int nb,
                    int rows, int waves, int64_t grid, hipStream_t s) {
    const dim3 gd((unsigned)grid), bd((unsigned)(64 * waves));
    const size_t lds = waves > 1 ? sizeof(float) * (size_t)rows * waves : 0;
    switch (qtype) {
        case kTypeQ5K: gemv_q5_k_kernel<4><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows); break;
        case kTypeQ6K:
            if (cpl == 4) gemv_q6_k_kernel<4, 4><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            else if (cpl == 2) gemv_q6_k_kernel<2, U><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            else gemv_q6_k_kernel<1, U><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            break;
        case kTypeQ80:
            if (cpl == 4) gemv_q8_0_kernel<4, U><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            else if (cpl == 2) gemv_q8_0_kernel<2, U><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            else gemv_q8_0_kernel<1, U><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            break;
        case kTypeQ10:
            if (cpl == 2) gemv_q1_0_kernel<2, U><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            else gemv_q1_0_kernel<1, U><<<gd, bd, lds, s>>>(w, x, y, n, nb, rows);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool gemv_supported(int qtype, int64_t n, int64_t k) {
    const Fmt f = fmt_of(qtype);
    if (f.belems == 0 || n <= 0 || k <= 0 || k % f.belems) return false;
    return pick_cpl(qtype, k / f.belems) != 0;
}

hipError_t launch_gemv(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k,
                       GemvPlan* plan, hipStream_t stream) {
    const Fmt f = fmt_of(qtype);
    if (f.belems == 0 || k % f.belems) return hipErrorInvalidValue;
    if (n <= 0) return hipSuccess;
    const int64_t nb = k / f.belems;
    GemvPlan p = plan ? *plan : GemvPlan{};
    if (qtype == kTypeQ6K && (p.cpl <= 0 || p.cpl == kQ6KRingUnit) && q6k_ring_ok(w, nb)) {
        p.cpl = kQ6KRingUnit;
        p.waves = (int)((nb * 8 + 63) / 64);
        if (p.rows_per_wg <= 0) p.rows_per_wg = pick_rows_q6k(n, p.waves);
        if (!q4k_rows_ok(p.rows_per_wg)) return hipErrorInvalidConfiguration;
        p.unroll = 4;
        p.grid = (n + p.rows_per_wg - 1) / p.rows_per_wg;
        if (p.grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        if (plan) *plan = p;
        return launch_q6k_ring(p.unroll, p.rows_per_wg, p.waves, p.grid, w, x, y, n, (int)nb, stream);
    }
    if (qtype == kTypeQ6K && p.cpl == kQ6KRingUnit) return hipErrorInvalidValue;   // layout not eligible
    if (qtype == kTypeQ10 && (p.cpl == kQ10MxUnit || (p.cpl <= 0 && gemv_q10_mx_default(w, n, k)))) {
        p.cpl = kQ10MxUnit;
        if (!gemv_q10_mx_ok(w, k)) return hipErrorInvalidValue;   // layout not eligible
        if (!plan_gemv_q10_mx(n, k, &p.unroll, &p.rows_per_wg)) return hipErrorInvalidConfiguration;
        p.waves = (int)((nb + p.unroll - 1) / p.unroll);
        p.grid = (n + p.rows_per_wg - 1) / p.rows_per_wg;
        if (plan) *plan = p;
        return launch_gemv_q10_mx(w, x, y, n, k, p.unroll, p.rows_per_wg, stream);
    }
    if (qtype == kTypeQ10 && (p.cpl <= 0 || p.cpl == kQ10RingUnit) && q10_ring_ok(w, nb)) {
        p.cpl = kQ10RingUnit;
        p.waves = (int)((nb * 4 + 63) / 64);
        if (p.rows_per_wg <= 0) p.rows_per_wg = pick_rows_q6k(n, p.waves);
        if (!q4k_rows_ok(p.rows_per_wg)) return hipErrorInvalidConfiguration;
        p.unroll = p.unroll >= p.rows_per_wg ? p.rows_per_wg : 4;
        p.grid = (n + p.rows_per_wg - 1) / p.rows_per_wg;
        if (p.grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        if (plan) *plan = p;
        return launch_q10_ring(p.unroll, p.rows_per_wg, p.waves, p.grid, w, x, y, n, (int)nb, stream);
    }
    if (qtype == kTypeQ10 && p.cpl == kQ10RingUnit) return hipErrorInvalidValue;   // layout not eligible
    if (qtype == kTypeQ80 && (p.cpl <= 0 || p.cpl == kQ80RingUnit) && q80_ring_ok(w, nb)) {
        p.cpl = kQ80RingUnit;
        p.waves = (int)((nb * 2 + 63) / 64);
        if (p.rows_per_wg <= 0) p.rows_per_wg = pick_rows_q6k(n, p.waves);
        if (!q4k_rows_ok(p.rows_per_wg)) return hipErrorInvalidConfiguration;
        p.unroll = p.unroll >= p.rows_per_wg ? p.rows_per_wg : 4;
        p.grid = (n + p.rows_per_wg - 1) / p.rows_per_wg;
        if (p.grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        if (plan) *plan = p;
        return launch_q80_ring(p.unroll, p.rows_per_wg, p.waves, p.grid, w, x, y, n, (int)nb, stream);
    }
    if (qtype == kTypeQ80 && p.cpl == kQ80RingUnit) return hipErrorInvalidValue;   // layout not eligible
    if (p.cpl <= 0) p.cpl = pick_cpl(qtype, nb);
    if (!cpl_valid(qtype, p.cpl)) return hipErrorInvalidValue;
    const int64_t lanes = nb * lanes_per_block(qtype, p.cpl);
    if (lanes > max_lanes(qtype, p.cpl)) return hipErrorInvalidConfiguration;
    p.waves = (int)((lanes + 63) / 64);
    if (qtype == kTypeQ4K) {
        if (p.slices > 1) return hipErrorInvalidConfiguration;   // every row in one workgroup
        p.slices = 1;
        if (p.rows_per_wg <= 0) p.rows_per_wg = pick_rows_q4k(n, p.waves);
        if (!q4k_rows_ok(p.rows_per_wg)) return hipErrorInvalidConfiguration;
        p.unroll = q4k_ring(p.cpl, p.unroll > 0 ? p.unroll : 3);
        p.grid = (n + p.rows_per_wg - 1) / p.rows_per_wg;
        if (p.grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
        if (plan) *plan = p;
        return launch_q4k(p.cpl, p.unroll, p.rows_per_wg, p.waves, p.grid, w, x, y, n, (int)nb, stream);
    }
    if (p.rows_per_wg <= 0) p.rows_per_wg = pick_rows(n, p.waves);
    if (p.unroll != 4 && p.unroll != 8) p.unroll = p.rows_per_wg >= 8 ? 8 : 4;
    if (p.unroll == 8 && !unroll8_ok(qtype, p.cpl)) p.unroll = 4;
    p.grid = (n + p.rows_per_wg - 1) / p.rows_per_wg;
    if (p.grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    if (plan) *plan = p;
    if (p.unroll == 8)
        return launch_u<8>(qtype, p.cpl, w, x, y, n, (int)nb, p.rows_per_wg, p.waves, p.grid, stream);
    return launch_u<4>(qtype, p.cpl, w, x, y, n, (int)nb, p.rows_per_wg, p.waves, p.grid, stream);
}

bool gemv_swiglu_fusable(int qtype_gate, const uint8_t* wgate, int qtype_up, const uint8_t* wup, int64_t k) {
    return qtype_gate == kTypeQ4K && qtype_up == kTypeQ4K && k > 0 && k % kQKElems == 0 &&
           (k / kQKElems) * 8 <= 1024 && !(reinterpret_cast<uintptr_t>(wgate) & 15) &&
           !(reinterpret_cast<uintptr_t>(wup) & 15);
}

// Rows per matrix of the two-matrix ring: half of what the single-matrix
// rule gives their 2n rows (a workgroup runs the same row count), in the
// instantiated set.
static int pair_rows(int64_t n, int waves) {
    int R = pick_rows_q4k(2 * n, waves) / 2;
    if (R < 1) R = 1;
    if (R == 3) R = 2;
    return R;
}

template <int R>
static void swiglu_go(int64_t grid, int waves, const uint8_t* wgate, const uint8_t* wup, const float* x,
                      float* gateup, float* act, int64_t inter, int nb, hipStream_t s) {
    gemv_swiglu_kernel<R><<<dim3((unsigned)grid), dim3((unsigned)(64 * waves)), 0, s>>>(wgate, wup, x, gateup, act,
                                                                                         inter, nb);
}

hipError_t launch_gemv_swiglu(const uint8_t* wgate, const uint8_t* wup, const float* x, float* gateup, float* act,
                              int64_t inter, int64_t k, hipStream_t s) {
    if (inter <= 0) return hipSuccess;
    if (!gemv_swiglu_fusable(kTypeQ4K, wgate, kTypeQ4K, wup, k)) return hipErrorInvalidValue;
    const int64_t nb = k / kQKElems;
    const int waves = (int)((nb * 8 + 63) / 64);
    const int R = pair_rows(inter, waves);
    const int64_t grid = (inter + R - 1) / R;
    if (grid > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    switch (R) {
        case 1: swiglu_go<1>(grid, waves, wgate, wup, x, gateup, act, inter, (int)nb, s); break;
        case 2: swiglu_go<2>(grid, waves, wgate, wup, x, gateup, act, inter, (int)nb, s); break;
        case 4: swiglu_go<4>(grid, waves, wgate, wup, x, gateup, act, inter, (int)nb, s); break;
        case 7: swiglu_go<7>(grid, waves, wgate, wup, x, gateup, act, inter, (int)nb, s); break;
        case 8: swiglu_go<8>(grid, waves, wgate, wup, x, gateup, act, inter, (int)nb, s); break;
        default: return hipErrorInvalidConfiguration;
    }
    return hipGetLastError();
}

bool gemv_group_fusable(int count, const int* qtypes, const uint8_t* const* w, int64_t k) {
    // one matrix has nothing to fuse: it takes frq_dev_gemv's own kernel
    // (the matrix cores for a large Q4_K matrix)
    if (count < 2 || count > kGemvGroupMax || k <= 0 || k % kQKElems) return false;
    const int64_t nb = k / kQKElems;
    if (nb * 8 > 1024) return false;
    for (int i = 0; i < count; ++i) {
        if (qtypes[i] == kTypeQ4K) {
            if (reinterpret_cast<uintptr_t>(w[i]) & 15) return false;
        } else if (qtypes[i] == kTypeQ6K) {
            if (!q6k_ring_ok(w[i], nb)) return false;
        } else {
            return false;
        }
    }
    return true;
}

template <int R>
static void group_go(int64_t grid, int waves, const GemvGroup& g, const float* x, int nb, hipStream_t s) {
    gemv_group_kernel<R><<<dim3((unsigned)grid), dim3((unsigned)(64 * waves)), 0, s>>>(g, x, nb);
}

template <int R>
static void pair_go(int64_t grid, int waves, const uint8_t* w0, const uint8_t* w1, const float* x, float* y0, float* y1,
                    int64_t n, int nb, hipStream_t s) {
    gemv_pair_kernel<R><<<dim3((unsigned)grid), dim3((unsigned)(64 * waves)), 0, s>>>(w0, w1, x, y0, y1, n, nb);
}

hipError_t launch_gemv_group(int count, const int* qtypes, const uint8_t* const* w, const int64_t* n, float* const* y,
                             const float* x, int64_t k, hipStream_t s, int* fused) {
    if (fused) *fused = 0;
    if (count < 1 || count > kGemvGroupMax) return hipErrorInvalidValue;
    if (!gemv_group_fusable(count, qtypes, w, k)) {
        for (int i = 0; i < count; ++i) {
            GemvPlan p;
            const hipError_t e = launch_gemv(qtypes[i], w[i], x, y[i], n[i], k, &p, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const int64_t nb = k / kQKElems;
    const int waves = (int)((nb * 8 + 63) / 64);
    int64_t total = 0;
    for (int i = 0; i < count; ++i) {
        if (n[i] < 0) return hipErrorInvalidValue;
        total += n[i];
    }
    if (total == 0) return hipSuccess;
    // rows per workgroup for the whole group, by the single-matrix Q4_K rule
    const int R = pick_rows_q4k(total, waves);
    GemvGroup g{};
    int64_t wg = 0;
    int used = 0;
    for (int i = 0; i < count; ++i) {
        if (n[i] == 0) continue;                      // empty segment: no workgroups
        g.w[used] = w[i];
        g.y[used] = y[i];
        g.n[used] = n[i];
        g.qtype[used] = qtypes[i];
        g.wg_begin[used] = wg;
        wg += (n[i] + R - 1) / R;
        ++used;
    }
    g.count = used;
    if (wg > 0x7FFFFFFF) return hipErrorInvalidConfiguration;
    if (used == 2 && g.qtype[0] == kTypeQ4K && g.qtype[1] == kTypeQ4K && g.n[0] == g.n[1]) {
        // two Q4_K matrices of one shape (gate|up): one ring over both
        const int RP = pair_rows(g.n[0], waves);
        const int64_t grid = (g.n[0] + RP - 1) / RP;
        switch (RP) {
            case 1: pair_go<1>(grid, waves, g.w[0], g.w[1], x, g.y[0], g.y[1], g.n[0], (int)nb, s); break;
            case 2: pair_go<2>(grid, waves, g.w[0], g.w[1], x, g.y[0], g.y[1], g.n[0], (int)nb, s); break;
            case 4: pair_go<4>(grid, waves, g.w[0], g.w[1], x, g.y[0], g.y[1], g.n[0], (int)nb, s); break;
            case 7: pair_go<7>(grid, waves, g.w[0], g.w[1], x, g.y[0], g.y[1], g.n[0], (int)nb, s); break;
            case 8: pair_go<8>(grid, waves, g.w[0], g.w[1], x, g.y[0], g.y[1], g.n[0], (int)nb, s); break;
            default: return hipErrorInvalidConfiguration;
        }
        if (fused) *fused = 1;
        return hipGetLastError();
    }
    switch (R) {
        case 1: group_go<1>(wg, waves, g, x, (int)nb, s); break;
        case 2: group_go<2>(wg, waves, g, x, (int)nb, s); break;
        case 4: group_go<4>(wg, waves, g, x, (int)nb, s); break;
        case 7: group_go<7>(wg, waves, g, x, (int)nb, s); break;
        case 8: group_go<8>(wg, waves, g, x, (int)nb, s); break;
        case 14: group_go<14>(wg, waves, g, x, (int)nb, s); break;
        case 16: group_go<16>(wg, waves, g, x, (int)nb, s); break;
        default: return hipErrorInvalidConfiguration;
    }
    if (fused) *fused = 1;
    return hipGetLastError();
}

}  // namespace frq
