// Prefill GEMM on the gfx950 matrix cores:
//   Y[M, N] (fp32) = X[M, K] (bf16) . W[N, K]^T, W = raw Q4_K, Q6_K or Q8_0 blocks.
//
// The reference prefills by re-running the matvec for every token
// (matmul_<q>_batched, _C.cpp:154-283): W is dequantized M times and there
// is no reuse. Here W is dequantized once per output tile into LDS as bf16
// and multiplied with v_mfma_f32_32x32x16_bf16 (fp32 accumulation). The
// kernel is one template; only the W staging (which raw bytes a thread
// loads, and how it turns them into 16 bf16 weights) depends on the format.
//
// Precision contract: W values are the exact fp32 dequant (the same
// arithmetic as the dequant kernels) rounded to bf16 (nearest even);
// X is taken as given in bf16; products and sums are fp32. The result equals
// fp64 X . bf16(W)^T to fp32 accumulation error.
//
// Tiling: a workgroup (8 waves, two per SIMD) owns a 256 (M) x 128 (N) tile of
// Y and walks K in steps of 64 (one Q4_K group: 32 qs bytes per row). Wave
// (wm, wn) owns the 64 x 64 sub-tile at (64 wm, 64 wn): 2 x 2 MFMA tiles of
// 32 x 32, 64 fp32 accumulators per lane. Per K-step the X tile [256][64]
// bf16 and the W tile [128][64] (dequantized, 16 weights of one row per
// thread) pass through LDS, double buffered; LDS rows are padded to 72 bf16
// (144 B) so a fragment read by 32 lanes of consecutive rows spreads over
// the banks.
// Schedule (ping-pong): the two waves of a SIMD (w and w + 4) sit in
// different groups, group g = the waves with wn = g, and the groups take turns
// between workgroup barriers. In one phase a wave issues its K-step's 16
// MFMAs from registers (with the global loads for a later tile and the
// dequant arithmetic between them); in the next it reads its next K-step's
// fragments from LDS and writes its group's half of a later tile (X rows
// 128 g .. 128 g + 127, W rows 64 g .. 64 g + 63). So one wave's MFMAs run
// while its SIMD partner waits on LDS, instead of both waves of a SIMD
// reaching the LDS round trip together.
// MFMA operand layouts (32x32x16, 8 bf16 per lane): A lane l holds row l%32,
// k = 8*(l/32) .. +7; B lane l holds column l%32, same k; D register r of lane
// l is row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
// Native vector, not HIP's uint4 class: values of the class type held across
// the K loop's barrier stay in scratch memory; native vectors go to registers.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 128, kBK = 64;
constexpr int kLds = kBK + 8;   // bf16 per LDS row

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// W staging per format. A K-step is 64 consecutive k of 128 rows; thread
// (row wr, quarter wq) stages 16 weights of row wr. load() issues the global
// reads for step `kb` (first k of the step), convert() dequantizes them (same
// rounding sequence as the format's dequant kernel) into 16 bf16 in two
// registers of four words, and put() writes those into bf16 LDS row `dst`.
template <int QT>
struct WFmt;

// Q4_K: the step is one 32-byte qs group g; the quarter wq owns qs bytes
// 8wq .. 8wq+7, whose low nibbles are k = 8wq + i (sub-block 2g) and high
// nibbles k = 32 + 8wq + i (sub-block 2g + 1) (gguf.py:209-219).
template <>
struct WFmt<kTypeQ4K> {
    static constexpr int kBytes = kQ4KBytes, kElems = kQKElems;
    struct Raw {
        u32x4 h;
        u32x2 q;
    };
    // rs covers the workgroup's W rows; voff = the row's byte offset, the
    // K-step's block and group offsets go in as scalars
    __device__ static void load(Raw& r, __amdgpu_buffer_rsrc_t rs, uint32_t voff, int kb, int wq) {
        const int sblk = (kb >> 8) * kQ4KBytes;
        r.h = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)voff, sblk, 0));
        r.q = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, (int)(voff + 16 + 8 * wq),
                                                                            sblk + 32 * ((kb >> 6) & 3), 0));
    }
    // scale/min pairs 2g, 2g+1 (get_scale_min_k4, gguf.py:135-163) as
    // (s0, t0, s1, t1), without a branch: bytes o, o+1 of scales[0..3] and
    // [4..7] (g < 2), or the nibbles of scales[8 + o], [9 + o] with their high
    // bits (g >= 2), o = 2 (g % 2). Codes enter as q * u (fp8 pair conversion
    // of the nibble bytes, u a power of two) and the scale as d * sc / u, so
    // fma(s, q u, -t) is fl(d*sc*q - dmin*m): d*sc*q is exact, one rounding,
    // the dequant's bits.
    __device__ static f32x4 scales(const Raw& r, int kb, float u_inv) {
        const int g = (kb >> 6) & 3;
        const uint32_t o = 2u * (uint32_t)(g & 1);
        const uint32_t P = __builtin_amdgcn_perm(r.h[2], r.h[1], o | ((o + 1) << 8) | ((o + 4) << 16) | ((o + 5) << 24));
        const uint32_t Q = __builtin_amdgcn_perm(r.h[3], r.h[3], o | ((o + 1) << 8) | (o << 16) | ((o + 1) << 24));
        const uint32_t lo4 = (Q & 0x00000F0Fu) | ((Q >> 4) & 0x0F0F0000u);
        const uint32_t lowsel = 0u - (uint32_t)(g < 2);   // all ones for g < 2: a blend, not a branch
        const uint32_t scm = ((P & 0x3F3F3F3Fu) & lowsel) |
                             ((lo4 | ((P >> 2) & 0x30303030u)) & ~lowsel);
        const float d = f16_bits_to_f32(r.h[0]), dmin = f16_bits_to_f32(r.h[0] >> 16);
        const float du = d * u_inv;
        return f32x4{du * byte_f(scm, 0), dmin * byte_f(scm, 2), du * byte_f(scm, 1), dmin * byte_f(scm, 3)};
    }
    // the 16 weights as bf16: a = k 8wq .. +7 (low nibbles), b = k 32 + 8wq .. +7
    __device__ static void weights(const Raw& r, const f32x4& sc, u32x4& a, u32x4& b) {
        const float s0 = sc[0], t0 = sc[1], s1 = sc[2], t1 = sc[3];
        const uint32_t qw[2] = {r.q[0], r.q[1]};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {                          // bytes 4h .. 4h+3 of the quarter
            float f[8];
            nibbles8_fp8(qw[h], f);                            // f[0..3] low nibbles, f[4..7] high
            lo[2 * h] = pack_bf16(__builtin_fmaf(s0, f[0], -t0), __builtin_fmaf(s0, f[1], -t0));
            lo[2 * h + 1] = pack_bf16(__builtin_fmaf(s0, f[2], -t0), __builtin_fmaf(s0, f[3], -t0));
            hi[2 * h] = pack_bf16(__builtin_fmaf(s1, f[4], -t1), __builtin_fmaf(s1, f[5], -t1));
            hi[2 * h + 1] = pack_bf16(__builtin_fmaf(s1, f[6], -t1), __builtin_fmaf(s1, f[7], -t1));
        }
        a = u32x4{lo[0], lo[1], lo[2], lo[3]};
        b = u32x4{hi[0], hi[1], hi[2], hi[3]};
    }
    __device__ static void convert(const Raw& r, int kb, int, float u_inv, u32x4& a, u32x4& b) {
        weights(r, scales(r, kb, u_inv), a, b);
    }
    __device__ static void put(uint16_t* dst, int wq, const u32x4& a, const u32x4& b) {
        *reinterpret_cast<u32x4*>(dst + 8 * wq) = a;
        *reinterpret_cast<u32x4*>(dst + 32 + 8 * wq) = b;
    }
};

// Q8_0: the step is two 34-byte blocks; quarter wq owns elements
// 16 (wq & 1) .. +15 of block wq >> 1, i.e. k = 16 wq + i: y = fl(q * d).
template <>
struct WFmt<kTypeQ80> {
    static constexpr int kBytes = kQ80Bytes, kElems = kQ80Elems;
    struct Raw {
        uint32_t d;
        uint32_t q[4];
    };
    __device__ static void load(Raw& r, const uint8_t* wrow, int kb, int wq) {
        const uint8_t* bp = wrow + (int64_t)((kb >> 5) + (wq >> 1)) * kQ80Bytes;
        r.d = ld_u16(bp);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.q[i] = ld_u32_a2(bp + 2 + 16 * (wq & 1) + 4 * i);
    }
    __device__ static void convert(const Raw& r, int, int, float, u32x4& a, u32x4& b) {
        const float d = f16_bits_to_f32(r.d);
        uint32_t o[8];
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const uint32_t v = r.q[p >> 1] >> (16 * (p & 1));
            o[p] = pack_bf16((float)(int)(int8_t)(v & 0xFFu) * d, (float)(int)(int8_t)((v >> 8) & 0xFFu) * d);
        }
        a = u32x4{o[0], o[1], o[2], o[3]};
        b = u32x4{o[4], o[5], o[6], o[7]};
    }
    __device__ static void put(uint16_t* dst, int wq, const u32x4& a, const u32x4& b) {
        *reinterpret_cast<u32x4*>(dst + 16 * wq) = a;
        *reinterpret_cast<u32x4*>(dst + 16 * wq + 8) = b;
    }
};

// Q6_K: the step is 64 k of one half h of a block: elements 128h + 32ks + l
// for ks = 2kp, 2kp+1 (kp = which 64 of the half). Quarter wq takes
// ks = 2kp + (wq >> 1) and l = 16 (wq & 1) .. +15, i.e. k = 16 wq + i:
// q = nibble of ql[64h + 32 (ks & 1) + l] (high nibble for ks >= 2) | bits
// 2ks, 2ks+1 of qh[32h + l] << 4; y = fl(fl(d * sc[8h + l/16 + 2ks]) * (q - 32))
// (gguf.py:401-419). Fields are only 2-byte aligned (210-byte blocks).
template <>
struct WFmt<kTypeQ6K> {
    static constexpr int kBytes = kQ6KBytes, kElems = kQKElems;
    // ql and qh bytes of the quarter come from 20-byte windows aligned down to
    // 4 bytes (the fields start at 0 or 2 mod 4; both windows share the
    // misalignment, as their offsets differ by a multiple of 4) and are
    // funnel-shifted into place; the windows stay inside the block.
    struct Raw {
        u32x4 ql;
        u32x4 qh;
        uint32_t ql4, qh4, sh, sc, d;
    };
    __device__ static void load(Raw& r, const uint8_t* wrow, int kb, int wq) {
        const uint8_t* bp = wrow + (int64_t)(kb >> 8) * kQ6KBytes;
        const int kt4 = (kb & 255) >> 6, h = kt4 >> 1, ks = 2 * (kt4 & 1) + (wq >> 1), l0 = 16 * (wq & 1);
        const uint8_t* pl = bp + 64 * h + 32 * (ks & 1) + l0;
        const uint8_t* ph = bp + 128 + 32 * h + l0;
        const uintptr_t mis = reinterpret_cast<uintptr_t>(pl) & 3;
        const uint8_t* al = pl - mis;
        const uint8_t* ah = ph - mis;
        r.ql = *reinterpret_cast<const u32x4*>(al);
        r.ql4 = *reinterpret_cast<const uint32_t*>(al + 16);
        r.qh = *reinterpret_cast<const u32x4*>(ah);
        r.qh4 = *reinterpret_cast<const uint32_t*>(ah + 16);
        r.sh = 8u * (uint32_t)mis;
        r.sc = bp[192 + 8 * h + (wq & 1) + 2 * ks];
        r.d = ld_u16(bp + 208);
    }
    // half H of convert(): words 4H .. 4H + 3 (k = 16 wq + 8H .. + 7)
    template <int H>
    __device__ static void convert_half(const Raw& r, int kb, int wq, u32x4& v) {
        const int kt4 = (kb & 255) >> 6, ks = 2 * (kt4 & 1) + (wq >> 1);
        const float s = f16_bits_to_f32(r.d) * (float)(int)(int8_t)(r.sc & 0xFFu);
        const float m = -32.0f * s;
        const uint32_t lw[5] = {r.ql[0], r.ql[1], r.ql[2], r.ql[3], r.ql4};
        const uint32_t hw[5] = {r.qh[0], r.qh[1], r.qh[2], r.qh[3], r.qh4};
        const uint32_t nsh = ks >= 2 ? 4u : 0u, hsh = 2u * (uint32_t)ks;
        uint32_t o[4];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int c = 2 * H + cc;
            const uint32_t l = __builtin_amdgcn_alignbit(lw[c + 1], lw[c], r.sh);
            const uint32_t hb = __builtin_amdgcn_alignbit(hw[c + 1], hw[c], r.sh);
            const uint32_t q = ((l >> nsh) & 0x0F0F0F0Fu) | (((hb >> hsh) & 0x03030303u) << 4);
            o[2 * cc] = pack_bf16(__builtin_fmaf(byte_f(q, 0), s, m), __builtin_fmaf(byte_f(q, 1), s, m));
            o[2 * cc + 1] = pack_bf16(__builtin_fmaf(byte_f(q, 2), s, m), __builtin_fmaf(byte_f(q, 3), s, m));
        }
        v = u32x4{o[0], o[1], o[2], o[3]};
    }
    template <int H>
    __device__ static void put_half(uint16_t* dst, int wq, const u32x4& v) {
        *reinterpret_cast<u32x4*>(dst + 16 * wq + 8 * H) = v;
    }
    __device__ static void convert(const Raw& r, int kb, int wq, float, u32x4& a, u32x4& b) {
        const int kt4 = (kb & 255) >> 6, ks = 2 * (kt4 & 1) + (wq >> 1);
        const float s = f16_bits_to_f32(r.d) * (float)(int)(int8_t)(r.sc & 0xFFu);
        const float m = -32.0f * s;                         // exact: a power-of-two multiple
        const uint32_t lw[5] = {r.ql[0], r.ql[1], r.ql[2], r.ql[3], r.ql4};
        const uint32_t hw[5] = {r.qh[0], r.qh[1], r.qh[2], r.qh[3], r.qh4};
        const uint32_t nsh = ks >= 2 ? 4u : 0u, hsh = 2u * (uint32_t)ks;
        uint32_t o[8];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t l = __builtin_amdgcn_alignbit(lw[c + 1], lw[c], r.sh);
            const uint32_t hb = __builtin_amdgcn_alignbit(hw[c + 1], hw[c], r.sh);
            // q = low or high nibble of ql | bits 2ks, 2ks + 1 of qh << 4 (0 .. 63 per byte)
            const uint32_t q = ((l >> nsh) & 0x0F0F0F0Fu) | (((hb >> hsh) & 0x03030303u) << 4);
            // fl(s * (q - 32)) = fma(q, s, -32 s): the exact value, rounded once
            o[2 * c] = pack_bf16(__builtin_fmaf(byte_f(q, 0), s, m), __builtin_fmaf(byte_f(q, 1), s, m));
            o[2 * c + 1] = pack_bf16(__builtin_fmaf(byte_f(q, 2), s, m), __builtin_fmaf(byte_f(q, 3), s, m));
        }
        a = u32x4{o[0], o[1], o[2], o[3]};
        b = u32x4{o[4], o[5], o[6], o[7]};
    }
    __device__ static void put(uint16_t* dst, int wq, const u32x4& a, const u32x4& b) {
        *reinterpret_cast<u32x4*>(dst + 16 * wq) = a;
        *reinterpret_cast<u32x4*>(dst + 16 * wq + 8) = b;
    }
};

// S > 1 splits K: split s of an output tile runs K-steps [s * K/(64S), +K/(64S))
// and writes its fp32 partial tile to plane s of `part`; a second, small
// kernel adds the planes in split order (deterministic, and the kernel
// boundary makes every partial visible whichever XCD wrote it).
// L: K-steps between a tile's global loads and the phase that dequantizes it
// (1, or 2 when the K-step count per split is a multiple of four).
//
// Phases (group 0's numbering; group 1 runs the same sequence one phase
// later): phase 2t issues the MFMAs of step t, phase 2t + 1 reads the
// fragments of tile t + 1 and writes the group's half of tile t + 2. Tile u
// lives in LDS buffer u % 2: group 0 writes its half in global phase 2u - 3,
// group 1 in 2u - 2; group 0 reads it in 2u - 1, group 1 in 2u; the buffer is
// rewritten from phase 2u + 1 on. Every access is separated from a
// conflicting one by at least one barrier.
typedef uint16_t XTile[kBM * kLds];
typedef uint16_t WTile[kBN * kLds];
// The workgroup's LDS tiles, named directly in the tile body (a pointer
// passed in would be a generic address: 64-bit arithmetic and spills).
__shared__ __attribute__((aligned(16))) XTile xs[2];
__shared__ __attribute__((aligned(16))) WTile ws[2];

// One workgroup's output tile (M-tile mt, N-tile nt, K-split `split` of S):
// y[m * ldy + n] for its rows and columns, or with S > 1 plane `split` of
// `part` (M x N, dense).
template <int QT, int L>
__device__ __forceinline__ void gemm_tile(const uint8_t* __restrict__ w, const uint16_t* __restrict__ x,
                                          float* __restrict__ y, int ldy, float* __restrict__ part, int M, int N,
                                          int K, int S, int mt, int nt, int split) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 3, wn = wave >> 2;
    const int grp = __builtin_amdgcn_readfirstlane(wn);
    const int n0 = nt * kBN, m0 = mt * kBM;
    using F = WFmt<QT>;
    const int64_t row_bytes = (int64_t)(K / F::kElems) * F::kBytes;
    const int ksteps = K / kBK / S;                    // a multiple of NS (chosen by the host)
    const int kbase = split * ksteps;

    // The group's half of a tile: X rows 128 grp + xr + 32 j (8 threads of 16 B
    // per row), W row 64 grp + wr, quarter wq.
    const int gt = tid & 255;
    const int xc = gt & 7, xr = 128 * grp + (gt >> 3);
    const int wr = 64 * grp + (gt >> 2), wq = gt & 3;
    const float u_inv = 1.0f / fp8_unit();
    // X (and Q4_K W) through buffer resources over the tile's rows: per-thread
    // offsets are constants and the K-step's offset a scalar, so a load needs
    // no address arithmetic. Rows past M or N read as zeros (their outputs
    // are not stored); the host keeps the offsets below 2^31.
    const int mrows = M - m0 < kBM ? M - m0 : kBM;
    const auto xrs = buffer_rsrc(x + (int64_t)m0 * K, (uint32_t)((int64_t)mrows * K * 2));
    uint32_t xoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xoff[j] = (uint32_t)(((int64_t)(xr + 32 * j) * K + 8 * xc) * 2);
    const int nrows = N - n0 < kBN ? N - n0 : kBN;
    const auto wrs = buffer_rsrc(w + (int64_t)n0 * row_bytes, (uint32_t)((int64_t)nrows * row_bytes));
    const uint32_t wvoff = (uint32_t)((int64_t)wr * row_bytes);
    const uint8_t* wrow = w + (int64_t)(n0 + wr < N ? n0 + wr : N - 1) * row_bytes;

    struct Stage {
        u32x4 x[4];
        typename F::Raw w;
    };
    constexpr int NS = L == 2 ? 4 : 2;                 // staging sets, a power of two
    static_assert(L == 1 || L == 2, "loads one or two K-steps ahead");
    Stage st[NS];
    const int last = ksteps - 1;
    // Tiles past the last one repeat it (into an LDS buffer nothing reads
    // again), so loads and LDS writes stay unconditional and the compiler's
    // wait before an LDS write covers one staging set only.
    auto kb_of = [&](int u) __attribute__((always_inline)) { return (kbase + (u < last ? u : last)) * kBK; };
    auto load_half = [&](Stage& sg, int u) __attribute__((always_inline)) {
        const int kb = kb_of(u);
        static_for<0, 4>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            sg.x[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)xoff[j], kb * 2, 0));
        });
        if constexpr (QT == kTypeQ4K) F::load(sg.w, wrs, wvoff, kb, wq);
        else F::load(sg.w, wrow, kb, wq);
    };
    auto put_x = [&](const Stage& sg, int buf) __attribute__((always_inline)) {
        static_for<0, 4>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            *reinterpret_cast<u32x4*>(&xs[buf][(xr + 32 * j) * kLds + 8 * xc]) = sg.x[j];
        });
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

    bf16x8 fa[kBK / 16][2], fb[kBK / 16][2];           // one K-step's fragments
    u32x4 wa, wb;                                      // the next W half, as bf16
    // Q4_K with loads two steps ahead: the memory phase decodes the scales of
    // the tile the next MFMA phase dequantizes, after its own LDS traffic, so
    // the MFMA phase only applies them (70.5 -> 70.0 us at 512 x 14336 x 4096).
    constexpr bool kPipe = QT == kTypeQ4K && L == 2;
    f32x4 sc_next = {0.f, 0.f, 0.f, 0.f};
    // Q6_K: the MFMA phase converts the first half of the W weights, the
    // memory phase the second half after its other LDS traffic (512 x 4096 x
    // 14336: 93.0 -> 90.6 us)
    constexpr bool kHalves = QT == kTypeQ6K;

    // MFMA phase of step t: the global loads for tile uld = t + 2 + L, the
    // dequant of tile udq = t + 2's W half into wa, wb, and the step's MFMAs.
    auto mfma_phase = [&](Stage& sld, int uld, const Stage& sdq, int udq) __attribute__((always_inline)) {
        load_half(sld, uld);
        if constexpr (kPipe) F::weights(sdq.w, sc_next, wa, wb);
        else if constexpr (kHalves) F::template convert_half<0>(sdq.w, kb_of(udq), wq, wa);
        else F::convert(sdq.w, kb_of(udq), wq, u_inv, wa, wb);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk)
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk][mi], fb[kk][ni], acc[mi][ni], 0, 0, 0);
    };
    // Memory phase: the fragments of buffer rbuf, then the group's half of
    // tile ust, staging set sst (X) and wa, wb (W), into buffer wbuf; then
    // (Q4_K, L = 2) the scales of tile unx from set snx.
    auto mem_phase = [&](int rbuf, const Stage& sst, int wbuf, int ust, const Stage& snx, int unx) __attribute__((always_inline)) {
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int kof = 16 * kk + 8 * (lane >> 5);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
                fa[kk][mi] = *reinterpret_cast<const bf16x8*>(&xs[rbuf][(64 * wm + 32 * mi + (lane & 31)) * kLds + kof]);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                fb[kk][ni] = *reinterpret_cast<const bf16x8*>(&ws[rbuf][(64 * wn + 32 * ni + (lane & 31)) * kLds + kof]);
        }
        put_x(sst, wbuf);
        if constexpr (kHalves) {
            F::template put_half<0>(&ws[wbuf][wr * kLds], wq, wa);
            __builtin_amdgcn_sched_barrier(0);
            F::template convert_half<1>(sst.w, kb_of(ust), wq, wb);
            F::template put_half<1>(&ws[wbuf][wr * kLds], wq, wb);
        } else {
            F::put(&ws[wbuf][wr * kLds], wq, wa, wb);
        }
        if constexpr (kPipe) {
            __builtin_amdgcn_sched_barrier(0);
            sc_next = F::scales(snx.w, kb_of(unx), u_inv);
        } else {
            (void)snx;
            (void)unx;
        }
    };
    // A phase ends at a workgroup barrier; sched_barrier(0) keeps the
    // scheduler from moving MFMAs or memory operations across it.
    auto phase_end = []() __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    };

    // Prologue: tiles 0 .. L loaded, tile 0 whole in LDS (both groups), the W
    // half of tile 1 converted, the loads for tile 1 + L issued.
    static_for<0, L + 1>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        load_half(st[i], i);
    });
    put_x(st[0], 0);
    F::convert(st[0].w, kb_of(0), wq, u_inv, wa, wb);
    F::put(&ws[0][wr * kLds], wq, wa, wb);
    F::convert(st[1].w, kb_of(1), wq, u_inv, wa, wb);
    load_half(st[(1 + L) % NS], 1 + L);
    __syncthreads();
    // group 1 lags one phase: one barrier before the sequence, group 0 one after
    if (grp == 1) phase_end();
    mem_phase(0, st[1], 1, 1, st[2 % NS], 2);
    phase_end();
    for (int t0 = 0; t0 < ksteps; t0 += NS) {
        static_for<0, NS>([&](auto jc) {
            constexpr int j = decltype(jc)::value;      // t % NS: staging sets; t % 2: LDS buffers
            const int t = t0 + j;
            mfma_phase(st[(j + 2 + L) % NS], t + 2 + L, st[(j + 2) % NS], t + 2);
            phase_end();
            mem_phase((j + 1) & 1, st[(j + 2) % NS], j & 1, t + 2, st[(j + 3) % NS], t + 3);
            phase_end();
        });
    }
    if (grp == 0) phase_end();

    float* out = S == 1 ? y : part + (int64_t)split * M * N;
    const int ldo = S == 1 ? ldy : N;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int n = n0 + 64 * wn + 32 * ni + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + 64 * wm + 32 * mi + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M && n < N) out[(int64_t)m * ldo + n] = acc[mi][ni][r];
            }
        }
}

// 1-D grid, M-tile fastest: workgroups are dealt to the 8 XCDs round-robin,
// so with 2 (or 4, 8) M-tiles each XCD only ever needs its own M-tile of X
// (2 MB at M-tile 256, K 4096), which then stays in that XCD's L2. S > 1:
// a split's partial tile goes to plane `split` of `part`, and
// gemm_split_reduce_kernel adds the planes after the kernel.
template <int QT, int L>
__global__ void __launch_bounds__(512) gemm_bf16_kernel(const uint8_t* __restrict__ w,
                                                             const uint16_t* __restrict__ x,
                                                             float* __restrict__ y, int M, int N, int K, int S,
                                                             float* __restrict__ part) {
    const int mtiles = (M + kBM - 1) / kBM;
    const int mt = (int)(blockIdx.x % mtiles), rest = (int)(blockIdx.x / mtiles);
    const int split = rest % S, nt = rest / S;
    gemm_tile<QT, L>(w, x, y, N, part, M, N, K, S, mt, nt, split);
}

// Up to four matrices that multiply the same x in one launch (a fused q|k|v
// projection): segment i owns workgroups [wg_begin_i, wg_begin_{i+1}), laid
// out as the single-matrix kernel's grid, and its format picks the tile
// body with a wave-uniform branch (the bodies share the LDS).
template <int L>
__global__ void __launch_bounds__(512) gemm_bf16_group_kernel(GemmGroup g, const uint16_t* __restrict__ x, int M,
                                                                   int K, int S) {
    const int64_t b = blockIdx.x;
    int i = 0;
#pragma unroll
    for (int t = 1; t < kGemmGroupMax; ++t)
        if (t < g.count && b >= g.wg_begin[t]) i = t;
    const int N = (int)g.n[i];
    const int mtiles = (M + kBM - 1) / kBM;
    const int local = (int)(b - g.wg_begin[i]);
    const int mt = local % mtiles, rest = local / mtiles;
    const int split = rest % S, nt = rest / S;
    const int ldy = (int)g.ldy[i];
    switch (g.qtype[i]) {
        case kTypeQ4K: gemm_tile<kTypeQ4K, L>(g.w[i], x, g.y[i], ldy, g.part[i], M, N, K, S, mt, nt, split); break;
        case kTypeQ6K: gemm_tile<kTypeQ6K, L>(g.w[i], x, g.y[i], ldy, g.part[i], M, N, K, S, mt, nt, split); break;
        default: gemm_tile<kTypeQ80, L>(g.w[i], x, g.y[i], ldy, g.part[i], M, N, K, S, mt, nt, split); break;
    }
}

// y[i] = part[0][i] + part[1][i] + ... + part[S-1][i], in that order (the
// same bits however the splits were scheduled); 4 elements per thread, the
// planes loaded eight at a time (sum_planes).
__global__ void __launch_bounds__(256) gemm_split_reduce_kernel(const float* __restrict__ part, float* __restrict__ y,
                                                                int S, int64_t count) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i + 4 <= count) {
        const f32x4 v = sum_planes<f32x4>(
            [&](int q) { return *reinterpret_cast<const f32x4*>(part + q * count + i); }, S);
        *reinterpret_cast<f32x4*>(y + i) = v;
    } else {
        for (int64_t e = i; e < count; ++e) y[e] = sum_planes<float>([&](int q) { return part[q * count + e]; }, S);
    }
}

// The same sum with rows of `cols` elements written `ldy` floats apart.
__global__ void __launch_bounds__(256) gemm_split_reduce_strided_kernel(const float* __restrict__ part,
                                                                        float* __restrict__ y, int S, int64_t count,
                                                                        int64_t cols, int64_t ldy) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    y[(i / cols) * ldy + i % cols] = sum_planes<float>([&](int q) { return part[q * count + i]; }, S);
}

// The split sums of a group: element e of segment i (e - e_begin_i = r n_i + c)
// goes to y_i[r ldy_i + c], the planes added in split order.
__global__ void __launch_bounds__(256) gemm_split_reduce_group_kernel(GemmGroup g, int64_t M, int S, int64_t total) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= total) return;
    int i = 0;
#pragma unroll
    for (int t = 1; t < kGemmGroupMax; ++t)
        if (t < g.count && e >= g.e_begin[t]) i = t;
    const int64_t local = e - g.e_begin[i], n = g.n[i], count = M * n;
    const float* p = g.part[i] + local;
    g.y[i][(local / n) * g.ldy[i] + local % n] = sum_planes<float>([&](int q) { return p[q * count]; }, S);
}

// The same with four consecutive elements per thread, where every n_i and
// ldy_i is a multiple of 4 and every y_i 16-byte aligned (then no group of
// four crosses a row, and every load and store is one 16-byte access).
__global__ void __launch_bounds__(256) gemm_split_reduce_group4_kernel(GemmGroup g, int64_t M, int S, int64_t total) {
    const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (e >= total) return;
    int i = 0;
#pragma unroll
    for (int t = 1; t < kGemmGroupMax; ++t)
        if (t < g.count && e >= g.e_begin[t]) i = t;
    const int64_t local = e - g.e_begin[i], n = g.n[i], count = M * n;
    const float* p = g.part[i] + local;
    const f32x4 v = sum_planes<f32x4>([&](int q) { return *reinterpret_cast<const f32x4*>(p + q * count); }, S);
    *reinterpret_cast<f32x4*>(g.y[i] + (local / n) * g.ldy[i] + local % n) = v;
}

}  // namespace

bool gemm_bf16_supported(int qtype, int64_t m, int64_t n, int64_t k) {
    // K-steps of 64 come in pairs (the loop is unrolled by two or four); k <=
    // 2^22 keeps the X and W buffer offsets of a tile below 2^31
    const int64_t kq = qtype == kTypeQ80 ? 128 : (qtype == kTypeQ4K || qtype == kTypeQ6K) ? kQKElems : 0;
    return kq > 0 && m > 0 && n > 0 && k > 0 && k % kq == 0 && m <= 0x7FFFFFFF && n <= 0x7FFFFFFF &&
           k <= (int64_t)1 << 22 && ((n + kBN - 1) / kBN) * ((m + kBM - 1) / kBM) <= 0x7FFFFFFF;
}

// K-splits for a GEMM shape: the largest S in {1, 2, 4, 8} that keeps the grid
// within one round of 256 one-per-CU workgroups (tiles * S <= 256) and every
// split at an even count of at least 4 K-steps. Shapes that fill the GPU are
// not split: that would only trade tail balance for partial-sum traffic.
// 512 x 14336 x 4096: 1; 512 x 4096 x 14336: 4; 512 x 1024 x 4096: 8.
static int splits_for_tiles(int64_t tiles, int64_t k) {
    const int64_t kCUs = 256;
    const int64_t ksteps = k / kBK;
    int best = 1;
    for (int sp = 2; sp <= 8; sp *= 2) {
        if (ksteps % (2 * sp) || ksteps / sp < 4 || tiles * sp > kCUs) break;
        best = sp;
    }
    return best;
}

int gemm_bf16_splits(int64_t m, int64_t n, int64_t k) {
    return splits_for_tiles(((n + kBN - 1) / kBN) * ((m + kBM - 1) / kBM), k);
}

// A group splits K for its total tile count (q|k|v of Llama-3-8B at m = 512:
// 96 tiles, 2 splits, where q alone takes 4 and k or v alone 8).
int gemm_bf16_group_splits(int count, const int64_t* n, int64_t m, int64_t k) {
    int64_t tiles = 0;
    for (int i = 0; i < count; ++i) tiles += ((n[i] + kBN - 1) / kBN) * ((m + kBM - 1) / kBM);
    return splits_for_tiles(tiles, k);
}

size_t gemm_bf16_group_scratch(int count, const int64_t* n, int64_t m, int64_t k) {
    const int sp = gemm_bf16_group_splits(count, n, m, k);
    if (sp == 1) return 0;
    size_t cols = 0;
    for (int i = 0; i < count; ++i) cols += (size_t)n[i];
    return (size_t)sp * (size_t)m * cols * sizeof(float);
}

size_t gemm_bf16_scratch(int64_t m, int64_t n, int64_t k) {
    const int sp = gemm_bf16_splits(m, n, k);
    return sp > 1 ? (size_t)sp * (size_t)m * (size_t)n * sizeof(float) : 0;
}

hipError_t launch_split_reduce(const float* part, float* y, int splits, int64_t rows, int64_t cols, int64_t ldy,
                               hipStream_t stream) {
    const int64_t count = rows * cols;
    if (count <= 0) return hipSuccess;
    if (ldy == cols) {
        const int64_t threads = (count + 3) / 4;
        gemm_split_reduce_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream>>>(part, y, splits,
                                                                                                     count);
    } else {
        gemm_split_reduce_strided_kernel<<<dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream>>>(
            part, y, splits, count, cols, ldy);
    }
    return hipGetLastError();
}

hipError_t launch_gemm_bf16(int qtype, const uint8_t* w, const uint16_t* x, float* y, int64_t m, int64_t n, int64_t k,
                            hipStream_t stream, float* part) {
    if (!gemm_bf16_supported(qtype, m, n, k)) return hipErrorInvalidValue;
    int sp = gemm_bf16_splits(m, n, k);
    if (sp > 1 && !part) sp = 1;                           // no scratch: one split
    const int64_t tiles = ((n + kBN - 1) / kBN) * ((m + kBM - 1) / kBM);
    if (tiles * sp > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 grid((unsigned)(tiles * sp)), block(512);
    // loads two K-steps ahead where the step count per split is a multiple of four
    const bool ahead2 = (k / kBK / sp) % 4 == 0;
    switch (qtype) {
        case kTypeQ4K:
            if (ahead2) gemm_bf16_kernel<kTypeQ4K, 2><<<grid, block, 0, stream>>>(w, x, y, (int)m, (int)n, (int)k, sp, part);
            else gemm_bf16_kernel<kTypeQ4K, 1><<<grid, block, 0, stream>>>(w, x, y, (int)m, (int)n, (int)k, sp, part);
            break;
        case kTypeQ6K:
            if (ahead2) gemm_bf16_kernel<kTypeQ6K, 2><<<grid, block, 0, stream>>>(w, x, y, (int)m, (int)n, (int)k, sp, part);
            else gemm_bf16_kernel<kTypeQ6K, 1><<<grid, block, 0, stream>>>(w, x, y, (int)m, (int)n, (int)k, sp, part);
            break;
        case kTypeQ80:
            if (ahead2) gemm_bf16_kernel<kTypeQ80, 2><<<grid, block, 0, stream>>>(w, x, y, (int)m, (int)n, (int)k, sp, part);
            else gemm_bf16_kernel<kTypeQ80, 1><<<grid, block, 0, stream>>>(w, x, y, (int)m, (int)n, (int)k, sp, part);
            break;
        default: return hipErrorInvalidValue;
    }
    if (sp > 1) {
        const int64_t count = m * n, threads = (count + 3) / 4;
        gemm_split_reduce_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream>>>(part, y, sp, count);
    }
    return hipGetLastError();
}

hipError_t launch_gemm_bf16_group(int count, const int* qtypes, const uint8_t* const* w, const int64_t* n,
                                  float* const* y, const int64_t* ldy, const uint16_t* x, int64_t m, int64_t k,
                                  hipStream_t stream, float* part) {
    if (count < 1 || count > kGemmGroupMax) return hipErrorInvalidValue;
    for (int i = 0; i < count; ++i)
        if (!gemm_bf16_supported(qtypes[i], m, n[i], k) || ldy[i] < n[i] || ldy[i] > 0x7FFFFFFF)
            return hipErrorInvalidValue;
    int sp = gemm_bf16_group_splits(count, n, m, k);
    if (sp > 1 && !part) sp = 1;                           // no scratch: one split
    GemmGroup g{};
    g.count = count;
    const int64_t mtiles = (m + kBM - 1) / kBM;
    int64_t wg = 0, e = 0;
    float* pp = part;
    for (int i = 0; i < count; ++i) {
        g.w[i] = w[i];
        g.y[i] = y[i];
        g.n[i] = n[i];
        g.ldy[i] = ldy[i];
        g.qtype[i] = qtypes[i];
        g.wg_begin[i] = wg;
        g.e_begin[i] = e;
        g.part[i] = sp > 1 ? pp : nullptr;
        wg += ((n[i] + kBN - 1) / kBN) * mtiles * sp;
        e += m * n[i];
        if (sp > 1) pp += (int64_t)sp * m * n[i];
    }
    if (wg > 0x7FFFFFFF) return hipErrorInvalidValue;
    const bool ahead2 = (k / kBK / sp) % 4 == 0;
    if (ahead2) gemm_bf16_group_kernel<2><<<dim3((unsigned)wg), dim3(512), 0, stream>>>(g, x, (int)m, (int)k, sp);
    else gemm_bf16_group_kernel<1><<<dim3((unsigned)wg), dim3(512), 0, stream>>>(g, x, (int)m, (int)k, sp);
    if (sp > 1) {
        bool vec4 = true;
        for (int i = 0; i < count; ++i)
            vec4 = vec4 && n[i] % 4 == 0 && ldy[i] % 4 == 0 && (reinterpret_cast<uintptr_t>(y[i]) & 15) == 0;
        if (vec4)
            gemm_split_reduce_group4_kernel<<<dim3((unsigned)((e / 4 + 255) / 256)), dim3(256), 0, stream>>>(g, m, sp, e);
        else
            gemm_split_reduce_group_kernel<<<dim3((unsigned)((e + 255) / 256)), dim3(256), 0, stream>>>(g, m, sp, e);
    }
    return hipGetLastError();
}

}  // namespace frq
