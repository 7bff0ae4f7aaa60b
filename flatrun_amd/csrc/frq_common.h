// Shared device helpers for the gfx950 GGUF kernels.
//
// Block formats (GGML type id, bytes, elements), as in the reference's type
// table src/flatrun/backend/gguf.py:59-86:
//   Q8_0  id 8   34 B /  32   [d f16][qs i8 x32]
//   Q4_K  id 12 144 B / 256   [d f16][dmin f16][scales 12][qs 128]
//   Q5_K  id 13 176 B / 256   [d f16][dmin f16][scales 12][qh 32][qs 128]
//   Q6_K  id 14 210 B / 256   [ql 128][qh 64][scales i8 x16][d f16]
//   Q1_0  id 41  18 B / 128   [d f16][qs 16]  (1 sign bit per element, LSB first)
//   Q4_0  id 2   18 B /  32   [d f16][qs 16]
//   Q5_0  id 6   22 B /  32   [d f16][qh 4][qs 16]
//   Q5_1  id 7   24 B /  32   [d f16][m f16][qh 4][qs 16]
//
// All code here is compiled with -ffp-contract=off: every product and sum
// rounds on its own exactly where it is written, which the bit-exact dequant
// relies on. Kernels that want an FMA call __builtin_fmaf explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frq {

template <int V>
struct Int {
    static constexpr int value = V;
};

// Calls f(Int<J>{}) for J = B .. E-1 with J a compile-time constant, so array
// indices derived from J stay constant and the arrays stay in registers.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(Int<B>{});
        static_for<B + 1, E>(f);
    }
}

constexpr int kQ80Bytes = 34, kQ80Elems = 32;
constexpr int kQ4KBytes = 144, kQ5KBytes = 176, kQ6KBytes = 210, kQKElems = 256;
constexpr int kQ10Bytes = 18, kQ10Elems = 128;
constexpr int kQ40Bytes = 18, kQ50Bytes = 22, kQ51Bytes = 24;   // 32 elements each

// Raw (untyped) buffer descriptor over [base, base + bytes). Loads through it
// take a 32-bit VGPR byte offset against a base held in scalar registers, so
// a lane pays no 64-bit address arithmetic, and an access past `bytes` reads
// zeros instead of touching memory. Word 3 is the gfx9-family raw-access
// setting (32-bit data format, no swizzle, no index).
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferWord3);
}
__device__ __forceinline__ uint4 bload_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void bload_b96(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t (&wv)[3]) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b96(r, (int)off, 0, 0);
    wv[0] = v[0];
    wv[1] = v[1];
    wv[2] = v[2];
}
__device__ __forceinline__ uint32_t bload_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

// IEEE binary16 -> binary32. v_cvt_f32_f16 is exact for every finite input,
// subnormals included (f16 denormals are enabled in the default FP mode).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
    return (float)v;
}

// 6-bit (scale, min) pair j of a K-quant 12-byte scale field, given as three
// little-endian dwords s0 = bytes 0..3, s1 = bytes 4..7, s2 = bytes 8..11
// (get_scale_min_k4: gguf.py:135-163, q4_k.h:89-110).
__device__ __forceinline__ void k4_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                             uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int b = 8 * (j - 4);
        sc = ((s2 >> b) & 15u) | (((s0 >> (b + 6)) & 3u) << 4);
        m = ((s2 >> (b + 4)) & 15u) | (((s1 >> (b + 6)) & 3u) << 4);
    }
}

// Four bytes starting at a 2-byte aligned device address (Q8_0 / Q6_K / Q1_0
// blocks are only 2-byte aligned inside a row): one dword load when the
// address is 4-aligned, else two 16-bit loads. Never touches a byte outside
// [p, p + 4), so the last field of the last block cannot read past the end
// of the buffer.
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
    if ((reinterpret_cast<uintptr_t>(p) & 3) == 0) return *reinterpret_cast<const uint32_t*>(p);
    const uint32_t lo = *reinterpret_cast<const uint16_t*>(p);
    const uint32_t hi = *reinterpret_cast<const uint16_t*>(p + 2);
    return lo | (hi << 16);
}

// Bitwise ops the optimiser cannot see through. After a plain `w & 0x0F0F0F0F`
// LLVM knows every byte is < 16 and rewrites each later byte -> float
// conversion as a bit-field extract plus v_cvt_f32_ubyte0 (2 VALU ops per
// element); hiding the mask keeps the single-op v_cvt_f32_ubyte{0,1,2,3}.
__device__ __forceinline__ uint32_t vand(uint32_t a, uint32_t mask) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "s"(mask), "v"(a));
    return r;
}
// (a & mask) | c
__device__ __forceinline__ uint32_t vand_or(uint32_t a, uint32_t mask, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(c));
    return r;
}
// Both nibble planes of a qs dword as eight floats: f[0..3] = the low nibbles
// of bytes 0..3, f[4..7] = 16 * the high nibbles. One asm block, so the eight
// conversions issue back to back and the FMAs that consume them come later;
// left to itself the compiler pairs every conversion with its FMA, and the
// FMA then waits on the conversion it follows.
// Masks come in registers: kernels that give each lane its own plane order
// (see the Q4_K GEMV) pass per-lane masks, f[0..3] then being the lane's
// "own" plane.
__device__ __forceinline__ void nibbles8(uint32_t w, float (&f)[8], uint32_t mask_a = 0x0F0F0F0Fu,
                                         uint32_t mask_b = 0xF0F0F0F0u) {
    uint32_t lo, hi;
    asm("v_and_b32 %0, %10, %12\n\t"
        "v_and_b32 %1, %11, %12\n\t"
        "v_cvt_f32_ubyte0 %2, %0\n\t"
        "v_cvt_f32_ubyte0 %6, %1\n\t"
        "v_cvt_f32_ubyte1 %3, %0\n\t"
        "v_cvt_f32_ubyte1 %7, %1\n\t"
        "v_cvt_f32_ubyte2 %4, %0\n\t"
        "v_cvt_f32_ubyte2 %8, %1\n\t"
        "v_cvt_f32_ubyte3 %5, %0\n\t"
        "v_cvt_f32_ubyte3 %9, %1"
        : "=&v"(lo), "=&v"(hi), "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3]), "=&v"(f[4]), "=&v"(f[5]),
          "=&v"(f[6]), "=&v"(f[7])
        : "v"(mask_a), "v"(mask_b), "v"(w));
}

// SwiGLU's silu(g) * u with the forwarder's operations and roundings
// (model/qwen2.py:1703-1740): e = exp(-g); e = e + 1; e = 1 / e; e = e * g;
// e * u -- each rounded, no FMA, the reciprocal a correctly rounded division.
__device__ __forceinline__ float silu_mul(float g, float u) {
    float e = expf(-g);
    e = e + 1.0f;
    e = 1.0f / e;
    e = e * g;
    return e * u;
}

// The value of the fp8 (e4m3) code 1: a power of two u such that a byte
// holding q < 16 converts to q * u exactly (codes below 8 are subnormal,
// 8 .. 15 have the smallest exponent; both read as q * u).
__device__ __forceinline__ float fp8_unit() {
    return __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0];
}

// The eight nibbles of w as q * fp8_unit(): f[0..3] the low nibbles of bytes
// 0..3, f[4..7] the high ones. Seven VALU operations for eight values.
__device__ __forceinline__ void nibbles8_fp8(uint32_t w, float (&f)[8]) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false), b = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
    const auto c = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false), e = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
    f[0] = a[0]; f[1] = a[1]; f[2] = b[0]; f[3] = b[1];
    f[4] = c[0]; f[5] = c[1]; f[6] = e[0]; f[7] = e[1];
}

// Four 6-bit Q6_K codes q as the signed bytes 4 (q - 32), converted to float
// exactly (one sign-extending byte-select convert each): lo holds the low
// nibbles at bits 2..5 of each byte, hi2 the two high bits at bits 6, 7 with
// the upper one flipped (so bit 7 is the sign of q - 32). Byte value:
// 4 lo + 64 (hi ^ 2) read as int8 = 4 (lo + 16 hi - 32).
__device__ __forceinline__ void q6_quad_signed(uint32_t lo, uint32_t hi2, float (&f)[4]) {
    uint32_t t, q;
    asm("v_and_b32 %0, %6, %7\n\t"
        "v_and_or_b32 %1, %8, %9, %0\n\t"
        "v_cvt_f32_i32_sdwa %2, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f32_i32_sdwa %3, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f32_i32_sdwa %4, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f32_i32_sdwa %5, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=&v"(t), "=&v"(q), "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3])
        : "s"(0xC0C0C0C0u), "v"(hi2), "v"(lo), "s"(0x3C3C3C3Cu));
}

// Byte b of w as float: one v_cvt_f32_ubyte<b>.
__device__ __forceinline__ float byte_f(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
// Four DPP steps reduce each 16-lane row, two cross-row swizzles finish.
// Only for controls that give every lane a source inside its row (quad_perm,
// row_half_mirror, row_mirror): the old value is never used, so it is left
// undefined and the compiler folds the move into the add that consumes it.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float acc, float v) {
    // acc + v[src lane]; rows outside ROW_MASK keep acc unchanged (old = 0).
    return acc + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                        0xF, false));
}

// Sum over the 64 lanes of a wavefront, in VALU only (no LDS round trip):
// four DPP steps give every lane its 16-lane row sum, then row_bcast:15 and
// row_bcast:31 fold rows 0..3 upwards. Only lane 63 holds the total.
__device__ __forceinline__ float wave_sum_lane63(float v) {
    v += dpp_mov<0xB1>(v);           // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);           // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);          // row_half_mirror
    v += dpp_mov<0x140>(v);          // row_mirror: every lane holds its row's sum
    v = dpp_add<0x142, 0xA>(v, v);   // row_bcast:15 -> rows 1, 3 add rows 0, 2
    v = dpp_add<0x143, 0xC>(v, v);   // row_bcast:31 -> rows 2, 3 add lane 31
    return v;
}

// Issue priority by row progress, for the row-ring GEMV bodies. A SIMD's
// instruction arbiter serves its oldest ready wavefront first, vector memory
// instructions included, so without priorities the wavefronts dispatched
// last in a workgroup receive their first rows only when the older ones have
// finished theirs, and the workgroup ends with a few wavefronts running
// alone, each limited by its own issue chain (clock stamps per row at
// 3584 x 18944: the last two of ten wavefronts finished 11k cycles after the
// first four). A wavefront at row j of R runs at priority 3 - 4j/R, so the
// ones behind issue and load first and the workgroup's wavefronts advance
// together. s_setprio changes only this wavefront's arbitration priority.
template <bool ON, int R, int J>
__device__ __forceinline__ void row_priority() {
    if constexpr (ON) __builtin_amdgcn_s_setprio(3 - (4 * J) / R);
}

// The four in-row DPP steps of wave_sum_lane63: every lane ends with the sum
// of its 16-lane DPP row. Callers park the four row sums (lanes 15, 31, 47,
// 63) in LDS and add them with the other waves' in a fixed order, which
// saves the two row_bcast steps and their zeroed operands per reduction.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// load(0) + load(1) + ... + load(S - 1), added in that order (fixed bits),
// with the loads issued eight at a time before they are added: the sum of S
// split-K partial planes with eight loads in flight instead of one round
// trip per plane.
template <typename V, typename Load>
__device__ __forceinline__ V sum_planes(Load load, int S) {
    V v = load(0);
    int q = 1;
    for (; q + 8 <= S; q += 8) {
        V t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = load(q + u);
#pragma unroll
        for (int u = 0; u < 8; ++u) v += t[u];
    }
    for (; q < S; ++q) v += load(q);
    return v;
}

// Decoded per-lane constants for the two 6-bit (scale, min) pairs 2g, 2g+1
// of a K-quant block (get_scale_min_k4, gguf.py:135-163). With s0, s1, s2 the
// three scale dwords:
//   j < 4 : sc = bits [8j, 8j+6) of s0,          m = same bits of s1
//   j >= 4: sc = bits [8(j-4), +4) of s2 | bits [8(j-4)+6, +2) of s0 << 4
//           m  = bits [8(j-4)+4, +4) of s2 | bits [8(j-4)+6, +2) of s1 << 4
// One v_bfe with lane-variable offset/width covers both cases; the high-bit
// term has width 0 for j < 4.
struct ScaleDecode {
    bool hi;                  // g >= 2: low bits come from s2
    uint32_t o_sc, o_m, w_a;  // offsets / width of the low-bit field (pair 2g)
    uint32_t o_b, w_b;        // offset / width of the high-bit field (pair 2g)

    __device__ __forceinline__ explicit ScaleDecode(int g) {
        hi = g >= 2;
        const uint32_t j = 2 * g;
        o_sc = hi ? 8 * (j - 4) : 8 * j;
        o_m = hi ? 8 * (j - 4) + 4 : 8 * j;
        w_a = hi ? 4 : 6;
        o_b = hi ? 8 * (j - 4) + 6 : 0;
        w_b = hi ? 2 : 0;
    }

    // pair 2g -> (sc0, m0), pair 2g+1 -> (sc1, m1); the second pair's fields
    // sit 8 bits above the first's.
    __device__ __forceinline__ void operator()(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc0, uint32_t& m0,
                                               uint32_t& sc1, uint32_t& m1) const {
        const uint32_t a_sc = hi ? s2 : s0, a_m = hi ? s2 : s1;
        sc0 = __builtin_amdgcn_ubfe(a_sc, o_sc, w_a) | (__builtin_amdgcn_ubfe(s0, o_b, w_b) << 4);
        sc1 = __builtin_amdgcn_ubfe(a_sc, o_sc + 8, w_a) | (__builtin_amdgcn_ubfe(s0, o_b + 8, w_b) << 4);
        m0 = __builtin_amdgcn_ubfe(a_m, o_m, w_a) | (__builtin_amdgcn_ubfe(s1, o_b, w_b) << 4);
        m1 = __builtin_amdgcn_ubfe(a_m, o_m + 8, w_a) | (__builtin_amdgcn_ubfe(s1, o_b + 8, w_b) << 4);
    }
};

// One (scale, min) pair j of a K-quant block per lane (same fields as
// k4_scale_min): lanes that share a block decode one pair each and read the
// others' with DPP instead of all decoding every pair they use.
struct PairDecode {
    bool hi;                          // j >= 4: low bits come from s2
    uint32_t o_sc, o_m, w_a, o_b, w_b;

    __device__ __forceinline__ explicit PairDecode(int j) {
        hi = j >= 4;
        const uint32_t b = hi ? 8u * (uint32_t)(j - 4) : 8u * (uint32_t)j;
        o_sc = b;
        o_m = hi ? b + 4 : b;
        w_a = hi ? 4 : 6;
        o_b = hi ? b + 6 : 0;
        w_b = hi ? 2 : 0;
    }
    __device__ __forceinline__ void operator()(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc,
                                               uint32_t& m) const {
        const uint32_t a_sc = hi ? s2 : s0, a_m = hi ? s2 : s1;
        sc = __builtin_amdgcn_ubfe(a_sc, o_sc, w_a) | (__builtin_amdgcn_ubfe(s0, o_b, w_b) << 4);
        m = __builtin_amdgcn_ubfe(a_m, o_m, w_a) | (__builtin_amdgcn_ubfe(s1, o_b, w_b) << 4);
    }
};

template <int CPL>
struct Q4KRow {
    uint4 hd;
    uint4 q[CPL];
};

}  // namespace frq
