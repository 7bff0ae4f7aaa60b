// Shared device helpers for the gfx950 GGUF kernels.
//
// Block formats (GGML type id, bytes, elements), as in the reference's type
// table src/flatrun/backend/gguf.py:59-86:
//   Q8_0  id 8   34 B /  32   [d f16][qs i8 x32]
//   Q4_K  id 12 144 B / 256   [d f16][dmin f16][scales 12][qs 128]
//   Q5_K  id 13 176 B / 256   [d f16][dmin f16][scales 12][qh 32][qs 128]
//   Q6_K  id 14 210 B / 256   [ql 128][qh 64][scales i8 x16][d f16]
//   Q1_0  id 41  18 B / 128   [d f16][qs 16]  (1 sign bit per element, LSB first)
//
// All code here is compiled with -ffp-contract=off: every product and sum
// rounds on its own exactly where it is written, which the bit-exact dequant
// relies on. Kernels that want an FMA call __builtin_fmaf explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frq {

constexpr int kQ80Bytes = 34, kQ80Elems = 32;
constexpr int kQ4KBytes = 144, kQ5KBytes = 176, kQ6KBytes = 210, kQKElems = 256;
constexpr int kQ10Bytes = 18, kQ10Elems = 128;

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
// Byte b of w as float: one v_cvt_f32_ubyte<b>.
__device__ __forceinline__ float byte_f(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
// Four DPP steps reduce each 16-lane row, two cross-row swizzles finish.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
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

}  // namespace frq
