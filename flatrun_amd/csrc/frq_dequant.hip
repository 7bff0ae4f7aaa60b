// GGUF block dequant kernels for gfx950: raw blocks in HBM -> fp32, or fp16.
//
// Bit-exact contract with the reference NumPy decoders
// (src/flatrun/dequant/gguf.py), which fixes the rounding sequence:
//   Q8_0  fl32(q * d)                                     gguf.py:112-127
//   Q4_K  fl32(fl32(fl32(d*sc) * q) - fl32(dmin*m))       gguf.py:166-220
//   Q5_K  fl32(fl64(fl32(d*sc) * v) - fl32(dmin*m))       gguf.py:223-263
//   Q6_K  fl32(fl32(d*sc) * (q - 32))                     gguf.py:365-420
//   Q1_0  +d / -d by bit, LSB first                       gguf.py:266-299
//   Q4_0  fl32((q - 8) * d)                               gguf.py:81-107
//   Q5_0  fl32((q - 16) * d), q = nibble | qh bit << 4    gguf.py:302-330
//   Q5_1  fl32(fl32(d * q) + m)                           gguf.py:333-362
// (every product above except Q4_K's and Q5_K's is exact in fp32: an fp16
// scale times an integer of at most 6 bits).
// This translation unit is built with -ffp-contract=off, so none of the
// products above is fused into the following add.
//
// Work mapping: one thread writes four consecutive fp32 outputs (one
// dwordx4 store), so each store instruction of a wavefront writes 1 KiB of
// contiguous fp32; the kernel is bound by the 4 B/element write stream. With fp16 output every thread writes eight (one dwordx4
// store of 2 B elements: two four-output decodes for the other formats).
// Four outputs always share one scale, so each decode reads one scale pair.
// A ragged last block (element count not a multiple of the block) is decoded
// and the tail trimmed, as the reference's _finish does (gguf.py:61-73).
// fp16 output: the reference decodes into an fp32 array and _finish casts it
// (astype, round to nearest even; dequant_handle's default dtype is float16,
// loader.py:51-88), so each fp32 value above is rounded to fp16 once with
// v_cvt_f16_f32 (nearest even, overflow to inf, fp16 subnormals kept) and
// stored as 2 B/element.
#include <type_traits>

#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {

// Output stores are non-temporal (`nt`): a dequantized matrix is written
// once and not read again by this kernel, and streaming it past the caches
// saves 4-9 % against ordinary write-allocating stores, with weights and
// outputs both cold (Q4_K 18944 x 3584 to fp32: 64.4 -> 61.3 us; Q6_K
// 152064 x 3584: 521-524 -> 491-494 us; fp16 Q6_K 304 -> 290 us). The
// stores also leave the last-level cache to the weights, so a weight that
// is read again soon after (a few hundred MB of them) stays cached.
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store4(float* __restrict__ y, int64_t e0, int64_t n, float v0, float v1,
                                       float v2, float v3) {
    if (e0 + 3 < n && ((reinterpret_cast<uintptr_t>(y + e0) & 15) == 0)) {
        __builtin_nontemporal_store(f32x4v{v0, v1, v2, v3}, reinterpret_cast<f32x4v*>(y + e0));
    } else {
        if (e0 + 0 < n) y[e0 + 0] = v0;
        if (e0 + 1 < n) y[e0 + 1] = v1;
        if (e0 + 2 < n) y[e0 + 2] = v2;
        if (e0 + 3 < n) y[e0 + 3] = v3;
    }
}

// fp16 bits of an fp32 value, rounded to nearest even. The conversion is its
// own instruction: left to itself the compiler folds "multiply, then
// convert" into v_fma_mix*_f16, which rounds the exact product once to fp16
// (the reference rounds to fp32 first) and turns a -0 product into +0.
__device__ __forceinline__ uint32_t f16_bits(float v) {
    uint32_t r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(v));
    return r & 0xFFFFu;
}

__device__ __forceinline__ void store4(uint16_t* __restrict__ y, int64_t e0, int64_t n, float v0, float v1,
                                       float v2, float v3) {
    const uint32_t h0 = f16_bits(v0), h1 = f16_bits(v1), h2 = f16_bits(v2), h3 = f16_bits(v3);
    if (e0 + 3 < n && ((reinterpret_cast<uintptr_t>(y + e0) & 7) == 0)) {
        __builtin_nontemporal_store(u32x2v{h0 | (h1 << 16), h2 | (h3 << 16)}, reinterpret_cast<u32x2v*>(y + e0));
    } else {
        if (e0 + 0 < n) y[e0 + 0] = (uint16_t)h0;
        if (e0 + 1 < n) y[e0 + 1] = (uint16_t)h1;
        if (e0 + 2 < n) y[e0 + 2] = (uint16_t)h2;
        if (e0 + 3 < n) y[e0 + 3] = (uint16_t)h3;
    }
}

__device__ __forceinline__ void store8(float* __restrict__ y, int64_t e0, int64_t n, const float (&v)[8]) {
    store4(y, e0, n, v[0], v[1], v[2], v[3]);
    store4(y, e0 + 4, n, v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void store8(uint16_t* __restrict__ y, int64_t e0, int64_t n, const float (&v)[8]) {
    uint32_t h[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) h[c] = f16_bits(v[c]);
    if (e0 + 7 < n && ((reinterpret_cast<uintptr_t>(y + e0) & 15) == 0)) {
        __builtin_nontemporal_store(
            u32x4v{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)},
            reinterpret_cast<u32x4v*>(y + e0));
    } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
            if (e0 + c < n) y[e0 + c] = (uint16_t)h[c];
    }
}

__device__ __forceinline__ float ub(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

// k4_scale_min for a pair index j that differs between the lanes of a wave:
// both forms computed and one selected, so no branch stands between the
// block's loads and the whole 16-byte header stays one load.
__device__ __forceinline__ void k4_scale_min_sel(uint32_t s0, uint32_t s1, uint32_t s2, int j, uint32_t& sc,
                                                 uint32_t& m) {
    const uint32_t b = 8u * (uint32_t)(j & 3);
    const uint32_t lo_sc = (s0 >> b) & 63u, lo_m = (s1 >> b) & 63u;
    const uint32_t hi_sc = ((s2 >> b) & 15u) | (((s0 >> (b + 6)) & 3u) << 4);
    const uint32_t hi_m = ((s2 >> (b + 4)) & 15u) | (((s1 >> (b + 6)) & 3u) << 4);
    sc = j < 4 ? lo_sc : hi_sc;
    m = j < 4 ? lo_m : hi_m;
}

// Decoders: v = the elements e0 .. e0 + E - 1 (E = 8 for Q4_K / Q5_K with
// fp16 output, whose eight share one sub-block, else 4), all inside the
// allocated blocks for any e0 < n that is a multiple of the outputs per
// thread (every block holds a multiple of 8 elements).

// Q4_K and Q5_K: E = 4 or 8 outputs, all in one 32-element sub-block. fp32
// output takes E = 4, one 16-byte store per thread, so every store
// instruction of a wave writes 1 KiB contiguous (E = 8 with two stores per
// thread measured 79 against 72 us for 18944 x 3584); fp16 output takes
// E = 8, whose eight halves are one 16-byte store.
template <int E_>
struct DecQ4K {
    static constexpr int E = E_;
    __device__ static void decode(const uint8_t* __restrict__ w, int64_t e0, float (&v)[E_]) {
        const int64_t b = e0 / kQKElems;
        const int o = (int)(e0 % kQKElems);
        const int j = o >> 5, i = o & 31, g = j >> 1;
        const uint8_t* blk = w + b * kQ4KBytes;
        const uint4 hd = *reinterpret_cast<const uint4*>(blk);
        uint32_t sc, m;
        k4_scale_min_sel(hd.y, hd.z, hd.w, j, sc, m);
        const float s = f16_bits_to_f32(hd.x) * (float)sc;
        const float t = f16_bits_to_f32(hd.x >> 16) * (float)m;
        const uint32_t sh = (j & 1) ? 4u : 0u;
        if constexpr (E_ == 8) {
            const uint2 qq = *reinterpret_cast<const uint2*>(blk + 16 + 32 * g + i);
            const uint32_t q0 = (qq.x >> sh) & 0x0F0F0F0Fu, q1 = (qq.y >> sh) & 0x0F0F0F0Fu;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                v[c] = s * ub(q0, c) - t;
                v[4 + c] = s * ub(q1, c) - t;
            }
        } else {
            const uint32_t q0 = (*reinterpret_cast<const uint32_t*>(blk + 16 + 32 * g + i) >> sh) & 0x0F0F0F0Fu;
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c] = s * ub(q0, c) - t;
        }
    }
};

template <int E_>
struct DecQ5K {
    static constexpr int E = E_;
    __device__ static void decode(const uint8_t* __restrict__ w, int64_t e0, float (&v)[E_]) {
        const int64_t b = e0 / kQKElems;
        const int o = (int)(e0 % kQKElems);
        const int j = o >> 5, i = o & 31, g = j >> 1;
        const uint8_t* blk = w + b * kQ5KBytes;
        const uint4 hd = *reinterpret_cast<const uint4*>(blk);
        uint32_t sc, m;
        k4_scale_min_sel(hd.y, hd.z, hd.w, j, sc, m);
        const double s = (double)(f16_bits_to_f32(hd.x) * (float)sc);   // fl32(d*sc), widened exactly
        const double t = (double)(f16_bits_to_f32(hd.x >> 16) * (float)m);
        const uint32_t sh = (j & 1) ? 4u : 0u;
        uint32_t qw[2], hw[2];
        if constexpr (E_ == 8) {
            const uint2 qq = *reinterpret_cast<const uint2*>(blk + 48 + 32 * g + i);
            const uint2 hh = *reinterpret_cast<const uint2*>(blk + 16 + i);
            qw[0] = qq.x, qw[1] = qq.y, hw[0] = hh.x, hw[1] = hh.y;
        } else {
            qw[0] = *reinterpret_cast<const uint32_t*>(blk + 48 + 32 * g + i);
            hw[0] = *reinterpret_cast<const uint32_t*>(blk + 16 + i);
            qw[1] = hw[1] = 0;
        }
#pragma unroll
        for (int p = 0; p < E_ / 4; ++p) {
            const uint32_t q = ((qw[p] >> sh) & 0x0F0F0F0Fu) | (((hw[p] >> j) & 0x01010101u) << 4);   // q4 + 16*bit
#pragma unroll
            for (int c = 0; c < 4; ++c) v[4 * p + c] = (float)(s * (double)((q >> (8 * c)) & 0xFFu) - t);
        }
    }
};

// Q6_K: E = 4 (fp32 output) or 8 (fp16) consecutive elements 128h + 32k + l
// .. + E - 1, which share one 16-element scale (l is a multiple of E).
template <int E_>
struct DecQ6K {
    static constexpr int E = E_;
    __device__ static void decode(const uint8_t* __restrict__ w, int64_t e0, float (&v)[E_]) {
        const int64_t b = e0 / kQKElems;
        const int o = (int)(e0 % kQKElems);
        const int h = o >> 7, k = (o >> 5) & 3, l = o & 31;   // element 128h + 32k + l
        const uint8_t* blk = w + b * kQ6KBytes;
        const int sc = (int)(int8_t)blk[192 + 8 * h + (l >> 4) + 2 * k];
        const float s = f16_bits_to_f32(ld_u16(blk + 208)) * (float)sc;
#pragma unroll
        for (int p = 0; p < E_ / 4; ++p) {
            uint32_t nib = ld_u32_a2(blk + 64 * h + 32 * (k & 1) + l + 4 * p);
            nib = ((k >= 2) ? (nib >> 4) : nib) & 0x0F0F0F0Fu;
            const uint32_t hb = (ld_u32_a2(blk + 128 + 32 * h + l + 4 * p) >> (2 * k)) & 0x03030303u;
            const uint32_t q = nib | (hb << 4);
#pragma unroll
            for (int c = 0; c < 4; ++c) v[4 * p + c] = s * (ub(q, c) - 32.0f);
        }
    }
};

struct DecQ80 {
    static constexpr int E = 4;
    __device__ static void decode(const uint8_t* __restrict__ w, int64_t e0, float (&v)[4]) {
        const int64_t b = e0 / kQ80Elems;
        const int o = (int)(e0 % kQ80Elems);
        const uint8_t* blk = w + b * kQ80Bytes;
        const float d = f16_bits_to_f32(ld_u16(blk));
        const uint32_t q = ld_u32_a2(blk + 2 + o);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = (float)(int)(int8_t)((q >> (8 * c)) & 0xFFu) * d;
    }
};

struct DecQ10 {
    static constexpr int E = 4;
    __device__ static void decode(const uint8_t* __restrict__ w, int64_t e0, float (&v)[4]) {
        const int64_t b = e0 / kQ10Elems;
        const int o = (int)(e0 % kQ10Elems);
        const uint8_t* blk = w + b * kQ10Bytes;
        const float d = f16_bits_to_f32(ld_u16(blk));
        const uint32_t bits = (uint32_t)blk[2 + (o >> 3)] >> (o & 7);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = ((bits >> c) & 1u) ? d : -d;
    }
};

// Q4_0 / Q5_0 / Q5_1: 32-element blocks; byte j of qs holds element j in its
// low nibble and element j + 16 in its high nibble; for Q5_x the 5th bit of
// element j (j < 16) is bit j of the little-endian qh word and of element
// j + 16 bit j + 16. Four outputs are four consecutive elements of one half:
// bytes 4p .. 4p+3 of qs (p = offset / 4 within the half).
template <int BB, int QS_OFF, bool FIVE, bool MIN>
struct DecQ32 {
    static constexpr int E = 4;
    __device__ static void decode(const uint8_t* __restrict__ w, int64_t e0, float (&v)[4]) {
        const int64_t b = e0 / 32;
        const int o = (int)(e0 % 32);
        const int half = o >> 4, j0 = o & 15;
        const uint8_t* blk = w + b * BB;
        const float d = f16_bits_to_f32(ld_u16(blk));
        const uint32_t qs = ld_u32_a2(blk + QS_OFF + j0);
        uint32_t qh = 0;
        if constexpr (FIVE) qh = ld_u32_a2(blk + (MIN ? 4 : 2)) >> (16 * half + j0);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint32_t q = (qs >> (8 * c + 4 * half)) & 15u;
            if constexpr (FIVE) q |= ((qh >> c) & 1u) << 4;
            if constexpr (MIN) {
                const float m = f16_bits_to_f32(ld_u16(blk + 2));
                v[c] = d * (float)q + m;
            } else {
                v[c] = (float)((int)q - (FIVE ? 16 : 8)) * d;
            }
        }
    }
};

// Outputs per thread: the decoder's E for fp32 (one 16-byte store per four);
// eight for fp16 (two 4-output decodes, one 16-byte store).
template <typename Dec, typename T>
constexpr int per_thread() {
    return (sizeof(T) == 2 || Dec::E == 8) ? 8 : 4;
}

template <typename Dec, typename T>
__device__ __forceinline__ void dequant_one(const uint8_t* __restrict__ w, T* __restrict__ y, int64_t n, int64_t e0) {
    constexpr int P = per_thread<Dec, T>();
    if constexpr (P == 8) {
        float v[8];
        if constexpr (Dec::E == 8) {
            Dec::decode(w, e0, v);
        } else {
            float a[4], b[4];
            Dec::decode(w, e0, a);
            Dec::decode(w, e0 + 4, b);   // e0 + 4 < the allocated elements (see above)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                v[c] = a[c];
                v[4 + c] = b[c];
            }
        }
        store8(y, e0, n, v);
    } else {
        float v[4];
        Dec::decode(w, e0, v);
        store4(y, e0, n, v[0], v[1], v[2], v[3]);
    }
}

// U groups of P outputs per thread, one grid width apart: every store
// instruction of a wave still writes contiguous memory, and the U groups'
// loads are in flight together, which keeps more bytes moving per wave.
// U = 2 for fp32 output (18944 x 3584: Q4_K 71 -> 66 us, Q4_0 70 -> 63,
// Q5_0 79 -> 72; Q6_K 152064 x 3584 563 -> 530), except Q8_0, whose wider
// blocks already keep the stream busy (64 vs 65 us); U = 1 for fp16 (Q6_K
// 359 vs 364 us at U = 2).
template <typename Dec, typename T, int U>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ w, T* __restrict__ y, int64_t n) {
    constexpr int P = per_thread<Dec, T>();
    const int64_t stride = (int64_t)P * gridDim.x * blockDim.x;
    const int64_t e0 = P * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t e = e0 + u * stride;
        if (e < n) dequant_one<Dec, T>(w, y, n, e);
    }
}

__global__ void __launch_bounds__(256) fill_kernel(float* __restrict__ y, float v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = v;
}

hipError_t launch_fill(float* y, float value, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    fill_kernel<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream>>>(y, value, n);
    return hipGetLastError();
}

// Plain streaming copy (16 B per lane, grid-stride). Used to calibrate the
// HBM traffic counters against a kernel whose traffic is known exactly.
__global__ void __launch_bounds__(256) copy16_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                     int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

hipError_t launch_copy(void* dst, const void* src, int64_t bytes, hipStream_t stream) {
    if (bytes <= 0) return hipSuccess;
    const int64_t n16 = bytes / 16;
    const int64_t blocks = (n16 + 255) / 256;
    copy16_kernel<<<dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, stream>>>(
        static_cast<uint4*>(dst), static_cast<const uint4*>(src), n16);
    return hipGetLastError();
}

// Plain streaming read: a contiguous slice per workgroup, 16 B per lane and
// eight loads in flight per lane, folded into a 32-bit XOR; workgroup b
// stores its XOR in out[b] (no atomics) and workgroup 0 zeroes the words past
// the grid. The read-only reference point beside copy16: a GEMV reads its
// weights once and writes almost nothing.
constexpr int kReadUnroll = 8;
__global__ void __launch_bounds__(256) read_xor_kernel(const uint4* __restrict__ src, int64_t n16,
                                                       uint32_t* __restrict__ out) {
    __shared__ uint32_t red[4];
    const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const int64_t b = (int64_t)blockIdx.x * per;
    const int64_t e = b + per < n16 ? b + per : n16;
    uint32_t r = 0;
    for (int64_t i = b + threadIdx.x; i < e; i += 256 * kReadUnroll) {
        uint4 v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) {
            const int64_t j = i + 256 * u;
            v[u] = j < e ? src[j] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) r ^= (v[u].x ^ v[u].y) ^ (v[u].z ^ v[u].w);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) r ^= (uint32_t)__shfl_xor((int)r, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = (red[0] ^ red[1]) ^ (red[2] ^ red[3]);
    if (blockIdx.x == 0)
        for (int i = (int)gridDim.x + (int)threadIdx.x; i < kReadXorWords; i += 256) out[i] = 0;
}

hipError_t launch_read_xor(const void* src, int64_t bytes, uint32_t* out, hipStream_t stream) {
    const int64_t n16 = bytes > 0 ? bytes / 16 : 0;
    const int64_t blocks = n16 > 0 ? (n16 + 255) / 256 : 1;
    read_xor_kernel<<<dim3((unsigned)(blocks < kReadXorWords ? blocks : kReadXorWords)), dim3(256), 0, stream>>>(
        static_cast<const uint4*>(src), n16, out);
    return hipGetLastError();
}

template <typename Dec, typename T>
void go_dequant(const uint8_t* w, T* y, int64_t n, hipStream_t stream) {
    constexpr int P = per_thread<Dec, T>();
    constexpr int U = (sizeof(T) == 4 && !std::is_same<Dec, DecQ80>::value) ? 2 : 1;
    const int64_t threads = ((n + P - 1) / P + U - 1) / U;
    dequant_kernel<Dec, T, U><<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream>>>(w, y, n);
}

template <typename T>
hipError_t launch_dequant_t(int qtype, const uint8_t* w, T* y, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    switch (qtype) {
        case kTypeQ4K: go_dequant<DecQ4K<sizeof(T) == 2 ? 8 : 4>>(w, y, n, stream); break;
        case kTypeQ5K: go_dequant<DecQ5K<sizeof(T) == 2 ? 8 : 4>>(w, y, n, stream); break;
        case kTypeQ6K: go_dequant<DecQ6K<sizeof(T) == 2 ? 8 : 4>>(w, y, n, stream); break;
        case kTypeQ80: go_dequant<DecQ80>(w, y, n, stream); break;
        case kTypeQ10: go_dequant<DecQ10>(w, y, n, stream); break;
        case kTypeQ40: go_dequant<DecQ32<kQ40Bytes, 2, false, false>>(w, y, n, stream); break;
        case kTypeQ50: go_dequant<DecQ32<kQ50Bytes, 6, true, false>>(w, y, n, stream); break;
        case kTypeQ51: go_dequant<DecQ32<kQ51Bytes, 8, true, true>>(w, y, n, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant(int qtype, const uint8_t* w, float* y, int64_t n, hipStream_t stream) {
    return launch_dequant_t(qtype, w, y, n, stream);
}

hipError_t launch_dequant_f16(int qtype, const uint8_t* w, uint16_t* y, int64_t n, hipStream_t stream) {
    return launch_dequant_t(qtype, w, y, n, stream);
}

}  // namespace frq
