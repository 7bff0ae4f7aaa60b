// SwiGLU activation between a decoder block's gate|up and down projections:
//   out[r, i] = silu(gate[r, i]) * up[r, i],  silu(g) = g / (1 + exp(-g)),
// with gate and up the two halves of one row of the grouped gate|up output
// (row r at gateup + r * ld_in: gate in [0, inter), up in [inter, 2 inter)).
// The operations and their fp32 roundings follow the forwarder's in-place
// NumPy chain (model/qwen2.py:1703-1740): e = exp(-g); e = e + 1; e = 1 / e;
// e = e * g; e = e * up -- each one rounded, no FMA (-ffp-contract=off), the
// reciprocal a correctly rounded division. Only exp differs from NumPy's by
// its last-place rounding (expf here, NumPy's own SIMD exp there), so results
// agree within a few ulp; exp(-g) overflowing to +inf gives 0 * g, as there.
#include "frq_common.h"
#include "frq_kernels.h"

namespace frq {
namespace {

__global__ void __launch_bounds__(256) silu_mul_kernel(const float* __restrict__ gateup, int64_t ld_in,
                                                       float* __restrict__ out, int64_t ld_out, int64_t rows,
                                                       int64_t inter) {
    const int64_t per_row = inter;
    const int64_t total = rows * per_row;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / per_row, c = i - r * per_row;
        const float* row = gateup + r * ld_in;
        out[r * ld_out + c] = silu_mul(row[c], row[inter + c]);
    }
}

}  // namespace

hipError_t launch_silu_mul(const float* gateup, int64_t ld_in, float* out, int64_t ld_out, int64_t rows,
                           int64_t inter, hipStream_t stream) {
    const int64_t total = rows * inter;
    if (total <= 0) return hipSuccess;
    const int64_t blocks = (total + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 8192 ? blocks : 8192);
    silu_mul_kernel<<<grid, 256, 0, stream>>>(gateup, ld_in, out, ld_out, rows, inter);
    return hipGetLastError();
}

}  // namespace frq
