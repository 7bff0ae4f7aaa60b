/*
 * frq.h -- C ABI of libfrq_hip.so, the gfx950 GGUF dequant + matvec library.
 *
 * Plain pointers and sizes only; no exceptions cross this boundary. Every
 * entry point returns an frq_status; on failure frq_last_error() returns a
 * thread-local message. Python reaches the library through ctypes
 * (flatrun_amd/_lib.py).
 *
 * Two families:
 *
 *  1. Host-buffer entry points, one per function of the reference's pybind11
 *     module flatrun_native._C (src/flatrun_native/_C.cpp:455-488). Inputs
 *     and outputs are host memory; the library stages them through device
 *     memory, runs the HIP kernels and copies the result back before
 *     returning. Validation and messages follow _C.cpp; a failure the
 *     reference reports as std::runtime_error is returned as
 *     FRQ_ERR_SHAPE / FRQ_ERR_SIZE so the facade can raise RuntimeError,
 *     the exception the reference runtime falls back on
 *     (src/flatrun/runtime/backend.py:259-268).
 *
 *  2. Device entry points (frq_dev_*): raw GGUF blocks, x and y already in
 *     device memory, work enqueued on a caller-given hipStream_t (NULL = the
 *     null stream), nothing copied. This is the decode-time hot path.
 *
 * Quant types are GGML type ids (src/flatrun/backend/gguf.py:59-86):
 *   FRQ_Q8_0 = 8 (34 B / 32), FRQ_Q4_K = 12 (144 B / 256),
 *   FRQ_Q5_K = 13 (176 B / 256), FRQ_Q6_K = 14 (210 B / 256),
 *   FRQ_Q1_0 = 41 (18 B / 128),
 *   FRQ_Q4_0 = 2 (18 B / 32), FRQ_Q5_0 = 6 (22 B / 32), FRQ_Q5_1 = 7
 *   (24 B / 32): dequant only (the reference decodes them in NumPy,
 *   dequant/gguf.py:81-107, 302-362; no native matvec exists for them).
 *
 * Numerics: dequant is bit-exact with the reference NumPy decoders
 * (src/flatrun/dequant/gguf.py); matmul accumulates in fp32 and is held to
 * 1e-5 relative error (normwise and componentwise) against the reference
 * NumPy / native matvec.
 */
#ifndef FRQ_H
#define FRQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    FRQ_OK = 0,
    FRQ_ERR_INVALID = 1,      /* bad argument (null pointer, unknown type, ...) */
    FRQ_ERR_SHAPE = 2,        /* shape / ndim rule of _C.cpp violated          */
    FRQ_ERR_SIZE = 3,         /* weight byte count does not match (n, k)       */
    FRQ_ERR_UNSUPPORTED = 4,  /* valid request this library does not plan       */
    FRQ_ERR_NO_DEVICE = 5,    /* no HIP device visible                          */
    FRQ_ERR_HIP = 6,          /* HIP runtime error                              */
    FRQ_ERR_ALIGN = 7         /* device pointer misaligned for its format       */
} frq_status;

enum { FRQ_Q4_0 = 2, FRQ_Q5_0 = 6, FRQ_Q5_1 = 7, FRQ_Q8_0 = 8, FRQ_Q4_K = 12, FRQ_Q5_K = 13, FRQ_Q6_K = 14,
       FRQ_Q1_0 = 41 };

/* ---------------------------------------------------------------- general */

/* Build identifier. Replaces _C.version (_C.cpp:449-451). */
const char* frq_version(void);

/* Always 0: this library has no NEON path. Replaces _C.is_neon (_C.cpp:441-447). */
int frq_is_neon(void);

/* Message of the last failed call on this thread ("" if none). */
const char* frq_last_error(void);

/* Number of visible HIP devices (0 on a machine without a GPU). */
int frq_device_count(int* count);

/* Bytes and elements per block of a GGML type id
 * (src/flatrun/backend/gguf.py:59-103). */
int frq_block_info(int qtype, int64_t* block_bytes, int64_t* block_elems);

/* ---------------------------------------------- host-buffer entry points
 * weight: raw GGUF block bytes, weight_bytes long (host memory).
 * out:    caller-allocated float32 host buffer of the result size.        */

/* dequant_q4_k(weight, (out, in)) -> f32 (out, in). _C.cpp:47-86. */
int frq_dequant_q4_k(const uint8_t* weight, size_t weight_bytes, int64_t out_dim, int64_t in_dim, float* out);
/* dequant_q8_0(weight, (out, in)). _C.cpp:285-320. */
int frq_dequant_q8_0(const uint8_t* weight, size_t weight_bytes, int64_t out_dim, int64_t in_dim, float* out);
/* dequant_q6_k(weight, (out, in)). _C.cpp:363-398. */
int frq_dequant_q6_k(const uint8_t* weight, size_t weight_bytes, int64_t out_dim, int64_t in_dim, float* out);

/* Generic dequant of any supported type with the NumPy decoders' size rule
 * (ceil-div blocks, tail trimmed): replaces dequant_q8_0 / q4_k / q5_k /
 * q6_k / q1_0 of src/flatrun/dequant/gguf.py:112,166,223,266,365 for the
 * Q5_K and Q1_0 formats the native module lacks. */
int frq_dequant(int qtype, const uint8_t* weight, size_t weight_bytes, int64_t n_elems, float* out);

/* The same decode with float16 output (fp16 bit patterns in `out`):
 * dequant_handle's default dtype, loader.py:51-88, whose decoders fill an
 * fp32 array that _finish casts with astype (gguf.py:61-73): each fp32
 * value rounded once to nearest even, overflow to inf, subnormals kept. */
int frq_dequant_f16(int qtype, const uint8_t* weight, size_t weight_bytes, int64_t n_elems, uint16_t* out);

/* matmul_q4_k(x[k], weight, n, k) -> out[n]. _C.cpp:99-132. */
int frq_matmul_q4_k(const float* x, size_t x_len, const uint8_t* weight, size_t weight_bytes, size_t n, size_t k,
                    float* out);
/* matmul_q4_k_batched(x[seq, k], weight, n, k) -> out[seq, n]. _C.cpp:154-197.
 * x_ndim is the ndim of the caller's array (must be 2), x_cols its shape[1]. */
int frq_matmul_q4_k_batched(const float* x, int x_ndim, size_t seq, size_t x_cols, const uint8_t* weight,
                            size_t weight_bytes, size_t n, size_t k, float* out);
/* matmul_q8_0. _C.cpp:326-357. */
int frq_matmul_q8_0(const float* x, size_t x_len, const uint8_t* weight, size_t weight_bytes, size_t n, size_t k,
                    float* out);
/* matmul_q8_0_batched. _C.cpp:199-242. */
int frq_matmul_q8_0_batched(const float* x, int x_ndim, size_t seq, size_t x_cols, const uint8_t* weight,
                            size_t weight_bytes, size_t n, size_t k, float* out);
/* matmul_q6_k. _C.cpp:404-435. */
int frq_matmul_q6_k(const float* x, size_t x_len, const uint8_t* weight, size_t weight_bytes, size_t n, size_t k,
                    float* out);
/* matmul_q6_k_batched. _C.cpp:244-283. */
int frq_matmul_q6_k_batched(const float* x, int x_ndim, size_t seq, size_t x_cols, const uint8_t* weight,
                            size_t weight_bytes, size_t n, size_t k, float* out);

/* Generic host matmul for every supported type (adds Q5_K and Q1_0, whose
 * reference path is dequant + `w @ x`, runtime/backend.py:203-213):
 * x is seq rows of k floats, out is seq rows of n floats. */
int frq_matmul(int qtype, const float* x, size_t seq, const uint8_t* weight, size_t weight_bytes, size_t n, size_t k,
               float* out);

/* ---------------------------------------------------- device entry points
 * All pointers are device pointers; stream is a hipStream_t (NULL = null
 * stream). Q4_K / Q5_K weights must be 16-byte aligned, the others 2-byte
 * aligned; x and y 16-byte / 4-byte aligned.                              */

/* y[n_elems] = dequant(w). Same numerics as frq_dequant. */
int frq_dev_dequant(int qtype, const void* w, size_t w_bytes, int64_t n_elems, float* y, void* stream);
/* y[n_elems] = fp16(dequant(w)). Same numerics as frq_dequant_f16; y 2-byte aligned. */
int frq_dev_dequant_f16(int qtype, const void* w, size_t w_bytes, int64_t n_elems, uint16_t* y, void* stream);

/* y[b, n] = W[n, k] . x[b, k] for b < batch: the decode matvec of
 * matmul_<q> / matmul_<q>_batched (_C.cpp:99-283) on device buffers.
 * Q4_K with n > 1280, k <= 16384 or so (whole rows in one workgroup) and
 * rows that one round of at most 256 workgroups covers (w and x 16-byte
 * aligned) runs on the matrix cores, where they measured 5 % or more faster
 * than the element-wise kernel: int8 MFMA on the 4-bit codes and on x written per
 * 32-element sub-block as a 60-bit fixed-point number relative to the
 * sub-block's max |x| (eight 8-bit digits), exact integer sums of q x and
 * of x, then per sub-block
 *   T_s = d*sc_s * sum(q x) - dmin*m_s * sum(x)
 * formed exactly in fp64 and summed per lane in fp64, rounded to fp32 once.
 * Every x within 2^36 of its sub-block's max |x| is carried exactly; a
 * block whose x is not (a wider range, |x| >= 2^30, inf, NaN) is computed
 * per weight in fp32 (w = fl(fl(d*sc)*q) - fl(dmin*m), q4_k.h:153-185).
 * (frq_dev_gemv_tuned can also run it on rows split in two halves of k over
 * two workgroups that combine in a fixed order through per-row slots in the
 * stream's scratch.) The other shapes and formats run on element-wise
 * kernels whose every product is w_j x_j with the weight
 * itself (Q4_K / Q5_K: w = fma(d*sc, q, -dmin*m), the dequantized bits;
 * Q6_K / Q8_0: signed codes under the block scale; Q1_0: +-d).
 * Error: for every finite x, row i is within the fp32 accumulation bound
 *   c * 2^-24 * sum_j |w_ij x_j|   (c a small multiple of the summation
 * depth), which the tests hold to 1e-5 of sum_j |w_ij x_j| (componentwise)
 * and of max |y| (normwise) -- including outliers x_j on weights that are
 * exactly zero while their scales are not (d*sc*q = dmin*m), where a sum
 * written as s * sum(q x) - t * sum(x) in fp32 would cancel.
 * batch >= 2 with Q4_K, Q6_K or Q8_0 (x 16-byte aligned, k a multiple of the
 * block) is one fp32-contract GEMM that reads W once per 32 or 64 rows of x:
 * bf16 matrix cores on exact integer codes (Q4_K q - c with c the code
 * nearest dmin*m / d*sc, so every term stays within 3 |w_j x_j|) and on x
 * split into three bf16 pieces (all 24 bits of every x in {0} U
 * [2^-100, 2^100]), fp32 sums per sub-block, then the sub-block scales in
 * fp32 -- the same error bound, other bits than one row at a time. A row of
 * x with any value outside that range (tiny, subnormal, huge, inf, NaN) is
 * computed again weight by weight in fp64 (one rounding; inf and NaN as
 * IEEE arithmetic has them) by a second kernel. A few
 * rows run a small-M matvec instead, W read once per launch: Q4_K with 4
 * rows (k <= 24576), or 5 to 8 rows where k <= 8192, in one launch of the
 * fp32 matrix-core matvec (per-weight dequant, each product fused into an
 * fp32 sum by v_mfma_f32_4x4x1_16b_f32; a row's bits independent of the
 * other rows and of its position); otherwise (Q4_K, Q8_0: up to 6 rows;
 * Q6_K: up to 10) the element-wise small-M matvec, one launch per two or
 * three rows (Q4_K with per-weight fp32 arithmetic as one row, a row's bits
 * the same in any batch this kernel takes; Q6_K and Q8_0 with the bits of a
 * batch-1 call); up to 3 rows that neither takes run one GEMV per row. Few output
 * tiles split k over workgroups whose fp32 partials a second kernel adds in
 * a fixed order (scratch of the stream). Q5_K and Q1_0 run one matvec per
 * row. */
int frq_dev_gemv(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                 int64_t batch, void* stream);

/* frq_dev_gemv that allocates nothing. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and results (bit for bit) as frq_dev_gemv; the scratch
 * that frq_dev_gemv grows per stream is one fixed device array of
 * FRQ_NOALLOC_SCRATCH_BYTES per GPU instead (held until the process ends):
 * 1 MiB of row-exchange slots (8 bytes per output row of a Q4_K matrix whose
 * rows are split over two workgroups: n <= 131072; no default shape splits
 * rows so today) and 3 MiB of split-K partials (n x slices x 4 bytes, rows
 * longer than one workgroup). A batch-1 shape that needs more is refused
 * with FRQ_ERR_UNSUPPORTED before anything is launched. A batch that takes
 * a small-M matvec (see frq_dev_gemv) needs no scratch; a batch that takes
 * the batched GEMM (more rows of Q4_K, Q6_K, Q8_0) keeps one flag word per row of x
 * in the 3 MiB and splits k only as far as its partials (splits x batch x n
 * x 4 bytes) fit beside them, so neither is refused (up to 786432 rows); where the GEMM splits less than
 * frq_dev_gemv would, the bits differ from frq_dev_gemv's within the same
 * bound. Any other batch runs one GEMV per row and is refused as batch 1
 * would be (for example 2 or 3 rows of Q4_K with k > 24576). Every call on a GPU shares that GPU's array: calls that overlap
 * on one GPU (different streams or threads) race; calls ordered on one
 * stream do not. The first call on a device clears the slots with a kernel
 * on `stream`; every launch leaves them zero. */
#define FRQ_NOALLOC_SCRATCH_BYTES (4u << 20)
int frq_dev_gemv_noalloc(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                         int64_t batch, void* stream);

/* Launch geometry of one GEMV, for tuning sweeps and profiling. Fields set
 * to 0 are chosen by the library; on return every field holds what ran.
 *   kernel        FRQ_GEMV_AUTO, FRQ_GEMV_SPLITK (one wavefront per
 *                 (row block, K-slice) work item, deterministic split-K
 *                 fixup) or FRQ_GEMV_ROWS (one workgroup spans all of k)
 *                 or FRQ_GEMV_MX (the matrix-core kernel, Q4_K, k <= 32768:
 *                 `rows` = output rows per workgroup (<= 16 per tile),
 *                 `cpl` = 16-row tiles per wavefront (1 or 2), `slices` =
 *                 workgroups per row (1: k <= 16384, or 2 halves of k),
 *                 `unroll` = load depth: 1 = each wavefront issues block
 *                 j + 1's weight loads before block j's products, >= its
 *                 blocks = all of them before its x split; 0 = choose)
 *                 or FRQ_GEMV_MB (Q4_K, fp32 products on the matrix cores,
 *                 the kernel batches of 2 .. 8 rows of x take: `rows` =
 *                 rows per workgroup (<= 16), `unroll` = pairs of blocks
 *                 per wavefront (1 .. 3, at most 16 wavefronts cover k);
 *                 0 = choose). AUTO takes the kernel frq_dev_gemv takes.
 *                 Other values are refused with FRQ_ERR_INVALID.
 *   cpl           work unit per lane (format specific); with ROWS and
 *                 Q1_0, 16 selects the matrix-core Q1_0 kernel (`rows` <=
 *                 16 per workgroup, `unroll` = 128-element blocks per
 *                 wavefront: 1, 2, 4 or 8)
 *   rows          rows per work item (SPLITK) / per workgroup (ROWS)
 *   unroll        rows per load batch
 *   slices        K-slices per row: output for SPLITK; 1 for the ROWS
 *                 kernels (an input of 0 or 1; anything else is rejected)
 *   waves_per_wg  wavefronts per workgroup (output)
 *   items         work items / workgroups launched (output)              */
enum { FRQ_GEMV_AUTO = 0, FRQ_GEMV_SPLITK = 1, FRQ_GEMV_ROWS = 2, FRQ_GEMV_MX = 4, FRQ_GEMV_MB = 8 };
typedef struct {
    int32_t kernel, cpl, rows, unroll, slices, waves_per_wg;
    int64_t items;
} frq_gemv_config;

/* Several matrices that multiply the same x, with one launch where possible
 * (replaces the forwarder's per-projection matmul calls followed by
 * np.concatenate of their outputs: q/k/v model/qwen2.py:1510-1519, gate/up
 * model/qwen2.py:1690-1702).
 *   count        1 .. 4 matrices; qtypes[i], w[i], w_bytes[i], n[i] as for
 *                frq_dev_gemv; all share k and x (batch rows of k floats)
 *   y[i]         output base of matrix i for batch row 0; row b goes to
 *                y[i] + b * (y_stride ? y_stride : n[i]) floats, so with
 *                y[i] = out + (n[0] + .. + n[i-1]) and y_stride = sum of n
 *                the result is the concatenation [W_0 x | W_1 x | ...]
 * One launch per batch row when there are two or more matrices, every one
 * Q4_K (16-byte aligned) or Q6_K (4-byte aligned, even block count per row),
 * and k <= 32768 (frq_gemv_group_fusable). That launch computes every row with the
 * element-wise kernels, bit for bit what they give on each matrix alone;
 * frq_dev_gemv on a Q4_K matrix that it sends to the matrix cores agrees
 * with it to the fp32 accumulation tolerance, not bit for bit. Otherwise
 * the group is one frq_dev_gemv launch per matrix. */
int frq_dev_gemv_group(int count, const int* qtypes, const void* const* w, const size_t* w_bytes, const int64_t* n,
                       const float* x, int64_t k, float* const* y, int64_t batch, int64_t y_stride, void* stream);
/* 1 if frq_dev_gemv_group would fuse these matrices into one launch, else 0. */
int frq_gemv_group_fusable(int count, const int* qtypes, const void* const* w, int64_t k);

/* frq_dev_gemv with an explicit launch geometry (batch 1). */
int frq_dev_gemv_tuned(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                       frq_gemv_config* cfg, void* stream);

/* Q4_K prefill GEMM on the matrix cores: y[m, n] = x[m, k] . W[n, k]^T, where
 * x holds bf16 bit patterns (row-major), W is raw Q4_K blocks (n rows of k/256
 * blocks) and y is fp32 row-major. W values are the exact fp32 dequant rounded
 * to bf16 (nearest even); products and sums are fp32. Replaces, for
 * activations already in bf16, the per-token loop of matmul_q4_k_batched
 * (_C.cpp:154-197), which re-dequantizes W for every row of x. Device
 * pointers (w, x 16-byte aligned); k a multiple of 256, at most 4194304. */
int frq_dev_gemm_q4_k_bf16(const void* w, size_t w_bytes, const uint16_t* x_bf16, float* y, int64_t m, int64_t n,
                           int64_t k, void* stream);
/* Same with host buffers (copied to the device and back on every call). */
int frq_gemm_q4_k_bf16(const uint16_t* x_bf16, const uint8_t* w, size_t w_bytes, int64_t m, int64_t n, int64_t k,
                       float* y);
/* The same GEMM for any of Q4_K, Q6_K, Q8_0 (qtype); k a multiple of 256
 * (Q4_K, Q6_K) or 128 (Q8_0) and at most 4194304 (FRQ_ERR_UNSUPPORTED
 * beyond); w 16-byte aligned (Q4_K) or 2-byte aligned.
 * Replaces, for bf16 activations, matmul_q6_k_batched (_C.cpp:244-283) and
 * matmul_q8_0_batched (_C.cpp:199-242) as well. Shapes with too few output
 * tiles to fill the GPU (e.g. n = 1024 or 4096 at m = 512) split K over
 * several workgroups and add the partials in a fixed order (deterministic);
 * the partials live in scratch grown once per (device, stream). */
int frq_dev_gemm_bf16(int qtype, const void* w, size_t w_bytes, const uint16_t* x_bf16, float* y, int64_t m,
                      int64_t n, int64_t k, void* stream);
int frq_gemm_bf16(int qtype, const uint16_t* x_bf16, const uint8_t* w, size_t w_bytes, int64_t m, int64_t n,
                  int64_t k, float* y);
/* Up to 4 matrices that multiply the same x (a fused q|k|v projection at
 * prefill) in one GEMM launch, plus one launch adding the K-split partials
 * where the group splits K. No reference counterpart: the reference's
 * forwarder calls one batched matmul per projection (model/qwen2.py:1510-1519);
 * this is those calls with x read by one launch.
 *   count      1 .. 4; qtypes[i], w[i], w_bytes[i], n[i] as for
 *              frq_dev_gemm_bf16, all sharing m, k and x (m rows of k bf16)
 *   y[i]       output of matrix i: row r at y[i] + r * (y_stride ? y_stride : n[i])
 *              floats, so y[i] = out + (n[0] + .. + n[i-1]) with y_stride the sum
 *              of n gives the concatenation [X W_0^T | X W_1^T | ...]
 * The K-split is chosen for the group's total tile count; with the split a
 * matrix would get alone, its outputs are those of frq_dev_gemm_bf16 bit for
 * bit, else they agree to the fp32 accumulation tolerance. A group with one
 * matrix and a dense output is frq_dev_gemm_bf16. Status codes as
 * frq_dev_gemm_bf16. */
int frq_dev_gemm_bf16_group(int count, const int* qtypes, const void* const* w, const size_t* w_bytes,
                            const int64_t* n, const uint16_t* x_bf16, int64_t m, int64_t k, float* const* y,
                            int64_t y_stride, void* stream);

/* dst = src on the device with a plain 16-byte-per-lane streaming kernel:
 * the reference point for calibrating HBM traffic counters (bytes a
 * multiple of 16, both pointers 16-byte aligned). No reference counterpart. */
int frq_dev_copy(void* dst, const void* src, size_t bytes, void* stream);

/* A plain 16-byte-per-lane streaming read of src[0, bytes) (a multiple of
 * 16, src 16-byte aligned) that folds its 32-bit words by XOR: workgroup b
 * writes the XOR of its contiguous slice to out[b], and the words of out past
 * the grid are zeroed, so the XOR of the FRQ_READ_XOR_WORDS device words of
 * out is the XOR of all of src. The read-only reference point for the GEMV
 * kernels, which read their weights once and write almost nothing; also a
 * checksum of device data. No reference counterpart. */
enum { FRQ_READ_XOR_WORDS = 2048 };
int frq_dev_read_xor(const void* src, size_t bytes, uint32_t* out, void* stream);

/* The SwiGLU activation between a decoder block's gate|up and down
 * projections, on device: out[r * ld_out + i] = silu(g) * u with
 * g = gateup[r * ld_in + i], u = gateup[r * ld_in + inter + i] (the grouped
 * gate|up output, gate first) for r < rows, i < inter; ld_in >= 2 inter,
 * ld_out >= inter, 4-byte aligned. The fp32 operations of the forwarder's
 * NumPy chain in its order (exp(-g), + 1, reciprocal, * g, * u;
 * model/qwen2.py:1703-1740); only exp's last-place rounding differs. */
int frq_dev_silu_mul(const float* gateup, int64_t ld_in, float* out, int64_t ld_out, int64_t rows, int64_t inter,
                     void* stream);

/* A decoder block's gate and up projections and their SwiGLU activation
 * (replaces the forwarder's gate and up matmuls, their np.concatenate and
 * the in-place SwiGLU chain, model/qwen2.py:1690-1740): for each of `batch`
 * rows of x (k floats apart), gateup[r * 2 inter + [0, inter)] = W_gate x_r,
 * gateup[r * 2 inter + [inter, 2 inter)] = W_up x_r and
 * act[r * inter + i] = silu(gate_i) * up_i, with W_gate and W_up
 * [inter x k] blocks of qtype_gate / qtype_up. The results are bit for bit
 * those of frq_dev_gemv_group over the two matrices (y_stride 2 inter)
 * followed by frq_dev_silu_mul. With batch 1, both matrices Q4_K (16-byte
 * aligned) and 8 lanes per block covering k (k <= 32768), it is one launch:
 * each workgroup computes the same rows of both matrices and applies the
 * activation; otherwise those two calls. Status codes as frq_dev_gemv. */
int frq_dev_gemv_swiglu(int qtype_gate, const void* w_gate, size_t gate_bytes, int qtype_up, const void* w_up,
                        size_t up_bytes, int64_t inter, const float* x, int64_t k, float* gateup, float* act,
                        int64_t batch, void* stream);
/* 1 if frq_dev_gemv_swiglu runs these two matrices and the activation as one
 * launch at batch 1, else 0. */
int frq_gemv_swiglu_fusable(int qtype_gate, const void* w_gate, int qtype_up, const void* w_up, int64_t k);

/* ------------------------------------------- memory, streams and events
 * Thin wrappers so a ctypes caller needs no other HIP binding. Streams are
 * created at the default priority.                                         */
int frq_set_device(int device);
int frq_malloc(void** ptr, size_t bytes);
int frq_free(void* ptr);
int frq_host_alloc(void** ptr, size_t bytes);      /* pinned host memory */
int frq_host_free(void* ptr);
int frq_memcpy_h2d(void* dst, const void* src, size_t bytes);
int frq_memcpy_d2h(void* dst, const void* src, size_t bytes);
int frq_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream);
int frq_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream);
int frq_memset_async(void* dst, int value, size_t bytes, void* stream);
int frq_stream_create(void** stream);
int frq_stream_destroy(void* stream);
int frq_stream_synchronize(void* stream);
int frq_stream_wait_event(void* stream, void* event);
int frq_event_create(void** event);
int frq_event_destroy(void* event);
int frq_event_record(void* event, void* stream);
int frq_event_synchronize(void* event);
int frq_event_elapsed_ms(float* ms, void* start, void* stop);
int frq_device_synchronize(void);

/* ------------------------------------------------------------ HIP graphs
 * Record a fixed launch sequence once and replay it with one call: a decode
 * step issues one GEMV per weight (224 for a 32-layer Llama block stack),
 * and replay removes the per-launch host cost. Capture runs on a stream made
 * by frq_stream_create (not the null stream), in thread-local mode. Entry
 * points that allocate on first use (the split-K scratch of very long rows
 * and of split GEMMs, the host workspace) must have run once for the shape
 * before capture.
 * Scratch lifetime: each (device, stream) has its own scratch; it grows when
 * a later call on that stream needs more, and the buffers it replaces stay
 * allocated (a graph captured earlier still launches on them) until
 * frq_stream_destroy, which synchronises the stream and frees them. Destroy
 * the graphs captured on a stream before destroying the stream.
 * Captured work records kernels only (no memset nodes). No reference
 * counterpart: the reference calls its matmuls one by one from Python.     */
int frq_stream_begin_capture(void* stream);
/* Ends the capture and instantiates it; *graph_exec receives the handle. */
int frq_stream_end_capture(void* stream, void** graph_exec);
int frq_graph_launch(void* graph_exec, void* stream);
int frq_graph_destroy(void* graph_exec);

#ifdef __cplusplus
}
#endif

#endif /* FRQ_H */
