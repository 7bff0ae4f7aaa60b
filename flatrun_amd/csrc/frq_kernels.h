// Launchers shared between the kernel translation units and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frq {

// GGML type ids (src/flatrun/backend/gguf.py:59-86).
constexpr int kTypeQ80 = 8;
constexpr int kTypeQ4K = 12;
constexpr int kTypeQ5K = 13;
constexpr int kTypeQ6K = 14;
constexpr int kTypeQ10 = 41;
constexpr int kTypeQ40 = 2;     // dequant only
constexpr int kTypeQ50 = 6;     // dequant only
constexpr int kTypeQ51 = 7;     // dequant only

// Launch geometry of one GEMV: lanes per row, waves per workgroup, rows per
// workgroup and the per-format work unit chosen for it.
struct GemvPlan {
    int cpl = 0;            // format-specific work unit per lane (see frq_gemv.hip)
    int waves = 0;          // wavefronts per workgroup
    int rows_per_wg = 0;    // output rows owned by one workgroup
    int unroll = 0;         // rows whose loads are issued together
    int slices = 0;         // 1: every row in one workgroup (0 = choose; nothing else is accepted)
    int64_t grid = 0;       // workgroups
};

// y[0, n) = value, by kernel (no hipMemset node if the caller captures a graph).
hipError_t launch_fill(float* y, float value, int64_t n, hipStream_t stream);

// dst[0, bytes) = src[0, bytes); bytes a multiple of 16, both 16-byte aligned.
hipError_t launch_copy(void* dst, const void* src, int64_t bytes, hipStream_t stream);

// out[0, kReadXorWords) = per-workgroup XORs of the 32-bit words of
// src[0, bytes) (zeros past the grid): the XOR of all of out is the XOR of
// all of src. bytes a multiple of 16, src 16-byte aligned.
constexpr int kReadXorWords = 2048;
hipError_t launch_read_xor(const void* src, int64_t bytes, uint32_t* out, hipStream_t stream);

hipError_t launch_dequant(int qtype, const uint8_t* w, float* y, int64_t n_elems, hipStream_t stream);
// The same values rounded to fp16 (nearest even), stored as fp16 bit patterns.
hipError_t launch_dequant_f16(int qtype, const uint8_t* w, uint16_t* y, int64_t n_elems, hipStream_t stream);

// y[n] = W[n, k] . x[k] with fp32 accumulation. `plan` may be pre-filled
// (cpl/rows_per_wg/unroll > 0) to override the heuristic; on return it holds
// the geometry that was launched.
hipError_t launch_gemv(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k,
                       GemvPlan* plan, hipStream_t stream);

// Checks that a GEMV of this shape can be planned; returns false with no launch otherwise.
bool gemv_supported(int qtype, int64_t n, int64_t k);

// Q4_K GEMV on the matrix cores (frq_gemv_mx.hip), batch 1: k a multiple of
// 256, x and w 16-byte aligned. A workgroup owns `rows` output rows (tiles of
// <= 16 rows, 1 or 2 per wavefront) and the whole row (ksplit 1) or one half
// of it (ksplit 2: two workgroups per row set, combined through one 64-bit
// slot per row that must be zero before a launch; every launch leaves it
// zero, and launches sharing slots must be ordered, e.g. one stream).
// Wavefronts own `blocks` consecutive 256-element blocks of the range.
// plan_gemv_mx fills the fields left <= 0 and checks the rest. It runs for
// Q4_K with n > 1280 (gemv_mx_eligible); the default path takes it where it
// measured 5 % or more faster than the element-wise kernel: whole rows in one
// round of <= 256 workgroups (gemv_mx_default).
struct MxPlan {
    int rows = 0;      // output rows per workgroup (<= 16 * tiles)
    int tiles = 0;     // 16-row MFMA tiles per wavefront: 1 or 2
    int ksplit = 0;    // workgroups per row set: 1 or 2
    int depth = 0;     // blocks whose weight loads a wavefront issues before its x split: 1 (then
                       // block j + 1's loads before block j's products) or all of them; 0 = choose
    int blocks = 0;    // blocks per wavefront (derived, <= 4)
    int waves = 0;     // wavefronts per workgroup (derived)
    int64_t grid = 0;  // workgroups (derived)
};
bool plan_gemv_mx(int64_t n, int64_t k, MxPlan* plan);
size_t gemv_mx_slot_bytes(const MxPlan& plan, int64_t n);
bool gemv_mx_eligible(int qtype, const uint8_t* w, const float* x, int64_t n, int64_t k);
bool gemv_mx_default(int qtype, const uint8_t* w, const float* x, int64_t n, int64_t k);
hipError_t launch_gemv_mx(const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, const MxPlan& plan,
                          uint64_t* slots, hipStream_t stream);

// Q1_0 GEMV on the matrix cores (frq_gemv_mx.hip), batch 1: a workgroup owns
// TR <= 16 rows and all of k, each wavefront L (1, 2, 4 or 8) consecutive
// 128-element blocks, at most 16 wavefronts. w 4-byte aligned with an even
// block count (gemv_q10_mx_ok). plan_gemv_q10_mx fills L / TR left <= 0 and
// checks them.
bool gemv_q10_mx_ok(const uint8_t* w, int64_t k);
// The default path's choice between this kernel and the element-wise ring.
bool gemv_q10_mx_default(const uint8_t* w, int64_t n, int64_t k);
bool plan_gemv_q10_mx(int64_t n, int64_t k, int* L, int* TR);
hipError_t launch_gemv_q10_mx(const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int L, int TR,
                              hipStream_t stream);

// Matvec of m = 2 .. kGemvMrMax rows of x at once (frq_gemv_mr.hip), Q4_K,
// Q6_K or Q8_0: Y[r * ldy + i] = sum_j W[i, j] X[r * k + j]; W read once for
// the m rows. Q4_K: per-weight fp32 arithmetic of the single-row element-wise
// order; Q6_K / Q8_0: each row with the bits of the single-row ring kernel.
// Needs x 16-byte aligned; Q4_K: W 16-byte aligned, k <= 24576; Q6_K: W
// 4-byte aligned, an even block count, k <= 24576; Q8_0: W 4-byte aligned, an
// even block count, k <= 16384 (gemv_mr_ok).
constexpr int kGemvMrMax = 3;
bool gemv_mr_ok(int qtype, const uint8_t* w, const float* x, int64_t k);
hipError_t launch_gemv_mr(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int m,
                          int64_t ldy, hipStream_t stream);

// Q4_K matvec of m = 1 .. kGemvMbMax rows of x with fp32 products on the
// matrix cores (frq_gemv_mb.hip): Y[r * ldy + i] = sum_j W[i, j] X[r * k + j],
// W read once. Per-weight fp32 arithmetic (w = fma(s, q, -t), every product
// fused into an fp32 sum); a row's bits depend on its own x only. Needs W and
// x 16-byte aligned. The plan fills what is 0: nbp block pairs per wavefront
// (waves = ceil(pairs / nbp) <= 16: k <= 24576 at m <= 4, k <= 8192 at m 5 .. 8),
// rows per workgroup (<= 16).
constexpr int kGemvMbMax = 8;
struct MbPlan {
    int nbp = 0, rows = 0;         // inputs (0: choose)
    int cg = 1, waves = 0, groups = 0;
    int64_t grid = 0;
};
bool plan_gemv_mb(int64_t n, int64_t k, int m, MbPlan* p);
bool gemv_mb_ok(const uint8_t* w, const float* x, int64_t k);
hipError_t launch_gemv_mb(const uint8_t* w, const float* x, float* y, int64_t n, int64_t k, int m, int64_t ldy,
                          const MbPlan& p, hipStream_t stream);

// Grouped GEMV: y_i[n_i] = W_i[n_i, k] . x[k] for up to kGemvGroupMax
// matrices sharing x (q/k/v, gate/up), in ONE launch when every W_i is Q4_K
// (16-byte aligned) or Q6_K (4-byte aligned, even block count) and 8 lanes
// per block cover k (k <= 32768); otherwise one launch per matrix. Outputs
// are bit-identical to separate launch_gemv calls either way. *fused tells
// which path ran.
constexpr int kGemvGroupMax = 4;
struct GemvGroup {
    const uint8_t* w[kGemvGroupMax];
    float* y[kGemvGroupMax];
    int64_t n[kGemvGroupMax];
    int64_t wg_begin[kGemvGroupMax];   // first workgroup of each segment
    int qtype[kGemvGroupMax];
    int count;
};
bool gemv_group_fusable(int count, const int* qtypes, const uint8_t* const* w, int64_t k);
hipError_t launch_gemv_group(int count, const int* qtypes, const uint8_t* const* w, const int64_t* n, float* const* y,
                             const float* x, int64_t k, hipStream_t stream, int* fused = nullptr);

// Split-K, software-pipelined GEMV (frq_gemv_sk.hip). Fields left <= 0 are
// chosen by plan_gemv_sk.
struct SplitKPlan {
    int cpl = 0;             // work unit per lane (format specific)
    int rows = 0;            // rows per work item (one wavefront), <= 64
    int unroll = 0;          // rows per load batch (2 or 4)
    int slices = 0;          // K-slices per row (derived)
    int unit_base = 0;       // work units per slice (derived; first unit_rem slices get one more)
    int unit_rem = 0;
    int64_t row_blocks = 0;  // ceil(n / rows) (derived)
    int64_t items = 0;       // work items = wavefronts launched (derived)
};

bool gemv_sk_supported(int qtype);
bool plan_gemv_sk(int qtype, int64_t n, int64_t k, SplitKPlan* plan);
// Device scratch a plan needs (both 0 when slices == 1): `counter_bytes` of
// per-row-block counters, which must be zero before the first launch and
// which every launch leaves zero (keep them in memory nothing else writes),
// and `partial_bytes` for n * slices partial sums.
void gemv_sk_scratch(const SplitKPlan& plan, int64_t n, size_t* partial_bytes, size_t* counter_bytes);
hipError_t launch_gemv_sk(int qtype, const uint8_t* w, const float* x, float* y, int64_t n, int64_t k,
                          const SplitKPlan& plan, float* partials, uint32_t* counters, hipStream_t stream);

// Prefill GEMM on the matrix cores (frq_gemm.hip): y[m, n] = x[m, k] (bf16
// bits, row-major) . W[n, k]^T (raw Q4_K, Q6_K or Q8_0 blocks) with W rounded
// to bf16 and fp32 accumulation. x 16-byte aligned; w 16-byte aligned for
// Q4_K, 2-byte for the others; k a multiple of 256 (Q4_K, Q6_K) or 128 (Q8_0).
// Shapes with too few 256 x 128 output tiles to fill the GPU split K
// (gemm_bf16_splits): each split writes an fp32 partial plane of `part`
// (gemm_bf16_scratch bytes) and a second kernel adds the planes in split
// order. Launches sharing `part` must be ordered (one stream). With null
// scratch the GEMM runs unsplit.
bool gemm_bf16_supported(int qtype, int64_t m, int64_t n, int64_t k);
int gemm_bf16_splits(int64_t m, int64_t n, int64_t k);
size_t gemm_bf16_scratch(int64_t m, int64_t n, int64_t k);
hipError_t launch_gemm_bf16(int qtype, const uint8_t* w, const uint16_t* x, float* y, int64_t m, int64_t n, int64_t k,
                            hipStream_t stream, float* part = nullptr);

// The same GEMM for up to kGemmGroupMax matrices W_i[n_i, k] that multiply
// the same x, in one launch (and one split-adding launch when K is split):
// y_i[r * ldy_i + c]. The K-split is chosen for the group's total tile count
// (gemm_bf16_group_splits); with the same split a matrix's outputs are those
// of its own launch bit for bit. Every segment passes gemm_bf16_supported.
constexpr int kGemmGroupMax = 4;
struct GemmGroup {
    const uint8_t* w[kGemmGroupMax];
    float* y[kGemmGroupMax];
    float* part[kGemmGroupMax];        // segment i's partial planes (split > 1)
    int64_t n[kGemmGroupMax];
    int64_t ldy[kGemmGroupMax];
    int64_t wg_begin[kGemmGroupMax];   // first workgroup of each segment
    int64_t e_begin[kGemmGroupMax];    // first element of each segment in the split-adding kernel
    int qtype[kGemmGroupMax];
    int count;
};
int gemm_bf16_group_splits(int count, const int64_t* n, int64_t m, int64_t k);
size_t gemm_bf16_group_scratch(int count, const int64_t* n, int64_t m, int64_t k);
hipError_t launch_gemm_bf16_group(int count, const int* qtypes, const uint8_t* const* w, const int64_t* n,
                                  float* const* y, const int64_t* ldy, const uint16_t* x, int64_t m, int64_t k,
                                  hipStream_t stream, float* part);

// y[r * ldy + c] = part[0][i] + ... + part[splits-1][i], i = r * cols + c, for
// the rows x cols elements of the partial planes, in split order.
hipError_t launch_split_reduce(const float* part, float* y, int splits, int64_t rows, int64_t cols, int64_t ldy,
                               hipStream_t stream);

// Batched matvec with the fp32 contract on the matrix cores (frq_gemm_f32.hip):
// y[m, n] = x[m, k] (fp32, row-major) . W[n, k]^T (raw Q4_K, Q6_K or Q8_0) with
// W as exact integer codes, x as three bf16 pieces and the sub-block scales in
// fp32; W is read once per tile of 32, 64 or 128 rows of x; rows of y are
// ldy >= n floats apart. x 16-byte aligned, w
// 16-byte (Q4_K) / 2-byte aligned; k a multiple of 256 (Q4_K, Q6_K) or 32
// (Q8_0). Few output tiles split K (gemm_f32_splits, at most `part_cap`
// bytes of partials): fp32 partial planes in `part` added in split order by
// a second kernel; `part` also holds one flag word per row of x (rows with
// values outside the bf16 pieces' range, computed again by the second
// kernel in fp64), so it is never null (gemm_f32_scratch bytes); launches
// sharing `part` must be ordered. The split count is a function of (qtype, m, n, k, part capacity) only, so
// results do not depend on which scratch a call gets beyond its capacity.
bool gemm_f32_supported(int qtype, int64_t m, int64_t n, int64_t k);
int gemm_f32_splits(int qtype, int64_t m, int64_t n, int64_t k, size_t part_cap = SIZE_MAX);
size_t gemm_f32_scratch(int qtype, int64_t m, int64_t n, int64_t k, size_t part_cap = SIZE_MAX);
hipError_t launch_gemm_f32(int qtype, const uint8_t* w, const float* x, float* y, int64_t m, int64_t n, int64_t k,
                           int64_t ldy, hipStream_t stream, float* part, size_t part_cap);

// out[r, i] = silu(gateup[r, i]) * gateup[r, inter + i] for r < rows, rows of
// gateup ld_in floats apart and of out ld_out apart (frq_act.hip).
// Gate and up of a SwiGLU block and its activation in one launch (batch 1,
// both Q4_K, 16-byte aligned, k a multiple of 256 with 8 lanes per block
// covering it): gateup[0, 2 inter) = [W_gate x | W_up x] with the grouped
// launch's bits, act[i] = silu(gate[i]) * up[i] with silu_mul's.
bool gemv_swiglu_fusable(int qtype_gate, const uint8_t* wgate, int qtype_up, const uint8_t* wup, int64_t k);
hipError_t launch_gemv_swiglu(const uint8_t* wgate, const uint8_t* wup, const float* x, float* gateup, float* act,
                              int64_t inter, int64_t k, hipStream_t s);

hipError_t launch_silu_mul(const float* gateup, int64_t ld_in, float* out, int64_t ld_out, int64_t rows,
                           int64_t inter, hipStream_t stream);

// Scratch a caller brings in place of the stream registry's: exchange slots
// (zero before a launch, left zero by every launch) and split-K partials.
struct FixedScratch {
    uint64_t* slots = nullptr;
    size_t slot_bytes = 0;
    float* part = nullptr;
    size_t part_bytes = 0;
};
// frq_dev_gemv with its scratch taken from `fixed` (frq_api.cpp); allocates
// nothing and refuses shapes that need more than `fixed` holds.
int dev_gemv_fixed(int qtype, const void* w, size_t w_bytes, const float* x, float* y, int64_t n, int64_t k,
                   int64_t batch, void* stream, const FixedScratch& fixed);
// Sets the calling thread's error message and returns FRQ_ERR_UNSUPPORTED / FRQ_ERR_HIP.
int fail_unsupported(const char* msg);
int fail_hip(hipError_t e, const char* what);

}  // namespace frq
