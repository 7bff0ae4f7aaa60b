/*
 * C restatement of the reference's scalar native kernels (oracle; test-only).
 *
 * TEST INFRASTRUCTURE ONLY. Built into oracle/liboracle.so by oracle/Makefile
 * and loaded through ctypes by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py. The shipped library never links it.
 *
 * It restates, with the x86 (non-NEON) semantics the reference has on the
 * GPU host, the scalar kernels of src/flatrun_native/kernels/:
 *   fp16 -> fp32 bit conversion               q4_k.h:55-80
 *   6-bit scale/min unpack                    q4_k.h:89-110
 *   Q4_K block dequant / fused dot / matmul   q4_k.h:116-144, 153-185, 427-449
 *   Q6_K fused dot / dequant / matmul         q6_k.h:44-95, 128-170, 180-201
 *   Q8_0 fused dot / dequant / matmul         q8_0.h:36-51, 157-172, 187-208
 * Accumulation order is the reference's: one fp32 accumulator per block,
 * element order as written there, block partials summed into the row
 * accumulator in block order. Built with -ffp-contract=off so no product is
 * fused into an add (x86-64 without -mfma never fuses either).
 *
 * The *_mt variants split rows over POSIX threads the way matmul_q4_k_mt
 * (q4_k.h:464-511) does; each row keeps the single-thread order, so the
 * output is identical to the single-thread one.
 *
 * Parity pins: bit-exact against the reference's own compiled _C module
 * (oracle/_ref) and against tests/golden/ref_native_vectors.npz.
 */
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static float h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t f = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (f << 13);           /* inf / nan, payload kept */
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (f << 13);    /* normal: rebias 15 -> 127 */
    } else if (f == 0) {
        bits = sign;                                     /* signed zero */
    } else {
        /* subnormal. IEEE value is f * 2^-24, i.e. biased exponent 113 - sh
         * after sh normalising shifts. The reference (q4_k.h:64-70) uses
         * 127 - 15 - sh = 112 - sh, which is half the IEEE value; this
         * restatement keeps the reference's formula so it stays bit-exact
         * with the reference's native build. NumPy's float16 -> float32
         * cast (and the GPU kernels) give the IEEE value. */
        int sh = 0;
        while (!(f & 0x400u)) { f <<= 1; ++sh; }
        bits = sign | ((uint32_t)(112 - sh) << 23) | ((f & 0x3FFu) << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

float oracle_fp16_to_fp32(uint16_t h) { return h2f(h); }

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static void k4_scales(const uint8_t* q, float sc[8], float m[8]) {
    for (int j = 0; j < 4; ++j) {
        sc[j] = (float)(q[j] & 63);
        m[j] = (float)(q[j + 4] & 63);
        sc[j + 4] = (float)((q[j + 8] & 15) | ((q[j] >> 6) << 4));
        m[j + 4] = (float)((q[j + 8] >> 4) | ((q[j + 4] >> 6) << 4));
    }
}

/* ---------------------------------------------------------------- Q4_K */

static void q4k_block_dequant(const uint8_t* blk, float* y) {
    float d = h2f(rd16(blk)), dmin = h2f(rd16(blk + 2));
    float sc[8], m[8];
    k4_scales(blk + 4, sc, m);
    const uint8_t* qs = blk + 16;
    for (int g = 0; g < 4; ++g) {
        float s0 = d * sc[2 * g], s1 = d * sc[2 * g + 1];
        float t0 = dmin * m[2 * g], t1 = dmin * m[2 * g + 1];
        for (int i = 0; i < 32; ++i) {
            uint8_t b = qs[32 * g + i];
            y[64 * g + i] = s0 * (float)(b & 15) - t0;
            y[64 * g + 32 + i] = s1 * (float)(b >> 4) - t1;
        }
    }
}

static float q4k_block_dot(const uint8_t* blk, const float* x) {
    float d = h2f(rd16(blk)), dmin = h2f(rd16(blk + 2));
    float sc[8], m[8];
    k4_scales(blk + 4, sc, m);
    const uint8_t* qs = blk + 16;
    float acc = 0.0f;
    for (int g = 0; g < 4; ++g) {
        float s0 = d * sc[2 * g], s1 = d * sc[2 * g + 1];
        float t0 = dmin * m[2 * g], t1 = dmin * m[2 * g + 1];
        for (int i = 0; i < 32; ++i) {
            uint8_t b = qs[32 * g + i];
            acc += (s0 * (float)(b & 15) - t0) * x[64 * g + i];        /* lo, then hi */
            acc += (s1 * (float)(b >> 4) - t1) * x[64 * g + 32 + i];
        }
    }
    return acc;
}

/* ---------------------------------------------------------------- Q6_K */

static int q6k_val(const uint8_t* ql, uint8_t qhb, int l, int k) {
    int nib = (k & 1) ? ql[l + 32] : ql[l];
    nib = (k >= 2) ? (nib >> 4) : (nib & 15);
    return nib | (((qhb >> (2 * k)) & 3) << 4);
}

static void q6k_block_dequant(const uint8_t* blk, float* y) {
    float d = h2f(rd16(blk + 208));
    const int8_t* sc = (const int8_t*)(blk + 192);
    for (int h = 0; h < 2; ++h) {
        const uint8_t* ql = blk + 64 * h;
        const uint8_t* qh = blk + 128 + 32 * h;
        for (int l = 0; l < 32; ++l)
            for (int k = 0; k < 4; ++k)
                y[128 * h + 32 * k + l] =
                    d * (float)sc[8 * h + l / 16 + 2 * k] * ((float)q6k_val(ql, qh[l], l, k) - 32.0f);
    }
}

static float q6k_block_dot(const uint8_t* blk, const float* x) {
    float d = h2f(rd16(blk + 208));
    const int8_t* sc = (const int8_t*)(blk + 192);
    float acc = 0.0f;
    for (int h = 0; h < 2; ++h) {          /* l-major: four groups per l */
        const uint8_t* ql = blk + 64 * h;
        const uint8_t* qh = blk + 128 + 32 * h;
        for (int l = 0; l < 32; ++l)
            for (int k = 0; k < 4; ++k) {
                float q = (float)q6k_val(ql, qh[l], l, k) - 32.0f;
                acc += d * (float)sc[8 * h + l / 16 + 2 * k] * q * x[128 * h + 32 * k + l];
            }
    }
    return acc;
}

/* ---------------------------------------------------------------- Q8_0 */

static void q8_0_block_dequant(const uint8_t* blk, float* y) {
    float d = h2f(rd16(blk));
    for (int i = 0; i < 32; ++i) y[i] = d * (float)(int8_t)blk[2 + i];
}

static float q8_0_block_dot(const uint8_t* blk, const float* x) {
    float d = h2f(rd16(blk));
    float acc = 0.0f;
    for (int i = 0; i < 32; ++i) acc += d * (float)(int8_t)blk[2 + i] * x[i];
    return acc;
}

/* --------------------------------------------------------- tensor level */

typedef float (*dot_fn)(const uint8_t*, const float*);

struct fmt { int bbytes, belems; dot_fn dot; void (*deq)(const uint8_t*, float*); };
static const struct fmt F_Q4K = {144, 256, q4k_block_dot, q4k_block_dequant};
static const struct fmt F_Q6K = {210, 256, q6k_block_dot, q6k_block_dequant};
static const struct fmt F_Q80 = {34, 32, q8_0_block_dot, q8_0_block_dequant};

static void rows(const struct fmt* f, const uint8_t* w, const float* x, float* y,
                 size_t r0, size_t r1, size_t k) {
    size_t nb = k / (size_t)f->belems;
    for (size_t i = r0; i < r1; ++i) {
        const uint8_t* row = w + i * nb * (size_t)f->bbytes;
        float acc = 0.0f;
        for (size_t b = 0; b < nb; ++b) acc += f->dot(row + b * f->bbytes, x + b * f->belems);
        y[i] = acc;
    }
}

struct job { const struct fmt* f; const uint8_t* w; const float* x; float* y; size_t r0, r1, k; };
static void* run_job(void* p) {
    struct job* j = (struct job*)p;
    rows(j->f, j->w, j->x, j->y, j->r0, j->r1, j->k);
    return NULL;
}

static void matmul_mt(const struct fmt* f, const uint8_t* w, const float* x, float* y,
                      size_t n, size_t k, int nthr) {
    if (nthr < 1) nthr = 1;
    if ((size_t)nthr > n) nthr = (int)(n ? n : 1);
    if (nthr == 1) { rows(f, w, x, y, 0, n, k); return; }
    pthread_t th[256];
    struct job jobs[256];
    if (nthr > 256) nthr = 256;
    size_t chunk = (n + nthr - 1) / nthr;
    int started = 0;
    for (int t = 0; t < nthr; ++t) {
        size_t r0 = (size_t)t * chunk, r1 = r0 + chunk < n ? r0 + chunk : n;
        if (r0 >= r1) break;
        jobs[t] = (struct job){f, w, x, y, r0, r1, k};
        if (pthread_create(&th[t], NULL, run_job, &jobs[t]) != 0) { run_job(&jobs[t]); th[t] = 0; }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t) if (th[t]) pthread_join(th[t], NULL);
}

static void deq(const struct fmt* f, const uint8_t* raw, size_t nblocks, float* out) {
    for (size_t b = 0; b < nblocks; ++b) f->deq(raw + b * f->bbytes, out + b * f->belems);
}

void oracle_dequant_q4_k(const uint8_t* raw, size_t nblocks, float* out) { deq(&F_Q4K, raw, nblocks, out); }
void oracle_dequant_q6_k(const uint8_t* raw, size_t nblocks, float* out) { deq(&F_Q6K, raw, nblocks, out); }
void oracle_dequant_q8_0(const uint8_t* raw, size_t nblocks, float* out) { deq(&F_Q80, raw, nblocks, out); }

void oracle_matmul_q4_k(const uint8_t* w, const float* x, float* y, size_t n, size_t k, int nthr) { matmul_mt(&F_Q4K, w, x, y, n, k, nthr); }
void oracle_matmul_q6_k(const uint8_t* w, const float* x, float* y, size_t n, size_t k, int nthr) { matmul_mt(&F_Q6K, w, x, y, n, k, nthr); }
void oracle_matmul_q8_0(const uint8_t* w, const float* x, float* y, size_t n, size_t k, int nthr) { matmul_mt(&F_Q80, w, x, y, n, k, nthr); }
