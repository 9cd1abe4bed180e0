/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the GGUF quantized-matmul path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or the timed CPU baseline). The
 * product (reflex_amd/) never links it and has no CPU fallback.
 *
 * Every function restates the reference's algorithm (paths relative to the
 * reference checkout):
 *   - le_f16 / get_scale_min_k4 / dequantize_block_{q4_k,q6_k,q8_0,q8_1} /
 *     dequantize: src/dequant.rs:33-47, :220-240, :339-367, :414-444, :53-161
 *   - host_matmul (f64 accumulation, f32 result): src/model/quant_resident_tests.rs:709-729
 *   - reference test generators synthetic_q4k / synthetic_q6k / synthetic_q8_0 /
 *     activations: quant_resident_tests.rs:907-925, quant_mma_tests.rs:64-84,
 *     quant_resident_tests.rs:669-692, quant_resident_tests.rs:40-52
 *   - route_top_k_with_norm: src/moe.rs:47-98
 *   - silu_and_mul: src/kernels_cuda/silu_and_mul.cu:7-23
 *   - rmsnorm: src/kernels_cuda/rmsnorm.cu:18-55, rmsnorm.cuh:17-41
 *   - moe_gather / moe_scatter_add: src/kernels_cuda/elementwise.cu:175-222
 *   - quantize_q8_1: the Q8_1 activation block (layout dequant.rs:228-240:
 *     d f16, s f16, qs[32]) filled by ggml's published quantize_row_q8_1_ref
 *     (ggml-quants.c: d = amax/127, id = 1/d, q = roundf(x*id), s = d*sum(q)).
 *     The reference has no activation quantizer; this is the north star's spec.
 *   - block_dots: the per-32 int32 dot products sum(qa*qw) that the MMQ kernel's
 *     int8 MFMA produces, qw being the weight's centered integer code (Q4_K
 *     nibble - 8, Q6_K (q6-32) times its 16-run scale, Q8_0 int8) as read
 *     from the same bytes the dequant formulas above read.
 *
 * Build with -ffp-contract=off so `d1 * q - m1` rounds twice, as Rust does.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256

/* ggml type ids (src/gguf.rs:124-152). */
enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 8, T_Q8_1 = 9, T_Q4K = 12, T_Q6K = 14 };

/* ---------- f16 <-> f32 (half 2.7.1 semantics: exact widening, RNE narrowing) ---------- */

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: normalise */
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0));
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1F) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t half_m = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

static float le_f16(const uint8_t* b) { return oracle_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }

/* dequant.rs:39-47 */
void oracle_get_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* dequant.rs:339-367 */
static void dq_q4_k(const uint8_t* block, float* y) {
    float d = le_f16(block);
    float min = le_f16(block + 2);
    const uint8_t* scales = block + 4;
    const uint8_t* q = block + 16;
    int is = 0;
    for (int j = 0; j < QK_K; j += 64) {
        uint8_t sc, m;
        oracle_get_scale_min_k4(is, scales, &sc, &m);
        float d1 = d * (float)sc;
        float m1 = min * (float)m;
        oracle_get_scale_min_k4(is + 1, scales, &sc, &m);
        float d2 = d * (float)sc;
        float m2 = min * (float)m;
        for (int l = 0; l < 32; l++) y[l] = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) y[32 + l] = d2 * (float)(q[l] >> 4) - m2;
        q += 32;
        is += 2;
        y += 64;
    }
}

/* dequant.rs:414-444: y = d * sc * q, evaluated left to right ((d*sc)*q). */
static void dq_q6_k(const uint8_t* block, float* y) {
    const uint8_t* ql = block;
    const uint8_t* qh = block + 128;
    const int8_t* sc = (const int8_t*)(block + 192);
    float d = le_f16(block + 208);
    for (int n = 0; n < QK_K; n += 128) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            uint8_t h = qh[l];
            int q1 = (int)((ql[l] & 0xF) | (((h >> 0) & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

/* dequant.rs:220-226 */
static void dq_q8_0(const uint8_t* block, float* y) {
    float d = le_f16(block);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)block[2 + j] * d;
}

/* dequant.rs:234-240 (s at bytes 2..4 is not used for values) */
static void dq_q8_1(const uint8_t* block, float* y) {
    float d = le_f16(block);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)block[4 + j] * d;
}

/*
 * dequant.rs:53-161. Returns the number of values written (element_count,
 * truncated from whole blocks), or -1 for a type with no dequantizer here
 * (the reference's Unknown-type error). `out` must hold nb*block_elems floats.
 */
long oracle_dequantize(int ty, const uint8_t* bytes, size_t nbytes, uint64_t element_count, float* out) {
    size_t bb, be;
    void (*f)(const uint8_t*, float*);
    switch (ty) {
        case T_F32: {
            size_t n = nbytes / 4;
            memcpy(out, bytes, n * 4);
            return (long)(element_count < n ? element_count : n);
        }
        case T_F16: {
            size_t n = nbytes / 2;
            for (size_t i = 0; i < n; i++) out[i] = le_f16(bytes + 2 * i);
            return (long)(element_count < n ? element_count : n);
        }
        case T_Q8_0: bb = 34; be = 32; f = dq_q8_0; break;
        case T_Q8_1: bb = 36; be = 32; f = dq_q8_1; break;
        case T_Q4K: bb = 144; be = QK_K; f = dq_q4_k; break;
        case T_Q6K: bb = 210; be = QK_K; f = dq_q6_k; break;
        default: return -1;
    }
    size_t nb = nbytes / bb;
    for (size_t i = 0; i < nb; i++) f(bytes + i * bb, out + i * be);
    size_t total = nb * be;
    return (long)(element_count < total ? element_count : total);
}

/* ---------- activation quantization (Q8_1, per 32) ---------- */

/*
 * x: [rows][k] f32, k % 32 == 0. qs: [rows][k] int8. ds: [rows][k/32][2] f16 bits
 * (d, s). d = amax/127 in f32, id = d ? 1/d : 0, q = roundf(x*id) (half away
 * from zero), stored d = f16(d), s = f16(sum(x) * id) with the sum taken in
 * f32 in the device kernel's order: p_j = ((x[4j]+x[4j+1])+x[4j+2])+x[4j+3],
 * then ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)).
 */
void oracle_quantize_q8_1(const float* x, long rows, long k, int8_t* qs, uint16_t* ds) {
    long nblk = k / 32;
    for (long r = 0; r < rows; r++) {
        for (long b = 0; b < nblk; b++) {
            const float* xb = x + r * k + b * 32;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) {
                float a = fabsf(xb[j]);
                if (a > amax) amax = a;
            }
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int j = 0; j < 32; j++) {
                float v = xb[j] * id;
                int q = (int)roundf(v);
                qs[r * k + b * 32 + j] = (int8_t)q;
            }
            float p[8];
            for (int j = 0; j < 8; j++) p[j] = ((xb[4 * j] + xb[4 * j + 1]) + xb[4 * j + 2]) + xb[4 * j + 3];
            float sum = ((p[0] + p[4]) + (p[2] + p[6])) + ((p[1] + p[5]) + (p[3] + p[7]));
            ds[(r * nblk + b) * 2 + 0] = oracle_f32_to_f16(d);
            ds[(r * nblk + b) * 2 + 1] = oracle_f32_to_f16(sum * id);
        }
    }
}

/* Integer weight code of element e (0..255) of a Q4_K / Q6_K block, or of a
 * Q8_0 block (e < 32): Q4_K nibble - 8, Q6_K q6 - 32, Q8_0 q. */
static int wcode(int ty, const uint8_t* blk, int e) {
    if (ty == T_Q4K) {
        int g = e / 64, r = e % 64;
        uint8_t b = blk[16 + 32 * g + (r % 32)];
        return (r < 32 ? (b & 0xF) : (b >> 4)) - 8; /* centered: the MMQ kernel's B operand */
    }
    if (ty == T_Q6K) {
        int n = e / 128, r = e % 128, t = r / 32, l = r % 32;
        uint8_t ql = blk[64 * n + l + ((t & 1) ? 32 : 0)];
        uint8_t qh = blk[128 + 32 * n + l];
        int lo = (t & 2) ? (ql >> 4) : (ql & 0xF);
        return (int)(lo | (((qh >> (2 * t)) & 3) << 4)) - 32;
    }
    return (int)(int8_t)blk[2 + e];
}

/* Q6_K: the int8 scale of element e's 16-run (sc[8n + l/16 + 2t]); 1 otherwise. */
static int wscale(int ty, const uint8_t* blk, int e) {
    if (ty != T_Q6K) return 1;
    int n = e / 128, r = e % 128, t = r / 32, l = r % 32;
    return (int)(int8_t)blk[192 + 8 * n + l / 16 + 2 * t];
}

/*
 * Per-32 integer dots: out[m][n][kb] = sum_{j<32} qa[m][32kb+j] * code(W[n], 32kb+j)
 * (for Q6_K each code is multiplied by its 16-run's int8 scale, which the MMQ
 * kernel folds into its 32-block dot).
 * w: n rows of k/QK blocks (row-major). Returns -1 for an unsupported type.
 */
int oracle_block_dots(int ty, const uint8_t* w, long n, long k, const int8_t* qa, long m, int32_t* out) {
    long bb, qk;
    if (ty == T_Q4K) { bb = 144; qk = 256; }
    else if (ty == T_Q6K) { bb = 210; qk = 256; }
    else if (ty == T_Q8_0) { bb = 34; qk = 32; }
    else return -1;
    long nb = k / qk, nkb = k / 32;
    int* codes = (int*)malloc(sizeof(int) * (size_t)k);
    for (long row = 0; row < n; row++) {
        for (long b = 0; b < nb; b++)
            for (long e = 0; e < qk; e++) codes[b * qk + e] = wcode((int)ty, w + (row * nb + b) * bb, (int)e) * wscale((int)ty, w + (row * nb + b) * bb, (int)e);
        for (long mm = 0; mm < m; mm++) {
            for (long kb = 0; kb < nkb; kb++) {
                int32_t s = 0;
                for (int j = 0; j < 32; j++) s += (int32_t)qa[mm * k + kb * 32 + j] * codes[kb * 32 + j];
                out[(mm * n + row) * nkb + kb] = s;
            }
        }
    }
    free(codes);
    return 0;
}

/* quant_resident_tests.rs:709-729: y[r][o] = (f32) sum_i (f64)x[r][i] * (f64)w[o][i]. */
void oracle_host_matmul(const float* x, const float* w, long rows, long in_f, long out_f, float* y) {
#pragma omp parallel for schedule(static)
    for (long o = 0; o < out_f; o++) {
        const float* wo = w + o * in_f;
        for (long r = 0; r < rows; r++) {
            const float* xr = x + r * in_f;
            double s = 0.0;
            for (long i = 0; i < in_f; i++) s += (double)xr[i] * (double)wo[i];
            y[r * out_f + o] = (float)s;
        }
    }
}

/* ---------- the reference's test generators (xorshift64) ---------- */

static uint64_t xs_next(uint64_t* s) {
    *s ^= *s << 13;
    *s ^= *s >> 7;
    *s ^= *s << 17;
    return *s;
}

/* quant_resident_tests.rs:907-925 */
void oracle_synthetic_q4k(long in_f, long out_f, uint64_t seed, uint8_t* out) {
    long blocks = in_f / QK_K * out_f;
    uint64_t s = (seed * 0x9E3779B97F4A7C15ull) | 1ull;
    uint8_t* p = out;
    for (long b = 0; b < blocks; b++) {
        for (int i = 0; i < 2; i++) {
            float v = ((float)(xs_next(&s) >> 40) / (float)(1ull << 24)) * 0.01f + 1e-4f;
            uint16_t h = oracle_f32_to_f16(v);
            *p++ = (uint8_t)(h & 0xFF);
            *p++ = (uint8_t)(h >> 8);
        }
        for (int i = 0; i < 140; i++) *p++ = (uint8_t)xs_next(&s);
    }
}

/* quant_mma_tests.rs:64-84 */
void oracle_synthetic_q6k(long in_f, long out_f, uint64_t seed, uint8_t* out) {
    long blocks = in_f / QK_K * out_f;
    uint64_t s = (seed * 0x9E3779B97F4A7C15ull) | 1ull;
    uint8_t* p = out;
    for (long b = 0; b < blocks; b++) {
        for (int i = 0; i < 208; i++) *p++ = (uint8_t)xs_next(&s);
        float d;
        if (b % 16 == 0) d = 0.0f;
        else if (b % 16 == 1) d = -2e-4f;
        else d = ((float)(xs_next(&s) >> 40) / (float)(1ull << 24)) * 4e-4f + 1e-6f;
        uint16_t h = oracle_f32_to_f16(d);
        *p++ = (uint8_t)(h & 0xFF);
        *p++ = (uint8_t)(h >> 8);
    }
}

/* quant_resident_tests.rs:669-692 */
void oracle_synthetic_q8_0(long in_f, long out_f, uint64_t seed, uint8_t* out) {
    long blocks = in_f / 32 * out_f;
    uint64_t s = (seed * 0x9E3779B97F4A7C15ull) | 1ull;
    uint8_t* p = out;
    for (long b = 0; b < blocks; b++) {
        uint16_t h;
        if (b % 16 == 0) {
            h = 0;
        } else if (b % 16 == 1) {
            h = (uint16_t)(xs_next(&s) % 0x3FF + 1);
        } else {
            float v = ((float)(xs_next(&s) >> 40) / (float)(1ull << 24)) * 0.02f + 1e-4f;
            h = oracle_f32_to_f16((xs_next(&s) & 1) == 0 ? v : -v);
        }
        *p++ = (uint8_t)(h & 0xFF);
        *p++ = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; i++) *p++ = (uint8_t)xs_next(&s);
    }
}

/* quant_resident_tests.rs:40-52: LCG activations in [-1, 1). */
void oracle_activations(long n, uint64_t seed, float* out) {
    uint64_t s = seed * 6364136223846793005ull + 1442695040888963407ull;
    for (long i = 0; i < n; i++) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        out[i] = ((float)(s >> 40) / (float)(1ull << 24)) * 2.0f - 1.0f;
    }
}

/* ---------- MoE host pieces ---------- */

/*
 * moe.rs:47-98. Writes k (expert, weight) pairs sorted by probability
 * descending, ties to the lower index. Returns 0, or -1 on the reference's
 * error conditions (empty logits, k out of range, non-finite / non-positive mass).
 */
int oracle_route_top_k(const float* logits, long n, long k, int normalize, int32_t* idx, float* w) {
    if (n <= 0 || k <= 0 || k > n) return -1;
    float maxl = -INFINITY;
    for (long i = 0; i < n; i++) maxl = fmaxf(maxl, logits[i]);
    float* probs = (float*)malloc(sizeof(float) * (size_t)n);
    float sum = 0.0f;
    for (long i = 0; i < n; i++) {
        probs[i] = expf(logits[i] - maxl);
        sum += probs[i];
    }
    if (!isfinite(sum) || sum <= 0.0f) {
        free(probs);
        return -1;
    }
    for (long i = 0; i < n; i++) probs[i] = probs[i] / sum;
    /* selection of the k best by (prob desc, index asc): O(n*k), n is the expert count */
    char* taken = (char*)calloc((size_t)n, 1);
    for (long t = 0; t < k; t++) {
        long best = -1;
        for (long i = 0; i < n; i++) {
            if (taken[i]) continue;
            if (best < 0 || probs[i] > probs[best]) best = i;
        }
        taken[best] = 1;
        idx[t] = (int32_t)best;
        w[t] = probs[best];
    }
    free(taken);
    int rc = 0;
    if (normalize) {
        float ts = 0.0f;
        for (long t = 0; t < k; t++) ts += w[t];
        if (!isfinite(ts) || ts <= 0.0f) rc = -1;
        else
            for (long t = 0; t < k; t++) w[t] = w[t] / ts;
    }
    free(probs);
    return rc;
}

/* silu_and_mul.cu:7-23 */
void oracle_silu_and_mul(const float* gate, const float* up, float* out, long n) {
    for (long i = 0; i < n; i++) {
        float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/*
 * rmsnorm.cu:18-55 with rmsnorm.cuh:17-41: per row, sum_sq accumulated in
 * index order as fused multiply-adds (nvcc contracts `sum_sq += v * v`, as
 * rmsnorm.cuh:4-5 states), r = 1 / sqrtf(sum_sq / hidden + eps), and
 * y = (x * r) * w (two roundings).
 */
void oracle_rmsnorm(const float* x, const float* w, float* y, long rows, long k, float eps) {
    for (long r = 0; r < rows; r++) {
        const float* xr = x + r * k;
        float sum_sq = 0.0f;
        for (long i = 0; i < k; i++) sum_sq = fmaf(xr[i], xr[i], sum_sq);
        const float inv = 1.0f / sqrtf(sum_sq / (float)k + eps);
        for (long i = 0; i < k; i++) y[r * k + i] = (xr[i] * inv) * w[i];
    }
}

/* ---------- CPU baseline: dequant restatement + f32 matmul ---------- */

/*
 * The reference's CPU path for one GEMM (dequant::dequantize then an f32 host
 * matmul), row-parallel over `threads` OpenMP threads. x: [rows][k], y: [rows][n].
 */
int oracle_cpu_dequant_matmul(int ty, const uint8_t* w, long n, long k, const float* x, long rows, float* y,
                              int threads) {
    long bb, qk;
    if (ty == T_Q4K) { bb = 144; qk = 256; }
    else if (ty == T_Q6K) { bb = 210; qk = 256; }
    else if (ty == T_Q8_0) { bb = 34; qk = 32; }
    else return -1;
    long row_bytes = k / qk * bb;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#endif
#pragma omp parallel
    {
        float* wrow = (float*)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
        for (long o = 0; o < n; o++) {
            oracle_dequantize(ty, w + o * row_bytes, (size_t)row_bytes, (uint64_t)k, wrow);
            for (long r = 0; r < rows; r++) {
                const float* xr = x + r * k;
                float s = 0.0f;
                for (long i = 0; i < k; i++) s += xr[i] * wrow[i];
                y[r * n + o] = s;
            }
        }
        free(wrow);
    }
    return 0;
}
