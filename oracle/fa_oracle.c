/*
 * fa_oracle.c -- CPU oracle for GGML_OP_FLASH_ATTN_EXT and for the KV-cache
 * write before it, GGML_OP_SET_ROWS (ora_set_rows, at the end of this file).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py
 * may load it.  The product path (libmxfa) never links or calls it.
 *
 * What it restates.  acestep.cpp builds every attention node with
 * ggml_flash_attn_ext(q, k, v, mask, scale, 0, 0) + GGML_PREC_F32
 * (reference src/qwen3-lm.h:465-469, :789-794; src/dit-graph.h:227-231,
 * :348-352; src/qwen3-enc.h:195-199).  The arithmetic of that op lives in the
 * ggml submodule, which is EMPTY in the reference checkout
 * (/root/reference/ggml, .gitmodules:1-3, revision unpinned: update.sh:3-5).
 * The ggml CPU kernel (ggml-cpu ops.cpp,
 * ggml_compute_forward_flash_attn_ext_f16_one_chunk, upstream ggml late 2025)
 * is therefore restated from its published algorithm:
 *
 *   per output row (iq1 query, iq2 head, iq3 batch):
 *     Q (F32) is converted to K's vec-dot type (F16 for F16 K, BF16 for BF16 K,
 *     Q8_0 for Q8_0 K) before the KQ dot;
 *     M = -inf, S = 0; accumulator is fp16 (VKQ16) when V is F16, else fp32;
 *     for every key ic: mv = slope*mask[ic]; if mv == -inf skip the key
 *     (K and V are not read); s = dot(K[ic], Qconv)*scale (+softcap) + mv;
 *     if s > M: ms = exp(Mold - s), M = s, acc *= ms; else vs = exp(s - M);
 *     acc += vs*V[ic] (rounded to fp16 every step when V is F16);
 *     S = S*ms + vs;
 *     out = acc * (S == 0 ? 0 : 1/S) written to dst[DV, Nh, Sq, B].
 *
 * The SIMD reduction orders follow ggml's x86 AVX2 code paths (the "haswell"
 * CPU variant): 4x8-lane fp32 accumulators for the F16 dot, 4x8 for BF16,
 * 8 int32 lane partials for the Q8_0 dot, round-half-even Q8_0 quantisation
 * with id = 127/amax.  Real ggml picks its SIMD variant at run time, so the
 * exact bit pattern of its sums is NOT pinned here ("parity unpinned" at the
 * last-ulp level); what is pinned (tests/test_oracle.py) is everything a
 * plausible mistake would break: the fp64 closed form on tiny shapes, the
 * GQA head map, the mask broadcast and -inf skip, the output permutation and
 * the special cases (single key, uniform V, key permutation, scale 0, fully
 * masked row -> 0).
 *
 * ora_fa_exact() is an independent fp64 two-pass softmax reference of the
 * same op (the non-FA path of the reference, qwen3-enc.h:101-112 /
 * dit-graph.h:123-134: mul_mat(K,Q) -> soft_max_ext(mask, scale) ->
 * mul_mat(V^T, P) -> permute(0,2,1,3)).
 *
 * Tensor descriptors follow ggml: ne[0] is the innermost dimension, nb[] are
 * byte strides.  Type ids are ggml's: F32=0, F16=1, Q8_0=8, BF16=30.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#define ORA_X86 1
#else
#define ORA_X86 0
#endif

enum { ORA_F32 = 0, ORA_F16 = 1, ORA_Q8_0 = 8, ORA_BF16 = 30 };
#define QK8_0 32
#define Q8_0_BYTES 34

typedef struct {
    int32_t     type;
    int64_t     ne[4];
    size_t      nb[4];
    const void *data;
} ora_tensor;

/* ------------------------------------------------------------------------ */
/* Scalar codecs.  fp16 = IEEE binary16 with round-to-nearest-even (what     */
/* F16C's _cvtss_sh(x, 0) and ggml's GGML_CPU_FP32_TO_FP16 produce); bf16 =   */
/* round-to-nearest-even of the top 16 bits, NaN kept quiet (ggml's           */
/* ggml_compute_fp32_to_bf16).                                                */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float ora_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24 is exact in fp32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t ora_f2h(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf or NaN */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (ax < 0x38800000u) {                        /* result subnormal or 0 */
        if (ax < 0x33000000u) return (uint16_t)sign;  /* < 2^-25: to zero */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                 /* 14..24 */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ax - 0x38000000u;                 /* rebias 127 -> 15 */
    uint32_t lsb = (r >> 13) & 1u;
    r += 0xfffu + lsb;
    return (uint16_t)(sign | (r >> 13));
}

float ora_bf2f(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t ora_f2bf(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 64u);
    return (uint16_t)((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

void ora_f32_to_f16(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ora_f2h(x[i]);
}
void ora_f16_to_f32(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ora_h2f(x[i]);
}
void ora_f32_to_bf16(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ora_f2bf(x[i]);
}
void ora_bf16_to_f32(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = ora_bf2f(x[i]);
}

/* Q8_0 block: fp16 d, then 32 int8 qs (34 bytes, ggml block_q8_0).
 * Quantiser as in ggml's AVX2 quantize_row_q8_0: amax over the block,
 * d = amax/127 stored as fp16, q = round_half_even(x * (127/amax)). */
void ora_quantize_q8_0(const float *x, uint8_t *y, int64_t n) {
    for (int64_t ib = 0; ib < n / QK8_0; ib++) {
        const float *xb = x + ib * QK8_0;
        uint8_t *yb = y + ib * Q8_0_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.f;
        const float id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        uint16_t dh = ora_f2h(d);
        memcpy(yb, &dh, 2);
        for (int j = 0; j < QK8_0; j++) {
            float v = nearbyintf(xb[j] * id);      /* default FE_TONEAREST */
            yb[2 + j] = (uint8_t)(int8_t)(int)v;
        }
    }
}

void ora_dequantize_q8_0(const uint8_t *x, float *y, int64_t n) {
    for (int64_t ib = 0; ib < n / QK8_0; ib++) {
        const uint8_t *xb = x + ib * Q8_0_BYTES;
        uint16_t dh;
        memcpy(&dh, xb, 2);
        const float d = ora_h2f(dh);
        for (int j = 0; j < QK8_0; j++) y[ib * QK8_0 + j] = (float)(int8_t)xb[2 + j] * d;
    }
}

/* ------------------------------------------------------------------------ */
/* Vector kernels in ggml's x86 AVX2 reduction order.  Each has a scalar     */
/* form with the identical sequence of IEEE operations (per-lane fma, the    */
/* same pairwise tree), so both forms give identical bits; the AVX2 form is  */
/* only used for speed when the host has AVX2+FMA+F16C.                      */
/* ------------------------------------------------------------------------ */

/* ggml_vec_dot_f16: GGML_F16_STEP=32, EPR=8 -> sum[4][8] fp32, fma per lane;
 * reduce sum0+=sum2, sum1+=sum3, sum0+=sum1; then 8->4 (lo+hi), hadd, hadd;
 * leftover elements accumulated in double. */
static float dot_f16_scalar(int64_t n, const uint16_t *x, const uint16_t *y) {
    float sum[4][8] = {{0}};
    const int64_t np = n & ~(int64_t)31;
    for (int64_t i = 0; i < np; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++)
                sum[j][l] = fmaf(ora_h2f(x[i + 8 * j + l]), ora_h2f(y[i + 8 * j + l]), sum[j][l]);
    for (int l = 0; l < 8; l++) { sum[0][l] += sum[2][l]; sum[1][l] += sum[3][l]; }
    for (int l = 0; l < 8; l++) sum[0][l] += sum[1][l];
    float t0[4];
    for (int l = 0; l < 4; l++) t0[l] = sum[0][l] + sum[0][l + 4];
    float t1a = t0[0] + t0[1], t1b = t0[2] + t0[3];
    double sumf = (double)(t1a + t1b);
    for (int64_t i = np; i < n; i++) sumf += (double)(ora_h2f(x[i]) * ora_h2f(y[i]));
    return (float)sumf;
}

/* ggml_vec_dot_bf16 (AVX2 branch): c1..c4 += x*y (mul then add, not fused)
 * on 8 lanes each; c1 = (c1+c3)+(c2+c4); 8->4 (hi+lo); movehl; movehdup. */
static float dot_bf16_scalar(int64_t n, const uint16_t *x, const uint16_t *y) {
    float c[4][8] = {{0}};
    int64_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++) {
                float p = ora_bf2f(x[i + 8 * j + l]) * ora_bf2f(y[i + 8 * j + l]);
                c[j][l] = p + c[j][l];
            }
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = (c[0][l] + c[2][l]) + (c[1][l] + c[3][l]);
    float g[4];
    for (int l = 0; l < 4; l++) g[l] = s[l + 4] + s[l];
    float g0 = g[0] + g[2], g1 = g[1] + g[3];
    double sumf = (double)(g0 + g1);
    for (; i < n; i++) sumf += (double)(ora_bf2f(x[i]) * ora_bf2f(y[i]));
    return (float)sumf;
}

/* ggml_vec_dot_q8_0_q8_0 (AVX2): per block, 8 int32 lane partials (lane j
 * sums products 4j..4j+3), converted to float, acc[j] = fma(dx*dy, p[j],
 * acc[j]); hsum_float_8: (hi+lo) -> r0+r2, r1+r3 -> sum. */
static float dot_q8_0_scalar(int64_t n, const uint8_t *x, const uint8_t *y) {
    float acc[8] = {0};
    for (int64_t ib = 0; ib < n / QK8_0; ib++) {
        const uint8_t *xb = x + ib * Q8_0_BYTES, *yb = y + ib * Q8_0_BYTES;
        uint16_t dx, dy;
        memcpy(&dx, xb, 2);
        memcpy(&dy, yb, 2);
        const float d = ora_h2f(dx) * ora_h2f(dy);
        for (int j = 0; j < 8; j++) {
            int32_t p = 0;
            for (int t = 0; t < 4; t++)
                p += (int32_t)(int8_t)xb[2 + 4 * j + t] * (int32_t)(int8_t)yb[2 + 4 * j + t];
            acc[j] = fmaf(d, (float)p, acc[j]);
        }
    }
    float r[4];
    for (int l = 0; l < 4; l++) r[l] = acc[l + 4] + acc[l];
    float a = r[0] + r[2], b = r[1] + r[3];
    return a + b;
}

/* ggml_vec_mad_f16 (F16C path): y = fp16(fma(fp32(x), v, fp32(y))). */
static void mad_f16_scalar(int64_t n, uint16_t *y, const uint16_t *x, float v) {
    for (int64_t i = 0; i < n; i++) y[i] = ora_f2h(fmaf(ora_h2f(x[i]), v, ora_h2f(y[i])));
}
/* ggml_vec_scale_f16: y = fp16(fp32(y) * v). */
static void scale_f16_scalar(int64_t n, uint16_t *y, float v) {
    for (int64_t i = 0; i < n; i++) y[i] = ora_f2h(ora_h2f(y[i]) * v);
}

#if ORA_X86
__attribute__((target("avx2,fma,f16c")))
static float dot_f16_avx2(int64_t n, const uint16_t *x, const uint16_t *y) {
    __m256 sum[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    const int64_t np = n & ~(int64_t)31;
    for (int64_t i = 0; i < np; i += 32)
        for (int j = 0; j < 4; j++) {
            __m256 ax = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x + i + 8 * j)));
            __m256 ay = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i + 8 * j)));
            sum[j] = _mm256_fmadd_ps(ax, ay, sum[j]);
        }
    sum[0] = _mm256_add_ps(sum[0], sum[2]);
    sum[1] = _mm256_add_ps(sum[1], sum[3]);
    sum[0] = _mm256_add_ps(sum[0], sum[1]);
    __m128 t0 = _mm_add_ps(_mm256_castps256_ps128(sum[0]), _mm256_extractf128_ps(sum[0], 1));
    __m128 t1 = _mm_hadd_ps(t0, t0);
    double sumf = (double)_mm_cvtss_f32(_mm_hadd_ps(t1, t1));
    for (int64_t i = np; i < n; i++) sumf += (double)(ora_h2f(x[i]) * ora_h2f(y[i]));
    return (float)sumf;
}

__attribute__((target("avx2,fma,f16c")))
static void mad_f16_avx2(int64_t n, uint16_t *y, const uint16_t *x, float v) {
    const __m256 vx = _mm256_set1_ps(v);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 ax = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x + i)));
        __m256 ay = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i)));
        ay = _mm256_fmadd_ps(ax, vx, ay);
        _mm_storeu_si128((__m128i *)(y + i), _mm256_cvtps_ph(ay, 0));
    }
    for (; i < n; i++) y[i] = ora_f2h(fmaf(ora_h2f(x[i]), v, ora_h2f(y[i])));
}

__attribute__((target("avx2,fma,f16c")))
static void scale_f16_avx2(int64_t n, uint16_t *y, float v) {
    const __m256 vx = _mm256_set1_ps(v);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 ay = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(y + i)));
        _mm_storeu_si128((__m128i *)(y + i), _mm256_cvtps_ph(_mm256_mul_ps(ay, vx), 0));
    }
    for (; i < n; i++) y[i] = ora_f2h(ora_h2f(y[i]) * v);
}

/* dot_bf16 with AVX2: the same lanes, the same mul-then-add per lane and the
 * same reduction as dot_bf16_scalar, so the bits agree. */
__attribute__((target("avx2,fma,f16c")))
static float dot_bf16_avx2(int64_t n, const uint16_t *x, const uint16_t *y) {
    __m256 c[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    int64_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 4; j++) {
            const __m256i xi = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(x + i + 8 * j)));
            const __m256i yi = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(y + i + 8 * j)));
            const __m256 p = _mm256_mul_ps(_mm256_castsi256_ps(_mm256_slli_epi32(xi, 16)),
                                           _mm256_castsi256_ps(_mm256_slli_epi32(yi, 16)));
            c[j] = _mm256_add_ps(p, c[j]);
        }
    float cl[4][8];
    for (int j = 0; j < 4; j++) _mm256_storeu_ps(cl[j], c[j]);
    float s[8];
    for (int l = 0; l < 8; l++) s[l] = (cl[0][l] + cl[2][l]) + (cl[1][l] + cl[3][l]);
    float g[4];
    for (int l = 0; l < 4; l++) g[l] = s[l + 4] + s[l];
    float g0 = g[0] + g[2], g1 = g[1] + g[3];
    double sumf = (double)(g0 + g1);
    for (; i < n; i++) sumf += (double)(ora_bf2f(x[i]) * ora_bf2f(y[i]));
    return (float)sumf;
}

/* fp32 accumulator step y[d] = fma(v16[d], s, y[d]) for an F16 or BF16 row
 * (the scalar form converts the row, then fmaf per element: same bits). */
__attribute__((target("avx2,fma,f16c")))
static void mad_f32_avx2(int64_t n, float *y, const uint16_t *x, int is_bf16, float v) {
    const __m256 vv = _mm256_set1_ps(v);
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        const __m128i xh = _mm_loadu_si128((const __m128i *)(x + i));
        const __m256 ax = is_bf16 ? _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(xh), 16))
                                  : _mm256_cvtph_ps(xh);
        _mm256_storeu_ps(y + i, _mm256_fmadd_ps(ax, vv, _mm256_loadu_ps(y + i)));
    }
    for (; i < n; i++) y[i] = fmaf(is_bf16 ? ora_bf2f(x[i]) : ora_h2f(x[i]), v, y[i]);
}

static int g_have_avx2 = -1;
static int have_avx2(void) {
    if (g_have_avx2 < 0) {
        __builtin_cpu_init();
        g_have_avx2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
                      __builtin_cpu_supports("f16c");
    }
    return g_have_avx2;
}
#else
static int have_avx2(void) { return 0; }
#endif

/* Force the scalar forms (used by tests to prove both forms agree). */
static int g_force_scalar = 0;
void ora_set_force_scalar(int on) { g_force_scalar = on; }
int ora_simd_available(void) { return have_avx2(); }

static inline int use_simd(void) { return !g_force_scalar && have_avx2(); }

static float dot_f16(int64_t n, const uint16_t *x, const uint16_t *y) {
#if ORA_X86
    if (use_simd()) return dot_f16_avx2(n, x, y);
#endif
    return dot_f16_scalar(n, x, y);
}
static void mad_f16(int64_t n, uint16_t *y, const uint16_t *x, float v) {
#if ORA_X86
    if (use_simd()) { mad_f16_avx2(n, y, x, v); return; }
#endif
    mad_f16_scalar(n, y, x, v);
}
static float dot_bf16(int64_t n, const uint16_t *x, const uint16_t *y) {
#if ORA_X86
    if (use_simd()) return dot_bf16_avx2(n, x, y);
#endif
    return dot_bf16_scalar(n, x, y);
}
/* returns 1 when it handled the row (F16 / BF16 row and SIMD available) */
static int mad_f32_row(int64_t n, float *y, const uint16_t *x, int is_bf16, float v) {
#if ORA_X86
    if (use_simd()) { mad_f32_avx2(n, y, x, is_bf16, v); return 1; }
#endif
    (void)n; (void)y; (void)x; (void)is_bf16; (void)v;
    return 0;
}
static void scale_f16(int64_t n, uint16_t *y, float v) {
#if ORA_X86
    if (use_simd()) { scale_f16_avx2(n, y, v); return; }
#endif
    scale_f16_scalar(n, y, v);
}

/* Exposed for tests: one dot / mad step on caller buffers. */
float ora_dot_f16(int64_t n, const uint16_t *x, const uint16_t *y) { return dot_f16(n, x, y); }
float ora_dot_bf16(int64_t n, const uint16_t *x, const uint16_t *y) { return dot_bf16(n, x, y); }
float ora_dot_q8_0(int64_t n, const uint8_t *x, const uint8_t *y) { return dot_q8_0_scalar(n, x, y); }
void ora_mad_f16(int64_t n, uint16_t *y, const uint16_t *x, float v) { mad_f16(n, y, x, v); }

/* ------------------------------------------------------------------------ */
/* Shape checks shared by both oracles (ggml_flash_attn_ext's asserts).      */
/* ------------------------------------------------------------------------ */
static int check_shapes(const ora_tensor *q, const ora_tensor *k, const ora_tensor *v,
                        const ora_tensor *mask) {
    if (!q || !k || !v) return -1;
    if (q->type != ORA_F32) return -2;
    if (k->type != ORA_F16 && k->type != ORA_BF16 && k->type != ORA_Q8_0) return -2;
    if (v->type != ORA_F16 && v->type != ORA_BF16 && v->type != ORA_Q8_0 && v->type != ORA_F32) return -2;
    if (q->ne[0] != k->ne[0]) return -3;                 /* DK */
    if (k->ne[1] != v->ne[1]) return -3;                 /* Skv */
    if (k->ne[2] <= 0 || q->ne[2] % k->ne[2] || q->ne[2] % v->ne[2]) return -3;
    if (k->ne[3] <= 0 || q->ne[3] % k->ne[3] || q->ne[3] % v->ne[3]) return -3;
    if ((k->type == ORA_Q8_0 && k->ne[0] % QK8_0) || (v->type == ORA_Q8_0 && v->ne[0] % QK8_0)) return -3;
    if (mask) {
        if (mask->type != ORA_F16) return -2;
        if (mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1]) return -3;
        if (mask->ne[2] <= 0 || mask->ne[3] <= 0) return -3;
        if (q->ne[2] % mask->ne[2] || q->ne[3] % mask->ne[3]) return -3;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* ggml-CPU-semantics oracle.                                                */
/* ------------------------------------------------------------------------ */
typedef struct {
    const ora_tensor *q, *k, *v, *mask;
    float scale, max_bias, softcap;
    int acc_f32;   /* 1: fp32 VKQ accumulator even for F16 V */
    float *dst;
    int64_t nrows;
    int nth, ith;
} ggml_job;

static void *ggml_rows(void *arg) {
    ggml_job *J = (ggml_job *)arg;
    const ora_tensor *q = J->q, *k = J->k, *v = J->v, *mask = J->mask;
    const int64_t DK = k->ne[0], DV = v->ne[0];
    const int64_t neq1 = q->ne[1], neq2 = q->ne[2], neq3 = q->ne[3];
    const int64_t nek1 = k->ne[1];
    const int64_t rk2 = neq2 / k->ne[2], rk3 = neq3 / k->ne[3];
    const int64_t rv2 = neq2 / v->ne[2], rv3 = neq3 / v->ne[3];
    float scale = J->scale;
    const float max_bias = J->max_bias, softcap = J->softcap;
    const int acc16 = (v->type == ORA_F16) && !J->acc_f32;
    if (softcap != 0.0f) scale /= softcap;
    const uint32_t n_head = (uint32_t)neq2;
    const uint32_t n_head_log2 = 1u << (uint32_t)floor(log2((double)n_head));
    const float m0 = powf(2.0f, -(max_bias) / (float)n_head_log2);
    const float m1 = powf(2.0f, -(max_bias / 2.0f) / (float)n_head_log2);

    float *VKQ32 = (float *)calloc((size_t)DV, sizeof(float));
    float *V32 = (float *)calloc((size_t)DV, sizeof(float));
    uint16_t *VKQ16 = (uint16_t *)calloc((size_t)DV, sizeof(uint16_t));
    uint8_t *Qq = (uint8_t *)calloc((size_t)DK * 4 + 64, 1);   /* converted Q */
    const int64_t dr = (J->nrows + J->nth - 1) / J->nth;
    const int64_t ir0 = dr * J->ith;
    const int64_t ir1 = ir0 + dr < J->nrows ? ir0 + dr : J->nrows;

    for (int64_t ir = ir0; ir < ir1; ir++) {
        const int64_t iq3 = ir / (neq2 * neq1);
        const int64_t iq2 = (ir - iq3 * neq2 * neq1) / neq1;
        const int64_t iq1 = ir - iq3 * neq2 * neq1 - iq2 * neq1;
        const uint32_t h = (uint32_t)iq2;
        const float slope = (max_bias > 0.0f)
            ? (h < n_head_log2 ? powf(m0, (float)(h + 1)) : powf(m1, (float)(2 * (h - n_head_log2) + 1)))
            : 1.0f;
        float S = 0.0f, M = -INFINITY;
        if (acc16) memset(VKQ16, 0, (size_t)DV * 2);
        else memset(VKQ32, 0, (size_t)DV * 4);

        const uint16_t *mp = mask
            ? (const uint16_t *)((const char *)mask->data + iq1 * mask->nb[1] +
                                 (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3])
            : NULL;
        const int64_t ik3 = iq3 / rk3, ik2 = iq2 / rk2;
        const int64_t iv3 = iq3 / rv3, iv2 = iq2 / rv2;
        const float *pq = (const float *)((const char *)q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3]);
        if (k->type == ORA_F16) ora_f32_to_f16(pq, (uint16_t *)Qq, DK);
        else if (k->type == ORA_BF16) ora_f32_to_bf16(pq, (uint16_t *)Qq, DK);
        else ora_quantize_q8_0(pq, Qq, DK);

        for (int64_t ic = 0; ic < nek1; ic++) {
            const float mv = mp ? slope * ora_h2f(mp[ic]) : 0.0f;
            if (mv == -INFINITY) continue;
            const char *kd = (const char *)k->data + ic * k->nb[1] + ik2 * k->nb[2] + ik3 * k->nb[3];
            float s;
            if (k->type == ORA_F16) s = dot_f16(DK, (const uint16_t *)kd, (const uint16_t *)Qq);
            else if (k->type == ORA_BF16) s = dot_bf16(DK, (const uint16_t *)kd, (const uint16_t *)Qq);
            else s = dot_q8_0_scalar(DK, (const uint8_t *)kd, Qq);
            s = s * scale;
            if (softcap != 0.0f) s = softcap * tanhf(s);
            s += mv;
            const float Mold = M;
            float ms = 1.0f, vs = 1.0f;
            const char *vd = (const char *)v->data + ic * v->nb[1] + iv2 * v->nb[2] + iv3 * v->nb[3];
            if (acc16) {
                if (s > M) {
                    M = s;
                    ms = expf(Mold - M);
                    scale_f16(DV, VKQ16, ms);
                } else {
                    vs = expf(s - M);
                }
                mad_f16(DV, VKQ16, (const uint16_t *)vd, vs);
            } else {
                if (s > M) {
                    M = s;
                    ms = expf(Mold - M);
                    for (int64_t d = 0; d < DV; d++) VKQ32[d] *= ms;
                } else {
                    vs = expf(s - M);
                }
                if ((v->type == ORA_F16 || v->type == ORA_BF16) &&
                    mad_f32_row(DV, VKQ32, (const uint16_t *)vd, v->type == ORA_BF16, vs)) {
                    S = S * ms + vs;
                    continue;
                }
                const float *vrow;
                if (v->type == ORA_F16) { ora_f16_to_f32((const uint16_t *)vd, V32, DV); vrow = V32; }
                else if (v->type == ORA_BF16) { ora_bf16_to_f32((const uint16_t *)vd, V32, DV); vrow = V32; }
                else if (v->type == ORA_Q8_0) { ora_dequantize_q8_0((const uint8_t *)vd, V32, DV); vrow = V32; }
                else vrow = (const float *)vd;
                for (int64_t d = 0; d < DV; d++) VKQ32[d] = fmaf(vrow[d], vs, VKQ32[d]);
            }
            S = S * ms + vs;
        }
        if (acc16)
            for (int64_t d = 0; d < DV; d++) VKQ32[d] = ora_h2f(VKQ16[d]);
        const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
        float *out = J->dst + ((iq3 * neq1 + iq1) * neq2 + iq2) * DV;
        for (int64_t d = 0; d < DV; d++) out[d] = VKQ32[d] * S_inv;
    }
    free(VKQ32); free(V32); free(VKQ16); free(Qq);
    return NULL;
}

/* dst: contiguous F32 [DV, Nh, Sq, B] (ggml's permuted FA output).
 * acc_f32 = 0: ggml's CPU kernel as it is (fp16 running accumulator for F16
 * V).  acc_f32 = 1: the same algorithm with an fp32 accumulator for every V
 * type (V rows converted to fp32 per key, as ggml already does for non-F16
 * V) -- the "fp32 accumulate" form of the op. */
int ora_fa_ggml_ex(const ora_tensor *q, const ora_tensor *k, const ora_tensor *v, const ora_tensor *mask,
                   float scale, float max_bias, float softcap, int acc_f32, float *dst, int n_threads) {
    int rc = check_shapes(q, k, v, mask);
    if (rc) return rc;
    if (n_threads < 1) n_threads = 1;
    const int64_t nrows = q->ne[1] * q->ne[2] * q->ne[3];
    ggml_job *jobs = (ggml_job *)calloc((size_t)n_threads, sizeof(ggml_job));
    pthread_t *th = (pthread_t *)calloc((size_t)n_threads, sizeof(pthread_t));
    for (int t = 0; t < n_threads; t++) {
        jobs[t] = (ggml_job){q, k, v, mask, scale, max_bias, softcap, acc_f32, dst, nrows, n_threads, t};
        if (t > 0) pthread_create(&th[t], NULL, ggml_rows, &jobs[t]);
    }
    ggml_rows(&jobs[0]);
    for (int t = 1; t < n_threads; t++) pthread_join(th[t], NULL);
    free(jobs); free(th);
    return 0;
}

int ora_fa_ggml(const ora_tensor *q, const ora_tensor *k, const ora_tensor *v, const ora_tensor *mask,
                float scale, float max_bias, float softcap, float *dst, int n_threads) {
    return ora_fa_ggml_ex(q, k, v, mask, scale, max_bias, softcap, 0, dst, n_threads);
}

/* ------------------------------------------------------------------------ */
/* fp64 exact reference (two-pass softmax).  q_round = 1 first rounds Q to  */
/* K's vec-dot type exactly like ggml (isolates the kernel's own error).    */
/* Keys with mask == -inf are excluded; a row with no key gives 0.          */
/* ------------------------------------------------------------------------ */
typedef struct {
    const ora_tensor *q, *k, *v, *mask;
    double scale, max_bias, softcap;
    int q_round;
    double *dst;
    int64_t nrows;
    int nth, ith;
} exact_job;

static void load_row_f64(const ora_tensor *t, const char *p, int64_t n, double *out, float *tmp) {
    if (t->type == ORA_F32) { for (int64_t i = 0; i < n; i++) out[i] = ((const float *)p)[i]; return; }
    if (t->type == ORA_F16) ora_f16_to_f32((const uint16_t *)p, tmp, n);
    else if (t->type == ORA_BF16) ora_bf16_to_f32((const uint16_t *)p, tmp, n);
    else ora_dequantize_q8_0((const uint8_t *)p, tmp, n);
    for (int64_t i = 0; i < n; i++) out[i] = tmp[i];
}

static void *exact_rows(void *arg) {
    exact_job *J = (exact_job *)arg;
    const ora_tensor *q = J->q, *k = J->k, *v = J->v, *mask = J->mask;
    const int64_t DK = k->ne[0], DV = v->ne[0];
    const int64_t neq1 = q->ne[1], neq2 = q->ne[2], neq3 = q->ne[3];
    const int64_t nek1 = k->ne[1];
    const int64_t rk2 = neq2 / k->ne[2], rk3 = neq3 / k->ne[3];
    const int64_t rv2 = neq2 / v->ne[2], rv3 = neq3 / v->ne[3];
    const uint32_t n_head = (uint32_t)neq2;
    const uint32_t n_head_log2 = 1u << (uint32_t)floor(log2((double)n_head));
    const double m0 = pow(2.0, -(J->max_bias) / n_head_log2);
    const double m1 = pow(2.0, -(J->max_bias / 2.0) / n_head_log2);
    double scale = J->scale;
    if (J->softcap != 0.0) scale /= J->softcap;

    double *qd = (double *)malloc(sizeof(double) * (size_t)DK);
    double *kd = (double *)malloc(sizeof(double) * (size_t)DK);
    double *vd = (double *)malloc(sizeof(double) * (size_t)DV);
    double *acc = (double *)malloc(sizeof(double) * (size_t)DV);
    double *sc = (double *)malloc(sizeof(double) * (size_t)nek1);
    float *tmp = (float *)malloc(sizeof(float) * (size_t)(DK > DV ? DK : DV));
    uint8_t *qq = (uint8_t *)malloc((size_t)DK * 4 + 64);
    /* fp64 copies of the K and V rows of the (kv head, kv batch) plane the
     * current row reads; rows go to threads in contiguous runs, so a plane
     * is converted once per run instead of once per query row */
    double *kpl = (double *)malloc(sizeof(double) * (size_t)(nek1 * DK));
    double *vpl = (double *)malloc(sizeof(double) * (size_t)(nek1 * DV));
    int64_t k_plane = -1, v_plane = -1;
    const int64_t dr = (J->nrows + J->nth - 1) / J->nth;
    const int64_t ir0 = dr * J->ith;
    const int64_t ir1 = ir0 + dr < J->nrows ? ir0 + dr : J->nrows;

    for (int64_t ir = ir0; ir < ir1; ir++) {
        const int64_t iq3 = ir / (neq2 * neq1);
        const int64_t iq2 = (ir - iq3 * neq2 * neq1) / neq1;
        const int64_t iq1 = ir - iq3 * neq2 * neq1 - iq2 * neq1;
        const uint32_t h = (uint32_t)iq2;
        {
            const int64_t kp = (iq3 / rk3) * k->ne[2] + iq2 / rk2, vp = (iq3 / rv3) * v->ne[2] + iq2 / rv2;
            if (kp != k_plane) {
                for (int64_t ic = 0; ic < nek1; ic++)
                    load_row_f64(k, (const char *)k->data + ic * k->nb[1] + (iq2 / rk2) * k->nb[2] +
                                        (iq3 / rk3) * k->nb[3], DK, kpl + ic * DK, tmp);
                k_plane = kp;
            }
            if (vp != v_plane) {
                for (int64_t ic = 0; ic < nek1; ic++)
                    load_row_f64(v, (const char *)v->data + ic * v->nb[1] + (iq2 / rv2) * v->nb[2] +
                                        (iq3 / rv3) * v->nb[3], DV, vpl + ic * DV, tmp);
                v_plane = vp;
            }
        }
        const double slope = (J->max_bias > 0.0)
            ? (h < n_head_log2 ? pow(m0, h + 1) : pow(m1, 2 * (h - n_head_log2) + 1)) : 1.0;
        const float *pq = (const float *)((const char *)q->data + iq1 * q->nb[1] + iq2 * q->nb[2] + iq3 * q->nb[3]);
        if (!J->q_round) {
            for (int64_t i = 0; i < DK; i++) qd[i] = pq[i];
        } else if (k->type == ORA_F16) {
            for (int64_t i = 0; i < DK; i++) qd[i] = ora_h2f(ora_f2h(pq[i]));
        } else if (k->type == ORA_BF16) {
            for (int64_t i = 0; i < DK; i++) qd[i] = ora_bf2f(ora_f2bf(pq[i]));
        } else {
            ora_quantize_q8_0(pq, qq, DK);
            ora_dequantize_q8_0(qq, tmp, DK);
            for (int64_t i = 0; i < DK; i++) qd[i] = tmp[i];
        }
        const uint16_t *mp = mask
            ? (const uint16_t *)((const char *)mask->data + iq1 * mask->nb[1] +
                                 (iq2 % mask->ne[2]) * mask->nb[2] + (iq3 % mask->ne[3]) * mask->nb[3])
            : NULL;
        double M = -INFINITY;
        for (int64_t ic = 0; ic < nek1; ic++) {
            double mv = mp ? slope * (double)ora_h2f(mp[ic]) : 0.0;
            if (mv == -INFINITY) { sc[ic] = -INFINITY; continue; }
            const double *kr = kpl + ic * DK;
            double s = 0.0;
            for (int64_t i = 0; i < DK; i++) s += kr[i] * qd[i];
            s *= scale;
            if (J->softcap != 0.0) s = J->softcap * tanh(s);
            s += mv;
            sc[ic] = s;
            if (s > M) M = s;
        }
        for (int64_t d = 0; d < DV; d++) acc[d] = 0.0;
        double S = 0.0;
        if (M != -INFINITY) {
            for (int64_t ic = 0; ic < nek1; ic++) {
                if (sc[ic] == -INFINITY) continue;
                const double p = exp(sc[ic] - M);
                const double *vr = vpl + ic * DV;
                for (int64_t d = 0; d < DV; d++) acc[d] += p * vr[d];
                S += p;
            }
        }
        double *out = J->dst + ((iq3 * neq1 + iq1) * neq2 + iq2) * DV;
        for (int64_t d = 0; d < DV; d++) out[d] = S == 0.0 ? 0.0 : acc[d] / S;
    }
    free(qd); free(kd); free(vd); free(acc); free(sc); free(tmp); free(qq); free(kpl); free(vpl);
    return NULL;
}

int ora_fa_exact(const ora_tensor *q, const ora_tensor *k, const ora_tensor *v, const ora_tensor *mask,
                 double scale, double max_bias, double softcap, int q_round, double *dst, int n_threads) {
    int rc = check_shapes(q, k, v, mask);
    if (rc) return rc;
    if (n_threads < 1) n_threads = 1;
    const int64_t nrows = q->ne[1] * q->ne[2] * q->ne[3];
    exact_job *jobs = (exact_job *)calloc((size_t)n_threads, sizeof(exact_job));
    pthread_t *th = (pthread_t *)calloc((size_t)n_threads, sizeof(pthread_t));
    for (int t = 0; t < n_threads; t++) {
        jobs[t] = (exact_job){q, k, v, mask, scale, max_bias, softcap, q_round, dst, nrows, n_threads, t};
        if (t > 0) pthread_create(&th[t], NULL, exact_rows, &jobs[t]);
    }
    exact_rows(&jobs[0]);
    for (int t = 1; t < n_threads; t++) pthread_join(th[t], NULL);
    free(jobs); free(th);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* GGML_OP_SET_ROWS (the KV-cache write), restated from ggml's published CPU  */
/* kernel (ggml-cpu ops.cpp, ggml_compute_forward_set_rows_f32, upstream      */
/* ggml late 2025; the ggml submodule is empty in the reference checkout).   */
/* The reference calls it at src/qwen3-lm.h:453-454 (F32 [D, S, Nkv] rows    */
/* into the F16 [D, max_seq, Nkv] cache, row ids [S] broadcast over Nkv) and  */
/* :776-777 ([D, 1, Nkv, N] rows into N cache sets, row ids [1, 1, N]).       */
/*                                                                            */
/*   for i03 < ne03, i02 < ne02, i < ne01:                                    */
/*     i1 = rows[i, i02 % rows.ne1, i03 % rows.ne2]   (I64 or I32)            */
/*     dst[:, i1, i02, i03] = from_float(src[:, i, i02, i03])                 */
/*                                                                            */
/* from_float: F32 copy, F16 / BF16 with the codecs above, Q8_0 with          */
/* ora_quantize_q8_0.  ggml asserts 0 <= i1 < dst.ne1; here such a row is     */
/* skipped and counted (the GPU kernel skips it too).                         */
/* Returns the number of skipped rows, or -1 when the shapes do not form a    */
/* set_rows node.                                                             */
/* ------------------------------------------------------------------------ */
int64_t ora_set_rows(const ora_tensor *dst, const ora_tensor *src, const ora_tensor *rows) {
    const int64_t D = src->ne[0];
    if (src->type != ORA_F32 || (rows->type != 26 && rows->type != 27)) return -1;
    if (dst->ne[0] != D || dst->ne[2] != src->ne[2] || dst->ne[3] != src->ne[3]) return -1;
    if (src->ne[1] != rows->ne[0] || rows->ne[1] < 1 || rows->ne[2] < 1 || rows->ne[3] != 1) return -1;
    if (src->ne[2] % rows->ne[1] || src->ne[3] % rows->ne[2]) return -1;
    if (dst->type == ORA_Q8_0 && D % QK8_0) return -1;
    if (dst->type != ORA_F32 && dst->type != ORA_F16 && dst->type != ORA_BF16 && dst->type != ORA_Q8_0)
        return -1;
    int64_t skipped = 0;
    for (int64_t i03 = 0; i03 < src->ne[3]; i03++)
        for (int64_t i02 = 0; i02 < src->ne[2]; i02++)
            for (int64_t i = 0; i < src->ne[1]; i++) {
                const char *ip = (const char *)rows->data + i * rows->nb[0] +
                                 (i02 % rows->ne[1]) * rows->nb[1] + (i03 % rows->ne[2]) * rows->nb[2];
                int64_t i1;
                if (rows->type == 27) memcpy(&i1, ip, 8);
                else { int32_t t; memcpy(&t, ip, 4); i1 = t; }
                if (i1 < 0 || i1 >= dst->ne[1]) { skipped++; continue; }
                const float *x = (const float *)((const char *)src->data + i * src->nb[1] +
                                                 i02 * src->nb[2] + i03 * src->nb[3]);
                char *y = (char *)dst->data + i1 * dst->nb[1] + i02 * dst->nb[2] + i03 * dst->nb[3];
                switch (dst->type) {
                    case ORA_F32: memcpy(y, x, (size_t)D * 4); break;
                    case ORA_F16:
                        for (int64_t j = 0; j < D; j++) { uint16_t h = ora_f2h(x[j]); memcpy(y + 2 * j, &h, 2); }
                        break;
                    case ORA_BF16:
                        for (int64_t j = 0; j < D; j++) { uint16_t h = ora_f2bf(x[j]); memcpy(y + 2 * j, &h, 2); }
                        break;
                    default: ora_quantize_q8_0(x, (uint8_t *)y, D); break;
                }
            }
    return skipped;
}

/* ------------------------------------------------------------------------ */
/* Pre-attention work of a layer (reference src/qwen3-lm.h:418-441,           */
/* src/dit-graph.h:177-225): rms_norm * weight, NEOX rope, V clamp -- the     */
/* restatement of ggml's published CPU ops (ggml-cpu ops.cpp,                 */
/* ggml_compute_forward_rms_norm_f32, ggml_compute_forward_rope_f32 with      */
/* ggml_rope_cache_init / rope_yarn at ext_factor 0, freq_scale 1,            */
/* attn_factor 1, NEOX pairs (i, i + n_dims/2)); upstream ggml late 2025.    */
/*   rms_norm: sum (double) of x*x (float), mean = sum/n, scale =             */
/*     1/sqrtf(mean + eps), y = x*scale, then y*w (ggml_mul);                 */
/*   rope: theta_scale = powf(base, -2/n_dims); theta_0 = p; theta_{i+1} =    */
/*     theta_i * theta_scale (float); c = cosf(theta_i), s = sinf(theta_i);  */
/*     y_i = x_i c - x_{i+n/2} s, y_{i+n/2} = x_i s + x_{i+n/2} c.            */
/* Inputs: rows of 128 floats; q [B][S][Nh][128] (row (b, s, h) at             */
/* q + ((b*S + s)*Nh + h)*128), k/v likewise with Nkv; pos [S] or [B][S].     */
/* Outputs (F32, before the 16-bit cast) in the same layouts.                 */
/* ------------------------------------------------------------------------ */
static void norm_rope_row(const float *x, const float *w, int pos, float eps, float theta_scale, float *y) {
    double sum = 0.0;
    for (int i = 0; i < 128; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / 128);
    const float scale = 1.0f / sqrtf(mean + eps);
    float t[128];
    for (int i = 0; i < 128; i++) t[i] = x[i] * scale;
    for (int i = 0; i < 128; i++) t[i] = t[i] * w[i];
    float theta = (float)pos;
    for (int i = 0; i < 64; i++) {
        const float c = cosf(theta), s = sinf(theta);
        const float x0 = t[i], x1 = t[i + 64];
        y[i] = x0 * c - x1 * s;
        y[i + 64] = x0 * s + x1 * c;
        theta *= theta_scale;
    }
}

/* The same QK-RMSNorm without the rotation (DiT cross-attention,
 * dit-graph.h:326-333): rms_norm(x, eps) * w for n rows of 128. */
static void norm_row(const float *x, const float *w, float eps, float *y) {
    double sum = 0.0;
    for (int i = 0; i < 128; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / 128);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < 128; i++) {
        const float t = x[i] * scale;
        y[i] = t * w[i];
    }
}

void ora_qk_norm(const float *x, const float *w, int64_t n_rows, float eps, float *y) {
    for (int64_t r = 0; r < n_rows; r++) norm_row(x + r * 128, w, eps, y + r * 128);
}

void ora_qk_norm_rope(const float *q, const float *k, const float *v, const float *qw, const float *kw,
                      const int32_t *pos, int pos_per_batch, int Nh, int Nkv, int S, int B, float eps,
                      float freq_base, int clamp_v, float *q_o, float *k_o, float *v_o) {
    const float theta_scale = powf(freq_base, -2.0f / 128.0f);
    for (int b = 0; b < B; b++)
        for (int s = 0; s < S; s++) {
            const int p = pos[(pos_per_batch ? b * S : 0) + s];
            for (int h = 0; h < Nh; h++) {
                const size_t o = (((size_t)b * S + s) * Nh + h) * 128;
                norm_rope_row(q + o, qw, p, eps, theta_scale, q_o + o);
            }
            for (int h = 0; h < Nkv; h++) {
                const size_t o = (((size_t)b * S + s) * Nkv + h) * 128;
                norm_rope_row(k + o, kw, p, eps, theta_scale, k_o + o);
                for (int i = 0; i < 128; i++) {
                    float x = v[o + i];
                    if (clamp_v) x = fminf(fmaxf(x, -65504.0f), 65504.0f);
                    v_o[o + i] = x;
                }
            }
        }
}
