/*
 * adam8_oracle.c -- CPU restatement of rollfast's 8-bit AdamW step.
 *
 * TEST INFRASTRUCTURE ONLY.  The HIP library's results are compared against
 * this restatement.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product (rollfast_amd/)
 * never links, imports or calls it.
 *
 * Every function follows the reference algorithm literally (searchsorted +
 * nearest-with-ties-to-lower, literal f32 operation order, no FMA
 * contraction: build with -ffp-contract=off) and cites the reference file
 * and line it restates.  Paths are relative to the rollfast source tree.
 *
 * Pinning (what fixes each function independently of this file):
 *   orc_codebook            closed form, checked in tests against an
 *                           independent float64 linspace build + reference
 *                           test facts (zero point 127/0, endpoints).
 *   orc_quantize_*          brute-force argmin over all 256 entries with
 *                           ties to the lower index; reference error bounds
 *                           (tests/test_adam8.py:42,65,84).
 *   orc_dequantize          closed form cb[code] * scale.
 *   orc_adam8_leaf          float64 textbook AdamW (fallback leaves, tight
 *                           tolerance) and the reference's adamw8-vs-adamw
 *                           tolerance test (tests/test_adam8.py:121-149).
 *   orc_sr_bf16             exhaustive over all 2^16 noise values (exact
 *                           expectation), sub-ulp KAT (tests/test_utils.py:89).
 *   orc_threefry2x32        Random123 known-answer vectors.
 *   bit layout of jax.random.bits / split (threefry_partitionable) and
 *   the f32 pow inside the bias correction: parity unpinned (JAX absent).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------- bits -- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* f32 -> bf16, round to nearest even; NaN keeps its sign and becomes the
 * canonical quiet NaN (the convention of XLA's CPU bf16 conversion). */
static inline uint16_t f32_to_bf16_rne(float x)
{
    uint32_t u = f2u(x);
    if (isnan(x)) return (uint16_t)((u >> 16) & 0x8000u) | 0x7FC0u;
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7FFFu + lsb;
    return (uint16_t)(u >> 16);
}
static inline float bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

/* f32 -> IEEE binary16 (astype(float16)), round to nearest even: overflow
 * from 65520 up goes to Inf, magnitudes below 2^-14 become subnormal
 * multiples of 2^-24 (or zero), NaN stays NaN with its sign and the top
 * payload bits, quiet. */
static inline uint16_t f32_to_f16_rne(float x)
{
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);       /* |x| >= 65520 (or Inf) */
    if (a < 0x38800000u) {                                          /* |x| < 2^-14 */
        float k = rintf(u2f(a) * 16777216.0f);                      /* |x| / 2^-24, exact scale */
        return (uint16_t)(sign | (uint32_t)k);                      /* k = 1024 is 2^-14 itself */
    }
    a += 0x0FFFu + ((a >> 13) & 1u);                                /* 23 -> 10 mantissa bits */
    return (uint16_t)(sign | ((a - 0x38000000u) >> 13));            /* exponent bias 127 -> 15 */
}

static inline float f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f;                /* m * 2^-24, exact */
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* utils.py:342-371 _stochastic_round_bf16: noise = bits & 0xFFFF, zero noise
 * for |x| >= Inf bit pattern, (x + noise) & 0xFFFF0000. */
static inline uint16_t sr_bf16_from_bits(float x, uint32_t bits)
{
    uint32_t u = f2u(x);
    uint32_t noise = bits & 0xFFFFu;
    if ((u & 0x7FFFFFFFu) >= 0x7F800000u) noise = 0;
    return (uint16_t)(((u + noise) & 0xFFFF0000u) >> 16);
}

/* ------------------------------------------------------------ threefry -- */
/* Threefry-2x32 with 20 rounds (Salmon et al., SC'11, Random123).  This is
 * the block cipher under jax.random's default PRNG; its output is pinned
 * by the Random123 known-answer vectors in tests. */
static inline uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

ORC_API void orc_threefry2x32(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1,
                              uint32_t* y0, uint32_t* y1)
{
    static const int R[8] = {13, 15, 26, 6, 17, 29, 16, 24};
    uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
    uint32_t x0 = c0 + ks[0], x1 = c1 + ks[1];
    for (int blk = 0; blk < 5; ++blk) {
        for (int r = 0; r < 4; ++r) {
            x0 += x1;
            x1 = rotl32(x1, R[(blk & 1) * 4 + r]);
            x1 ^= x0;
        }
        x0 += ks[(blk + 1) % 3];
        x1 += ks[(blk + 2) % 3] + (uint32_t)(blk + 1);
    }
    *y0 = x0;
    *y1 = x1;
}

/* jax.random.bits(key, shape, uint32) under jax_threefry_partitionable
 * (default since JAX 0.5): element i (row-major flat index) uses the
 * counter (hi32(i), lo32(i)) and returns y0 ^ y1.  Layout parity unpinned. */
ORC_API void orc_random_bits(uint32_t k0, uint32_t k1, uint64_t offset, int64_t n, uint32_t* out)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t idx = offset + (uint64_t)i;
        uint32_t y0, y1;
        orc_threefry2x32(k0, k1, (uint32_t)(idx >> 32), (uint32_t)idx, &y0, &y1);
        out[i] = y0 ^ y1;
    }
}

/* Both words of threefry2x32(key, (hi32(c), lo32(c))) for the counters
 * c = offset .. offset+n-1.  The block stream of the library's packed bit
 * source (its opt-in RF_PACKED_BITS, which has no reference counterpart):
 * the Python wrapper picks the words and halves each element takes. */
ORC_API void orc_threefry_blocks(uint32_t k0, uint32_t k1, uint64_t offset, int64_t n, uint32_t* y0, uint32_t* y1)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t c = offset + (uint64_t)i;
        orc_threefry2x32(k0, k1, (uint32_t)(c >> 32), (uint32_t)c, &y0[i], &y1[i]);
    }
}

/* jax.random.split(key, num) under jax_threefry_partitionable: subkey i is
 * threefry2x32(key, (0, i)) as the pair (y0, y1). */
ORC_API void orc_split(uint32_t k0, uint32_t k1, int32_t num, uint32_t* out /* [num][2] */)
{
    for (int32_t i = 0; i < num; ++i)
        orc_threefry2x32(k0, k1, 0u, (uint32_t)i, &out[2 * i], &out[2 * i + 1]);
}

/* jax.random.uniform(key, shape, float32) mantissa mapping applied to raw
 * bits: (bits >> 9) | 0x3F800000 reinterpreted, minus 1.0. */
static inline float uniform_from_bits(uint32_t bits)
{
    float f = u2f((bits >> 9) | 0x3F800000u) - 1.0f;
    return f > 0.0f ? f : 0.0f;
}

/* ------------------------------------------------------------ codebook -- */
/* adam8.py:495-503 _linspace_bin_means (double arithmetic). */
static int linspace_bin_means(double start, double stop, int points, double* out)
{
    if (points <= 1) return 0;
    double step = (stop - start) / (double)(points - 1);
    for (int i = 0; i + 1 < points; ++i) {
        volatile double left = start + step * (double)i;
        volatile double right = start + step * (double)(i + 1);
        out[i] = (left + right) / 2.0;
    }
    return points - 1;
}

static int cmp_double(const void* a, const void* b)
{
    double x = *(const double*)a, y = *(const double*)b;
    return (x > y) - (x < y);
}

/* adam8.py:465-492 _dynamic_codebook_values, then jnp.asarray(float32)
 * (adam8.py:461-462): 256 sorted doubles rounded to f32. */
ORC_API void orc_codebook(int is_signed, float* out /* [256] */)
{
    double data[300];
    int nd = 0;
    const int total_bits = 8, max_exponent_bits = 7;
    const int non_sign_bits = total_bits - 1;
    for (int index = 0; index < max_exponent_bits; ++index) {
        int e = -(max_exponent_bits - 1) + index;
        double exponent_scale = (e == 0) ? 1.0 : pow(10.0, (double)e);
        int fraction_items = is_signed ? (1 << (index + non_sign_bits - max_exponent_bits)) + 1
                                       : (1 << (index + non_sign_bits - max_exponent_bits + 1)) + 1;
        double means[200];
        int nm = linspace_bin_means(0.1, 1.0, fraction_items, means);
        for (int j = 0; j < nm; ++j) data[nd++] = exponent_scale * means[j];
        if (is_signed)
            for (int j = 0; j < nm; ++j) data[nd++] = -exponent_scale * means[j];
    }
    /* additional_items = 2**(7-7) - 1 = 0: no extra entries (adam8.py:482). */
    data[nd++] = 0.0;
    data[nd++] = 1.0;
    qsort(data, (size_t)nd, sizeof(double), cmp_double);
    for (int i = 0; i < 256 && i < nd; ++i) out[i] = (float)data[i];
}

/* ------------------------------------------------- dtypes and flags -- */
enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_F16 = 2 };
enum { ORC_MOM_QUANT = 0, ORC_MOM_F32 = 1, ORC_MOM_BF16 = 2, ORC_MOM_F16 = 3 };
enum {
    ORC_NESTEROV = 1,       /* adam8.py:341-350 */
    ORC_DECAY = 2,          /* add_decayed_weights applies to this leaf */
    ORC_DECAY_WEAK = 4,     /* wd is a Python scalar: wd*p in the param dtype */
    ORC_LR = 8,             /* scale_by_learning_rate in the chain */
    ORC_MOMENT_SR = 16,     /* adamw8(stochastic_rounding=True) */
    ORC_PARAM_SR = 32,      /* apply_updates(stochastic=True) for bf16 params */
    ORC_APPLY = 64,         /* write params (fused step) instead of updates */
    ORC_STORE_SR = 512,     /* bf16 fallback moments stored with SR from mu_bits / nu_bits
                               (optim/adam.py:219-222, utils.py:374-409) */
    ORC_ZERO_DECAY = 1024,  /* optim/adam.py's own decay term with weight 0 before the
                               optax decay (adam.py:185-201 inside adamw, :380-404) */
    ORC_SCALE_BF16 = 2048,  /* quantized moments store scales.astype(bfloat16) (adam8.py:186) */
    ORC_SCALE_F16 = 4096,   /* ... astype(float16) */
};

static inline float load_val(int dtype, const void* p, int64_t e)
{
    if (dtype == ORC_BF16) return bf16_to_f32(((const uint16_t*)p)[e]);
    if (dtype == ORC_F16) return f16_to_f32(((const uint16_t*)p)[e]);
    return ((const float*)p)[e];
}

/* x rounded to a 16-bit dtype (nearest even) as its bit pattern. */
static inline uint16_t to_h16(int dtype, float x)
{
    return dtype == ORC_F16 ? f32_to_f16_rne(x) : f32_to_bf16_rne(x);
}

static inline float round_to(int dtype, float x)
{
    if (dtype == ORC_BF16) return bf16_to_f32(f32_to_bf16_rne(x));
    if (dtype == ORC_F16) return f16_to_f32(f32_to_f16_rne(x));
    return x;
}

/* A block scale as stored: scales.astype(scale_dtype) read back as f32
 * (adam8.py:186, :202); the codes use the f32 scale before this. */
static inline float stored_scale(int32_t flags, float s)
{
    if (flags & ORC_SCALE_BF16) return round_to(ORC_BF16, s);
    if (flags & ORC_SCALE_F16) return round_to(ORC_F16, s);
    return s;
}

/* ---------------------------------------------------------- quantizers -- */
enum { ORC_Q_SIGNED = 0, ORC_Q_UNSIGNED = 1, ORC_Q_SYMMETRIC = 2 };

/* jnp.searchsorted(codebook, q, side="left") (adam8.py:549): JAX sorts in a
 * total order with every NaN largest and -0 == +0. */
static inline int searchsorted_left(const float* cb, float q)
{
    if (isnan(q)) return 256;
    int lo = 0, hi = 256;
    while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (cb[mid] >= q) hi = mid; else lo = mid + 1;
    }
    return lo;
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* jnp.clip(x, lo, hi) = minimum(maximum(x, lo), hi) with NaN propagating. */
static inline float clipf(float x, float lo, float hi)
{
    if (isnan(x)) return x;
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* adam8.py:542-569 _quantize_to_codebook for one normalised element. */
static inline uint8_t quantize_to_codebook(const float* cb, float n, int sr, uint32_t bits)
{
    int ui = clampi(searchsorted_left(cb, n), 0, 255);
    int li = clampi(ui - 1, 0, 255);
    float lv = cb[li], uv = cb[ui];
    int upper;
    if (sr) {
        float den = uv - lv;
        float p = (den > 0.0f) ? (n - lv) / den : 0.0f;
        p = clipf(p, 0.0f, 1.0f);
        upper = uniform_from_bits(bits) < p;   /* jax.random.bernoulli: u < p */
    } else {
        upper = fabsf(uv - n) < fabsf(n - lv);  /* ties go to the lower index */
    }
    return (uint8_t)(upper ? ui : li);
}

/* jnp.max(jnp.abs(block)) with NaN propagation (adam8.py:142). */
static inline float block_absmax(const float* x, int64_t len)
{
    float m = 0.0f;
    for (int64_t j = 0; j < len; ++j) {
        float a = fabsf(x[j]);
        if (isnan(a)) return a;
        if (a > m) m = a;
    }
    return m;
}

/* adam8.py:113-187 quantize_blocks.  x has `size` elements; codes has
 * nblocks*block_size entries (padding included), scales nblocks.  For the
 * dynamic quantizers codes are uint8 codebook indices; for the symmetric
 * quantizer they are int8 values stored in the same byte buffer.  bits
 * (nblocks*block_size words, may be NULL when sr == 0) are the raw
 * jax.random.bits that bernoulli consumes, over the padded block array. */
ORC_API void orc_quantize(int quantizer, const float* x, int64_t size, int64_t block_size,
                          int sr, const uint32_t* bits, uint8_t* codes, float* scales, int scale_flags)
{
    int64_t nblocks = size > 0 ? (size + block_size - 1) / block_size : 1;
    float cb[256];
    if (quantizer != ORC_Q_SYMMETRIC) orc_codebook(quantizer == ORC_Q_SIGNED, cb);
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nblocks; ++b) {
        float* blk = (float*)malloc(sizeof(float) * (size_t)block_size);
        for (int64_t j = 0; j < block_size; ++j) {
            int64_t e = b * block_size + j;
            blk[j] = e < size ? x[e] : 0.0f;          /* jnp.pad with zeros */
        }
        float amax = block_absmax(blk, block_size);
        if (quantizer == ORC_Q_SYMMETRIC) {
            /* adam8.py:143-164 */
            float scale = (amax > 0.0f) ? amax / 127.0f : 1.0f;
            scales[b] = stored_scale(scale_flags, scale);
            for (int64_t j = 0; j < block_size; ++j) {
                float s = clipf(blk[j] / scale, -127.0f, 127.0f);
                float r;
                if (sr) {
                    /* adam8.py:456-458: floor + bernoulli(frac) */
                    float lo = floorf(s);
                    float p = s - lo;
                    r = lo + ((uniform_from_bits(bits[b * block_size + j]) < p) ? 1.0f : 0.0f);
                } else {
                    r = rintf(s);                      /* jnp.round: half to even */
                }
                codes[b * block_size + j] = (uint8_t)(int8_t)(isnan(r) ? 0 : (int)r);
            }
        } else {
            float scale = (amax > 0.0f) ? amax : 1.0f;  /* adam8.py:167 */
            scales[b] = stored_scale(scale_flags, scale);
            for (int64_t j = 0; j < block_size; ++j) {
                float n = clipf(blk[j] / scale, cb[0], cb[255]);   /* adam8.py:168 */
                uint32_t w = sr ? bits[b * block_size + j] : 0u;
                codes[b * block_size + j] = quantize_to_codebook(cb, n, sr, w);
            }
        }
        free(blk);
    }
}

/* adam8.py:190-204 dequantize_blocks: values * scales[:, None], unpadded. */
ORC_API void orc_dequantize(int quantizer, const uint8_t* codes, const float* scales,
                            int64_t size, int64_t block_size, float* out)
{
    float cb[256];
    if (quantizer != ORC_Q_SYMMETRIC) orc_codebook(quantizer == ORC_Q_SIGNED, cb);
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < size; ++e) {
        float s = scales[e / block_size];
        float v = quantizer == ORC_Q_SYMMETRIC ? (float)(int8_t)codes[e] : cb[codes[e]];
        out[e] = v * s;
    }
}

/* Nearest code of one normalised value (for exhaustive tests). */
ORC_API int orc_nearest_code(int quantizer, float n)
{
    float cb[256];
    orc_codebook(quantizer == ORC_Q_SIGNED, cb);
    return quantize_to_codebook(cb, clipf(n, cb[0], cb[255]), 0, 0u);
}

/* Nearest codes for an array of normalised values (vectorised, exhaustive
 * sweeps over f32 bit patterns). */
ORC_API void orc_nearest_codes_bits(int quantizer, uint32_t first_bits, int64_t count, uint8_t* out)
{
    float cb[256];
    orc_codebook(quantizer == ORC_Q_SIGNED, cb);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        float n = u2f(first_bits + (uint32_t)i);
        out[i] = quantize_to_codebook(cb, clipf(n, cb[0], cb[255]), 0, 0u);
    }
}

/* ui = clip(searchsorted_left(cb, clip(n, cb[0], cb[255])), 0, 255)
 * (adam8.py:549-550), the upper candidate of moment SR, for the normalised
 * values n given as the consecutive f32 bit patterns first_bits .. +count-1. */
ORC_API void orc_search_index_bits(int quantizer, uint32_t first_bits, int64_t count, uint16_t* out)
{
    float cb[256];
    orc_codebook(quantizer == ORC_Q_SIGNED, cb);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        float n = u2f(first_bits + (uint32_t)i);
        out[i] = (uint16_t)clampi(searchsorted_left(cb, clipf(n, cb[0], cb[255])), 0, 255);
    }
}

/* Nearest codes for an arbitrary list of normalised values given as f32
 * bit patterns. */
ORC_API void orc_nearest_codes_list(int quantizer, const uint32_t* bits, int64_t count, uint8_t* out)
{
    float cb[256];
    orc_codebook(quantizer == ORC_Q_SIGNED, cb);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        float n = u2f(bits[i]);
        out[i] = quantize_to_codebook(cb, clipf(n, cb[0], cb[255]), 0, 0u);
    }
}

/* ------------------------------------------------------------ the step -- */

/* one_minus_b1 weights the gradient in the first-moment EMA; the Nesterov
 * combination uses nest_one_minus_b1 (adam8.py:322-327 and :341-350 both use
 * the Python double 1.0 - b1; optim/adam.py computes the EMA weight in f32,
 * utils.py:327-335 _momentum_grad_scale, and the Nesterov weight in double,
 * adam.py:146-160). */
typedef struct {
    float b1, one_minus_b1, b2, one_minus_b2;
    float bc1, bc2, bc1_next;
    float eps, eps_root;
    float weight_decay, neg_lr;
    int32_t flags;
    float nest_one_minus_b1;
} orc_hparams;


/* Direction, decay, lr and apply for one element.  Follows adam8.py:352-362
 * (bias correction utils.py:318-324), optax add_decayed_weights (u + wd*p),
 * optax scale_by_learning_rate ((-lr) * u) and utils.py:648-708
 * apply_updates.  Returns the f32 update; writes the param when applying. */
static inline float direction_and_apply(const orc_hparams* hp, int pdtype, void* param, int64_t e,
                                        float m, float v, float g, uint32_t pbits, int* wrote,
                                        float* pnew_f32, uint16_t* pnew_bf16)
{
    float mhat;
    if (hp->flags & ORC_NESTEROV) {
        float mu_bc = m / hp->bc1_next;
        float g_bc = g / hp->bc1;
        float t1 = hp->b1 * mu_bc;
        float t2 = hp->nest_one_minus_b1 * g_bc;
        mhat = t1 + t2;
    } else {
        mhat = m / hp->bc1;
    }
    float vhat = v / hp->bc2;
    float den = sqrtf(vhat + hp->eps_root) + hp->eps;
    float u = mhat / den;
    float p = load_val(pdtype, param, e);
    if (hp->flags & ORC_ZERO_DECAY) {
        /* utils.py:79-90 with weight_decay_step = 0.0: update + 0.0 * f32(param) */
        float zp = 0.0f * p;
        u = u + zp;
    }
    if (hp->flags & ORC_DECAY) {
        float wdp;
        if ((pdtype == ORC_BF16 || pdtype == ORC_F16) && (hp->flags & ORC_DECAY_WEAK)) {
            /* Python-scalar wd times a bf16 (f16) array stays bf16 (f16),
             * JAX weak typing: the wd and the product each rounded once to
             * the param dtype (the product of two 16-bit values is exact in
             * f32). */
            float wd16 = round_to(pdtype, hp->weight_decay);
            wdp = round_to(pdtype, wd16 * p);
        } else {
            wdp = hp->weight_decay * p;
        }
        u = u + wdp;
    }
    if (hp->flags & ORC_LR) u = hp->neg_lr * u;
    *wrote = 0;
    if (hp->flags & ORC_APPLY) {
        *wrote = 1;
        if (pdtype == ORC_BF16) {
            float s = p + u;
            *pnew_bf16 = (hp->flags & ORC_PARAM_SR) ? sr_bf16_from_bits(s, pbits) : f32_to_bf16_rne(s);
        } else if (pdtype == ORC_F16) {
            *pnew_bf16 = f32_to_f16_rne(p + u);   /* (p + u).astype(float16), utils.py:700 */
        } else {
            *pnew_f32 = p + u;
        }
    }
    return u;
}

/*
 * One leaf of one step: scale_by_adam8.update_fn (adam8.py:304-389) followed
 * by the rest of the adamw8 chain (adam8.py:418-443) and, when ORC_APPLY is
 * set, rollfast.apply_updates (utils.py:648-708).
 *
 * Quantized moments: mu/nu are uint8 codes [nblocks*block_size] with f32
 * scales [nblocks]; fallback moments are f32 or bf16 arrays of n elements.
 * The bits arrays are raw jax.random.bits words: mu_bits/nu_bits over the
 * padded block array (moment SR), p_bits over the param (param SR).
 */
ORC_API void orc_adam8_leaf(const orc_hparams* hp,
                            int pdtype, void* param, int gdtype, const void* grad, int64_t n,
                            int mkind, void* mu, float* mu_scales, void* nu, float* nu_scales,
                            int64_t block_size,
                            const uint32_t* mu_bits, const uint32_t* nu_bits, const uint32_t* p_bits,
                            float* updates_out)
{
    if (mkind == ORC_MOM_QUANT) {
        float cbs[256], cbu[256];
        orc_codebook(1, cbs);
        orc_codebook(0, cbu);
        int64_t nblocks = n > 0 ? (n + block_size - 1) / block_size : 1;
        int msr = (hp->flags & ORC_MOMENT_SR) != 0;
#pragma omp parallel for schedule(static)
        for (int64_t b = 0; b < nblocks; ++b) {
            float* mb = (float*)malloc(sizeof(float) * (size_t)block_size);
            float* vb = (float*)malloc(sizeof(float) * (size_t)block_size);
            uint8_t* mc = (uint8_t*)mu + b * block_size;
            uint8_t* vc = (uint8_t*)nu + b * block_size;
            float ms = mu_scales[b], vs = nu_scales[b];
            for (int64_t j = 0; j < block_size; ++j) {
                int64_t e = b * block_size + j;
                if (e >= n) { mb[j] = 0.0f; vb[j] = 0.0f; continue; }
                float g = load_val(gdtype, grad, e);
                float mp = cbs[mc[j]] * ms;                  /* adam8.py:200-203 */
                float vp = cbu[vc[j]] * vs;
                float t1 = hp->b1 * mp, t2 = hp->one_minus_b1 * g;
                float m = t1 + t2;                           /* adam8.py:322-327 */
                float gg = g * g;
                float t3 = hp->b2 * vp, t4 = hp->one_minus_b2 * gg;
                float v = t3 + t4;                           /* adam8.py:328-335 */
                mb[j] = m;
                vb[j] = v;
                int wrote;
                float pf = 0.0f; uint16_t ph = 0;
                uint32_t pbits = (p_bits && (hp->flags & ORC_PARAM_SR)) ? p_bits[e] : 0u;
                float u = direction_and_apply(hp, pdtype, param, e, m, v, g, pbits, &wrote, &pf, &ph);
                if (wrote) {
                    if (pdtype != ORC_F32) ((uint16_t*)param)[e] = ph;
                    else ((float*)param)[e] = pf;
                } else if (updates_out) {
                    updates_out[e] = u;
                }
            }
            /* adam8.py:633-688 -> quantize_blocks on the un-bias-corrected
             * moments, padding zero-filled (adam8.py:137-141). */
            float am = block_absmax(mb, block_size), av = block_absmax(vb, block_size);
            float sm = (am > 0.0f) ? am : 1.0f, sv = (av > 0.0f) ? av : 1.0f;
            mu_scales[b] = stored_scale(hp->flags, sm);
            nu_scales[b] = stored_scale(hp->flags, sv);
            for (int64_t j = 0; j < block_size; ++j) {
                int64_t e = b * block_size + j;
                float nm = clipf(mb[j] / sm, cbs[0], cbs[255]);
                float nv = clipf(vb[j] / sv, cbu[0], cbu[255]);
                mc[j] = quantize_to_codebook(cbs, nm, msr, msr ? mu_bits[e] : 0u);
                vc[j] = quantize_to_codebook(cbu, nv, msr, msr ? nu_bits[e] : 0u);
            }
            free(mb);
            free(vb);
        }
    } else {
#pragma omp parallel for schedule(static)
        for (int64_t e = 0; e < n; ++e) {
            float g = load_val(gdtype, grad, e);
            int mdt = mkind == ORC_MOM_BF16 ? ORC_BF16 : (mkind == ORC_MOM_F16 ? ORC_F16 : ORC_F32);
            float mp = load_val(mdt, mu, e);
            float vp = load_val(mdt, nu, e);
            float t1 = hp->b1 * mp, t2 = hp->one_minus_b1 * g;
            float m = t1 + t2;
            float gg = g * g;
            float t3 = hp->b2 * vp, t4 = hp->one_minus_b2 * gg;
            float v = t3 + t4;
            int wrote;
            float pf = 0.0f; uint16_t ph = 0;
            uint32_t pbits = (p_bits && (hp->flags & ORC_PARAM_SR)) ? p_bits[e] : 0u;
            float u = direction_and_apply(hp, pdtype, param, e, m, v, g, pbits, &wrote, &pf, &ph);
            if (wrote) {
                if (pdtype != ORC_F32) ((uint16_t*)param)[e] = ph;
                else ((float*)param)[e] = pf;
            } else if (updates_out) {
                updates_out[e] = u;
            }
            /* adam8.py:688 moment.astype(fallback_dtype); optim/adam.py:219-222
             * stores bf16 moments with _tree_stochastic_cast instead. */
            if (mkind == ORC_MOM_BF16 && (hp->flags & ORC_STORE_SR)) {
                ((uint16_t*)mu)[e] = sr_bf16_from_bits(m, mu_bits[e]);
                ((uint16_t*)nu)[e] = sr_bf16_from_bits(v, nu_bits[e]);
            } else if (mdt != ORC_F32) {
                ((uint16_t*)mu)[e] = to_h16(mdt, m);
                ((uint16_t*)nu)[e] = to_h16(mdt, v);
            } else {
                ((float*)mu)[e] = m;
                ((float*)nu)[e] = v;
            }
        }
    }
}

/* utils.py:648-708 apply_updates for one leaf: bf16 params take
 * f32(p) + f32(u) then SR (fed bits) or RNE; f32 params take p + u. */
ORC_API void orc_apply_updates(int pdtype, void* param, const float* upd, int64_t n, int sr,
                               const uint32_t* bits)
{
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < n; ++e) {
        if (pdtype == ORC_BF16) {
            float s = bf16_to_f32(((uint16_t*)param)[e]) + upd[e];
            ((uint16_t*)param)[e] = sr ? sr_bf16_from_bits(s, bits[e]) : f32_to_bf16_rne(s);
        } else if (pdtype == ORC_F16) {
            float s = f16_to_f32(((uint16_t*)param)[e]) + upd[e];
            ((uint16_t*)param)[e] = f32_to_f16_rne(s);
        } else {
            ((float*)param)[e] = ((float*)param)[e] + upd[e];
        }
    }
}

/* optax.MultiSteps (optax >=0.2.8,<0.3.0, optax/_src/wrappers.py; the
 * wrapper of finetune/builders.py:1614-1620) for one leaf, in place on acc:
 *   mode 1 (use_grad_mean): acc + (grad - acc) / (n_acc + 1)  (Welford)
 *   mode 0 (sum):           grad + acc
 *   mode 2 (reset after an emitting step): (1 - emit) * acc = 0 * acc
 * JAX computes each in the promoted dtype of grad and acc: f32 unless both
 * are the same 16-bit type, whose every operation then rounds to nearest
 * even; the int32 count n_acc + 1 converts to that dtype.  The result is
 * stored in acc's dtype (the promoted one for the combinations MultiSteps
 * accepts). */
ORC_API void orc_accumulate(int mode, int32_t n_acc, int gdtype, const void* grad, int adtype, void* acc,
                            int64_t n)
{
    const int cdt = gdtype == adtype ? adtype : ORC_F32;
    const float div = round_to(cdt, (float)n_acc + 1.0f);
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < n; ++e) {
        const float a = load_val(adtype, acc, e);
        float r;
        if (mode == 2) {
            r = 0.0f * a;
        } else {
            const float g = load_val(gdtype, grad, e);
            if (mode == 1) {
                const float d = round_to(cdt, g - a);
                const float q = round_to(cdt, d / div);
                r = round_to(cdt, a + q);
            } else {
                r = round_to(cdt, g + a);
            }
        }
        if (adtype == ORC_F32)
            ((float*)acc)[e] = r;
        else
            ((uint16_t*)acc)[e] = to_h16(adtype, r);
    }
}

/* Check helper, not a restatement: the moment-SR kernels' probability
 * quotient from a reciprocal y of the gap d, q0 = a*y, r = fma(-d, q0, a),
 * p = fma(r, y, q0), over an array of a.  The tables test holds it to the
 * IEEE quotient a / d that adam8.py:558-560 computes. */
ORC_API void orc_recip_quotient(const float* a, int64_t n, float d, float y, float* out)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float q0 = a[i] * y;
        const float r = fmaf(-d, q0, a[i]);
        out[i] = fmaf(r, y, q0);
    }
}

/* utils.py:342-371 _stochastic_round_bf16 over an array with fed bits. */
ORC_API void orc_sr_bf16(const float* x, const uint32_t* bits, int64_t n, uint16_t* out)
{
#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < n; ++e) out[e] = sr_bf16_from_bits(x[e], bits[e]);
}

/* f32 -> f16 RNE over an array (astype(float16)) and back. */
ORC_API void orc_f32_to_f16(const float* x, int64_t n, uint16_t* out)
{
    for (int64_t e = 0; e < n; ++e) out[e] = f32_to_f16_rne(x[e]);
}

ORC_API void orc_f16_to_f32(const uint16_t* h, int64_t n, float* out)
{
    for (int64_t e = 0; e < n; ++e) out[e] = f16_to_f32(h[e]);
}

/* f32 -> bf16 RNE over an array (astype(bfloat16)). */
ORC_API void orc_f32_to_bf16(const float* x, int64_t n, uint16_t* out)
{
    for (int64_t e = 0; e < n; ++e) out[e] = f32_to_bf16_rne(x[e]);
}

ORC_API void orc_set_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

ORC_API int orc_get_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
