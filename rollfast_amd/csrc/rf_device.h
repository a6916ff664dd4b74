// rf_device.h -- gfx950 (MI355X, CDNA4) device code of the 8-bit AdamW step.
//
// One HBM pass per step: dequantize the blockwise 8-bit moments, Adam/AdamW
// update, requantize with per-block absmax scales, write the bf16/f32 params
// (round-to-nearest-even or stochastic rounding).
//
// Reference (rollfast, Python/JAX): src/rollfast/optim/adam8.py:113-204
// (quantize/dequantize), :304-443 (scale_by_adam8 update + adamw8 chain),
// :542-569 (codebook quantization); src/rollfast/utils.py:342-371 (bf16 SR),
// :648-708 (apply_updates).
//
// Execution model.  One wave64 owns one 2048-element quantization block:
// lane l holds elements [j*512 + 8l, j*512 + 8l + 8) for j = 0..3, so every
// global access is a fully coalesced 16-byte (params, grads) or 8-byte
// (codes) vector access, the block absmax is a wave-local reduction (no LDS
// round trip, no barrier), and the updated moments stay in VGPRs until the
// scale is known.  Workgroups are persistent (grid = CUs x occupancy) and
// walk a device-resident work list that covers every leaf of the pytree, so
// a whole parameter tree is one launch.  The codebooks and the requantization
// lookup tables (rf_tables.h) are staged into LDS once per workgroup.
//
// Compiled with -ffp-contract=off: the reference rounds every multiply and
// add separately; FMAs appear only where written explicitly.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "../../include/rfadam8.h"
#include "rf_tables.h"

namespace rf {

constexpr int WAVE = 64;
constexpr int WG = 256;  // four waves per workgroup
constexpr int WAVES_PER_WG = WG / WAVE;
constexpr int64_t FAST_BS = 2048;  // block size of the vectorised path
constexpr int64_t CHUNK = 2048;    // elements per fallback (unquantized moment) work unit

enum : int32_t { KIND_QFAST = 0, KIND_QGEN = 1, KIND_FALLBACK = 2 };

// Kernel-side scalars (derived from rf_adam8_hparams on the host).
struct KHp {
    float b1, omb1, b2, omb2;
    float bc1, bc2, bc1n;
    float rbc1, rbc2, rbc1n;  // f32 reciprocals for the default (non-exact) direction
    float eps, eps_root;
    float wd, wd16;           // f32(wd) and bf16(wd) as f32 (weak-typed decay of bf16 params)
    float neg_lr;             // f32(-lr), or 1.0 when the chain has no learning-rate scale
    uint32_t flags;
    uint32_t kmu0, kmu1, knu0, knu1, kp0, kp1;
};

// Work list: unit u belongs to the segment s with
// segs[s].unit_start <= u < segs[s+1].unit_start (a sentinel closes the list).
struct Seg {
    int64_t unit_start;
    int64_t first;  // first block (quantized) or chunk (fallback) index in the leaf
    int32_t leaf;
    int32_t kind;
    int64_t pad;
};
static_assert(sizeof(Seg) == 32, "Seg is 32 bytes");

typedef void (*adam_kernel_t)(const rf_adam8_leaf*, const Seg*, int64_t, KHp, const uint4*);

// ============================================================ helpers ====
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// f32 -> bf16 round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float x)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ float round_to_bf16(float x) { return bf16_bits_to_f32(f32_to_bf16_rne(x)); }

// utils.py:365-371: noise = bits & 0xFFFF; no noise for |x| >= Inf bits;
// (x_u32 + noise) & 0xFFFF0000 -> bf16 (exact truncation).
__device__ __forceinline__ uint32_t sr_bf16(float x, uint32_t bits)
{
    const uint32_t u = __float_as_uint(x);
    const uint32_t noise = ((u & 0x7FFFFFFFu) >= 0x7F800000u) ? 0u : (bits & 0xFFFFu);
    return (u + noise) >> 16;
}

// Threefry-2x32, 20 rounds (Salmon et al., SC'11): the block cipher under
// jax.random's default PRNG.
__device__ __forceinline__ void threefry2x32(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1,
                                             uint32_t& y0, uint32_t& y1)
{
    const uint32_t k2 = k0 ^ k1 ^ 0x1BD11BDAu;
    uint32_t x0 = c0 + k0, x1 = c1 + k1;
#define RF_TF_ROUND(r)                  \
    x0 += x1;                           \
    x1 = __builtin_rotateleft32(x1, r); \
    x1 ^= x0;
#define RF_TF_R0 RF_TF_ROUND(13) RF_TF_ROUND(15) RF_TF_ROUND(26) RF_TF_ROUND(6)
#define RF_TF_R1 RF_TF_ROUND(17) RF_TF_ROUND(29) RF_TF_ROUND(16) RF_TF_ROUND(24)
    RF_TF_R0 x0 += k1; x1 += k2 + 1u;
    RF_TF_R1 x0 += k2; x1 += k0 + 2u;
    RF_TF_R0 x0 += k0; x1 += k1 + 3u;
    RF_TF_R1 x0 += k1; x1 += k2 + 4u;
    RF_TF_R0 x0 += k2; x1 += k0 + 5u;
#undef RF_TF_R0
#undef RF_TF_R1
#undef RF_TF_ROUND
    y0 = x0;
    y1 = x1;
}

// jax.random.bits(key, shape, uint32)[i] with jax_threefry_partitionable:
// counter (hi32(i), lo32(i)), output y0 ^ y1.
__device__ __forceinline__ uint32_t jax_bits(uint32_t k0, uint32_t k1, uint64_t i)
{
    uint32_t y0, y1;
    threefry2x32(k0, k1, (uint32_t)(i >> 32), (uint32_t)i, y0, y1);
    return y0 ^ y1;
}

// jax.random.split(key, n)[i] with jax_threefry_partitionable.
__device__ __forceinline__ void jax_split(uint32_t k0, uint32_t k1, uint32_t i, uint32_t& o0, uint32_t& o1)
{
    threefry2x32(k0, k1, 0u, i, o0, o1);
}

// jax.random.uniform(float32) from raw bits: mantissa fill of [1, 2) minus 1.
__device__ __forceinline__ float uniform_from_bits(uint32_t bits)
{
    return __uint_as_float((bits >> 9) | 0x3F800000u) - 1.0f;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = max(x, (uint32_t)__shfl_xor((int)x, o, WAVE));
    return x;
}

__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ void stage_tables(uint8_t* lds, const uint4* __restrict__ tables)
{
    uint4* dst = (uint4*)lds;
    for (uint32_t i = threadIdx.x; i < TABLE_BYTES / 16; i += WG) dst[i] = tables[i];
    __syncthreads();
}

// --------------------------------------------------------- quantization --
// Literal restatement of quantize_blocks' element step (adam8.py:167-169,
// :542-569): n = clip(x / scale, cb[0], cb[255]), searchsorted-left, nearest
// with ties to the lower index, or Bernoulli SR.  Used for blocks whose scale
// is outside the fast range and for moment SR.
__device__ __forceinline__ uint32_t code_literal(const float* cb, float x, float scale, bool sr, uint32_t bits)
{
    float n = x / scale;      // IEEE division
    if (n != n) return 254u;  // NaN sorts last: ui = 255, li = 254, never upper
    n = n < cb[0] ? cb[0] : n;
    n = n > cb[255] ? cb[255] : n;
    uint32_t pos = 0;  // number of codebook entries < n (searchsorted left)
    for (uint32_t step = 128; step >= 1; step >>= 1)
        if (cb[pos + step - 1] < n) pos += step;
    const uint32_t ui = pos;
    const uint32_t li = ui > 0 ? ui - 1 : 0;
    const float lv = cb[li], uv = cb[ui];
    bool upper;
    if (sr) {
        const float den = uv - lv;
        float p = den > 0.0f ? (n - lv) / den : 0.0f;
        p = p < 0.0f ? 0.0f : (p > 1.0f ? 1.0f : p);
        upper = uniform_from_bits(bits) < p;
    } else {
        upper = fabsf(uv - n) < fabsf(n - lv);
    }
    return upper ? ui : li;
}

// x / s rounded to nearest even, from the per-block reciprocal rs = 1/s:
// exact for s >= FAST_SCALE_MIN and |x/s| >= 2^-25 (rf_tables.h).
__device__ __forceinline__ float div_by_scale(float x, float s, float rs)
{
    const float q0 = x * rs;
    const float r = __builtin_fmaf(-s, q0, x);
    return __builtin_fmaf(r, rs, q0);
}

// Signed dynamic codebook code of x in a block with scale s (fast path).
__device__ __forceinline__ uint32_t code_signed_fast(const uint8_t* lds, float x, float s, float rs)
{
    const float n = div_by_scale(x, s, rs);
    const uint32_t nb = __float_as_uint(n);
    const uint32_t neg = (uint32_t)((int32_t)nb >> 31);  // 0 or 0xFFFFFFFF
    const uint32_t sd = neg & REGION;
    const uint32_t cell = max((nb >> CELL_SHIFT) & 0xFFFFu, CELL_LO);
    const uint32_t cand = lds[L_POS + REG_CAND - CELL_LO + sd + cell];
    const float t = *(const float*)(lds + L_POS + REG_T + sd + cand * 4u);
    const uint32_t c = cand + (fabsf(n) >= t ? 1u : 0u);
    return (c ^ neg) + 127u - neg;  // n >= 0: 127 + c ; n < 0: 127 - c
}

// Unsigned dynamic codebook code of x >= 0 in a block with scale s (fast path).
__device__ __forceinline__ uint32_t code_unsigned_fast(const uint8_t* lds, float x, float s, float rs)
{
    const float n = div_by_scale(x, s, rs);
    const uint32_t nb = __float_as_uint(n) & 0x7FFFFFFFu;
    const uint32_t cell = max(nb >> CELL_SHIFT, CELL_LO);
    const uint32_t cand = lds[L_CANDU - CELL_LO + cell];
    const float t = *(const float*)(lds + L_TU + cand * 4u);
    return cand + (__uint_as_float(nb) >= t ? 1u : 0u);
}

__device__ __forceinline__ bool scale_is_fast(float s)
{
    return s >= FAST_SCALE_MIN && s <= 3.4028234663852886e38f;
}

// Block scale from the NaN-propagating absmax bit pattern (adam8.py:142,167):
// max > 0 ? max : 1 (a NaN max compares false and yields 1).
__device__ __forceinline__ float scale_from_absmax_bits(uint32_t amax)
{
    const float a = __uint_as_float(amax);
    return a > 0.0f ? a : 1.0f;
}

// ------------------------------------------------------ per-element step --
// Bias-corrected Adam direction (adam8.py:336-362, utils.py:318-324).
template <bool NEST, bool EXACT>
__device__ __forceinline__ float adam_direction(const KHp& h, float m, float v, float g)
{
    if constexpr (EXACT) {
        float mhat;
        if constexpr (NEST) {
            const float a = m / h.bc1n;
            const float b = g / h.bc1;
            const float t1 = h.b1 * a;
            const float t2 = h.omb1 * b;
            mhat = t1 + t2;
        } else {
            mhat = m / h.bc1;
        }
        const float vhat = v / h.bc2;
        const float den = sqrtf(vhat + h.eps_root) + h.eps;
        return mhat / den;
    } else {
        float mhat;
        if constexpr (NEST) {
            const float t1 = h.b1 * (m * h.rbc1n);
            const float t2 = h.omb1 * (g * h.rbc1);
            mhat = t1 + t2;
        } else {
            mhat = m * h.rbc1;
        }
        const float vhat = v * h.rbc2;
        const float den = __builtin_amdgcn_sqrtf(vhat + h.eps_root) + h.eps;
        return mhat * __builtin_amdgcn_rcpf(den);
    }
}

enum : int32_t { WD_OFF = 0, WD_F32 = 1, WD_BF16 = 2 };

// optax add_decayed_weights (u + wd*p) then scale_by_learning_rate ((-lr)*u).
__device__ __forceinline__ float decay_and_scale(const KHp& h, float u, float p, int32_t wd_mode)
{
    if (wd_mode == WD_BF16) {
        u = u + round_to_bf16(h.wd16 * p);  // bf16*bf16 is exact in f32: one rounding
    } else if (wd_mode == WD_F32) {
        const float wdp = h.wd * p;
        u = u + wdp;
    }
    return h.neg_lr * u;  // neg_lr == 1.0 when the chain has no lr scale (exact identity)
}

// EMA moment updates (adam8.py:322-335).
__device__ __forceinline__ void ema(const KHp& h, float mp, float vp, float g, float& m, float& v)
{
    const float t1 = h.b1 * mp;
    const float t2 = h.omb1 * g;
    m = t1 + t2;
    const float gg = g * g;
    const float t3 = h.b2 * vp;
    const float t4 = h.omb2 * gg;
    v = t3 + t4;
}

// ----------------------------------------------------------- vector I/O --
// Load 8 consecutive elements (16-byte aligned) as f32.
template <typename T>
__device__ __forceinline__ void load8(const void* base, int64_t e0, float (&x)[8])
{
    if constexpr (std::is_same<T, uint16_t>::value) {
        const uint4 w = *(const uint4*)((const uint16_t*)base + e0);
        const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = __uint_as_float(d[i] << 16);
            x[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
        }
    } else {
        const float4 a = *(const float4*)((const float*)base + e0);
        const float4 b = *(const float4*)((const float*)base + e0 + 4);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    }
}

__device__ __forceinline__ void store8_f32(void* base, int64_t e0, const float (&x)[8])
{
    float4* p = (float4*)((float*)base + e0);
    p[0] = make_float4(x[0], x[1], x[2], x[3]);
    p[1] = make_float4(x[4], x[5], x[6], x[7]);
}

__device__ __forceinline__ void store8_bf16(void* base, int64_t e0, const uint32_t (&h)[8])
{
    uint4 w;
    w.x = h[0] | (h[1] << 16);
    w.y = h[2] | (h[3] << 16);
    w.z = h[4] | (h[5] << 16);
    w.w = h[6] | (h[7] << 16);
    *(uint4*)((uint16_t*)base + e0) = w;
}

__device__ __forceinline__ void load8_u32(const uint32_t* base, int64_t e0, uint32_t (&x)[8])
{
    const uint4 a = *(const uint4*)(base + e0);
    const uint4 b = *(const uint4*)(base + e0 + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// Scalar element access with a runtime dtype (generic paths).
__device__ __forceinline__ float load1(const void* base, int32_t dtype, int64_t e)
{
    return dtype == RF_BF16 ? bf16_bits_to_f32(((const uint16_t*)base)[e]) : ((const float*)base)[e];
}

__device__ __forceinline__ void store1(void* base, int32_t dtype, int64_t e, float x)
{
    if (dtype == RF_BF16) ((uint16_t*)base)[e] = (uint16_t)f32_to_bf16_rne(x);
    else ((float*)base)[e] = x;
}

// Uniform per-unit context.
struct UnitCtx {
    const uint8_t* lds;
    int32_t wd_mode;
    bool fed;
    uint32_t kmu0, kmu1, knu0, knu1, kp0, kp1;  // per-leaf keys
};

// The param after the update (fused) for one element.
template <bool PSR, typename PT>
__device__ __forceinline__ uint32_t new_param_bits(float p, float u, uint32_t rbits)
{
    const float s = p + u;
    if constexpr (std::is_same<PT, uint16_t>::value) {
        if constexpr (PSR) return sr_bf16(s, rbits);
        else return f32_to_bf16_rne(s);
    } else {
        (void)rbits;
        return __float_as_uint(s);
    }
}

// One element of the update for the generic (scalar) paths: writes the new
// param (fused) or the f32 update.
template <bool APPLY, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void update_one(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e, const KHp& h,
                                           float mm, float vv, float g)
{
    float u = adam_direction<NEST, EXACT>(h, mm, vv, g);
    const bool need_p = APPLY || c.wd_mode != WD_OFF;
    const float p = need_p ? load1(L.param, L.param_dtype, e) : 0.0f;
    u = decay_and_scale(h, u, p, c.wd_mode);
    if constexpr (APPLY) {
        if (L.param_dtype == RF_BF16) {
            uint32_t rb = 0;
            if constexpr (PSR) rb = c.fed ? L.param_bits[e] : jax_bits(c.kp0, c.kp1, (uint64_t)e);
            ((uint16_t*)L.param)[e] = (uint16_t)new_param_bits<PSR, uint16_t>(p, u, rb);
        } else {
            ((float*)L.param)[e] = p + u;
        }
    } else {
        L.updates[e] = u;
    }
}

// Codes of elements [base, base+bs) of a quantized leaf by the literal search
// (or moment SR), recomputing the new moments from the old codes, which are
// still in place.  Scales are not written here.
template <bool MSR>
__device__ __noinline__ void requant_literal(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h,
                                             float sm, float sv, bool fast_m, bool fast_v)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t bs = L.block_size;
    const int64_t base = blk * bs;
    const int64_t nvalid = max((int64_t)0, min(bs, L.size - base));
    const float* cbs = (const float*)(c.lds + L_CBS);
    const float* cbu = (const float*)(c.lds + L_CBU);
    const float sm_old = L.mu_scales[blk];
    const float sv_old = L.nu_scales[blk];
    uint8_t* mcodes = (uint8_t*)L.mu;
    uint8_t* vcodes = (uint8_t*)L.nu;
    const float rsm = 1.0f / sm;
    const float rsv = 1.0f / sv;
    for (int64_t j = lane; j < bs; j += WAVE) {
        const int64_t e = base + j;
        float mm = 0.0f, vv = 0.0f;
        if (j < nvalid) {
            const float g = load1(L.grad, L.grad_dtype, e);
            ema(h, cbs[mcodes[e]] * sm_old, cbu[vcodes[e]] * sv_old, g, mm, vv);
        }
        uint32_t cm, cv;
        if (fast_m) {
            cm = code_signed_fast(c.lds, mm, sm, rsm);
        } else {
            uint32_t bits = 0;
            if constexpr (MSR) bits = c.fed ? L.mu_bits[e] : jax_bits(c.kmu0, c.kmu1, (uint64_t)e);
            cm = code_literal(cbs, mm, sm, MSR, bits);
        }
        if (fast_v) {
            cv = code_unsigned_fast(c.lds, vv, sv, rsv);
        } else {
            uint32_t bits = 0;
            if constexpr (MSR) bits = c.fed ? L.nu_bits[e] : jax_bits(c.knu0, c.knu1, (uint64_t)e);
            cv = code_literal(cbu, vv, sv, MSR, bits);
        }
        mcodes[e] = (uint8_t)cm;
        vcodes[e] = (uint8_t)cv;
    }
}

// ================================================ work units: quantized ====
// Full 2048-element block, vectorised (KIND_QFAST).
template <typename PT, typename GT, bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void unit_qfast(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h)
{
    constexpr int J = FAST_BS / 512;
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t base = blk * FAST_BS;
    const float* cbs = (const float*)(c.lds + L_CBS);
    const float* cbu = (const float*)(c.lds + L_CBU);
    const float sm_old = L.mu_scales[blk];
    const float sv_old = L.nu_scales[blk];
    const uint8_t* mcodes = (const uint8_t*)L.mu;
    const uint8_t* vcodes = (const uint8_t*)L.nu;
    const bool need_p = APPLY || c.wd_mode != WD_OFF;

    float m[J][8], v[J][8];
    uint32_t am = 0, av = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t e0 = base + j * 512 + lane * 8;
        const uint2 mc = *(const uint2*)(mcodes + e0);
        const uint2 vc = *(const uint2*)(vcodes + e0);
        float g[8], p[8];
        load8<GT>(L.grad, e0, g);
        if (need_p) {
            load8<PT>(L.param, e0, p);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) p[t] = 0.0f;
        }
        uint32_t rb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (PSR) {
            if (c.fed) {
                load8_u32(L.param_bits, e0, rb);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) rb[t] = jax_bits(c.kp0, c.kp1, (uint64_t)(e0 + t));
            }
        }
        float uo[8];
        uint32_t po[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t cm = ((t < 4 ? mc.x : mc.y) >> (8 * (t & 3))) & 0xFFu;
            const uint32_t cv = ((t < 4 ? vc.x : vc.y) >> (8 * (t & 3))) & 0xFFu;
            const float mp = cbs[cm] * sm_old;  // adam8.py:200-203
            const float vp = cbu[cv] * sv_old;
            float mm, vv;
            ema(h, mp, vp, g[t], mm, vv);
            m[j][t] = mm;
            v[j][t] = vv;
            am = max(am, __float_as_uint(mm) & 0x7FFFFFFFu);  // NaN bits sort above Inf
            av = max(av, __float_as_uint(vv));                 // v >= 0
            float u = adam_direction<NEST, EXACT>(h, mm, vv, g[t]);
            u = decay_and_scale(h, u, p[t], c.wd_mode);
            if constexpr (APPLY) po[t] = new_param_bits<PSR, PT>(p[t], u, rb[t]);
            else uo[t] = u;
        }
        if constexpr (APPLY) {
            if constexpr (std::is_same<PT, uint16_t>::value) {
                store8_bf16(L.param, e0, po);
            } else {
                float pf[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) pf[t] = __uint_as_float(po[t]);
                store8_f32(L.param, e0, pf);
            }
        } else {
            store8_f32(L.updates, e0, uo);
        }
    }

    // Requantization (adam8.py:633-688 -> quantize_blocks).
    am = wave_max_u32(am);
    av = wave_max_u32(av);
    const float sm = scale_from_absmax_bits(am);
    const float sv = scale_from_absmax_bits(av);
    const bool fast_m = !MSR && scale_is_fast(sm);
    const bool fast_v = !MSR && scale_is_fast(sv);
    if (!MSR && fast_m && fast_v) {
        const float rsm = 1.0f / sm;
        const float rsv = 1.0f / sv;
        uint8_t* mout = (uint8_t*)L.mu;
        uint8_t* vout = (uint8_t*)L.nu;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int64_t e0 = base + j * 512 + lane * 8;
            uint32_t cm[8], cv[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                cm[t] = code_signed_fast(c.lds, m[j][t], sm, rsm);
                cv[t] = code_unsigned_fast(c.lds, v[j][t], sv, rsv);
            }
            uint2 wm, wv;
            wm.x = cm[0] | (cm[1] << 8) | (cm[2] << 16) | (cm[3] << 24);
            wm.y = cm[4] | (cm[5] << 8) | (cm[6] << 16) | (cm[7] << 24);
            wv.x = cv[0] | (cv[1] << 8) | (cv[2] << 16) | (cv[3] << 24);
            wv.y = cv[4] | (cv[5] << 8) | (cv[6] << 16) | (cv[7] << 24);
            *(uint2*)(mout + e0) = wm;
            *(uint2*)(vout + e0) = wv;
        }
    } else {
        // Rare (tiny, Inf or NaN scales) or moment SR: recompute from the old
        // codes, which are untouched so far, and search literally.
        requant_literal<MSR>(c, L, blk, h, sm, sv, fast_m, fast_v);
    }
    if (lane == 0) {
        L.mu_scales[blk] = sm;
        L.nu_scales[blk] = sv;
    }
}

// Any block size, partial or unaligned blocks (KIND_QGEN).  The first pass
// finds the new absmax, the second recomputes the moments and writes the
// params/updates, then the codes are requantized from the old codes (still
// in place).  Elements past `size` are the reference's zero padding.
template <bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT>
__device__ __noinline__ void unit_qgen(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t bs = L.block_size;
    const int64_t base = blk * bs;
    const int64_t nvalid = max((int64_t)0, min(bs, L.size - base));
    const float* cbs = (const float*)(c.lds + L_CBS);
    const float* cbu = (const float*)(c.lds + L_CBU);
    const float sm_old = L.mu_scales[blk];
    const float sv_old = L.nu_scales[blk];
    const uint8_t* mcodes = (const uint8_t*)L.mu;
    const uint8_t* vcodes = (const uint8_t*)L.nu;

    uint32_t am = 0, av = 0;
    for (int64_t j = lane; j < nvalid; j += WAVE) {
        const int64_t e = base + j;
        const float g = load1(L.grad, L.grad_dtype, e);
        float mm, vv;
        ema(h, cbs[mcodes[e]] * sm_old, cbu[vcodes[e]] * sv_old, g, mm, vv);
        am = max(am, __float_as_uint(mm) & 0x7FFFFFFFu);
        av = max(av, __float_as_uint(vv));
        update_one<APPLY, PSR, NEST, EXACT>(c, L, e, h, mm, vv, g);
    }
    am = wave_max_u32(am);
    av = wave_max_u32(av);
    const float sm = scale_from_absmax_bits(am);
    const float sv = scale_from_absmax_bits(av);
    const bool fast_m = !MSR && scale_is_fast(sm);
    const bool fast_v = !MSR && scale_is_fast(sv);
    requant_literal<MSR>(c, L, blk, h, sm, sv, fast_m, fast_v);
    if (lane == 0) {
        L.mu_scales[blk] = sm;
        L.nu_scales[blk] = sv;
    }
}

// ============================================= work units: fallback ====
// Moments stored unquantized (adam8.py:620-630: size < min_size, a
// non-inexact dtype or quantize=False): elementwise update of a chunk.
template <bool APPLY, bool PSR, bool NEST, bool EXACT>
__device__ __noinline__ void unit_fallback(const UnitCtx& c, const rf_adam8_leaf& L, int64_t chunk, const KHp& h)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t base = chunk * CHUNK;
    const int64_t end = min(base + CHUNK, L.size);
    const int32_t mdt = L.moment_kind == RF_MOMENT_BF16 ? RF_BF16 : RF_F32;
    for (int64_t e = base + lane; e < end; e += WAVE) {
        const float g = load1(L.grad, L.grad_dtype, e);
        float mm, vv;
        ema(h, load1(L.mu, mdt, e), load1(L.nu, mdt, e), g, mm, vv);
        update_one<APPLY, PSR, NEST, EXACT>(c, L, e, h, mm, vv, g);
        store1(L.mu, mdt, e, mm);  // adam8.py:688 moment.astype(fallback_dtype)
        store1(L.nu, mdt, e, vv);
    }
}

// ======================================================== step kernel ====
template <bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT>
__global__ __launch_bounds__(WG) void k_adam8(const rf_adam8_leaf* __restrict__ leaves,
                                              const Seg* __restrict__ segs, int64_t total_units, KHp h,
                                              const uint4* __restrict__ tables)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[TABLE_BYTES];
    stage_tables(lds, tables);

    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    int32_t s = 0;
    int32_t cur_leaf = -1;
    UnitCtx c;
    c.lds = lds;
    c.fed = (h.flags & RF_FED_BITS) != 0;
    c.wd_mode = WD_OFF;
    c.kmu0 = c.kmu1 = c.knu0 = c.knu1 = c.kp0 = c.kp1 = 0;
    rf_adam8_leaf L;
    for (int64_t u = wave; u < total_units; u += nwaves) {
        while (segs[s + 1].unit_start <= u) ++s;
        const Seg sg = segs[s];
        if (sg.leaf != cur_leaf) {
            cur_leaf = sg.leaf;
            L = leaves[cur_leaf];
            const bool decay = (L.flags & RF_LEAF_DECAY) != 0;
            c.wd_mode = !decay ? WD_OFF
                               : ((L.param_dtype == RF_BF16 && (h.flags & RF_DECAY_WEAK)) ? WD_BF16 : WD_F32);
            if constexpr (MSR) {
                jax_split(h.kmu0, h.kmu1, (uint32_t)L.state_index, c.kmu0, c.kmu1);
                jax_split(h.knu0, h.knu1, (uint32_t)L.state_index, c.knu0, c.knu1);
            }
            if constexpr (PSR) jax_split(h.kp0, h.kp1, (uint32_t)L.param_index, c.kp0, c.kp1);
        }
        const int64_t idx = sg.first + (u - sg.unit_start);
        if (sg.kind == KIND_QFAST) {
            const int32_t pd = L.param_dtype, gd = L.grad_dtype;
            if (pd == RF_BF16) {
                if (gd == RF_BF16) unit_qfast<uint16_t, uint16_t, APPLY, MSR, PSR, NEST, EXACT>(c, L, idx, h);
                else unit_qfast<uint16_t, float, APPLY, MSR, PSR, NEST, EXACT>(c, L, idx, h);
            } else {
                if (gd == RF_BF16) unit_qfast<float, uint16_t, APPLY, MSR, PSR, NEST, EXACT>(c, L, idx, h);
                else unit_qfast<float, float, APPLY, MSR, PSR, NEST, EXACT>(c, L, idx, h);
            }
        } else if (sg.kind == KIND_QGEN) {
            unit_qgen<APPLY, MSR, PSR, NEST, EXACT>(c, L, idx, h);
        } else {
            unit_fallback<APPLY, PSR, NEST, EXACT>(c, L, idx, h);
        }
    }
}

}  // namespace rf
