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
// scale is known.  Waves walk a device-resident work list that covers every
// leaf of the pytree (unit u goes to wave u mod nwaves, about 16 units per
// wave), so a whole parameter tree is one launch.  The codebooks and the
// requantization lookup tables (rf_tables.h) are staged into LDS once per
// workgroup.
//
// Compiled with -ffp-contract=off: the reference rounds every multiply and
// add separately; FMAs appear only where written explicitly.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "../../include/rfadam8.h"
#include "rf_tables.h"

// Global-address-space views of the leaf's buffers.  The leaf table holds
// generic pointers, and an access through one compiles to a flat
// instruction, which counts against lgkmcnt as well as vmcnt: every later
// wait for an LDS read or a scalar load then also waits for the flat loads
// and stores in flight, and the element paths' batches of loads serialise.
// Through these views they compile to global_load/global_store, counted
// only by vmcnt.
// RF_LDS: the LDS address space (the DMA loads' destination operand).
#if defined(__HIP_DEVICE_COMPILE__)
#define RF_GLOBAL __attribute__((address_space(1)))
#define RF_LDS __attribute__((address_space(3)))
#else
#define RF_GLOBAL
#define RF_LDS
#endif

namespace rf {

constexpr int WAVE = 64;
constexpr int WG = 256;  // four waves per workgroup
constexpr int WAVES_PER_WG = WG / WAVE;
constexpr int64_t FAST_BS = 2048;  // block size of the vectorised path
constexpr int64_t CHUNK = 2048;    // elements per fallback (unquantized moment) work unit
// Element-wise fallback units (leaves' tails that are not whole aligned
// chunks): in fused launches 256 elements, one batch per lane, so a small
// leaf spreads over several waves; update-only launches keep whole chunks,
// the slots of Magma's partial sums.
constexpr int64_t EW_UNIT_FUSED = 256;
template <bool APPLY>
constexpr int64_t EW_UNIT = APPLY ? EW_UNIT_FUSED : CHUNK;

// Waves per SIMD the step kernel is register-allocated for (<= 512 / N VGPRs).
#ifndef RF_STEP_WAVES_PER_EU
#define RF_STEP_WAVES_PER_EU 3
#endif
// Prefetch the next block's first chunk during requantization (1) or not (0).
#ifndef RF_PREFETCH_NEXT
#define RF_PREFETCH_NEXT 1
#endif

enum : int32_t { KIND_QFAST = 0, KIND_QGEN = 1, KIND_FALLBACK = 2, KIND_FALLBACK_VEC = 3 };

struct Seg;

// Kernel-side scalars (derived from rf_adam8_hparams on the host).
struct KHp {
    float b1, omb1, b2, omb2;
    float bc1, bc2, bc1n;
    // Default (non-exact) direction u = m / (k1 * sqrt(v + er2) + k2) with
    // k1 = bc1 / sqrt(bc2), k2 = eps * bc1, er2 = eps_root * bc2: the same
    // quantity as (m/bc1) / (sqrt(v/bc2 + eps_root) + eps), fewer roundings.
    float k1, k2, er2;
    float nb1, nomb1, rsbc2;  // nesterov: b1/bc1_next, (1-b1)/bc1, 1/sqrt(bc2)
    float nomb1x;             // nesterov: f32(1 - b1) (double), exact path
    float eps, eps_root;
    float wd, wd16, wdh;      // f32(wd), bf16(wd) and f16(wd) as f32 (weak-typed decay of 16-bit params)
    float neg_lr;             // f32(-lr), or 1.0 when the chain has no learning-rate scale
    uint32_t flags;
    int32_t run;              // fast kernel: consecutive units a wave takes before its grid stride (>= 1)
    int32_t upd_nt;           // fast kernel: nontemporal f32 update and param stores (store8_f32_lines)
    uint32_t kmu0, kmu1, knu0, knu1, kp0, kp1;
    const float* clip;        // device (scale, norm) of global-norm clipping, or null
    const float* gate;        // device flag: 1 = every grad finite, 0 = reject the step; null = no gate
    const rf_adam8_group* groups;  // per-group lr, decay, EMA weight and keys (grouped launch), or null
    // Magma sums (optim/magma.py:15-132) written by the unquantized-moment
    // units of an update-only launch, or null: f64 triples (g·m', g·g, m'·m') per 2048-element chunk at
    // mpart[3 * (msegs[leaf].unit_start + chunk)].
    double* mpart;
    const Seg* msegs;
    // Learning-rate-folded direction of the fast kernel's nearest-rounding
    // bf16 step (device-derived by flr_setup, not set by the host):
    // k1l = k1 / neg_lr, k2l = k2 / neg_lr, wdl = neg_lr * bf16(wd) and
    // flr = 1 where those are in range for the one-ulp bound.
    float k1l, k2l, wdl;
    int32_t flr;
    // A generic list riding along with a bf16/bf16 fast launch: its first
    // gwgs workgroups run gen_list over gsegs (gunits units); 0 = none.
    const Seg* gsegs;
    int64_t gunits;
    int32_t gwgs;
};

// Work list: unit u belongs to the segment s with
// segs[s].unit_start <= u < segs[s+1].unit_start (a sentinel closes the list).
struct Seg {
    int64_t unit_start;
    int64_t first;  // first block (quantized) or chunk (fallback) index in the leaf
    int32_t leaf;
    int32_t kind;
    int32_t nseg;   // the list's sentinel index (its segment count), in every record
    int32_t lead;   // generic list: its leading quantized units, taken a workgroup each (in every record)
};
static_assert(sizeof(Seg) == 32, "Seg is 32 bytes");

typedef void (*adam_kernel_t)(const rf_adam8_leaf*, const Seg*, int64_t, KHp, const uint4*);

// ============================================================ helpers ====
// The segment of unit u (segs[s].unit_start <= u < segs[s + 1].unit_start),
// searched upward from s, which must not lie past it.  A unit in the same
// segment as the last costs one load.  Otherwise the wave's 64 lanes probe
// 64 evenly spaced segments of the bracket at once and the ballot narrows it
// 64-fold: one or two dependent loads for up to 4,096 segments, where a
// binary search paid log2(nseg).  Called by whole waves with uniform
// arguments; the result is uniform.
__device__ __forceinline__ int32_t seek_seg(const Seg* __restrict__ segs, int32_t nseg, int32_t s, int64_t u)
{
    if (segs[s + 1].unit_start > u) return s;
    int32_t lo = s + 1, hi = nseg;  // segs[lo].unit_start <= u < segs[hi].unit_start (the sentinel's)
    const int32_t lane = (int32_t)(threadIdx.x & (WAVE - 1));
    while (hi - lo > 1) {
        const int32_t step = (hi - lo + WAVE - 1) / WAVE;
        const int32_t i = lo + lane * step;  // lane 0 probes lo, known to be <= u
        const bool le = i < hi && segs[i].unit_start <= u;
        const uint64_t m = __builtin_amdgcn_ballot_w64(le);
        lo += (63 - __builtin_clzll(m)) * step;  // the last probe <= u
        hi = min(hi, lo + step);                 // the next probe (or hi) is > u
    }
    return lo;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// f32 -> bf16 round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float x)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ float round_to_bf16(float x) { return bf16_bits_to_f32(f32_to_bf16_rne(x)); }

// Two f32 -> bf16 (round to nearest even) in one v_cvt_pk_bf16_f32; the
// result is the packed pair (lo, hi).
typedef float rf_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 rf_bf2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi)
{
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((rf_f2){lo, hi}, rf_bf2));
}

// f16 (IEEE binary16) conversions: exact widening; narrowing rounds to
// nearest even with f16 subnormals kept (v_cvt_f32_f16 / v_cvt_f16_f32).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__device__ __forceinline__ uint32_t f32_to_f16_rne(float x)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}

__device__ __forceinline__ float round_to_f16(float x) { return f16_bits_to_f32(f32_to_f16_rne(x)); }

__device__ __forceinline__ uint32_t pack_f16x2_rne(float lo, float hi)
{
    return f32_to_f16_rne(lo) | (f32_to_f16_rne(hi) << 16);
}

// Element types of the templated units: float = f32, uint16_t = bf16 bit
// patterns, _Float16 = f16.
template <typename T>
constexpr bool IS_BF16 = std::is_same<T, uint16_t>::value;
template <typename T>
constexpr bool IS_F16 = std::is_same<T, _Float16>::value;

// Two f32 values rounded to the 16-bit type T (nearest even) and packed.
template <typename T>
__device__ __forceinline__ uint32_t pack_h16x2_rne(float lo, float hi)
{
    if constexpr (IS_F16<T>) return pack_f16x2_rne(lo, hi);
    else return pack_bf16x2_rne(lo, hi);
}

// f32 value of a 16-bit pattern of type T.
template <typename T>
__device__ __forceinline__ float h16_to_f32(uint32_t h)
{
    if constexpr (IS_F16<T>) return f16_bits_to_f32(h & 0xFFFFu);
    else return bf16_bits_to_f32(h & 0xFFFFu);
}

// utils.py:365-371: noise = bits & 0xFFFF; no noise for |x| >= Inf bits;
// (x_u32 + noise) & 0xFFFF0000 -> bf16 (exact truncation).  The word with
// the rounded bf16 in its high half (the low half is not cleared): the
// noise is added unconditionally (one add of the low half of the bits) and
// the sum kept only for finite x (one class compare and one select).
__device__ __forceinline__ uint32_t sr_bf16_hi(float x, uint32_t bits)
{
    const uint32_t u = __float_as_uint(x);
    const uint32_t r = u + (bits & 0xFFFFu);
    return __builtin_isfinite(x) ? r : u;
}

__device__ __forceinline__ uint32_t sr_bf16(float x, uint32_t bits) { return sr_bf16_hi(x, bits) >> 16; }

// The high halves of two words as one (lo's in bits 0-15): one byte permute.
__device__ __forceinline__ uint32_t pack_hi16x2(uint32_t lo, uint32_t hi)
{
    return __builtin_amdgcn_perm(hi, lo, 0x07060302u);  // bytes lo.2, lo.3, hi.2, hi.3
}

// Threefry-2x32, 20 rounds (Salmon et al., SC'11): the block cipher under
// jax.random's default PRNG.
__device__ __forceinline__ void threefry2x32(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1,
                                             uint32_t& y0, uint32_t& y1)
{
    const uint32_t k2 = k0 ^ k1 ^ 0x1BD11BDAu;
    uint32_t x0 = c0 + k0, x1 = c1 + k1;
// The empty asm pins x0 and x1 to one register each after every round:
// without it the compiler keeps x0 as a sum of two registers across rounds
// and spends a second add per round on it (about 89 instead of 69 VALU
// instructions per Threefry block).  The fourth round of each group takes
// the key injection before its pin: x1's xor and injection add become one
// v_xad_u32, and x0's injection, left unpinned for one round, joins the next
// round's add in a v_add3_u32 (64 instructions per block).
#define RF_TF_ROUND(r)                  \
    x0 += x1;                           \
    x1 = __builtin_rotateleft32(x1, r); \
    x1 ^= x0;                           \
    __asm__("" : "+v"(x0), "+v"(x1));
#define RF_TF_INJECT(r, ka, kb)                         \
    x0 += x1;                                           \
    x1 = (__builtin_rotateleft32(x1, r) ^ x0) + (kb);   \
    __asm__("" : "+v"(x1));                             \
    x0 += (ka);
#define RF_TF_R0(ka, kb) RF_TF_ROUND(13) RF_TF_ROUND(15) RF_TF_ROUND(26) RF_TF_INJECT(6, ka, kb)
#define RF_TF_R1(ka, kb) RF_TF_ROUND(17) RF_TF_ROUND(29) RF_TF_ROUND(16) RF_TF_INJECT(24, ka, kb)
    RF_TF_R0(k1, k2 + 1u)
    RF_TF_R1(k2, k0 + 2u)
    RF_TF_R0(k0, k1 + 3u)
    RF_TF_R1(k1, k2 + 4u)
    RF_TF_R0(k2, k0 + 5u)
#undef RF_TF_R0
#undef RF_TF_R1
#undef RF_TF_INJECT
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

// Packed bit source (RF_PACKED_BITS; no reference counterpart, opt-in): the
// stochastic roundings draw from whole Threefry-2x32-20 blocks instead of
// one block per 32-bit word.  Param rounding needs 16 bits per element, so
// element e of a leaf takes the 16-bit half (e & 1) of word (e & 2 ? y1 :
// y0) of the block at counter (hi32(e >> 2), lo32(e >> 2)) under the leaf's
// param key: a block per four elements.  The moments' draws take the 16-bit
// halves (e & 1) of y0 (first moment) and y1 (second moment) of the block at
// counter (hi32(e >> 1), lo32(e >> 1)) under the leaf's first-moment key: a
// block per pair of elements for both moments (packed_moment_block).  The
// param rounding reads the noise from the low 16 bits of the word.
__device__ __forceinline__ void packed_param_bits4(uint32_t k0, uint32_t k1, uint64_t e0, uint32_t* rb)
{
    uint32_t y0, y1;
    const uint64_t q = e0 >> 2;  // e0 is a multiple of 4
    threefry2x32(k0, k1, (uint32_t)(q >> 32), (uint32_t)q, y0, y1);
    rb[0] = y0;
    rb[1] = y0 >> 16;
    rb[2] = y1;
    rb[3] = y1 >> 16;
}

__device__ __forceinline__ uint32_t packed_param_bits1(uint32_t k0, uint32_t k1, uint64_t e)
{
    uint32_t y0, y1;
    const uint64_t q = e >> 2;
    threefry2x32(k0, k1, (uint32_t)(q >> 32), (uint32_t)q, y0, y1);
    const uint32_t w = (e & 2) ? y1 : y0;
    return (e & 1) ? (w >> 16) : w;
}

// The packed source's moment blocks.  Element e's main half is the 16-bit
// half (e & 1) of y0 (first moment) or y1 (second moment) of the main block,
// at counter (hi32(e >> 1), lo32(e >> 1)); its fill half is the same half of
// the fill block, at counter 2^63 + (e >> 1) (both under the leaf's
// first-moment key; a 2^63 element leaf would be needed for the two to
// meet).  bf16 storage rounding takes the main half as its 16 bits of
// noise.  The codes' Bernoulli draw takes the word (main << 16) | fill,
// whose top 23 bits make the uniform (uniform_from_bits): the main half and
// the fill's top 7 bits, so each draw takes the upper code with the
// probability the reference's 23-bit uniform gives.  The main half alone
// settles a draw unless the probability lies within 127/128 of a main-half
// step above it (probability 2^-16 per draw; packed_sr_main), and only
// then is the fill block computed.
__device__ __forceinline__ void packed_moment_block(uint32_t k0, uint32_t k1, uint64_t e, bool fill, uint32_t& y0,
                                                    uint32_t& y1)
{
    const uint64_t q = e >> 1;
    threefry2x32(k0, k1, (uint32_t)(q >> 32) | (fill ? 0x80000000u : 0u), (uint32_t)q, y0, y1);
}

__device__ __forceinline__ uint32_t half16(uint32_t w, uint64_t e)
{
    return (e & 1) ? (w >> 16) : (w & 0xFFFFu);
}

// jax.random.uniform(float32) from raw bits: mantissa fill of [1, 2) minus 1.
__device__ __forceinline__ float uniform_from_bits(uint32_t bits)
{
    // (bits >> 9) | 0x3F800000 as one funnel shift of (0x7F : bits) by 9
    return __uint_as_float(__builtin_amdgcn_alignbit(0x7Fu, bits, 9)) - 1.0f;
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}

// Wave-wide unsigned max (every lane active), returned wave-uniform: four
// DPP steps leave each 16-lane row's max in all of its lanes, then the four
// row maxima are combined in scalar registers.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x)
{
    x = max(x, dpp_u32<0xB1>(x));   // quad_perm [1,0,3,2]
    x = max(x, dpp_u32<0x4E>(x));   // quad_perm [2,3,0,1]
    x = max(x, dpp_u32<0x141>(x));  // row_half_mirror
    x = max(x, dpp_u32<0x140>(x));  // row_mirror
    const uint32_t r0 = __builtin_amdgcn_readlane(x, 0), r1 = __builtin_amdgcn_readlane(x, 16);
    const uint32_t r2 = __builtin_amdgcn_readlane(x, 32), r3 = __builtin_amdgcn_readlane(x, 48);
    return max(max(r0, r1), max(r2, r3));
}

// Four byte values (each < 256) packed little-endian: two shift-or steps and
// one byte permute, three instructions.
__device__ __forceinline__ uint32_t pack4_u8(uint32_t a, uint32_t b, uint32_t c, uint32_t d)
{
    const uint32_t lo = a | (b << 8);
    const uint32_t hi = c | (d << 8);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);  // bytes lo.0, lo.1, hi.0, hi.1
}

__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ double wave_sum_f64(double x)
{
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, WAVE);
    return x;
}

// Copies the first BYTES of a table image into the workgroup's LDS.
// Up to the 22 KB requantization tables: through registers, every load of a
// thread issued before its first LDS write, so a workgroup's start waits for
// one memory latency.  The 30 KB search image of moment-SR launches: through
// the LDS-DMA form of the global load (global_load_lds_dwordx4, gfx950),
// each lane's 16 bytes going from global memory straight to LDS at the
// instruction's LDS base + 16 * lane; a wave moves 1 KB per instruction, the
// waves take the 1 KB pieces in turn, the last piece's lanes past BYTES
// masked off.  The register form of that image held 32 VGPRs at the
// kernel's start, where the compiler spilled them (28 KB of scratch writes
// per workgroup); with the DMA form the moment-SR step ran 1 % faster, while
// the nearest-rounding step measured 0.3 % slower with it than with
// registers (same GPU, alternating runs).
template <uint32_t BYTES = TABLE_BYTES>
__device__ __forceinline__ void stage_tables(uint8_t* lds, const uint4* __restrict__ tables)
{
    static_assert(BYTES % 16 == 0, "tables are copied in 16-byte words");
    if constexpr (BYTES > TABLE_BYTES) {
        constexpr uint32_t PIECE = WAVE * 16;
        constexpr uint32_t NPIECE = (BYTES + PIECE - 1) / PIECE;
        const uint32_t wave = uniform_u32(threadIdx.x / WAVE);
        const uint32_t lane16 = (threadIdx.x & (WAVE - 1)) * 16u;
        const RF_GLOBAL uint8_t* src = (const RF_GLOBAL uint8_t*)tables;
        for (uint32_t k = wave; k < NPIECE; k += WAVES_PER_WG) {
            const uint32_t base = k * PIECE;
            if (base + lane16 < BYTES)
                __builtin_amdgcn_global_load_lds((const RF_GLOBAL void*)(src + base + lane16),
                                                 (RF_LDS void*)(lds + base), 16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): the DMA writes have reached LDS
    } else {
        constexpr uint32_t N = BYTES / 16;
        constexpr uint32_t FULL = N / WG, REM = N % WG;  // whole rounds of the workgroup, then a partial one
        uint4* dst = (uint4*)lds;
        uint4 t[FULL + 1];
#pragma unroll
        for (uint32_t k = 0; k < FULL; ++k) t[k] = tables[threadIdx.x + k * WG];
        if (REM && threadIdx.x < REM) t[FULL] = tables[threadIdx.x + FULL * WG];
#pragma unroll
        for (uint32_t k = 0; k < FULL; ++k) dst[threadIdx.x + k * WG] = t[k];
        if (REM && threadIdx.x < REM) dst[threadIdx.x + FULL * WG] = t[FULL];
    }
    __syncthreads();
}

// --------------------------------------------------------- quantization --
// Literal restatement of quantize_blocks' element step (adam8.py:167-169,
// :542-569): n = clip(x / scale, cb[0], cb[255]), searchsorted-left, nearest
// with ties to the lower index, or Bernoulli SR.  Used for blocks whose scale
// is outside the fast range, and by the generic (partial-block) units.
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

// Threshold-count candidates of a normalised value: the number of decision
// thresholds at or below the low end of n's cell (signed: per sign).
// Signed candidate-table index of n: the cell of |n| with the sign as bit
// CANDS_SIGN_SHIFT.
__device__ __forceinline__ uint32_t signed_cell(float n)
{
    const uint32_t nb = __float_as_uint(n);
    const uint32_t idx = __builtin_elementwise_sub_sat((nb >> CELL_SHIFT) & 0xFFFFu, CELL_LO);
    return ((nb >> (31 - CANDS_SIGN_SHIFT)) & CANDS_SIGN_STRIDE) | idx;
}

__device__ __forceinline__ uint32_t cand_signed(const uint8_t* lds, float n)
{
    return lds[L_CANDS + signed_cell(n)];
}

__device__ __forceinline__ uint32_t cand_unsigned(const uint8_t* lds, float n)
{
    return lds[L_CANDU + __builtin_elementwise_sub_sat(__float_as_uint(n) >> CELL_SHIFT, CELL_LO)];
}

// Stochastically rounded code of a normalised n (finite, |n| <= 1) from its
// searchsorted candidate `cand` (the search image's candidate byte of n's
// cell): _quantize_to_codebook's SR branch (adam8.py:549-564).
// ui = searchsorted_left(cb, n) = cand + (cb[cand] < n), li = ui - 1 (at
// least 0), p = (n - cb[li]) / (cb[ui] - cb[li]) (0 when the two coincide),
// upper code iff uniform(bits) < p.  sr_upper returns x = 65536 p: `rec`
// holds per ui >= 1 {cb[li], gap 2^-16, y 2^16} with y = RN(1/gap), and
// x = fma(r, y', q0) with q0 = a*y' and r = fma(-gap', q0, a) (a = n -
// cb[li]) is 65536 times a quotient that decides the Bernoulli draw as the
// IEEE quotient does for every uniform value (a reciprocal correctly
// rounded and one Markstein correction, scaled by powers of two; the tables
// test checks it against IEEE division over every gap).  Since cb[li] < n
// <= cb[ui], 0 <= x <= 65536 needs no clip.  ui = 0 (n <= cb[0], where the
// reference's clip leaves li = ui = 0) finds {-2, 0, 65536}: a = n + 2 >= 1
// and x = 2a 65536 exceeds every draw, so "upper" picks ui and the code
// ui - 1 + up needs no clamp (code_of_draw).
__device__ __forceinline__ float sr_upper(const float* cb, const float4* rec, uint32_t& cand, float n)
{
    const uint32_t ui = cand + (cb[cand] < n ? 1u : 0u);
    const float4 nb = rec[ui];
    const float a = n - nb.x;
    const float q0 = a * nb.z;
    const float r = __builtin_fmaf(-nb.y, q0, a);
    cand = ui;
    return __builtin_fmaf(r, nb.z, q0);
}

// uniform_from_bits(bits) * 65536, exactly: (bits >> 9) | 0x47800000 is
// 65536 (1 + k 2^-23) for k = bits >> 9.
__device__ __forceinline__ float uniform_from_bits_x65536(uint32_t bits)
{
    return __uint_as_float(__builtin_amdgcn_alignbit(0x8Fu, bits, 9)) - 65536.0f;
}

// ui - 1 + up, the code of a draw: one v_addc whose carry-in is up's lane
// mask (the ui = 0 record makes up true there).  Written as asm: from C the
// compiler emits a select and a clamped subtract, or, as ui minus the
// "lower" bit, keeps a batch's masks in scalar registers across the packed
// source's fill branch and spills.  The s_nop gives the two wait states a
// lane mask written by a vector compare needs before a vector instruction
// reads it as a carry, which the compiler cannot see inside the asm.
__device__ __forceinline__ uint32_t code_of_draw(uint32_t ui, uint64_t up_mask)
{
    uint32_t r;
    uint64_t carry_out;
    __asm__("s_nop 1\n\tv_addc_co_u32_e64 %0, %1, -1, %2, %3" : "=v"(r), "=s"(carry_out) : "v"(ui), "s"(up_mask));
    return r;
}

__device__ __forceinline__ uint32_t code_of_draw(uint32_t ui, bool up)
{
    return code_of_draw(ui, __builtin_amdgcn_ballot_w64(up));
}

// The code from ui and x = 65536 p (sr_upper) and a 32-bit draw.
__device__ __forceinline__ uint32_t sr_decide(uint32_t ui, float x, uint32_t bits)
{
    return code_of_draw(ui, uniform_from_bits_x65536(bits) < x);
}

__device__ __forceinline__ uint32_t sr_code(const float* cb, const float4* rec, uint32_t cand, float n,
                                            uint32_t bits)
{
    const float x = sr_upper(cb, rec, cand, n);
    return sr_decide(cand, x, bits);
}

// The packed source's draw from its main half m alone (packed_moment_block):
// the draw is k = 128 m + f (f, the fill's top 7 bits, below 128) and takes
// the upper code iff k 2^-23 < p, i.e. m + f / 128 < x = 65536 p (sr_upper's
// result).  m + 127/128 < x settles "upper" whatever f is, and m >= x
// settles "lower"; the lanes between the two are added to `open` (a lane
// mask), and the caller decides them with the fill (sr_decide on the whole
// word).  x - 127/128 is exact where it is not negative (127/128 is a
// multiple of x's ulp while x < 2^17) and negative otherwise, where "upper"
// is rightly not settled; the ui = 0 record's x >= 131072 settles "upper".
// The two compares stay lane masks, combined in scalar registers.
__device__ __forceinline__ uint32_t packed_sr_main(uint32_t ui, float x, uint32_t m, uint64_t& open)
{
    const float hm = (float)m;
    const uint64_t up = __builtin_amdgcn_ballot_w64(hm < x - 0.9921875f);
    const uint64_t below = __builtin_amdgcn_ballot_w64(hm < x);
    open |= below & ~up;
    return code_of_draw(ui, up);
}

// Signed dynamic codebook code of x in a block with scale s (fast path;
// |x| <= s, so |n| <= 1).
__device__ __forceinline__ uint32_t code_signed_fast(const uint8_t* lds, float x, float s, float rs)
{
    const float n = div_by_scale(x, s, rs);
    const uint32_t cand = lds[L_CANDS + signed_cell(n)];
    const float t = *(const float*)(lds + L_TS + cand * 4u);
    return cand + (n >= t ? 1u : 0u);
}

// Unsigned dynamic codebook code of x >= 0 in a block with scale s (fast path).
__device__ __forceinline__ uint32_t code_unsigned_fast(const uint8_t* lds, float x, float s, float rs)
{
    const float n = div_by_scale(x, s, rs);
    const uint32_t idx = __builtin_elementwise_sub_sat(__float_as_uint(n) >> CELL_SHIFT, CELL_LO);
    const uint32_t cand = lds[L_CANDU + idx];
    const float t = *(const float*)(lds + L_TU + cand * 4u);
    return cand + (n >= t ? 1u : 0u);
}

// Fast (table) requantization of a block: its absmax must be finite (a NaN
// absmax yields scale 1 but leaves NaN or |n| > 1 elements, which only the
// literal path handles) and the scale within the exact-division range.
__device__ __forceinline__ bool block_is_fast(uint32_t amax_bits, float s)
{
    return amax_bits < 0x7F800000u && s >= FAST_SCALE_MIN;
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
// ER = false: eps_root is zero and its term is left out of the hardware
// direction (v + 0 is v for every v the step forms: v >= +0 or NaN).
template <bool NEST, bool EXACT, bool ER = true>
__device__ __forceinline__ float adam_direction(const KHp& h, float m, float v, float g)
{
    if constexpr (EXACT) {
        float mhat;
        if constexpr (NEST) {
            const float a = m / h.bc1n;
            const float b = g / h.bc1;
            const float t1 = h.b1 * a;
            const float t2 = h.nomb1x * b;
            mhat = t1 + t2;
        } else {
            mhat = m / h.bc1;
        }
        const float vhat = v / h.bc2;
        const float den = sqrtf(vhat + h.eps_root) + h.eps;
        return mhat / den;
    } else {
        const float sv = __builtin_amdgcn_sqrtf(ER ? v + h.er2 : v);
        if constexpr (NEST) {
            const float mhat = h.nb1 * m + h.nomb1 * g;
            return mhat * __builtin_amdgcn_rcpf(__builtin_fmaf(sv, h.rsbc2, h.eps));
        } else {
            return m * __builtin_amdgcn_rcpf(__builtin_fmaf(sv, h.k1, h.k2));
        }
    }
}

enum : int32_t { WD_OFF = 0, WD_F32 = 1, WD_BF16 = 2, WD_F16 = 3 };

// optax add_decayed_weights (u + wd*p) then scale_by_learning_rate ((-lr)*u);
// `zero`: optim/adam.py's own weight-0 term u + 0*p first (RF_LEAF_ZERO_DECAY).
__device__ __forceinline__ float decay_and_scale(const KHp& h, float u, float p, int32_t wd_mode, bool zero = false)
{
    if (zero) {
        const float zp = 0.0f * p;  // NaN for a non-finite p, signed zero otherwise
        u = u + zp;
    }
    if (wd_mode == WD_BF16) {
        u = u + round_to_bf16(h.wd16 * p);  // bf16*bf16 is exact in f32: one rounding
    } else if (wd_mode == WD_F16) {
        u = u + round_to_f16(h.wdh * p);    // f16*f16 is exact in f32: one rounding
    } else if (wd_mode == WD_F32) {
        const float wdp = h.wd * p;
        u = u + wdp;
    }
    return h.neg_lr * u;  // neg_lr == 1.0 when the chain has no lr scale (exact identity)
}

// decay_and_scale over the 8 elements of a chunk with the mode fixed at
// compile time (a Python-scalar wd times bf16 params: two products per
// bf16 conversion instruction).
template <int WDM>
__device__ __forceinline__ void decay_and_scale8(const KHp& h, float (&u)[8], const float (&p)[8]);

// True where a fused param update p + u nearly cancels (|p + u| < |u| / 4096):
// only there can a few-ulp error in u move the rounded param by more than
// one bf16 ulp.
__device__ __forceinline__ bool cancels(float sum, float u)
{
    return fabsf(sum) * 4096.0f < fabsf(u);
}

// Exact-mode bf16 params from the hardware direction: true when s = p + upd
// (upd = lr * (a + w), a the hardware rcp/sqrt direction, w the weight
// decay term) rounds to the same bf16 (nearest even) as the IEEE
// computation would.  The hardware direction (f32 k1, k2, er2, v + er2,
// v_sqrt and v_rcp within 1 ulp, one FMA, one product) is within 4 * 2^-23
// relative of the exact quotient, the IEEE sequence (m / bc1, v / bc2,
// + eps_root, sqrt, + eps, the quotient) within 2.5 * 2^-23, so the two
// directions differ by at most about 2^-20.3 |a| (no cancellation inside
// the non-Nesterov direction; Nesterov's two-term numerator can cancel and
// is not taken here).  With the roundings of a + w, of the lr product and of
// both sums, and |lr a| <= |upd| (1 + 2^-22) + |lr w|, |w| <= |wd p| (1 +
// 2^-8), the two sums differ by less than
//   B = 2^-17 |upd| + c_w |p| + 2^-22 |s| + 2^-126,  c_w = 2^-17 |lr wd|
// (each term with a margin of 2x or more).  The rounding is settled when s
// is farther than B from the bf16 midpoint of its binade (s - mid is exact),
// B is below |s| 2^-10 (below 0x4000 ulps of s: neither the midpoint of the
// binade below nor a sign change is within reach) and |upd| < c_g = 2^100
// |lr| (the direction far from f32 overflow, where one of the two could be
// infinite; lr = 0 settles nothing).  NaN and Inf fail the tests.  Unsettled
// lanes are recomputed with IEEE arithmetic.
__device__ __forceinline__ bool rne_bf16_settled(float s, float upd, float p, float c_w, float c_g)
{
    const float b = __builtin_fmaf(0x1p-17f, fabsf(upd),
                                   __builtin_fmaf(c_w, fabsf(p), __builtin_fmaf(0x1p-22f, fabsf(s), 0x1p-126f)));
    const float mid = __uint_as_float((__float_as_uint(s) & 0xFFFF0000u) | 0x8000u);
    return fabsf(s - mid) > b && b < fabsf(s) * 0x1p-10f && fabsf(upd) < c_g;
}

// The learning-rate-folded step (fast kernel, bf16 params, nearest
// rounding, hardware direction, eps_root = 0, no Nesterov).  The reference
// forms p + (-lr) * (m / (sqrt(v/bc2) + eps) / bc1 + bf16(wd * p)) with a
// rounding after every operation (adam8.py:322-339, optax
// add_decayed_weights and scale_by_learning_rate, apply_updates).  With
// D' = sqrt(v) * k1l + k2l (k1l = k1 / -lr, k2l = k2 / -lr) and
// wdl = -lr * bf16(wd) the same quantity is
//   s = fma(m, rcp(D'), fma(wdl, p, p)),
// five instructions per element where the unfolded form takes nine.  Bound
// against the reference's f32 sum s_ref, for |p| <= 1024 |s| (elements
// beyond that nearly cancel and are recomputed with IEEE arithmetic):
// the direction term is within about 2^-20 of |lr a| relative (k1l, k2l,
// v_sqrt, the FMA, v_rcp, the product: seven roundings of at most one f32
// ulp, against the reference's 2.5 ulp quotient and two roundings), and
// |lr a| <= |s| + |p| + |lr wd p| <= 1026 |s|; the decay term differs by the
// reference's bf16 rounding of wd * p, at most 2^-8 |wd p|, which with
// |lr wd| <= 2^-14 is below 2^-12 |s|; fma(wdl, p, p) and the final FMA
// round twice more (2^-24 |p| + 2^-24 |s|).  In all |s - s_ref| < 2^-9.5 |s|,
// below half a bf16 ulp of s (a bf16 ulp exceeds 2^-8 |s|), so nearest-even
// and stochastic rounding of s and s_ref land at most one bf16 ulp apart.
// flr_setup derives the constants and clears flr where they leave that
// range (lr = 0, non-finite or extreme k1l or k2l, |lr wd| > 2^-14).
constexpr float FLR_CANCEL = 1024.0f;

__device__ __forceinline__ void flr_setup(KHp& h)
{
    const float k1l = h.k1 / h.neg_lr;
    const float k2l = h.k2 / h.neg_lr;
    const float wdl = h.neg_lr * h.wd16;
    h.k1l = k1l;
    h.k2l = k2l;
    h.wdl = wdl;
    const float a1 = fabsf(k1l), a2 = fabsf(k2l);
    h.flr = (a1 >= 0x1p-100f && a1 <= 0x1p63f && (a2 == 0.0f || (a2 >= 0x1p-100f && a2 <= 0x1p63f)) &&
             fabsf(wdl) <= 0x1p-14f)
                ? 1
                : 0;
}

// Active lanes where any of 8 sums nearly cancels: each compare's lane mask
// is OR-ed in scalar registers, with no per-lane flag materialised.
__device__ __forceinline__ uint64_t cancel_lanes8(const float (&sum)[8], const float (&u)[8])
{
    uint64_t r = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) r |= __builtin_amdgcn_ballot_w64(cancels(sum[t], u[t]));
    return r;
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


template <typename T>
__device__ __forceinline__ const RF_GLOBAL T* gload_ptr(const void* p, int64_t byte_off)
{
    return (const RF_GLOBAL T*)((const RF_GLOBAL uint8_t*)p + byte_off);
}

template <typename T>
__device__ __forceinline__ RF_GLOBAL T* gstore_ptr(void* p, int64_t byte_off)
{
    return (RF_GLOBAL T*)((RF_GLOBAL uint8_t*)p + byte_off);
}

// Native vectors for __builtin_nontemporal_store (HIP's uint2 / float4 are
// structs, which the builtin does not take).
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
typedef float nt_f32x4 __attribute__((ext_vector_type(4)));

// Streaming accesses of the fast block path and the stream probe (16-bit
// params and grads, codes): nontemporal loads and stores, every byte being
// touched once per step.  On a stream kernel with the step's byte mix and
// lane layout they moved 2.3 % more bytes per second than plain accesses
// (nontemporal loads alone or stores alone gained nothing or lost).
__device__ __forceinline__ uint4 ld_nt(const RF_GLOBAL uint4* p)
{
    const nt_u32x4 v = __builtin_nontemporal_load((const RF_GLOBAL nt_u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint2 ld_nt(const RF_GLOBAL uint2* p)
{
    const nt_u32x2 v = __builtin_nontemporal_load((const RF_GLOBAL nt_u32x2*)p);
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ void st_nt(RF_GLOBAL uint4* p, uint4 v)
{
    __builtin_nontemporal_store(nt_u32x4{v.x, v.y, v.z, v.w}, (RF_GLOBAL nt_u32x4*)p);
}

__device__ __forceinline__ void st_nt(RF_GLOBAL uint2* p, uint2 v)
{
    __builtin_nontemporal_store(nt_u32x2{v.x, v.y}, (RF_GLOBAL nt_u32x2*)p);
}

__device__ __forceinline__ void st_nt(RF_GLOBAL float4* p, float4 v)
{
    __builtin_nontemporal_store(nt_f32x4{v.x, v.y, v.z, v.w}, (RF_GLOBAL nt_f32x4*)p);
}


// A nontemporal 16-byte load through a generic pointer (the standalone
// stochastic rounding's input).  Plain accesses stay in the vector I/O
// helpers below: with them nontemporal, MultiSteps' accumulation over the
// Llama-7B tree ran 1.9x slower, and the other element-wise steps moved by
// less than their run-to-run spread.
__device__ __forceinline__ uint4 ldg_nt(const void* p)
{
    const nt_u32x4 v = __builtin_nontemporal_load((const nt_u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Element i of a T array, read or written through its global view.
template <typename T>
__device__ __forceinline__ T gld(const void* p, int64_t i)
{
    return ((const RF_GLOBAL T*)p)[i];
}

template <typename T>
__device__ __forceinline__ void gst(void* p, int64_t i, T v)
{
    ((RF_GLOBAL T*)p)[i] = v;
}

// ----------------------------------------------------------- vector I/O --
// These keep generic pointers: through the global views above the generic
// kernel's full-chunk fallback unit took 147 VGPRs instead of 128 (3 waves
// per SIMD instead of 4), and the full-precision AdamW step over the
// Llama-7B tree ran 2-4 % slower.
// Load 8 consecutive elements (16-byte aligned) as f32.
template <typename T>
__device__ __forceinline__ void load8(const void* base, int64_t e0, float (&x)[8])
{
    if constexpr (IS_BF16<T>) {
        const uint4 w = *(const uint4*)((const uint16_t*)base + e0);
        const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = __uint_as_float(d[i] << 16);
            x[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
        }
    } else if constexpr (IS_F16<T>) {
        const uint4 w = *(const uint4*)((const uint16_t*)base + e0);
        const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = f16_bits_to_f32(d[i] & 0xFFFFu);
            x[2 * i + 1] = f16_bits_to_f32(d[i] >> 16);
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

// 8 consecutive 16-bit patterns (bf16 or f16), 16-byte aligned.
// 8 bf16 / f16 values from words holding them in their high halves.
__device__ __forceinline__ void store8_hi16(void* base, int64_t e0, const uint32_t (&h)[8])
{
    uint4 w;
    w.x = pack_hi16x2(h[0], h[1]);
    w.y = pack_hi16x2(h[2], h[3]);
    w.z = pack_hi16x2(h[4], h[5]);
    w.w = pack_hi16x2(h[6], h[7]);
    *(uint4*)((uint16_t*)base + e0) = w;
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
    if (dtype == RF_BF16) return bf16_bits_to_f32(gld<uint16_t>(base, e));
    if (dtype == RF_F16) return f16_bits_to_f32(gld<uint16_t>(base, e));
    return gld<float>(base, e);
}

// x rounded to nearest even in a 16-bit dtype, or as is.
__device__ __forceinline__ void store1(void* base, int32_t dtype, int64_t e, float x)
{
    if (dtype == RF_BF16) gst<uint16_t>(base, e, (uint16_t)f32_to_bf16_rne(x));
    else if (dtype == RF_F16) gst<uint16_t>(base, e, (uint16_t)f32_to_f16_rne(x));
    else gst<float>(base, e, x);
}

// Round x to a param/grad dtype and back (nearest even).
__device__ __forceinline__ float round_to_dtype(float x, int32_t dtype)
{
    if (dtype == RF_BF16) return round_to_bf16(x);
    if (dtype == RF_F16) return round_to_f16(x);
    return x;
}

// Block scales stored as f32, bf16 or f16 (RF_LEAF_SCALE_* flags of the leaf):
// quantize_blocks computes the scale in f32, codes with it, and stores it as
// scales.astype(scale_dtype); dequantize_blocks reads f32(stored)
// (adam8.py:167-186, :202).
__device__ __forceinline__ float load_scale(const float* scales, uint32_t leaf_flags, int64_t b)
{
    if (leaf_flags & RF_LEAF_SCALE_BF16) return bf16_bits_to_f32(gld<uint16_t>(scales, b));
    if (leaf_flags & RF_LEAF_SCALE_F16) return f16_bits_to_f32(gld<uint16_t>(scales, b));
    return gld<float>(scales, b);
}

__device__ __forceinline__ void store_scale(float* scales, uint32_t leaf_flags, int64_t b, float s)
{
    if (leaf_flags & RF_LEAF_SCALE_BF16) gst<uint16_t>(scales, b, (uint16_t)f32_to_bf16_rne(s));
    else if (leaf_flags & RF_LEAF_SCALE_F16) gst<uint16_t>(scales, b, (uint16_t)f32_to_f16_rne(s));
    else gst<float>(scales, b, s);
}

// Uniform per-unit context.
struct UnitCtx {
    const uint8_t* lds;
    float* wtab;  // this wave's 512-float LDS region (dequant-and-decay tables)
    float* xbuf;  // update-only fast kernel: this wave's 512-float LDS region for the update stores
    int32_t wd_mode;
    bool fed;
    bool packed;      // RF_PACKED_BITS without fed bits
    bool zero;        // RF_LEAF_ZERO_DECAY of the current leaf (unquantized-moment units)
    bool clip;        // grads are scaled by the global-norm clipping factor
    float cs, cs16, csh;  // that factor as f32, rounded to bf16 and rounded to f16
    uint32_t kmu0, kmu1, knu0, knu1, kp0, kp1;  // per-leaf keys
    double* mpart;    // Magma partial sums (KHp::mpart) or null
    int64_t mbase;    // the current leaf's first chunk slot in mpart
};

// One lane's share of a unit's Magma sums (optim/magma.py:98-106: vdot of
// the raw update with the new first moment, and the two squared norms),
// accumulated in f64 from the f32 values the step computes.
struct MagmaAcc {
    double dot = 0.0, gg = 0.0, mm = 0.0;
    __device__ __forceinline__ void add(float g, float m)
    {
        const double gd = g, md = m;
        dot += gd * md;
        gg += gd * gd;
        mm += md * md;
    }
    // Wave sums stored as the unit's partial triple (every lane calls it).
    __device__ __forceinline__ void store(const UnitCtx& c, int64_t chunk)
    {
        const double a = wave_sum_f64(dot), b = wave_sum_f64(gg), d = wave_sum_f64(mm);
        if ((threadIdx.x & (WAVE - 1)) == 0) {
            double* out = c.mpart + 3 * (c.mbase + chunk);
            out[0] = a;
            out[1] = b;
            out[2] = d;
        }
    }
};

// Global-norm clipping of one gradient element (finetune/transforms.py:79-82,
// leaf * scale.astype(leaf.dtype)): f32 grads multiply in f32; bf16 (f16)
// grads by the bf16- (f16-) rounded factor, the exact product rounded once
// to the grad dtype.
__device__ __forceinline__ float clip1(const UnitCtx& c, float g, int32_t dtype)
{
    if (dtype == RF_BF16) return round_to_bf16(g * c.cs16);
    if (dtype == RF_F16) return round_to_f16(g * c.csh);
    return g * c.cs;
}

template <typename GT>
__device__ __forceinline__ void clip8(const UnitCtx& c, float (&g)[8])
{
    if (!c.clip) return;
    if constexpr (IS_BF16<GT>) {
#pragma unroll
        for (int t = 0; t < 8; t += 2) {
            const uint32_t w2 = pack_bf16x2_rne(g[t] * c.cs16, g[t + 1] * c.cs16);
            g[t] = __uint_as_float(w2 << 16);
            g[t + 1] = __uint_as_float(w2 & 0xFFFF0000u);
        }
    } else if constexpr (IS_F16<GT>) {
#pragma unroll
        for (int t = 0; t < 8; ++t) g[t] = round_to_f16(g[t] * c.csh);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) g[t] = g[t] * c.cs;
    }
}

// Clipped gradient element of the generic paths (runtime dtype).
__device__ __forceinline__ float load_grad1(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e)
{
    const float g = load1(L.grad, L.grad_dtype, e);
    return c.clip ? clip1(c, g, L.grad_dtype) : g;
}

// Kernel-start setup of the clipping factor (one scalar load per wave).
__device__ __forceinline__ void clip_context(UnitCtx& c, const KHp& h)
{
    c.clip = h.clip != nullptr;
    c.cs = 1.0f;
    c.cs16 = 1.0f;
    c.csh = 1.0f;
    if (c.clip) {
        c.cs = gld<float>(h.clip, 0);
        c.cs16 = round_to_bf16(c.cs);
        c.csh = round_to_f16(c.cs);
    }
}

// Random bits of the stochastic roundings, from the launch's source: fed
// arrays, the packed stream, or jax.random.bits of the leaf keys.
__device__ __forceinline__ uint32_t param_bits1(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e)
{
    if (c.fed) return gld<uint32_t>(L.param_bits, e);
    if (c.packed) return packed_param_bits1(c.kp0, c.kp1, (uint64_t)e);
    return jax_bits(c.kp0, c.kp1, (uint64_t)e);
}

// Eight consecutive param elements from e0, a multiple of 4.
__device__ __forceinline__ void param_bits8(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e0, uint32_t (&rb)[8])
{
    if (c.fed) {
        load8_u32(L.param_bits, e0, rb);
    } else if (c.packed) {
        packed_param_bits4(c.kp0, c.kp1, (uint64_t)e0, rb);
        packed_param_bits4(c.kp0, c.kp1, (uint64_t)e0 + 4, rb + 4);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) rb[t] = jax_bits(c.kp0, c.kp1, (uint64_t)(e0 + t));
    }
}

// Both moments' bf16 storage-rounding bits of element e (RF_LEAF_STORE_SR;
// the rounding reads the low 16 bits): fed, the packed source's main halves,
// or jax.random.bits of the moment keys.
__device__ __forceinline__ void moment_bits1(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e, uint32_t& bm,
                                             uint32_t& bv)
{
    if (c.fed) {
        bm = gld<uint32_t>(L.mu_bits, e);
        bv = gld<uint32_t>(L.nu_bits, e);
    } else if (c.packed) {
        uint32_t y0, y1;
        packed_moment_block(c.kmu0, c.kmu1, (uint64_t)e, false, y0, y1);
        bm = half16(y0, (uint64_t)e);
        bv = half16(y1, (uint64_t)e);
    } else {
        bm = jax_bits(c.kmu0, c.kmu1, (uint64_t)e);
        bv = jax_bits(c.knu0, c.knu1, (uint64_t)e);
    }
}

// The packed source's whole code draw of element e (packed_moment_block):
// (main << 16) | fill from y0 (first moment) or y1 (second moment).
template <bool SECOND>
__device__ __forceinline__ uint32_t packed_code_word(const UnitCtx& c, int64_t e)
{
    uint32_t y0, y1, z0, z1;
    packed_moment_block(c.kmu0, c.kmu1, (uint64_t)e, false, y0, y1);
    packed_moment_block(c.kmu0, c.kmu1, (uint64_t)e, true, z0, z1);
    return SECOND ? (half16(y1, (uint64_t)e) << 16) | half16(z1, (uint64_t)e)
                  : (half16(y0, (uint64_t)e) << 16) | half16(z0, (uint64_t)e);
}

// One moment's code-draw bits of element e (quantized: of the padded code
// arrays; the literal paths code the moments apart).
__device__ __forceinline__ uint32_t mu_bits1(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e)
{
    if (c.fed) return gld<uint32_t>(L.mu_bits, e);
    if (c.packed) return packed_code_word<false>(c, e);
    return jax_bits(c.kmu0, c.kmu1, (uint64_t)e);
}

__device__ __forceinline__ uint32_t nu_bits1(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e)
{
    if (c.fed) return gld<uint32_t>(L.nu_bits, e);
    if (c.packed) return packed_code_word<true>(c, e);
    return jax_bits(c.knu0, c.knu1, (uint64_t)e);
}

// The param after the update (fused) for one element.
template <bool PSR, typename PT>
__device__ __forceinline__ uint32_t new_param_bits(float p, float u, uint32_t rbits)
{
    const float s = p + u;
    if constexpr (IS_BF16<PT>) {
        if constexpr (PSR) return sr_bf16(s, rbits);
        else return f32_to_bf16_rne(s);
    } else if constexpr (IS_F16<PT>) {
        (void)rbits;  // apply_updates rounds non-bf16 params to nearest (utils.py:700)
        return f32_to_f16_rne(s);
    } else {
        (void)rbits;
        return __float_as_uint(s);
    }
}

// One element of the update for the generic (scalar) paths: writes the new
// param (fused) or the f32 update.
// `p` is the element's param, already loaded where APPLY or decay needs it
// (0 otherwise).
template <bool APPLY, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void update_one(const UnitCtx& c, const rf_adam8_leaf& L, int64_t e, const KHp& h,
                                           float mm, float vv, float g, float p)
{
    float u = adam_direction<NEST, EXACT>(h, mm, vv, g);
    u = decay_and_scale(h, u, p, c.wd_mode, c.zero);
    if constexpr (APPLY && !EXACT) {
        if (cancels(p + u, u))
            u = decay_and_scale(h, adam_direction<NEST, true>(h, mm, vv, g), p, c.wd_mode, c.zero);
    }
    if constexpr (APPLY) {
        if (L.param_dtype == RF_BF16) {
            uint32_t rb = 0;
            if constexpr (PSR) rb = param_bits1(c, L, e);
            gst<uint16_t>(L.param, e, (uint16_t)new_param_bits<PSR, uint16_t>(p, u, rb));
        } else if (L.param_dtype == RF_F16) {
            gst<uint16_t>(L.param, e, (uint16_t)f32_to_f16_rne(p + u));
        } else {
            gst<float>(L.param, e, p + u);
        }
    } else {
        gst<float>(L.updates, e, u);
    }
}

// Element-wise units take each lane's elements EW_BATCH at a time and issue
// all of a batch's loads before its arithmetic: one memory round trip per
// batch instead of one per element.
constexpr int EW_BATCH = 4;

// Old codes and grads of lane elements j0 + k*WAVE (k < B) of the block at
// `base`; elements at or past nvalid read as code 0 and grad 0.
template <int B>
__device__ __forceinline__ void load_batch(const UnitCtx& c, const rf_adam8_leaf& L, int64_t base, int64_t j0,
                                           int64_t nvalid, uint32_t (&cm)[B], uint32_t (&cv)[B], float (&g)[B])
{
#pragma unroll
    for (int k = 0; k < B; ++k) {
        const int64_t j = j0 + k * WAVE;
        cm[k] = cv[k] = 0u;
        g[k] = 0.0f;
        if (j < nvalid) {
            cm[k] = gld<uint8_t>(L.mu, base + j);
            cv[k] = gld<uint8_t>(L.nu, base + j);
            g[k] = load_grad1(c, L, base + j);
        }
    }
}

// A batch of B lane elements of a quantized block: old codes, grads and (the
// update pass) params.
template <int B>
struct QBatch {
    uint32_t cm[B], cv[B];
    float g[B], p[B];
};

// The coding pass of a partial or odd-sized block (the generic kernel), over
// the wave's elements [lo, hi) of the block: with the block's new absmax
// bits (am, av), every element, the padding past the leaf's end as zero
// (adam8.py:137-141), is coded from its moments, recomputed from the old
// codes and scales, which are still in place; the new scales are written
// where `scales` is set (one wave of the block).  The next batch's loads are
// issued before this batch's arithmetic and stores, so a batch does not wait
// for the previous batch's stores.
template <bool MSR, int B>
__device__ __forceinline__ void literal_code(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h,
                                             float sm_old, float sv_old, uint32_t am, uint32_t av, int64_t lo,
                                             int64_t hi, bool scales)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t bs = L.block_size;
    const int64_t base = blk * bs;
    const int64_t nvalid = max((int64_t)0, min(bs, L.size - base));
    const float* cbs = (const float*)(c.lds + L_CBS);
    const float* cbu = (const float*)(c.lds + L_CBU);
    const float sm = scale_from_absmax_bits(am);
    const float sv = scale_from_absmax_bits(av);
    const bool fast_m = !MSR && block_is_fast(am, sm);
    const bool fast_v = !MSR && block_is_fast(av, sv);
    const float rsm = 1.0f / sm;
    const float rsv = 1.0f / sv;
    const int64_t nb = (hi - lo + B * WAVE - 1) / (B * WAVE);
    QBatch<B> cur{}, nxt{};
    if (nb > 0) load_batch<B>(c, L, base, lo + lane, nvalid, cur.cm, cur.cv, cur.g);
    for (int64_t i = 0; i < nb; ++i) {
        const int64_t j0 = lo + lane + i * (B * WAVE);
        if (i + 1 < nb) load_batch<B>(c, L, base, j0 + B * WAVE, nvalid, nxt.cm, nxt.cv, nxt.g);
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int64_t j = j0 + k * WAVE;
            if (j >= hi) continue;
            const int64_t e = base + j;
            float mm = 0.0f, vv = 0.0f;  // zero padding past the leaf's end
            if (j < nvalid) ema(h, cbs[cur.cm[k]] * sm_old, cbu[cur.cv[k]] * sv_old, cur.g[k], mm, vv);
            uint32_t cm, cv;
            if (fast_m) {
                cm = code_signed_fast(c.lds, mm, sm, rsm);
            } else {
                uint32_t bits = 0;
                if constexpr (MSR) bits = mu_bits1(c, L, e);
                cm = code_literal(cbs, mm, sm, MSR, bits);
            }
            if (fast_v) {
                cv = code_unsigned_fast(c.lds, vv, sv, rsv);
            } else {
                uint32_t bits = 0;
                if constexpr (MSR) bits = nu_bits1(c, L, e);
                cv = code_literal(cbu, vv, sv, MSR, bits);
            }
            gst<uint8_t>(L.mu, e, (uint8_t)cm);
            gst<uint8_t>(L.nu, e, (uint8_t)cv);
        }
        cur = nxt;
    }
    if (scales && lane == 0) {
        store_scale(L.mu_scales, L.flags, blk, sm);
        store_scale(L.nu_scales, L.flags, blk, sv);
    }
}

// Requantization of one block by the literal search (or moment SR): the new
// moments are recomputed from the old codes and scales, which are still in
// place, with the reference's NaN-propagating absmax (adam8.py:142), then
// every element is coded and the new scales are written.  Used inside the
// fast kernel for blocks whose scale leaves the fast range (zero-free tiny,
// Inf, NaN), with nearest or stochastic rounding.  B: elements per lane per
// batch (1 there, where this path is rare and registers are scarce).
template <bool MSR, int B = EW_BATCH>
__device__ __forceinline__ void requant_literal(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t bs = L.block_size;
    const int64_t base = blk * bs;
    const int64_t nvalid = max((int64_t)0, min(bs, L.size - base));
    const float* cbs = (const float*)(c.lds + L_CBS);
    const float* cbu = (const float*)(c.lds + L_CBU);
    const float sm_old = load_scale(L.mu_scales, L.flags, blk);
    const float sv_old = load_scale(L.nu_scales, L.flags, blk);
    uint32_t am = 0, av = 0;
    for (int64_t j0 = lane; j0 < nvalid; j0 += B * WAVE) {
        uint32_t cm[B], cv[B];
        float g[B];
        load_batch<B>(c, L, base, j0, nvalid, cm, cv, g);
#pragma unroll
        for (int k = 0; k < B; ++k) {
            if (j0 + k * WAVE < nvalid) {
                float mm, vv;
                ema(h, cbs[cm[k]] * sm_old, cbu[cv[k]] * sv_old, g[k], mm, vv);
                am = max(am, __float_as_uint(mm) & 0x7FFFFFFFu);
                av = max(av, __float_as_uint(vv));
            }
        }
    }
    am = wave_max_u32(am);
    av = wave_max_u32(av);
    const float sm = scale_from_absmax_bits(am);
    const float sv = scale_from_absmax_bits(av);
    const bool fast_m = !MSR && block_is_fast(am, sm);
    const bool fast_v = !MSR && block_is_fast(av, sv);
    const float rsm = 1.0f / sm;
    const float rsv = 1.0f / sv;
    for (int64_t j0 = lane; j0 < bs; j0 += B * WAVE) {
        uint32_t om[B], ov[B];
        float g[B];
        load_batch<B>(c, L, base, j0, nvalid, om, ov, g);
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int64_t j = j0 + k * WAVE;
            if (j >= bs) continue;
            const int64_t e = base + j;
            float mm = 0.0f, vv = 0.0f;  // zero padding past the leaf's end
            if (j < nvalid) ema(h, cbs[om[k]] * sm_old, cbu[ov[k]] * sv_old, g[k], mm, vv);
            uint32_t cm, cv;
            if (fast_m) {
                cm = code_signed_fast(c.lds, mm, sm, rsm);
            } else {
                uint32_t bits = 0;
                if constexpr (MSR) bits = mu_bits1(c, L, e);
                cm = code_literal(cbs, mm, sm, MSR, bits);
            }
            if (fast_v) {
                cv = code_unsigned_fast(c.lds, vv, sv, rsv);
            } else {
                uint32_t bits = 0;
                if constexpr (MSR) bits = nu_bits1(c, L, e);
                cv = code_literal(cbu, vv, sv, MSR, bits);
            }
            gst<uint8_t>(L.mu, e, (uint8_t)cm);
            gst<uint8_t>(L.nu, e, (uint8_t)cv);
        }
    }
    if (lane == 0) {
        store_scale(L.mu_scales, L.flags, blk, sm);
        store_scale(L.nu_scales, L.flags, blk, sv);
    }
}

// ================================================ work units: quantized ====

// 8 consecutive elements of a param/grad array in registers (16-byte words).
template <typename T>
struct Raw8 {
    uint4 w[sizeof(T) == 2 ? 1 : 2];
};

template <typename T>
__device__ __forceinline__ void raw8_load(Raw8<T>& r, const void* base, int64_t e0)
{
    const RF_GLOBAL uint4* p = gload_ptr<uint4>(base, e0 * (int64_t)sizeof(T));
    r.w[0] = p[0];
    if constexpr (sizeof(T) == 4) r.w[1] = p[1];
}

template <typename T>
__device__ __forceinline__ void raw8_unpack(const Raw8<T>& r, float (&x)[8])
{
    if constexpr (IS_BF16<T>) {
        const uint32_t d[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = __uint_as_float(d[i] << 16);
            x[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
        }
    } else if constexpr (IS_F16<T>) {
        const uint32_t d[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = f16_bits_to_f32(d[i] & 0xFFFFu);
            x[2 * i + 1] = f16_bits_to_f32(d[i] >> 16);
        }
    } else {
        const uint32_t d[8] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w, r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = __uint_as_float(d[i]);
    }
}


template <int WDM>
__device__ __forceinline__ void decay_and_scale8(const KHp& h, float (&u)[8], const float (&p)[8])
{
    if constexpr (WDM == WD_BF16) {
        // bf16(wd*p) as an f32 in one conversion: the pair (0, wd*p) packed
        // puts bf16(0) = 0 in the low half
#pragma unroll
        for (int t = 0; t < 8; ++t) u[t] = u[t] + __uint_as_float(pack_bf16x2_rne(0.0f, h.wd16 * p[t]));
    } else if constexpr (WDM == WD_F16) {
#pragma unroll
        for (int t = 0; t < 8; ++t) u[t] = u[t] + round_to_f16(h.wdh * p[t]);
    } else if constexpr (WDM == WD_F32) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float wdp = h.wd * p[t];
            u[t] = u[t] + wdp;
        }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) u[t] = h.neg_lr * u[t];  // scale_by_learning_rate
}

// Full 2048-element block, vectorised (KIND_QFAST).  WDM (weight-decay mode)
// is a template parameter so the per-element code has no branches.
//
// Per block the wave first tabulates, in its own LDS region, the decayed
// dequantized value of every code: TM[k] = fl(b1 * fl(cb_s[k] * s_m)) and
// TV[k] = fl(b2 * fl(cb_u[k] * s_v)) -- exactly the first product of each
// EMA (adam8.py:200-203, :322-335) -- so an element costs one table read per
// moment instead of a read and two multiplies.
// Registers of two in-flight 512-element chunks (codes, grads, params).
template <typename PT, typename GT>
struct ChunkSlots {
    uint2 mc[2], vc[2];
    Raw8<GT> graw[2];
    Raw8<PT> praw[2];
};

// Issue the loads of chunk j of block blk of leaf L into slot `slot`.
template <typename PT, typename GT, bool NEED_P>
__device__ __forceinline__ void issue_chunk(ChunkSlots<PT, GT>& sl, const rf_adam8_leaf& L, int64_t blk, int j,
                                            int slot)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t base = blk * FAST_BS;
    // Per-block uniform base pointers (SGPRs) + 32-bit lane offsets: the
    // global accesses need no 64-bit address arithmetic per lane.
    const RF_GLOBAL uint8_t* gB = (const RF_GLOBAL uint8_t*)L.grad + base * (int64_t)sizeof(GT);
    const RF_GLOBAL uint8_t* pB = (const RF_GLOBAL uint8_t*)L.param + base * (int64_t)sizeof(PT);
    const RF_GLOBAL uint8_t* mB = (const RF_GLOBAL uint8_t*)L.mu + base;
    const RF_GLOBAL uint8_t* vB = (const RF_GLOBAL uint8_t*)L.nu + base;
    const uint32_t eo = (uint32_t)(j * 512 + lane * 8);
    // 16-bit grads and params: one nontemporal 16-byte access per lane, a
    // wave covering whole cache lines.  f32 ones take two plain accesses
    // (each nontemporal instruction would cover half of every line it
    // touches; streams of those ran slower than plain, up to 1.9x).
    sl.mc[slot] = ld_nt((const RF_GLOBAL uint2*)(mB + eo));
    sl.vc[slot] = ld_nt((const RF_GLOBAL uint2*)(vB + eo));
    if constexpr (sizeof(GT) == 2) {
        sl.graw[slot].w[0] = ld_nt((const RF_GLOBAL uint4*)(gB + eo * 2));
    } else {
        sl.graw[slot].w[0] = *(const RF_GLOBAL uint4*)(gB + eo * 4);
        sl.graw[slot].w[1] = *(const RF_GLOBAL uint4*)(gB + eo * 4 + 16);
    }
    if constexpr (NEED_P) {
        if constexpr (sizeof(PT) == 2) {
            sl.praw[slot].w[0] = ld_nt((const RF_GLOBAL uint4*)(pB + eo * 2));
        } else {
            sl.praw[slot].w[0] = *(const RF_GLOBAL uint4*)(pB + eo * 4);
            sl.praw[slot].w[1] = *(const RF_GLOBAL uint4*)(pB + eo * 4 + 16);
        }
    }
}

// `have0`: slot 0 already holds chunk 0 of this block (prefetched by the
// previous unit).  `next_blk` >= 0: the wave's next unit is that block of
// the same leaf; its chunk 0 is loaded into slot 0 while this block is
// requantized, so the wave keeps memory traffic in flight through the
// arithmetic-only requantization phase.
// A lane's eight consecutive f32 values (chunk elements 8l .. 8l + 7) stored
// on whole cache lines: they pass through the wave's 512-float LDS region
// `xb`, and lane l stores elements 4l .. 4l + 3 and 256 + 4l .. 256 + 4l + 3
// of the 512-element chunk at `chunk` (eight consecutive f32 per lane would
// put each 16-byte store on half of every line it touches); nontemporal if
// `nt`.
__device__ __forceinline__ void store8_f32_lines(float* xb, RF_GLOBAL float4* chunk, int lane, const float (&x)[8],
                                                 bool nt)
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    *(float4*)(xb + lane * 8) = make_float4(x[0], x[1], x[2], x[3]);
    *(float4*)(xb + lane * 8 + 4) = make_float4(x[4], x[5], x[6], x[7]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float4 a = *(const float4*)(xb + lane * 4);
    const float4 b = *(const float4*)(xb + 256 + lane * 4);
    if (nt) {
        st_nt(chunk + lane, a);
        st_nt(chunk + 64 + lane, b);
    } else {
        chunk[lane] = a;
        chunk[64 + lane] = b;
    }
}

template <typename PT, typename GT, int WDM, bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT, bool ER,
          bool FLR = false>
__device__ __forceinline__ void unit_qfast(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h,
                                           ChunkSlots<PT, GT>& sl, bool have0, int64_t next_blk)
{
    static_assert(!FLR || (APPLY && IS_BF16<PT> && !NEST && !EXACT && !ER && (WDM == WD_BF16 || WDM == WD_OFF)),
                  "the learning-rate-folded step covers fused bf16 nearest or SR steps of the hardware direction");
    constexpr int J = FAST_BS / 512;
    constexpr bool NEED_P = APPLY || WDM != WD_OFF;
    constexpr bool H16P = sizeof(PT) == 2;  // bf16 or f16 params
    // Exact mode, fused, bf16 params rounded to nearest even, no Nesterov:
    // the hardware direction, with the IEEE one only where it could change
    // the rounded param (rne_bf16_settled).
    constexpr bool SETTLE = EXACT && APPLY && IS_BF16<PT> && !PSR && !NEST;
    constexpr bool IEEE_DIR = EXACT && !SETTLE;
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t base = blk * FAST_BS;
    const float sm_old = load_scale(L.mu_scales, L.flags, blk);
    const float sv_old = load_scale(L.nu_scales, L.flags, blk);
    RF_GLOBAL uint8_t* pB = (RF_GLOBAL uint8_t*)L.param + base * (int64_t)sizeof(PT);

    // Chunk j+1's loads are issued before chunk j's arithmetic: two chunks
    // (6 KB for bf16) in flight per wave without holding all four.
    if (!have0) issue_chunk<PT, GT, NEED_P>(sl, L, blk, 0, 0);

    {
        const float* cbs = (const float*)(c.lds + L_CBS);
        const float* cbu = (const float*)(c.lds + L_CBU);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int k = lane + 64 * r;
            c.wtab[k] = h.b1 * (cbs[k] * sm_old);
            c.wtab[256 + k] = h.b2 * (cbu[k] * sv_old);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    const float* TM = c.wtab;
    const float* TV = c.wtab + 256;

    float m[J][8], v[J][8];
    float amf = 0.0f;            // max |m| (v_max3 with |x| modifiers); with finite inputs no NaN can occur
    uint32_t av = 0;             // v >= 0: integer max of the bits, NaN-propagating
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t e0 = base + j * 512 + lane * 8;
        const uint32_t eo = (uint32_t)(j * 512 + lane * 8);
        const int slot = j & 1;
        if (j + 1 < J) issue_chunk<PT, GT, NEED_P>(sl, L, blk, j + 1, slot ^ 1);
        else if (next_blk >= 0) issue_chunk<PT, GT, NEED_P>(sl, L, next_blk, 0, 0);  // slot 0 is free
        float g[8], p[8];
        raw8_unpack<GT>(sl.graw[slot], g);
        clip8<GT>(c, g);
        if constexpr (NEED_P) {
            raw8_unpack<PT>(sl.praw[slot], p);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) p[t] = 0.0f;
        }
        float u[8], sum[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t cm = ((t < 4 ? sl.mc[slot].x : sl.mc[slot].y) >> (8 * (t & 3))) & 0xFFu;
            const uint32_t cv = ((t < 4 ? sl.vc[slot].x : sl.vc[slot].y) >> (8 * (t & 3))) & 0xFFu;
            const float t2 = h.omb1 * g[t];
            const float mm = TM[cm] + t2;
            const float gg = g[t] * g[t];
            const float t4 = h.omb2 * gg;
            const float vv = TV[cv] + t4;
            m[j][t] = mm;
            v[j][t] = vv;
            amf = fmaxf(amf, fabsf(mm));
            av = max(av, __float_as_uint(vv));
            if constexpr (FLR) {
                const float rr = __builtin_amdgcn_rcpf(__builtin_fmaf(__builtin_amdgcn_sqrtf(vv), h.k1l, h.k2l));
                const float pd = WDM == WD_BF16 ? __builtin_fmaf(h.wdl, p[t], p[t]) : p[t];
                sum[t] = __builtin_fmaf(mm, rr, pd);
            } else {
                u[t] = adam_direction<NEST, IEEE_DIR, ER>(h, mm, vv, g[t]);
            }
        }
        if constexpr (!FLR) decay_and_scale8<WDM>(h, u, p);
        if constexpr (FLR) {
            // |p| > FLR_CANCEL |s|: the sum nearly cancels the param, where
            // the folded form's few-ulp error could exceed half a bf16 ulp of
            // s; those elements take the IEEE direction and the reference's
            // operation order.  fma(-C, |s|, |p|) > 0 is that test exactly
            // (NaN never passes), its maximum over the chunk one compare.
            float dmax = __builtin_fmaf(-FLR_CANCEL, fabsf(sum[0]), fabsf(p[0]));
#pragma unroll
            for (int t = 1; t < 8; ++t) dmax = fmaxf(dmax, __builtin_fmaf(-FLR_CANCEL, fabsf(sum[t]), fabsf(p[t])));
            if (__builtin_amdgcn_ballot_w64(dmax > 0.0f) != 0) {
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    if (__builtin_fmaf(-FLR_CANCEL, fabsf(sum[t]), fabsf(p[t])) > 0.0f) {
                        float ue = adam_direction<NEST, true>(h, m[j][t], v[j][t], g[t]);
                        ue = decay_and_scale(h, ue, p[t], WDM);
                        sum[t] = p[t] + ue;
                    }
                }
            }
        }
        if constexpr (APPLY) {
            if constexpr (!FLR) {
#pragma unroll
                for (int t = 0; t < 8; ++t) sum[t] = p[t] + u[t];
            }
            if constexpr (SETTLE) {
                const float wd_eff = WDM == WD_BF16 ? h.wd16 : (WDM == WD_F32 ? h.wd : (WDM == WD_F16 ? h.wdh : 0.0f));
                const float c_w = fabsf(h.neg_lr * wd_eff) * 0x1p-17f;
                const float c_g = fabsf(h.neg_lr) * 0x1p100f;
                uint32_t open = 0;  // bit t: element t's rounding is not settled
#pragma unroll
                for (int t = 0; t < 8; ++t) open |= rne_bf16_settled(sum[t], u[t], p[t], c_w, c_g) ? 0u : 1u << t;
                if (__builtin_amdgcn_ballot_w64(open != 0) != 0) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        if (open & (1u << t)) {
                            float ue = adam_direction<NEST, true>(h, m[j][t], v[j][t], g[t]);
                            ue = decay_and_scale(h, ue, p[t], WDM);
                            sum[t] = p[t] + ue;
                        }
                    }
                }
            }
            if constexpr (!EXACT && !FLR) {
                // Hardware rcp/sqrt leave u a few f32 ulps from the IEEE
                // value; that moves the rounded param by more than one
                // bf16 ulp only where p + u nearly cancels.  Such chunks
                // (rare) are recomputed with IEEE arithmetic.
                if (cancel_lanes8(sum, u) != 0) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        if (cancels(sum[t], u[t])) {
                            float ue = adam_direction<NEST, true>(h, m[j][t], v[j][t], g[t]);
                            ue = decay_and_scale(h, ue, p[t], WDM);
                            sum[t] = p[t] + ue;
                        }
                    }
                }
            }
            if constexpr (H16P) {
                uint32_t w[4];
                if constexpr (PSR && IS_BF16<PT>) {
                    // the rounding bits (fed, or jax.random.bits of the
                    // leaf's param key) drawn after the arithmetic: they are
                    // not live through it
                    uint32_t rb[8];
                    param_bits8(c, L, e0, rb);
#pragma unroll
                    for (int t = 0; t < 8; t += 2)
                        w[t / 2] = pack_hi16x2(sr_bf16_hi(sum[t], rb[t]), sr_bf16_hi(sum[t + 1], rb[t + 1]));
                } else {
#pragma unroll
                    for (int t = 0; t < 8; t += 2) w[t / 2] = pack_h16x2_rne<PT>(sum[t], sum[t + 1]);
                }
                st_nt((RF_GLOBAL uint4*)(pB + eo * 2), make_uint4(w[0], w[1], w[2], w[3]));
            } else {
                store8_f32_lines(c.xbuf, (RF_GLOBAL float4*)(pB + j * 512 * 4), lane, sum, h.upd_nt != 0);
            }
        } else {
            // f32 updates on whole cache lines, nontemporal in launches of
            // many blocks (h.upd_nt), where no cache keeps them for the
            // apply that reads them next
            store8_f32_lines(c.xbuf, gstore_ptr<float4>(L.updates, (base + j * 512) * 4), lane, u, h.upd_nt != 0);
        }
    }

    // Requantization (adam8.py:633-688 -> quantize_blocks).
    const uint32_t am = wave_max_u32(__float_as_uint(amf));  // amf >= 0: bit order = value order
    av = wave_max_u32(av);
    const float sm = scale_from_absmax_bits(am);
    const float sv = scale_from_absmax_bits(av);
    // Non-finite old scales can make m NaN, which fmaxf would drop: those
    // blocks and tiny or non-finite new scales go the literal way.
    const bool old_finite = (__float_as_uint(sm_old) & 0x7FFFFFFFu) < 0x7F800000u &&
                            (__float_as_uint(sv_old) & 0x7FFFFFFFu) < 0x7F800000u;
    if (old_finite && block_is_fast(am, sm) && block_is_fast(av, sv)) {
        const float rsm = 1.0f / sm;
        const float rsv = 1.0f / sv;
        RF_GLOBAL uint8_t* mW = (RF_GLOBAL uint8_t*)L.mu + base;
        RF_GLOBAL uint8_t* vW = (RF_GLOBAL uint8_t*)L.nu + base;
        if constexpr (MSR) {
            // Bernoulli rounding between the searchsorted neighbours
            // (adam8.py:549-564) with the random bits of the padded
            // [nblocks, bs] moment arrays: fed, the packed stream, or
            // jax.random.bits of the leaf keys.  With one stream per
            // moment, the first moment is coded over the whole block
            // before the second, so that only one moment's bits, quotients
            // and candidates are live beside the block's values, and the
            // first moment's registers are free for the second's pass.
            // Moment-SR launches stage the search image: the candidates are
            // searchsorted counts.
            const float* cbs = (const float*)(c.lds + L_CBS);
            const float* cbu = (const float*)(c.lds + L_CBU);
            const float4* srs = (const float4*)(c.lds + L_SRS);
            const float4* sru = (const float4*)(c.lds + L_SRU);
            if (c.packed) {
                // A main block per pair of elements feeds both moments; each
                // chunk is coded for both at once, four elements (two
                // blocks) at a time so that few words are live.  A batch
                // whose main halves leave a draw open computes its two fill
                // blocks and decides every draw on the whole word.
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint32_t eo = (uint32_t)(j * 512 + lane * 8);
                    const uint64_t e0 = (uint64_t)(base + eo);
                    uint32_t wm[2], wv[2];
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        uint32_t ym[2], yv[2], um[4], uv[4], cm[4], cv[4];
                        float nm[4], nv[4], pm[4], pv[4];
#pragma unroll
                        for (int pr = 0; pr < 2; ++pr)
                            packed_moment_block(c.kmu0, c.kmu1, e0 + 4 * hh + 2 * pr, false, ym[pr], yv[pr]);
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            nm[t] = div_by_scale(m[j][4 * hh + t], sm, rsm);
                            nv[t] = div_by_scale(v[j][4 * hh + t], sv, rsv);
                        }
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            um[t] = cand_signed(c.lds, nm[t]);
                            uv[t] = cand_unsigned(c.lds, nv[t]);
                        }
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            pm[t] = sr_upper(cbs, srs, um[t], nm[t]);
                            pv[t] = sr_upper(cbu, sru, uv[t], nv[t]);
                        }
                        uint64_t open = 0;
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            cm[t] = packed_sr_main(um[t], pm[t], half16(ym[t >> 1], t), open);
                            cv[t] = packed_sr_main(uv[t], pv[t], half16(yv[t >> 1], t), open);
                        }
                        // a wave with an open draw decides all of its
                        // lanes' draws on whole words (the same codes
                        // wherever the main half settled them)
                        if (__builtin_expect(open != 0, 0)) {
                            uint32_t zm[2], zv[2];
#pragma unroll
                            for (int pr = 0; pr < 2; ++pr)
                                packed_moment_block(c.kmu0, c.kmu1, e0 + 4 * hh + 2 * pr, true, zm[pr], zv[pr]);
#pragma unroll
                            for (int t = 0; t < 4; ++t) {
                                cm[t] = sr_decide(um[t], pm[t], (half16(ym[t >> 1], t) << 16) | half16(zm[t >> 1], t));
                                cv[t] = sr_decide(uv[t], pv[t], (half16(yv[t >> 1], t) << 16) | half16(zv[t >> 1], t));
                            }
                        }
                        wm[hh] = pack4_u8(cm[0], cm[1], cm[2], cm[3]);
                        wv[hh] = pack4_u8(cv[0], cv[1], cv[2], cv[3]);
                    }
                    st_nt((RF_GLOBAL uint2*)(mW + eo), make_uint2(wm[0], wm[1]));
                    st_nt((RF_GLOBAL uint2*)(vW + eo), make_uint2(wv[0], wv[1]));
                }
            } else {
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint32_t eo = (uint32_t)(j * 512 + lane * 8);
                    uint32_t b[8], cc[8];
                    float n[8];
                    if (c.fed) {
                        load8_u32(L.mu_bits, base + eo, b);
                    } else {
#pragma unroll
                        for (int t = 0; t < 8; ++t) b[t] = jax_bits(c.kmu0, c.kmu1, (uint64_t)(base + eo + t));
                    }
#pragma unroll
                    for (int t = 0; t < 8; ++t) n[t] = div_by_scale(m[j][t], sm, rsm);
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] = cand_signed(c.lds, n[t]);
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] = sr_code(cbs, srs, cc[t], n[t], b[t]);
                    uint2 w;
                    w.x = pack4_u8(cc[0], cc[1], cc[2], cc[3]);
                    w.y = pack4_u8(cc[4], cc[5], cc[6], cc[7]);
                    st_nt((RF_GLOBAL uint2*)(mW + eo), w);
                }
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint32_t eo = (uint32_t)(j * 512 + lane * 8);
                    uint32_t b[8], cc[8];
                    float n[8];
                    if (c.fed) {
                        load8_u32(L.nu_bits, base + eo, b);
                    } else {
#pragma unroll
                        for (int t = 0; t < 8; ++t) b[t] = jax_bits(c.knu0, c.knu1, (uint64_t)(base + eo + t));
                    }
#pragma unroll
                    for (int t = 0; t < 8; ++t) n[t] = div_by_scale(v[j][t], sv, rsv);
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] = cand_unsigned(c.lds, n[t]);
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] = sr_code(cbu, sru, cc[t], n[t], b[t]);
                    uint2 w;
                    w.x = pack4_u8(cc[0], cc[1], cc[2], cc[3]);
                    w.y = pack4_u8(cc[4], cc[5], cc[6], cc[7]);
                    st_nt((RF_GLOBAL uint2*)(vW + eo), w);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const uint32_t eo = (uint32_t)(j * 512 + lane * 8);
                // Batched phases (normalise + cell, candidate reads,
                // threshold reads) keep 16 independent LDS reads in flight
                // instead of 16 dependent read pairs.
                float nm[8], nv[8], tm[8], tv[8];
                uint32_t cm[8], cv[8];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    nm[t] = div_by_scale(m[j][t], sm, rsm);
                    nv[t] = div_by_scale(v[j][t], sv, rsv);
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    cm[t] = cand_signed(c.lds, nm[t]);
                    cv[t] = cand_unsigned(c.lds, nv[t]);
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    tm[t] = *(const float*)(c.lds + L_TS + cm[t] * 4u);
                    tv[t] = *(const float*)(c.lds + L_TU + cv[t] * 4u);
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    cm[t] += nm[t] >= tm[t] ? 1u : 0u;
                    cv[t] += nv[t] >= tv[t] ? 1u : 0u;
                }
                uint2 wm, wv;
                wm.x = pack4_u8(cm[0], cm[1], cm[2], cm[3]);
                wm.y = pack4_u8(cm[4], cm[5], cm[6], cm[7]);
                wv.x = pack4_u8(cv[0], cv[1], cv[2], cv[3]);
                wv.y = pack4_u8(cv[4], cv[5], cv[6], cv[7]);
                st_nt((RF_GLOBAL uint2*)(mW + eo), wm);
                st_nt((RF_GLOBAL uint2*)(vW + eo), wv);
            }
        }
        if (lane == 0) {
            store_scale(L.mu_scales, L.flags, blk, sm);
            store_scale(L.nu_scales, L.flags, blk, sv);
        }
    } else {
        requant_literal<MSR, 1>(c, L, blk, h);
    }
}

// The vectorised block: the weight-decay mode (and, for the hardware
// direction, whether eps_root is zero) is resolved once per unit into a
// branch-free instance.
template <typename PT, typename GT, bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT, bool ER>
__device__ __forceinline__ void dispatch_qfast_wd(const UnitCtx& c, const rf_adam8_leaf& L, int64_t idx, const KHp& h,
                                                  ChunkSlots<PT, GT>& sl, bool have0, int64_t next_blk)
{
    const int32_t wdm = c.wd_mode;
    if constexpr (APPLY && IS_BF16<PT> && !NEST && !EXACT && !ER) {
        if (h.flr) {
            if (wdm == WD_BF16) {
                unit_qfast<PT, GT, WD_BF16, APPLY, MSR, PSR, NEST, EXACT, ER, true>(c, L, idx, h, sl, have0, next_blk);
                return;
            }
            if (wdm == WD_OFF) {
                unit_qfast<PT, GT, WD_OFF, APPLY, MSR, PSR, NEST, EXACT, ER, true>(c, L, idx, h, sl, have0, next_blk);
                return;
            }
        }
    }
    if constexpr (IS_BF16<PT>) {
        if (wdm == WD_BF16) {
            unit_qfast<PT, GT, WD_BF16, APPLY, MSR, PSR, NEST, EXACT, ER>(c, L, idx, h, sl, have0, next_blk);
            return;
        }
    }
    if constexpr (IS_F16<PT>) {
        if (wdm == WD_F16) {
            unit_qfast<PT, GT, WD_F16, APPLY, MSR, PSR, NEST, EXACT, ER>(c, L, idx, h, sl, have0, next_blk);
            return;
        }
    }
    if (wdm != WD_OFF) unit_qfast<PT, GT, WD_F32, APPLY, MSR, PSR, NEST, EXACT, ER>(c, L, idx, h, sl, have0, next_blk);
    else unit_qfast<PT, GT, WD_OFF, APPLY, MSR, PSR, NEST, EXACT, ER>(c, L, idx, h, sl, have0, next_blk);
}

template <typename PT, typename GT, bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void dispatch_qfast(const UnitCtx& c, const rf_adam8_leaf& L, int64_t idx, const KHp& h,
                                               ChunkSlots<PT, GT>& sl, bool have0, int64_t next_blk)
{
    if constexpr (!EXACT) {
        if (h.er2 == 0.0f) {
            dispatch_qfast_wd<PT, GT, APPLY, MSR, PSR, NEST, EXACT, false>(c, L, idx, h, sl, have0, next_blk);
            return;
        }
    }
    dispatch_qfast_wd<PT, GT, APPLY, MSR, PSR, NEST, EXACT, true>(c, L, idx, h, sl, have0, next_blk);
}

// Any block size, partial or unaligned blocks (KIND_QGEN): an update pass
// writes the params/updates and takes the new moments' absmax, then the
// coding pass recomputes the moments from the old codes (still in place) and
// requantizes them.  Elements past `size` are the reference's zero padding.
//
// The update pass of a partial or odd-sized block over the wave's valid
// elements [lo, hi): params updated, and the absmax bits of the new moments
// (the NaN-propagating max of adam8.py:142) reduced over the wave.  The next
// batch's loads are in flight behind each batch.
template <bool APPLY, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void qgen_update(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h,
                                            float sm_old, float sv_old, int64_t lo, int64_t hi, uint32_t& am,
                                            uint32_t& av)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t base = blk * (int64_t)L.block_size;
    const float* cbs = (const float*)(c.lds + L_CBS);
    const float* cbu = (const float*)(c.lds + L_CBU);
    const bool need_p = APPLY || c.wd_mode != WD_OFF;
    constexpr int B = EW_BATCH;
    const int64_t nb = (hi - lo + B * WAVE - 1) / (B * WAVE);
    auto load = [&](int64_t j0, QBatch<B>& q) {
        load_batch<B>(c, L, base, j0, hi, q.cm, q.cv, q.g);
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int64_t j = j0 + k * WAVE;
            q.p[k] = (need_p && j < hi) ? load1(L.param, L.param_dtype, base + j) : 0.0f;
        }
    };
    am = 0;
    av = 0;
    QBatch<B> cur{}, nxt{};
    if (nb > 0) load(lo + lane, cur);
    for (int64_t i = 0; i < nb; ++i) {
        const int64_t j0 = lo + lane + i * (B * WAVE);
        if (i + 1 < nb) load(j0 + B * WAVE, nxt);
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int64_t j = j0 + k * WAVE;
            if (j < hi) {
                float mm, vv;
                ema(h, cbs[cur.cm[k]] * sm_old, cbu[cur.cv[k]] * sv_old, cur.g[k], mm, vv);
                am = max(am, __float_as_uint(mm) & 0x7FFFFFFFu);
                av = max(av, __float_as_uint(vv));
                update_one<APPLY, PSR, NEST, EXACT>(c, L, base + j, h, mm, vv, cur.g[k], cur.p[k]);
            }
        }
        cur = nxt;
    }
    am = wave_max_u32(am);
    av = wave_max_u32(av);
}

// A partial or odd-sized block (KIND_QGEN) by the workgroup's waves
// together: the update pass, which also takes the new moments' absmax, then
// the coding pass; wave w updates and codes its quarter of the block
// (rounded up to whole batches), the four waves' absmax bits meet in LDS.  Called by every wave of the workgroup
// (it holds two barriers); `red` is 8 words of LDS.
template <bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void unit_qgen_wg(const UnitCtx& c, const rf_adam8_leaf& L, int64_t blk, const KHp& h,
                                             uint32_t* red)
{
    constexpr int64_t BW = EW_BATCH * WAVE;
    const int lane = threadIdx.x & (WAVE - 1);
    const int w = (int)uniform_u32(threadIdx.x / WAVE);
    const int64_t bs = L.block_size;
    const int64_t nvalid = max((int64_t)0, min(bs, L.size - blk * bs));
    const int64_t quarter = ((bs + WAVES_PER_WG - 1) / WAVES_PER_WG + BW - 1) / BW * BW;
    const int64_t lo = min(bs, w * quarter), hi = min(bs, lo + quarter);
    const float sm_old = load_scale(L.mu_scales, L.flags, blk);
    const float sv_old = load_scale(L.nu_scales, L.flags, blk);
    uint32_t am, av;
    qgen_update<APPLY, PSR, NEST, EXACT>(c, L, blk, h, sm_old, sv_old, lo, min(hi, nvalid), am, av);
    if (lane == 0) {
        red[2 * w] = am;
        red[2 * w + 1] = av;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < WAVES_PER_WG; ++k) {
        am = max(am, red[2 * k]);
        av = max(av, red[2 * k + 1]);
    }
    __syncthreads();  // red is free for the workgroup's next block
    literal_code<MSR, EW_BATCH>(c, L, blk, h, sm_old, sv_old, am, av, lo, hi, w == 0);
}

// ============================================= work units: fallback ====
// Moments stored unquantized (adam8.py:620-630: size < min_size, a
// non-inexact dtype or quantize=False): elementwise update of elements
// [base, end).  Magma's partial sums (update-only launches, whose units are
// whole chunks) go to the slot of chunk base / CHUNK.
template <bool APPLY, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void unit_fallback(const UnitCtx& c, const rf_adam8_leaf& L, int64_t base, int64_t end,
                                              const KHp& h)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int32_t mdt = L.moment_kind == RF_MOMENT_BF16 ? RF_BF16 : (L.moment_kind == RF_MOMENT_F16 ? RF_F16 : RF_F32);
    const bool store_sr = mdt == RF_BF16 && (L.flags & RF_LEAF_STORE_SR);
    const bool need_p = APPLY || c.wd_mode != WD_OFF || c.zero;
    const bool msum = !APPLY && c.mpart != nullptr;  // Magma sums: update-only launches
    MagmaAcc acc;
    // Batches of EW_BATCH elements per lane, the next batch's loads in flight
    // behind each batch's arithmetic and stores.
    struct Batch {
        float g[EW_BATCH], mo[EW_BATCH], vo[EW_BATCH], p[EW_BATCH];
    };
    auto load = [&](int64_t e0, Batch& b) {
#pragma unroll
        for (int k = 0; k < EW_BATCH; ++k) {
            const int64_t e = e0 + k * WAVE;
            b.g[k] = b.mo[k] = b.vo[k] = b.p[k] = 0.0f;
            if (e < end) {
                b.g[k] = load_grad1(c, L, e);
                b.mo[k] = load1(L.mu, mdt, e);
                b.vo[k] = load1(L.nu, mdt, e);
                if (need_p) b.p[k] = load1(L.param, L.param_dtype, e);
            }
        }
    };
    const int64_t nb = (end - base + EW_BATCH * WAVE - 1) / (EW_BATCH * WAVE);
    Batch cur{}, nxt{};
    if (nb > 0) load(base + lane, cur);
    for (int64_t i = 0; i < nb; ++i) {
        const int64_t e0 = base + lane + i * (EW_BATCH * WAVE);
        if (i + 1 < nb) load(e0 + EW_BATCH * WAVE, nxt);
        const float(&g)[EW_BATCH] = cur.g;
        const float(&mo)[EW_BATCH] = cur.mo;
        const float(&vo)[EW_BATCH] = cur.vo;
        const float(&p)[EW_BATCH] = cur.p;
#pragma unroll
        for (int k = 0; k < EW_BATCH; ++k) {
            const int64_t e = e0 + k * WAVE;
            if (e >= end) continue;
            float mm, vv;
            ema(h, mo[k], vo[k], g[k], mm, vv);
            if (msum) acc.add(g[k], mm);
            update_one<APPLY, PSR, NEST, EXACT>(c, L, e, h, mm, vv, g[k], p[k]);
            if (store_sr) {
                // optim/adam.py:219-222: _tree_stochastic_cast(moments, bfloat16, k1 | k2)
                uint32_t bm, bv;
                moment_bits1(c, L, e, bm, bv);
                gst<uint16_t>(L.mu, e, (uint16_t)sr_bf16(mm, bm));
                gst<uint16_t>(L.nu, e, (uint16_t)sr_bf16(vv, bv));
            } else {
                store1(L.mu, mdt, e, mm);  // adam8.py:688 moment.astype(fallback_dtype)
                store1(L.nu, mdt, e, vv);
            }
        }
        cur = nxt;
    }
    if (msum) acc.store(c, base / CHUNK);
}

// Full 2048-element chunk of a fallback (unquantized-moment) leaf whose
// buffers are 16-byte aligned (KIND_FALLBACK_VEC): lane l owns elements
// j*512 + 8l .. +7 of the chunk, so every access is a 16-byte vector access;
// the four chunks' loads are issued before any arithmetic.  Dtypes are
// template parameters (PT params, GT grads, MT moments: uint16_t = bf16).
template <typename PT, typename GT, typename MT, bool APPLY, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void unit_fallback_vec(const UnitCtx& c, const rf_adam8_leaf& L, int64_t chunk,
                                                  const KHp& h)
{
    constexpr int J = (int)(CHUNK / 512);
    constexpr bool BF16M = IS_BF16<MT>;
    constexpr bool H16M = sizeof(MT) == 2;  // bf16 or f16 moments
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t base = chunk * CHUNK;
    const int32_t wdm = c.wd_mode;
    const bool need_p = APPLY || wdm != WD_OFF || c.zero;
    const bool store_sr = BF16M && (L.flags & RF_LEAF_STORE_SR);
    const bool msum = !APPLY && c.mpart != nullptr;  // Magma sums: update-only launches
    MagmaAcc acc;

    // Two chunks in flight: chunk j+1's loads are issued into `nxt` before
    // chunk j's arithmetic on `cur`, and move to `cur` after it.  No buffer
    // is indexed by the chunk: with param SR (three Threefry streams
    // inlined) the compiler does not unroll this loop, and a slot index
    // j & 1 would put both buffers in scratch memory and wait for every
    // load at once.  Unrolled instances rename the moves away.
    struct Bufs {
        Raw8<GT> g;
        Raw8<PT> p;
        Raw8<MT> m, v;
    } cur, nxt;
    auto issue = [&](int j, Bufs& b) {
        const int64_t e0 = base + j * 512 + lane * 8;
        raw8_load<GT>(b.g, L.grad, e0);
        if (need_p) raw8_load<PT>(b.p, L.param, e0);
        raw8_load<MT>(b.m, L.mu, e0);
        raw8_load<MT>(b.v, L.nu, e0);
    };
    issue(0, cur);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int64_t e0 = base + j * 512 + lane * 8;
        if (j + 1 < J) issue(j + 1, nxt);
        float g[8], p[8], m[8], v[8], u[8];
        raw8_unpack<GT>(cur.g, g);
        clip8<GT>(c, g);
        if (need_p) {
            raw8_unpack<PT>(cur.p, p);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) p[t] = 0.0f;
        }
        raw8_unpack<MT>(cur.m, m);
        raw8_unpack<MT>(cur.v, v);
        cur = nxt;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            float mm, vv;
            ema(h, m[t], v[t], g[t], mm, vv);
            if (msum) acc.add(g[t], mm);
            m[t] = mm;
            v[t] = vv;
            u[t] = decay_and_scale(h, adam_direction<NEST, EXACT>(h, mm, vv, g[t]), p[t], wdm, c.zero);
        }
        if constexpr (APPLY) {
            float sum[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) sum[t] = p[t] + u[t];
            if constexpr (!EXACT) {
                if (cancel_lanes8(sum, u) != 0) {
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        if (cancels(sum[t], u[t]))
                            sum[t] = p[t] + decay_and_scale(h, adam_direction<NEST, true>(h, m[t], v[t], g[t]), p[t],
                                                            wdm, c.zero);
                    }
                }
            }
            if constexpr (sizeof(PT) == 2) {
                uint32_t hb[8];
                if constexpr (PSR && IS_BF16<PT>) {
                    uint32_t rb[8];
                    param_bits8(c, L, e0, rb);
#pragma unroll
                    for (int t = 0; t < 8; ++t) hb[t] = sr_bf16_hi(sum[t], rb[t]);
                    store8_hi16(L.param, e0, hb);
                } else {
#pragma unroll
                    for (int t = 0; t < 8; t += 2) {
                        const uint32_t w2 = pack_h16x2_rne<PT>(sum[t], sum[t + 1]);
                        hb[t] = w2 & 0xFFFFu;
                        hb[t + 1] = w2 >> 16;
                    }
                    store8_bf16(L.param, e0, hb);
                }
            } else {
                store8_f32(L.param, e0, sum);
            }
        } else {
            store8_f32(L.updates, e0, u);
        }
        // adam8.py:688 moment.astype(fallback_dtype) / optim/adam.py:219-222 SR storage
        if constexpr (H16M) {
            uint32_t hm[8], hv[8];
            if (BF16M && store_sr) {
                uint32_t bm[8], bv[8];
                if (c.packed) {
                    // e0 is a multiple of 8: a packed block per pair
#pragma unroll
                    for (int t = 0; t < 8; t += 2) {
                        uint32_t y0, y1;
                        packed_moment_block(c.kmu0, c.kmu1, (uint64_t)(e0 + t), false, y0, y1);
                        bm[t] = y0;
                        bm[t + 1] = y0 >> 16;
                        bv[t] = y1;
                        bv[t + 1] = y1 >> 16;
                    }
                } else {
#pragma unroll
                    for (int t = 0; t < 8; ++t) moment_bits1(c, L, e0 + t, bm[t], bv[t]);
                }
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    hm[t] = sr_bf16_hi(m[t], bm[t]);
                    hv[t] = sr_bf16_hi(v[t], bv[t]);
                }
                store8_hi16(L.mu, e0, hm);
                store8_hi16(L.nu, e0, hv);
            } else {
#pragma unroll
                for (int t = 0; t < 8; t += 2) {
                    const uint32_t wm = pack_h16x2_rne<MT>(m[t], m[t + 1]);
                    const uint32_t wv = pack_h16x2_rne<MT>(v[t], v[t + 1]);
                    hm[t] = wm & 0xFFFFu;
                    hm[t + 1] = wm >> 16;
                    hv[t] = wv & 0xFFFFu;
                    hv[t + 1] = wv >> 16;
                }
                store8_bf16(L.mu, e0, hm);
                store8_bf16(L.nu, e0, hv);
            }
        } else {
            store8_f32(L.mu, e0, m);
            store8_f32(L.nu, e0, v);
        }
    }
    if (msum) acc.store(c, chunk);
}

template <bool APPLY, bool PSR, bool NEST, bool EXACT>
__device__ __forceinline__ void dispatch_fallback_vec(const UnitCtx& c, const rf_adam8_leaf& L, int64_t chunk,
                                                      const KHp& h)
{
    // Vectorised instances for params and grads of one dtype; other mixes
    // take the element-wise unit (same arithmetic).
    // (param dtype, grad dtype, moment dtype) in base 4 (RF_F32/RF_BF16/RF_F16; moments by kind)
    const int32_t mk = L.moment_kind == RF_MOMENT_BF16 ? RF_BF16 : (L.moment_kind == RF_MOMENT_F16 ? RF_F16 : RF_F32);
    const int sel = L.param_dtype * 16 + L.grad_dtype * 4 + mk;
    constexpr int F = RF_F32 * 20, B = RF_BF16 * 20, H = RF_F16 * 20;  // params and grads of one dtype
    switch (sel) {
    case F + RF_F32: unit_fallback_vec<float, float, float, APPLY, PSR, NEST, EXACT>(c, L, chunk, h); break;
    case F + RF_BF16: unit_fallback_vec<float, float, uint16_t, APPLY, PSR, NEST, EXACT>(c, L, chunk, h); break;
    case B + RF_F32:
        unit_fallback_vec<uint16_t, uint16_t, float, APPLY, PSR, NEST, EXACT>(c, L, chunk, h);
        break;
    case B + RF_BF16:
        unit_fallback_vec<uint16_t, uint16_t, uint16_t, APPLY, PSR, NEST, EXACT>(c, L, chunk, h);
        break;
    case H + RF_F32:
        unit_fallback_vec<_Float16, _Float16, float, APPLY, PSR, NEST, EXACT>(c, L, chunk, h);
        break;
    case H + RF_F16:
        unit_fallback_vec<_Float16, _Float16, _Float16, APPLY, PSR, NEST, EXACT>(c, L, chunk, h);
        break;
    default:
        unit_fallback<APPLY, PSR, NEST, EXACT>(c, L, chunk * CHUNK, min(chunk * CHUNK + CHUNK, L.size), h);
        break;
    }
}

// ======================================================== step kernels ===
// The scalars of the leaf's group in a grouped launch (optax.multi_transform):
// hl is the launch's KHp with the group's learning rate, weight decay, EMA
// weight and moment keys.  Ungrouped launches keep hl == h.
__device__ __forceinline__ void group_hparams(KHp& hl, const KHp& h, const rf_adam8_leaf& L)
{
    if (h.groups == nullptr) return;
    const rf_adam8_group G = h.groups[L.group];
    hl.neg_lr = (h.flags & RF_LR) ? G.neg_lr : 1.0f;
    hl.wd = G.weight_decay;
    hl.wd16 = round_to_bf16(G.weight_decay);
    hl.wdh = round_to_f16(G.weight_decay);
    hl.omb1 = G.one_minus_b1;
    hl.kmu0 = G.key_mu[0];
    hl.kmu1 = G.key_mu[1];
    hl.knu0 = G.key_nu[0];
    hl.knu1 = G.key_nu[1];
}

// UNIFORM_KEYS: move the leaf's keys to scalar registers (the fast kernel;
// the generic kernel is short of scalar registers and would spill them).
template <bool UNIFORM_KEYS>
__device__ __forceinline__ void leaf_context(UnitCtx& c, const rf_adam8_leaf& L, const KHp& h, bool msr, bool psr)
{
    const bool decay = (L.flags & RF_LEAF_DECAY) != 0;
    const bool weak = (h.flags & RF_DECAY_WEAK) != 0;
    c.wd_mode = !decay ? WD_OFF
                       : (weak && L.param_dtype == RF_BF16) ? WD_BF16
                       : (weak && L.param_dtype == RF_F16) ? WD_F16 : WD_F32;
    c.zero = (L.flags & RF_LEAF_ZERO_DECAY) != 0;
    if (msr || (L.flags & RF_LEAF_STORE_SR)) {
        jax_split(h.kmu0, h.kmu1, (uint32_t)L.state_index, c.kmu0, c.kmu1);
        jax_split(h.knu0, h.knu1, (uint32_t)L.state_index, c.knu0, c.knu1);
    }
    if (psr) jax_split(h.kp0, h.kp1, (uint32_t)L.param_index, c.kp0, c.kp1);
    if constexpr (UNIFORM_KEYS) {
        // A wave's leaf is one leaf: its keys are wave-uniform.  Threefry's
        // register pins leave them in vector registers; moved to scalar
        // ones, the key-schedule constants of every later block are scalar
        // work.
        c.kmu0 = uniform_u32(c.kmu0);
        c.kmu1 = uniform_u32(c.kmu1);
        c.knu0 = uniform_u32(c.knu0);
        c.knu1 = uniform_u32(c.knu1);
        c.kp0 = uniform_u32(c.kp0);
        c.kp1 = uniform_u32(c.kp1);
    }
}

// optax.apply_if_finite's reject branch (zero updates, inner state kept),
// as the launch's units see it: the moments are left untouched; the fused
// step applies the zero update (apply_updates, utils.py:694-700: f32(p) + 0
// rounded to the param dtype, so only -0 params change, to +0; stochastic
// rounding of an exact value adds nothing); the update-only mode writes
// zero updates.
template <bool APPLY>
__device__ void reject_units(const rf_adam8_leaf* __restrict__ leaves, const Seg* __restrict__ segs,
                             int64_t total_units, int64_t wave, int64_t nwaves)
{
    const int lane = threadIdx.x & (WAVE - 1);
    int32_t s = 0;
    const int32_t nseg = segs[0].nseg;
    for (int64_t u = wave; u < total_units; u += nwaves) {
        s = seek_seg(segs, nseg, s, u);
        const Seg sg = segs[s];
        const rf_adam8_leaf& L = leaves[sg.leaf];
        const int64_t span = (sg.kind == KIND_QFAST || sg.kind == KIND_QGEN) ? (int64_t)L.block_size
                             : sg.kind == KIND_FALLBACK                    ? EW_UNIT<APPLY>
                                                                           : CHUNK;
        const int64_t base = (sg.first + (u - sg.unit_start)) * span;
        const int64_t end = min(base + span, L.size);
        for (int64_t e = base + lane; e < end; e += WAVE) {
            if constexpr (APPLY) {
                store1(L.param, L.param_dtype, e, load1(L.param, L.param_dtype, e) + 0.0f);
            } else {
                gst<float>(L.updates, e, 0.0f);
            }
        }
    }
}

__device__ __forceinline__ bool gate_rejects(const KHp& h) { return h.gate != nullptr && gld<float>(h.gate, 0) == 0.0f; }

template <bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT, bool VEC_ONLY>
__device__ __forceinline__ void gen_list(const rf_adam8_leaf* __restrict__ leaves, const Seg* __restrict__ segs,
                                         int64_t total_units, const KHp& h, const uint4* __restrict__ tables,
                                         uint8_t* lds, uint32_t* red, uint32_t bid, uint32_t nbid);

// Full 2048-element blocks of the leaves whose (param, grad) dtypes are
// (PT, GT) (uint16_t = bf16, float = f32): the hot kernel.  Waves walk the
// work list with a grid stride of one block per wave.  The bf16/bf16
// instances without moment SR also carry a step's generic list (partial
// blocks, small leaves) in their first h.gwgs workgroups (CARRIES_GEN), so
// that a tree of such leaves is one launch and the generic units'
// latency-bound work overlaps the blocks' streaming instead of running as a
// kernel of its own before them.  (With moment SR the added code made the
// compiler spill in the block path: 194 scratch instructions against 11.)
template <typename PT, typename GT, bool MSR>
constexpr bool CARRIES_GEN = IS_BF16<PT> && IS_BF16<GT> && !MSR;

template <typename PT, typename GT, bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(RF_STEP_WAVES_PER_EU))) void k_adam8(
    const rf_adam8_leaf* __restrict__ leaves, const Seg* __restrict__ segs, int64_t total_units, KHp h,
    const uint4* __restrict__ tables)
{
    // moment-SR launches stage the search image with its neighbour records
    constexpr uint32_t LDS_TABLES = MSR ? SEARCH_BYTES : TABLE_BYTES;
    __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_TABLES];
    __shared__ __attribute__((aligned(16))) float wtab[WAVES_PER_WG][512];
    uint32_t bid = blockIdx.x, nbid = gridDim.x;
    if constexpr (CARRIES_GEN<PT, GT, MSR>) {
        const uint32_t gw = (uint32_t)h.gwgs;
        if (bid < gw) {
            // the generic units do not use the per-wave tables: their
            // workgroup absmax words take the first of them
            gen_list<APPLY, MSR, PSR, NEST, EXACT, false>(leaves, h.gsegs, h.gunits, h, tables, lds,
                                                          (uint32_t*)&wtab[0][0], bid, gw);
            return;
        }
        bid -= gw;
        nbid -= gw;
    }
    stage_tables<LDS_TABLES>(lds, tables);

    const uint32_t wave_in_wg = uniform_u32(threadIdx.x / WAVE);
    const int64_t wave = (int64_t)bid * WAVES_PER_WG + wave_in_wg;
    const int64_t nwaves = (int64_t)nbid * WAVES_PER_WG;
    int32_t s = 0;
    const int32_t nseg = segs[0].nseg;
    int32_t cur_leaf = -1;
    UnitCtx c;
    c.lds = lds;
    c.wtab = wtab[wave_in_wg];
    c.xbuf = nullptr;
    if constexpr (!APPLY || sizeof(PT) == 4) {  // f32 updates or params: store8_f32_lines
        __shared__ __attribute__((aligned(16))) float xbuf[WAVES_PER_WG][512];
        c.xbuf = xbuf[wave_in_wg];
    }
    c.fed = (h.flags & RF_FED_BITS) != 0;
    c.packed = !c.fed && (h.flags & RF_PACKED_BITS) != 0;
    c.zero = false;  // quantized blocks only: RF_LEAF_ZERO_DECAY is refused for them
    c.mpart = nullptr;
    c.mbase = 0;
    if (gate_rejects(h)) {
        reject_units<APPLY>(leaves, segs, total_units, wave, nwaves);
        return;
    }
    clip_context(c, h);
    c.wd_mode = WD_OFF;
    c.kmu0 = c.kmu1 = c.knu0 = c.knu1 = c.kp0 = c.kp1 = 0;
    rf_adam8_leaf L;
    KHp hl = h;  // the current leaf's scalars (its group's, in a grouped launch)
    flr_setup(hl);
    ChunkSlots<PT, GT> sl;
    bool have0 = false;  // slot 0 holds chunk 0 of unit u
    // Wave w takes runs of h.run consecutive units: run r = w, w + nwaves, ...
    const int64_t run = h.run;
    const int64_t nruns = (total_units + run - 1) / run;
    for (int64_t r = wave; r < nruns; r += nwaves) {
        const int64_t u_end = min(r * run + run, total_units);
        for (int64_t u = r * run; u < u_end; ++u) {
            s = seek_seg(segs, nseg, s, u);
            const Seg sg = segs[s];
            if (sg.leaf != cur_leaf) {
                cur_leaf = sg.leaf;
                L = leaves[cur_leaf];
                if (h.groups != nullptr) {
                    group_hparams(hl, h, L);
                    flr_setup(hl);
                }
                leaf_context<true>(c, L, hl, MSR, PSR);
            }
            // The next unit of this wave, when it is a block of the same leaf
            // (this kernel's units are all full blocks; one segment per leaf).
            const int64_t un = u + 1 < u_end ? u + 1 : (r + nwaves) * run;
            int64_t next_blk = -1;
            if (RF_PREFETCH_NEXT && un < total_units && un < segs[s + 1].unit_start)
                next_blk = sg.first + (un - sg.unit_start);
            dispatch_qfast<PT, GT, APPLY, MSR, PSR, NEST, EXACT>(c, L, sg.first + (u - sg.unit_start), hl, sl,
                                                                 have0, next_blk);
            have0 = next_blk >= 0;
        }
    }
}

// The memory ceiling of the fused step (diagnostics; no reference
// counterpart): the fast kernel's work list, launch shape and lane layout,
// every byte the step moves per 2048-element block -- params, grads, both
// code arrays and both scales read; params, codes and scales written back
// unchanged -- and no arithmetic.  Two chunks in flight per wave, as in the
// step.  The empty asm statements make the loaded values opaque, so the
// compiler neither drops the grad loads nor folds a store of a loaded
// value into nothing.
__device__ __forceinline__ void opaque(uint32_t& x) { __asm__ volatile("" : "+v"(x)); }
__device__ __forceinline__ void opaque(uint2& x) { opaque(x.x); opaque(x.y); }
__device__ __forceinline__ void opaque(uint4& x) { opaque(x.x); opaque(x.y); opaque(x.z); opaque(x.w); }

template <typename PT, typename GT>
__device__ __forceinline__ void probe_block(const rf_adam8_leaf& L, int64_t blk)
{
    constexpr int J = FAST_BS / 512;
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t base = blk * FAST_BS;
    // (16-bit stored scales read back and stored again exactly)
    float sm = load_scale(L.mu_scales, L.flags, blk);
    float sv = load_scale(L.nu_scales, L.flags, blk);
    RF_GLOBAL uint8_t* pB = (RF_GLOBAL uint8_t*)L.param + base * (int64_t)sizeof(PT);
    RF_GLOBAL uint8_t* mW = (RF_GLOBAL uint8_t*)L.mu + base;
    RF_GLOBAL uint8_t* vW = (RF_GLOBAL uint8_t*)L.nu + base;
    ChunkSlots<PT, GT> sl;
    issue_chunk<PT, GT, true>(sl, L, blk, 0, 0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int slot = j & 1;
        const uint32_t eo = (uint32_t)(j * 512 + lane * 8);
        if (j + 1 < J) issue_chunk<PT, GT, true>(sl, L, blk, j + 1, slot ^ 1);
        uint2 mc = sl.mc[slot], vc = sl.vc[slot];
        uint4 p0 = sl.praw[slot].w[0];
        opaque(mc);
        opaque(vc);
        opaque(p0);
        opaque(sl.graw[slot].w[0]);
        if constexpr (sizeof(GT) == 4) opaque(sl.graw[slot].w[1]);
        if constexpr (sizeof(PT) == 2) {
            st_nt((RF_GLOBAL uint4*)(pB + eo * 2), p0);
        } else {
            uint4 p1 = sl.praw[slot].w[1];
            opaque(p1);
            *(RF_GLOBAL uint4*)(pB + eo * 4) = p0;
            *(RF_GLOBAL uint4*)(pB + eo * 4 + 16) = p1;
        }
        st_nt((RF_GLOBAL uint2*)(mW + eo), mc);
        st_nt((RF_GLOBAL uint2*)(vW + eo), vc);
    }
    uint32_t smb = __float_as_uint(sm), svb = __float_as_uint(sv);
    opaque(smb);
    opaque(svb);
    sm = __uint_as_float(smb);
    sv = __uint_as_float(svb);
    if (lane == 0) {
        store_scale(L.mu_scales, L.flags, blk, sm);
        store_scale(L.nu_scales, L.flags, blk, sv);
    }
}

template <typename PT, typename GT>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(RF_STEP_WAVES_PER_EU))) void k_stream_probe(
    const rf_adam8_leaf* __restrict__ leaves, const Seg* __restrict__ segs, int64_t total_units, int32_t run)
{
    const uint32_t wave_in_wg = uniform_u32(threadIdx.x / WAVE);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + wave_in_wg;
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    int32_t s = 0;
    const int32_t nseg = segs[0].nseg;
    int32_t cur_leaf = -1;
    rf_adam8_leaf L;
    const int64_t nruns = (total_units + run - 1) / run;
    for (int64_t r = wave; r < nruns; r += nwaves) {
        const int64_t u_end = min(r * run + run, total_units);
        for (int64_t u = r * run; u < u_end; ++u) {
            s = seek_seg(segs, nseg, s, u);
            const Seg sg = segs[s];
            if (sg.leaf != cur_leaf) {
                cur_leaf = sg.leaf;
                L = leaves[cur_leaf];
            }
            probe_block<PT, GT>(L, sg.first + (u - sg.unit_start));
        }
    }
}

// Everything else: quantized blocks of other sizes and partial or unaligned
// blocks (a workgroup each; two passes, literal requantization), then the
// leaves with unquantized (fallback) moments (a wave per unit).  Dtypes are
// read per leaf.
// VEC_ONLY: an instance for lists of full-chunk fallback units only (the
// full-precision AdamW trees).  Without the other unit kinds its plain
// instances take 126-127 VGPRs (4 waves per SIMD) as the compiler schedules
// them; with them, 133-135, which the mixed instances are held to 128 from
// (GEN_WAVES_PER_EU), the moment-SR, param-SR and Nesterov ones aside
// (138-151 VGPRs, 3 waves, where 4 would spill).  Measured on the Llama-7B
// tree, the full-precision step ran 8 % slower in the mixed kernel held to
// 128 VGPRs; the ragged tree's mixed lists 2.5 % faster held than not.
template <bool MSR, bool PSR, bool NEST, bool VEC_ONLY>
constexpr int GEN_WAVES_PER_EU = (VEC_ONLY || MSR || PSR || NEST) ? 1 : 4;

// The generic list's units over workgroups bid = 0 .. nbid - 1 of a launch:
// the generic kernel's whole grid, or the leading workgroups of a fast
// launch the list rides along with (k_adam8, KHp.gsegs).  `lds` holds at
// least TABLE_BYTES; `red` is 8 words of LDS.
template <bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT, bool VEC_ONLY>
__device__ __forceinline__ void gen_list(const rf_adam8_leaf* __restrict__ leaves, const Seg* __restrict__ segs,
                                         int64_t total_units, const KHp& h, const uint4* __restrict__ tables,
                                         uint8_t* lds, uint32_t* red, uint32_t bid, uint32_t nbid)
{
    // The list's leading quantized units go to workgroups bid, bid + nbid,
    // ...: only workgroups below nlead code a block, and only they stage the
    // tables (null: the list has no quantized units).  The others
    // (element-wise units of small leaves) start at once.
    const int64_t nlead = VEC_ONLY ? 0 : segs[0].lead;
    if (!VEC_ONLY && tables && (int64_t)bid < nlead) stage_tables(lds, tables);

    const int64_t wave = (int64_t)bid * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)nbid * WAVES_PER_WG;
    int32_t s = 0;
    const int32_t nseg = segs[0].nseg;
    int32_t cur_leaf = -1;
    UnitCtx c;
    c.lds = lds;
    c.wtab = nullptr;
    c.fed = (h.flags & RF_FED_BITS) != 0;
    c.packed = !c.fed && (h.flags & RF_PACKED_BITS) != 0;
    c.zero = false;
    c.mpart = h.mpart;
    c.mbase = 0;
    if (gate_rejects(h)) {
        reject_units<APPLY>(leaves, segs, total_units, wave, nwaves);
        return;
    }
    clip_context(c, h);
    c.wd_mode = WD_OFF;
    c.kmu0 = c.kmu1 = c.knu0 = c.knu1 = c.kp0 = c.kp1 = 0;
    rf_adam8_leaf L;
    KHp hl = h;  // the current leaf's scalars (its group's, in a grouped launch)
    // The list's leading quantized units (partial and odd-sized blocks, the
    // long ones), a workgroup each; then the rest a wave each, handed out
    // from the last waves down so that the workgroups of the first phase
    // take none when the workgroups cover every unit.
    for (int64_t q = bid; q < nlead; q += nbid) {
        s = seek_seg(segs, nseg, s, q);
        const Seg sg = segs[s];
        if (sg.leaf != cur_leaf) {
            cur_leaf = sg.leaf;
            L = leaves[cur_leaf];
            group_hparams(hl, h, L);
            leaf_context<false>(c, L, hl, MSR, PSR);
            if (h.mpart) c.mbase = h.msegs[cur_leaf].unit_start;
        }
        unit_qgen_wg<APPLY, MSR, PSR, NEST, EXACT>(c, L, sg.first + (q - sg.unit_start), hl, red);
    }
    for (int64_t u = nlead + (nwaves - 1 - wave); u < total_units; u += nwaves) {
        s = seek_seg(segs, nseg, s, u);
        const Seg sg = segs[s];
        if (sg.leaf != cur_leaf) {
            cur_leaf = sg.leaf;
            L = leaves[cur_leaf];
            group_hparams(hl, h, L);
            leaf_context<false>(c, L, hl, MSR, PSR);
            if (h.mpart) c.mbase = h.msegs[cur_leaf].unit_start;
        }
        const int64_t idx = sg.first + (u - sg.unit_start);
        if constexpr (VEC_ONLY) {
            dispatch_fallback_vec<APPLY, PSR, NEST, EXACT>(c, L, idx, hl);
        } else {
            // (the list's quantized units are all among the leading ones)
            if (sg.kind == KIND_FALLBACK_VEC) dispatch_fallback_vec<APPLY, PSR, NEST, EXACT>(c, L, idx, hl);
            else unit_fallback<APPLY, PSR, NEST, EXACT>(c, L, idx * EW_UNIT<APPLY>,
                                                         min(idx * EW_UNIT<APPLY> + EW_UNIT<APPLY>, L.size), hl);
        }
    }
}

template <bool APPLY, bool MSR, bool PSR, bool NEST, bool EXACT, bool VEC_ONLY = false>
__global__ __launch_bounds__(WG) __attribute__((amdgpu_waves_per_eu(GEN_WAVES_PER_EU<MSR, PSR, NEST, VEC_ONLY>)))
void k_adam8_gen(const rf_adam8_leaf* __restrict__ leaves,
                                                  const Seg* __restrict__ segs, int64_t total_units, KHp h,
                                                  const uint4* __restrict__ tables)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[TABLE_BYTES];
    __shared__ uint32_t red[2 * WAVES_PER_WG];  // absmax bits of a workgroup's block, per wave
    gen_list<APPLY, MSR, PSR, NEST, EXACT, VEC_ONLY>(leaves, segs, total_units, h, tables, lds, red, blockIdx.x,
                                                     gridDim.x);
}

}  // namespace rf
