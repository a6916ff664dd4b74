// rf_host.hip -- host side of librfadam8.so: lookup-table construction,
// per-device state, launch plans, the standalone quantize / dequantize / SR /
// apply kernels, and the C ABI declared in include/rfadam8.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "rf_device.h"

using namespace rf;

#define RF_VERSION "rfadam8 0.2.0 gfx950"

// ------------------------------------------------------------------ errors --
namespace {
thread_local std::string g_err;

rf_status fail(rf_status code, const std::string& msg)
{
    g_err = msg;
    return code;
}

#define HIP_TRY(expr)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (expr);                                                          \
        if (e_ != hipSuccess)                                                            \
            return fail(RF_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)
}  // namespace

// Instances of the step kernel (rf_adam8_inst.hip, one object per variant).
namespace rf {
adam_kernel_t rf_pick_adam8_a0_m0_e0(int dtype_combo, bool psr, bool nest);
adam_kernel_t rf_pick_adam8_a0_m0_e1(int dtype_combo, bool psr, bool nest);
adam_kernel_t rf_pick_adam8_a0_m1_e0(int dtype_combo, bool psr, bool nest);
adam_kernel_t rf_pick_adam8_a0_m1_e1(int dtype_combo, bool psr, bool nest);
adam_kernel_t rf_pick_adam8_a1_m0_e0(int dtype_combo, bool psr, bool nest);
adam_kernel_t rf_pick_adam8_a1_m0_e1(int dtype_combo, bool psr, bool nest);
adam_kernel_t rf_pick_adam8_a1_m1_e0(int dtype_combo, bool psr, bool nest);
adam_kernel_t rf_pick_adam8_a1_m1_e1(int dtype_combo, bool psr, bool nest);
}  // namespace rf

// ====================================================== standalone kernels ==
// 8 consecutive elements of an f32, bf16 or f16 array as f32 (16-byte aligned).
__device__ __forceinline__ void load8_dt(const void* base, int32_t dtype, int64_t e0, float (&x)[8])
{
    if (dtype == RF_BF16) load8<uint16_t>(base, e0, x);
    else if (dtype == RF_F16) load8<_Float16>(base, e0, x);
    else load8<float>(base, e0, x);
}

// Standalone quantize_blocks (adam8.py:113-187): one wave per block.  Fast
// path: 2048-element aligned blocks held in registers; otherwise two passes.
__global__ __launch_bounds__(WG) void k_quantize(int32_t quantizer, const void* __restrict__ x, int32_t x_dtype,
                                                 int64_t size, int64_t bs, int64_t nblocks, int32_t sr, uint32_t k0,
                                                 uint32_t k1, const uint32_t* __restrict__ bits,
                                                 uint8_t* __restrict__ values, void* __restrict__ scales,
                                                 int32_t scale_dtype, const uint4* __restrict__ tables,
                                                 int32_t vec_ok)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[TABLE_BYTES];
    stage_tables(lds, tables);
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    const float* cb = (const float*)(lds + (quantizer == RF_Q_DYNAMIC_UNSIGNED ? L_CBU : L_CBS));
    auto is_full = [&](int64_t b) { return vec_ok && bs == FAST_BS && b < nblocks && b * bs + bs <= size; };
    auto load_chunk = [&](int64_t b, int j, float (&r)[32]) {
        float t8[8];
        load8_dt(x, x_dtype, b * FAST_BS + j * 512 + lane * 8, t8);
#pragma unroll
        for (int t = 0; t < 8; ++t) r[j * 8 + t] = t8[t];
    };
    auto load_block = [&](int64_t b, float (&r)[32]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) load_chunk(b, j, r);
    };
    // Full 2048-blocks stream through one 32-value ring per lane: once chunk
    // j of a block is coded, its registers take chunk j of the wave's next
    // block, so the next block's loads are in flight while the rest of the
    // current one is coded.
    float xr[32];
    bool have = false;
    for (int64_t b = wave; b < nblocks; b += nwaves) {
        const int64_t base = b * bs;
        const int64_t nvalid = max((int64_t)0, min(bs, size - base));
        const bool full = is_full(b);
        uint32_t am = 0;
        if (full) {
            if (!have) load_block(b, xr);
#pragma unroll
            for (int i = 0; i < 32; ++i) am = max(am, __float_as_uint(xr[i]) & 0x7FFFFFFFu);
        } else {
            for (int64_t j = lane; j < nvalid; j += WAVE)
                am = max(am, __float_as_uint(load1(x, x_dtype, base + j)) & 0x7FFFFFFFu);
        }
        am = wave_max_u32(am);
        const float amax = __uint_as_float(am);
        float scale;
        if (quantizer == RF_Q_SYMMETRIC_INT8) scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        else scale = amax > 0.0f ? amax : 1.0f;
        if (lane == 0) store1(scales, scale_dtype, b, scale);  // scales.astype(scale_dtype) (adam8.py:186)
        const bool fast = !sr && quantizer != RF_Q_SYMMETRIC_INT8 && block_is_fast(am, scale);
        const float rs = 1.0f / scale;
        auto code_of = [&](float xv, int64_t e) -> uint32_t {
            if (quantizer == RF_Q_SYMMETRIC_INT8) {
                // adam8.py:143-164 and _round_scaled :446-458
                float s = xv / scale;
                s = s < -127.0f ? -127.0f : (s > 127.0f ? 127.0f : s);
                float r;
                if (sr) {
                    const uint32_t w = bits ? bits[e] : jax_bits(k0, k1, (uint64_t)e);
                    const float lo = floorf(s);
                    r = lo + (uniform_from_bits(w) < (s - lo) ? 1.0f : 0.0f);
                } else {
                    r = rintf(s);
                }
                return (uint32_t)(uint8_t)(int8_t)(r == r ? (int)r : 0);
            }
            if (fast) {
                if (quantizer == RF_Q_DYNAMIC_SIGNED) return code_signed_fast(lds, xv, scale, rs);
                return code_unsigned_fast(lds, xv > 0.0f ? xv : 0.0f, scale, rs);
            }
            uint32_t w = 0;
            if (sr) w = bits ? bits[e] : jax_bits(k0, k1, (uint64_t)e);
            return code_literal(cb, xv, scale, sr != 0, w);
        };
        if (full) {
            const bool next_full = is_full(b + nwaves);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t e0 = base + j * 512 + lane * 8;
                uint32_t cc[8];
                if (fast && quantizer != RF_Q_SYMMETRIC_INT8) {
                    // Batched phases: normalise, candidate reads, threshold
                    // reads (16 independent LDS reads in flight).
                    const bool sgn = quantizer == RF_Q_DYNAMIC_SIGNED;
                    float nv[8], tv[8];
#pragma unroll
                    for (int t = 0; t < 8; ++t) {
                        const float xv = xr[j * 8 + t];
                        nv[t] = div_by_scale(sgn ? xv : (xv > 0.0f ? xv : 0.0f), scale, rs);
                    }
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] = sgn ? cand_signed(lds, nv[t]) : cand_unsigned(lds, nv[t]);
#pragma unroll
                    for (int t = 0; t < 8; ++t) tv[t] = *(const float*)(lds + (sgn ? L_TS : L_TU) + cc[t] * 4u);
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] += nv[t] >= tv[t] ? 1u : 0u;
                } else {
#pragma unroll
                    for (int t = 0; t < 8; ++t) cc[t] = code_of(xr[j * 8 + t], e0 + t);
                }
                uint2 w;
                w.x = pack4_u8(cc[0], cc[1], cc[2], cc[3]);
                w.y = pack4_u8(cc[4], cc[5], cc[6], cc[7]);
                // nontemporal: the codes are not read again by this launch
                __builtin_nontemporal_store((nt_u32x2){w.x, w.y}, (nt_u32x2*)(values + e0));
                if (next_full) load_chunk(b + nwaves, j, xr);
            }
            have = next_full;
        } else {
            have = false;
            for (int64_t j = lane; j < bs; j += WAVE) {
                const int64_t e = base + j;
                const float xv = j < nvalid ? load1(x, x_dtype, e) : 0.0f;
                values[e] = (uint8_t)code_of(xv, e);
            }
        }
    }
}

// Standalone dequantize_blocks (adam8.py:190-204).  Vector path: each wave
// takes 1024-element tiles, two at a time; lane l owns elements
// 256k + 4l .. 256k + 4l + 3 (k = 0..3), so every code load reads 256
// contiguous bytes and every store writes 1 KB (f32) or 512 B (bf16)
// contiguous.  Requires a power-of-two block size (>= 4) and 4-byte aligned
// codes / 16-byte (f32) or 8-byte (bf16) aligned output.
__device__ __forceinline__ void dq_store4(void* out, int32_t out_dtype, int64_t e, const float (&o)[4])
{
    // nontemporal: the launch does not read its output back
    if (out_dtype == RF_BF16) {
        const nt_u32x2 w = {f32_to_bf16_rne(o[0]) | (f32_to_bf16_rne(o[1]) << 16),
                            f32_to_bf16_rne(o[2]) | (f32_to_bf16_rne(o[3]) << 16)};
        __builtin_nontemporal_store(w, (nt_u32x2*)((uint16_t*)out + e));
    } else if (out_dtype == RF_F16) {
        const nt_u32x2 w = {pack_f16x2_rne(o[0], o[1]), pack_f16x2_rne(o[2], o[3])};
        __builtin_nontemporal_store(w, (nt_u32x2*)((uint16_t*)out + e));
    } else {
        __builtin_nontemporal_store((nt_f32x4){o[0], o[1], o[2], o[3]}, (nt_f32x4*)((float*)out + e));
    }
}

__global__ __launch_bounds__(WG) void k_dequantize(int32_t quantizer, const uint8_t* __restrict__ values,
                                                   const void* __restrict__ scales, int32_t scale_dtype,
                                                   int64_t size, int64_t bs,
                                                   int32_t bs_log2, int32_t out_dtype, void* __restrict__ out,
                                                   const uint4* __restrict__ tables, int32_t vec_ok)
{
    __shared__ __attribute__((aligned(16))) float cb[256];
    const uint32_t off = quantizer == RF_Q_DYNAMIC_UNSIGNED ? L_CBU : L_CBS;
    for (int i = threadIdx.x; i < 64; i += WG) ((uint4*)cb)[i] = tables[off / 16 + i];
    __syncthreads();
    const bool sym = quantizer == RF_Q_SYMMETRIC_INT8;
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    const int64_t ntiles = vec_ok ? size / 1024 : 0;
    constexpr int T = 2;  // tiles per wave and iteration
    for (int64_t t0 = wave * T; t0 < ntiles; t0 += nwaves * T) {
        uint32_t w[T][4];
        float s[T][4];
#pragma unroll
        for (int u = 0; u < T; ++u) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t e = (t0 + u) * 1024 + k * 256 + lane * 4;
                if (t0 + u < ntiles) {
                    w[u][k] = *(const uint32_t*)(values + e);
                    s[u][k] = load1(scales, scale_dtype, e >> bs_log2);  // the 4 elements share a block (bs >= 4)
                }
            }
        }
#pragma unroll
        for (int u = 0; u < T; ++u) {
            if (t0 + u >= ntiles) break;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t e = (t0 + u) * 1024 + k * 256 + lane * 4;
                float o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t cbyte = (w[u][k] >> (8 * i)) & 0xFFu;
                    const float val = sym ? (float)(int8_t)cbyte : cb[cbyte];
                    o[i] = val * s[u][k];
                }
                dq_store4(out, out_dtype, e, o);
            }
        }
    }
    const int64_t tid = (int64_t)blockIdx.x * WG + threadIdx.x;
    const int64_t nthreads = (int64_t)gridDim.x * WG;
    for (int64_t e = ntiles * 1024 + tid; e < size; e += nthreads) {
        const uint32_t cbyte = values[e];
        const float val = sym ? (float)(int8_t)cbyte : cb[cbyte];
        store1(out, out_dtype, e, val * load1(scales, scale_dtype, e / bs));
    }
}

// Standalone _stochastic_round_bf16 (utils.py:342-371).  PACKED: the packed
// bit source (a Threefry block per four elements) instead of
// jax.random.bits.  Vector path: a wave takes two 1024-element tiles per
// iteration, each lane four consecutive elements per 256-element row (one
// 16-byte load; with the packed source exactly one block), all loads of the
// two tiles issued before the rounding; nontemporal loads and 8-byte stores.
template <bool PACKED>
__global__ __launch_bounds__(WG) void k_sr_bf16(const float* __restrict__ x, int64_t size, uint32_t k0,
                                                uint32_t k1, const uint32_t* __restrict__ bits,
                                                uint16_t* __restrict__ out, int32_t vec_ok)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    const int64_t ntiles = vec_ok ? size / 1024 : 0;
    constexpr int T = 2;  // tiles per wave and iteration
    for (int64_t t0 = wave * T; t0 < ntiles; t0 += nwaves * T) {
        float4 xv[T][4];
        uint4 fb[T][4];
#pragma unroll
        for (int u = 0; u < T; ++u) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t e = (t0 + u) * 1024 + k * 256 + lane * 4;
                if (t0 + u < ntiles) {
                    const uint4 w = ldg_nt(x + e);
                    xv[u][k] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z),
                                           __uint_as_float(w.w));
                    if (bits) fb[u][k] = ldg_nt(bits + e);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < T; ++u) {
            if (t0 + u >= ntiles) break;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t e = (t0 + u) * 1024 + k * 256 + lane * 4;
                uint32_t rb[4];
                if (bits) {
                    rb[0] = fb[u][k].x;
                    rb[1] = fb[u][k].y;
                    rb[2] = fb[u][k].z;
                    rb[3] = fb[u][k].w;
                } else if constexpr (PACKED) {
                    packed_param_bits4(k0, k1, (uint64_t)e, rb);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) rb[i] = jax_bits(k0, k1, (uint64_t)(e + i));
                }
                const nt_u32x2 w = {pack_hi16x2(sr_bf16_hi(xv[u][k].x, rb[0]), sr_bf16_hi(xv[u][k].y, rb[1])),
                                    pack_hi16x2(sr_bf16_hi(xv[u][k].z, rb[2]), sr_bf16_hi(xv[u][k].w, rb[3]))};
                __builtin_nontemporal_store(w, (nt_u32x2*)(out + e));
            }
        }
    }
    const int64_t tid = (int64_t)blockIdx.x * WG + threadIdx.x;
    const int64_t nthreads = (int64_t)gridDim.x * WG;
    for (int64_t e = ntiles * 1024 + tid; e < size; e += nthreads) {
        const uint32_t w = bits ? bits[e] : PACKED ? packed_param_bits1(k0, k1, (uint64_t)e) : jax_bits(k0, k1, (uint64_t)e);
        out[e] = (uint16_t)sr_bf16(x[e], w);
    }
}

// apply_updates over a leaf table (utils.py:648-708): f32(p) + f32(u), then
// stochastic rounding or round-to-nearest-even for bf16 params.
template <bool PACKED>
__device__ __forceinline__ uint32_t apply_bf16(float p, float u, bool stochastic, const uint32_t* bits, uint32_t lk0,
                                               uint32_t lk1, int64_t e)
{
    const float s = p + u;
    if (!stochastic) return f32_to_bf16_rne(s);
    const uint32_t w = bits      ? gld<uint32_t>(bits, e)
                       : PACKED ? packed_param_bits1(lk0, lk1, (uint64_t)e)
                                : jax_bits(lk0, lk1, (uint64_t)e);
    return sr_bf16(s, w);
}

// Work units of apply_updates: APPLY_UNIT consecutive elements of one leaf
// per wave (a ragged tree launches no idle workgroups).  On the Llama-7B
// tree (packed SR, one GPU, two processes each) units of 8192, 4096 and
// 2048 elements ran 10.50-10.59, 10.12-10.13 and 10.02-10.05 ms (the grid
// grows with the unit count); GPT-2-small's launch 215-222 us in each.
constexpr int64_t APPLY_UNIT = 2048;

// Four consecutive elements e0 .. e0 + 3 (e0 a multiple of 4, the buffer
// 16-byte aligned), read and written nontemporally: f32 values, uint32
// words, or 16-bit patterns as two words.
__device__ __forceinline__ void ld4_f32_nt(const void* base, int64_t e0, float (&x)[4])
{
    const nt_u32x4 v = __builtin_nontemporal_load((const nt_u32x4*)((const float*)base + e0));
    x[0] = __uint_as_float(v.x);
    x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z);
    x[3] = __uint_as_float(v.w);
}

__device__ __forceinline__ void ld4_u32_nt(const uint32_t* base, int64_t e0, uint32_t (&x)[4])
{
    const nt_u32x4 v = __builtin_nontemporal_load((const nt_u32x4*)(base + e0));
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
}

__device__ __forceinline__ nt_u32x2 ld4_h16_nt(const void* base, int64_t e0)
{
    return __builtin_nontemporal_load((const nt_u32x2*)((const uint16_t*)base + e0));
}

__device__ __forceinline__ void st4_h16_nt(void* base, int64_t e0, uint32_t w0, uint32_t w1)
{
    __builtin_nontemporal_store(nt_u32x2{w0, w1}, (nt_u32x2*)((uint16_t*)base + e0));
}

__device__ __forceinline__ void st4_f32_nt(void* base, int64_t e0, const float (&x)[4])
{
    __builtin_nontemporal_store(nt_f32x4{x[0], x[1], x[2], x[3]}, (nt_f32x4*)((float*)base + e0));
}

// `factor` (Magma's fused form, or null): each update is first taken as
// neg_lr * (factor[leaf] * u), the scaling rf_magma_scale would have done.
// Segment s of `segs` is leaf segs[s].leaf.  SR: stochastic rounding of bf16
// params (an instance of its own: the Threefry code would cost the
// nearest-even instance waves per SIMD); PACKED: its bits from the packed
// source.
template <bool SR, bool PACKED>
__global__ __launch_bounds__(WG) void k_apply(const rf_apply_leaf* __restrict__ leaves, const Seg* __restrict__ segs,
                                              int64_t nunits, uint32_t k0, uint32_t k1,
                                              const float* __restrict__ factor, float neg_lr)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    constexpr bool sr = SR;
    int32_t s = 0, cur = -1;
    const int32_t nseg = segs[0].nseg;
    rf_apply_leaf L{};
    float f = 1.0f;
    uint32_t lk0 = 0, lk1 = 0;
    bool vec = false;
    for (int64_t u_ = wave; u_ < nunits; u_ += nwaves) {
        s = seek_seg(segs, nseg, s, u_);
        if (segs[s].leaf != cur) {
            cur = segs[s].leaf;
            L = leaves[cur];
            f = factor ? factor[cur] : 1.0f;
            if (sr) {
                jax_split(k0, k1, (uint32_t)L.param_index, lk0, lk1);
                lk0 = uniform_u32(lk0);  // one leaf per unit: wave-uniform keys
                lk1 = uniform_u32(lk1);
            }
            vec = ((uintptr_t)L.param % 16 == 0) && ((uintptr_t)L.updates % 16 == 0) &&
                  (!L.bits || (uintptr_t)L.bits % 16 == 0);
        }
        const int64_t e_begin = (u_ - segs[s].unit_start) * APPLY_UNIT;
        const int64_t e_end = min(L.size, e_begin + APPLY_UNIT);
        // Whole groups of 512 elements: lane l takes elements 4l .. 4l + 3
        // and 256 + 4l .. 256 + 4l + 3 of a group, so that each load and
        // store instruction of the wave covers whole cache lines (16-bit
        // params 512 bytes, f32 updates and params 1 KB), all of them
        // nontemporal; the unit's last partial group goes element-wise.
        // (Eight consecutive elements per lane put each f32 access on half
        // of every line it touches.)
        const int64_t v_end = vec ? e_begin + ((e_end - e_begin) / 512) * 512 : e_begin;
        for (int64_t g0 = e_begin; g0 < v_end; g0 += 512) {
            int64_t e0[2];
            float u[2][4], p[2][4];
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) e0[hf] = g0 + hf * 256 + lane * 4;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) ld4_f32_nt(L.updates, e0[hf], u[hf]);
            if (L.param_dtype == RF_F32) {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) ld4_f32_nt(L.param, e0[hf], p[hf]);
            } else {
                nt_u32x2 w[2];
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) w[hf] = ld4_h16_nt(L.param, e0[hf]);
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const uint32_t d[2] = {w[hf].x, w[hf].y};
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        if (L.param_dtype == RF_F16) {
                            p[hf][2 * i] = f16_bits_to_f32(d[i] & 0xFFFFu);
                            p[hf][2 * i + 1] = f16_bits_to_f32(d[i] >> 16);
                        } else {
                            p[hf][2 * i] = __uint_as_float(d[i] << 16);
                            p[hf][2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
                        }
                    }
                }
            }
            if (factor) {
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int t = 0; t < 4; ++t) u[hf][t] = neg_lr * (f * u[hf][t]);
            }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                if (L.param_dtype == RF_F16) {
                    uint32_t h[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) h[t] = f32_to_f16_rne(p[hf][t] + u[hf][t]);  // no SR below bf16 (utils.py:700)
                    st4_h16_nt(L.param, e0[hf], h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                } else if (L.param_dtype == RF_BF16) {
                    uint32_t h[4];
                    if constexpr (SR) {
                        uint32_t rb[4];
                        if (L.bits) {
                            ld4_u32_nt(L.bits, e0[hf], rb);
                        } else if constexpr (PACKED) {
                            packed_param_bits4(lk0, lk1, (uint64_t)e0[hf], rb);  // e0: a multiple of 4
                        } else {
#pragma unroll
                            for (int t = 0; t < 4; ++t) rb[t] = jax_bits(lk0, lk1, (uint64_t)(e0[hf] + t));
                        }
#pragma unroll
                        for (int t = 0; t < 4; ++t) h[t] = sr_bf16_hi(p[hf][t] + u[hf][t], rb[t]);
                        st4_h16_nt(L.param, e0[hf], pack_hi16x2(h[0], h[1]), pack_hi16x2(h[2], h[3]));
                    } else {
#pragma unroll
                        for (int t = 0; t < 4; ++t) h[t] = f32_to_bf16_rne(p[hf][t] + u[hf][t]);
                        st4_h16_nt(L.param, e0[hf], h[0] | (h[1] << 16), h[2] | (h[3] << 16));
                    }
                } else {
                    float o[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) o[t] = p[hf][t] + u[hf][t];
                    st4_f32_nt(L.param, e0[hf], o);
                }
            }
        }
        for (int64_t e = v_end + lane; e < e_end; e += WAVE) {
            const float ue = gld<float>(L.updates, e);
            const float u = factor ? neg_lr * (f * ue) : ue;
            if (L.param_dtype == RF_F16) {
                const float p = f16_bits_to_f32(gld<uint16_t>(L.param, e));
                gst<uint16_t>(L.param, e, (uint16_t)f32_to_f16_rne(p + u));
            } else if (L.param_dtype == RF_BF16) {
                const float p = bf16_bits_to_f32(gld<uint16_t>(L.param, e));
                gst<uint16_t>(L.param, e, (uint16_t)apply_bf16<PACKED>(p, u, sr, L.bits, lk0, lk1, e));
            } else {
                gst<float>(L.param, e, gld<float>(L.param, e) + u);
            }
        }
    }
}

// optax.MultiSteps' gradient accumulation (finetune/builders.py:1614-1620):
// per element, in the promoted dtype of the grad and the accumulator (f32
// unless both are the same 16-bit type, whose every operation then rounds
// to nearest even), mean: acc + (g - acc) / (n_acc + 1) (Welford's running
// mean), sum: g + acc, zero: 0 * acc (MultiSteps' (1 - emit) * acc after an
// emitting step: a signed zero, NaN where acc was not finite); the result is
// stored in the accumulator's dtype.  Work units as in k_apply.
__device__ __forceinline__ float acc_op(int32_t mode, int32_t cdt, float g, float a, float div)
{
    if (mode == RF_ACC_MEAN) {
        const float d = round_to_dtype(g - a, cdt);
        const float q = round_to_dtype(d / div, cdt);
        return round_to_dtype(a + q, cdt);
    }
    return round_to_dtype(g + a, cdt);
}

__global__ __launch_bounds__(WG) void k_accumulate(const rf_accum_leaf* __restrict__ leaves,
                                                   const Seg* __restrict__ segs, int64_t nunits, int32_t mode,
                                                   int32_t n_acc)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    int32_t s = 0, cur = -1;
    const int32_t nseg = segs[0].nseg;
    rf_accum_leaf L{};
    int32_t cdt = RF_F32;
    float div = 1.0f;
    bool vec = false;
    for (int64_t u = wave; u < nunits; u += nwaves) {
        s = seek_seg(segs, nseg, s, u);
        if (segs[s].leaf != cur) {
            cur = segs[s].leaf;
            L = leaves[cur];
            cdt = L.grad_dtype == L.acc_dtype ? L.acc_dtype : RF_F32;
            div = round_to_dtype((float)n_acc + 1.0f, cdt);  // the int32 count promoted to the compute dtype
            vec = ((uintptr_t)L.grad % 16 == 0) && ((uintptr_t)L.acc % 16 == 0);
        }
        const int64_t e_begin = (u - segs[s].unit_start) * APPLY_UNIT;
        const int64_t e_end = min(L.size, e_begin + APPLY_UNIT);
        const int64_t v_end = vec ? e_begin + ((e_end - e_begin) / 8) * 8 : e_begin;
        for (int64_t e0 = e_begin + lane * 8; e0 < v_end; e0 += WAVE * 8) {
            float g[8], a[8];
            load8_dt(L.acc, L.acc_dtype, e0, a);
            if (mode == RF_ACC_ZERO) {
#pragma unroll
                for (int t = 0; t < 8; ++t) a[t] = 0.0f * a[t];
            } else {
                load8_dt(L.grad, L.grad_dtype, e0, g);
#pragma unroll
                for (int t = 0; t < 8; ++t) a[t] = acc_op(mode, cdt, g[t], a[t], div);
            }
            if (L.acc_dtype == RF_F32) {
                store8_f32(L.acc, e0, a);
            } else {
                uint32_t h[8];
#pragma unroll
                for (int t = 0; t < 8; t += 2) {
                    const uint32_t w2 = L.acc_dtype == RF_F16 ? pack_f16x2_rne(a[t], a[t + 1])
                                                              : pack_bf16x2_rne(a[t], a[t + 1]);
                    h[t] = w2 & 0xFFFFu;
                    h[t + 1] = w2 >> 16;
                }
                store8_bf16(L.acc, e0, h);
            }
        }
        for (int64_t e = v_end + lane; e < e_end; e += WAVE) {
            const float a = load1(L.acc, L.acc_dtype, e);
            const float r = mode == RF_ACC_ZERO ? 0.0f * a : acc_op(mode, cdt, load1(L.grad, L.grad_dtype, e), a, div);
            store1(L.acc, L.acc_dtype, e, r);
        }
    }
}

// Global-norm clipping pre-pass (finetune/transforms.py:57-82): sum of
// squares of the f32 grad values, in f64 per NORM_UNIT-element unit (exact
// products, negligible accumulation error), then per leaf rounded once to
// f32, then the leaf sums added in f32 in leaf order; norm = sqrtf(total),
// scale = min(1, max_norm / (norm + 1e-6)) with NaN propagating.
constexpr int64_t NORM_UNIT = 16384;

// Work units per wave of the work-list kernels (worklist_grid).
constexpr int64_t STEP_UNITS_PER_WAVE = 16;
// Launch shape of a step (step_grid): waves take runs of consecutive blocks
// before their grid stride, about `per_wave` units each, and the grid is a
// whole number of chip-fulls of workgroups.  The fused nearest-rounding
// steps of the hardware direction (the memory-bound instances) take runs of
// 2 and 8 units per wave; the others (stochastic rounding, the IEEE
// direction, update-only) runs of 4 and 16.  Both shapes in turn on one GPU
// (two processes each): the Llama-7B step 12.78 -> 12.51 ms, with f32
// params 20.1-20.6 -> 19.1-19.6 ms, the ragged tree 0.467-0.473 -> 0.457-
// 0.465 ms; under the short shape moment SR ran 1.3 %, exact mode 2 % and
// the update-only step 0.5 % slower.  Runs of 1 were 1-6 % slower than
// either, and earlier (plain accesses) runs of 4 beat one block per run and
// a free grid by 0.7 % (Llama-7B) to 11 % (the ragged tree).
struct StepShape {
    int32_t run;
    int64_t per_wave;
};
constexpr StepShape STEP_SHAPE_STREAM = {2, 8};
constexpr StepShape STEP_SHAPE_HEAVY = {4, 16};
// Launches of at least this many fast blocks per CU (64 per resident wave
// at 3 waves per SIMD: far more output than the caches hold) store f32
// updates and params nontemporally (KHp.upd_nt).
constexpr int64_t UPD_NT_MIN_BLOCKS_PER_CU = 64 * 12;
#ifndef RF_STEP_GRID_ROUNDS
#define RF_STEP_GRID_ROUNDS 1
#endif
constexpr bool STEP_GRID_ROUNDS = RF_STEP_GRID_ROUNDS != 0;

__global__ __launch_bounds__(WG) void k_gnorm_partial(const rf_adam8_leaf* __restrict__ leaves,
                                                      const Seg* __restrict__ nsegs, int64_t nunits,
                                                      double* __restrict__ part)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    int32_t s = 0;
    const int32_t nseg = nsegs[0].nseg;
    for (int64_t u = wave; u < nunits; u += nwaves) {
        s = seek_seg(nsegs, nseg, s, u);
        const Seg sg = nsegs[s];
        const rf_adam8_leaf& L = leaves[sg.leaf];
        const int64_t e_begin = (u - sg.unit_start) * NORM_UNIT;
        const int64_t e_end = min(L.size, e_begin + NORM_UNIT);
        double acc = 0.0;
        if (e_end - e_begin == NORM_UNIT && ((uintptr_t)L.grad & 15u) == 0) {
            for (int64_t e0 = e_begin + lane * 8; e0 < e_end; e0 += 512) {
                float x[8];
                if (L.grad_dtype == RF_BF16) load8<uint16_t>(L.grad, e0, x);
                else if (L.grad_dtype == RF_F16) load8<_Float16>(L.grad, e0, x);
                else load8<float>(L.grad, e0, x);
#pragma unroll
                for (int t = 0; t < 8; ++t) acc += (double)x[t] * (double)x[t];
            }
        } else {
            for (int64_t e = e_begin + lane; e < e_end; e += WAVE) {
                const double x = load1(L.grad, L.grad_dtype, e);
                acc += x * x;
            }
        }
        acc = wave_sum_f64(acc);
        if (lane == 0) part[u] = acc;
    }
}

__global__ __launch_bounds__(WG) void k_gnorm_leaf(const Seg* __restrict__ nsegs, int32_t nseg,
                                                   const double* __restrict__ part, double* __restrict__ leafsum)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    for (int64_t i = wave; i < nseg; i += nwaves) {
        double acc = 0.0;
        for (int64_t u = nsegs[i].unit_start + lane; u < nsegs[i + 1].unit_start; u += WAVE) acc += part[u];
        acc = wave_sum_f64(acc);
        if (lane == 0) leafsum[i] = acc;
    }
}

// clip = (scale, norm, finite as f32, finite as int32 bits).  A leaf's f64 sum of squares is finite
// exactly when all its grads are: squares of finite f32 values (< 2^256)
// cannot overflow an f64 sum, and an Inf or NaN element makes it Inf or NaN.
__global__ void k_gnorm_finish(const double* __restrict__ leafsum, int32_t nseg, float max_norm,
                               float* __restrict__ clip, float* __restrict__ out, int32_t* __restrict__ finite_out)
{
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float total = 0.0f;
    bool finite = true;
    for (int32_t i = 0; i < nseg; ++i) {
        const double ls = leafsum[i];
        finite = finite && __builtin_isfinite(ls);
        total = total + (float)ls;
    }
    const float norm = sqrtf(total);
    const float q = max_norm / (norm + 1e-6f);
    const float scale = (q < 1.0f || q != q) ? q : 1.0f;  // jnp.minimum(1.0, q): NaN propagates
    clip[0] = scale;
    clip[1] = norm;
    clip[2] = finite ? 1.0f : 0.0f;
    clip[3] = __int_as_float(finite ? 1 : 0);  // the int32 flag copied to the host
    if (out) {
        out[0] = scale;
        out[1] = norm;
    }
    if (finite_out) *finite_out = finite ? 1 : 0;
}

// ---------------------------------------------------------------- Magma --
// Momentum-aligned update masking of scale_by_adam(use_magma=True)
// (optim/magma.py:15-132).  Work units are NORM_UNIT-element ranges of a
// leaf; every leaf has a segment (empty leaves an empty one), so segment i is
// leaf i.


// Per-unit f64 partial sums of g*m', g*g and m'*m', m' = f32(b1*mu) +
// f32(omb1*g): the step's new first moment (utils.py:437-467).
__global__ __launch_bounds__(WG) void k_magma_partial(const rf_magma_leaf* __restrict__ leaves,
                                                      const Seg* __restrict__ segs, int64_t nunits, float b1,
                                                      float omb1, double* __restrict__ part)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    int32_t s = 0;
    const int32_t nseg = segs[0].nseg;
    for (int64_t u = wave; u < nunits; u += nwaves) {
        s = seek_seg(segs, nseg, s, u);
        const Seg sg = segs[s];
        const rf_magma_leaf& L = leaves[sg.leaf];
        const int64_t e_begin = (u - sg.unit_start) * NORM_UNIT;
        const int64_t e_end = min(L.size, e_begin + NORM_UNIT);
        double dot = 0.0, gg = 0.0, mm = 0.0;
        auto add = [&](float g, float mp) {
            const float t1 = b1 * mp;
            const float t2 = omb1 * g;
            const float m = t1 + t2;
            dot += (double)g * (double)m;
            gg += (double)g * (double)g;
            mm += (double)m * (double)m;
        };
        if (e_end - e_begin == NORM_UNIT && ((uintptr_t)L.grad & 15u) == 0 && ((uintptr_t)L.mu & 15u) == 0) {
            for (int64_t e0 = e_begin + lane * 8; e0 < e_end; e0 += 512) {
                float g[8], mp[8];
                load8_dt(L.grad, L.grad_dtype, e0, g);
                load8_dt(L.mu, L.mu_dtype, e0, mp);
#pragma unroll
                for (int t = 0; t < 8; ++t) add(g[t], mp[t]);
            }
        } else {
            for (int64_t e = e_begin + lane; e < e_end; e += WAVE)
                add(load1(L.grad, L.grad_dtype, e), load1(L.mu, L.mu_dtype, e));
        }
        dot = wave_sum_f64(dot);
        gg = wave_sum_f64(gg);
        mm = wave_sum_f64(mm);
        if (lane == 0) {
            part[3 * u] = dot;
            part[3 * u + 1] = gg;
            part[3 * u + 2] = mm;
        }
    }
}

// Leaf i's three sums from its units' partials: one workgroup per leaf
// (grid-strided over leaves), thread t summing units t, t + WG, ... with
// four in flight, then wave and workgroup sums.  The order depends only on
// WG, so a leaf's sums are the same on every run.
__global__ __launch_bounds__(WG) void k_magma_leaf(const Seg* __restrict__ segs, int32_t nseg,
                                                   const double* __restrict__ part, double* __restrict__ sums)
{
    __shared__ double red[WAVES_PER_WG][3];
    const int lane = threadIdx.x & (WAVE - 1);
    const int w = threadIdx.x / WAVE;
    for (int64_t i = blockIdx.x; i < nseg; i += gridDim.x) {
        double acc[3] = {0.0, 0.0, 0.0};
        const int64_t u1 = segs[i + 1].unit_start;
        int64_t u = segs[i].unit_start + threadIdx.x;
        for (; u + 3 * WG < u1; u += 4 * WG) {
            double t[4][3];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int k = 0; k < 3; ++k) t[j][k] = part[3 * (u + j * WG) + k];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int k = 0; k < 3; ++k) acc[k] += t[j][k];
        }
        for (; u < u1; u += WG)
#pragma unroll
            for (int k = 0; k < 3; ++k) acc[k] += part[3 * u + k];
#pragma unroll
        for (int k = 0; k < 3; ++k) acc[k] = wave_sum_f64(acc[k]);
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < 3; ++k) red[w][k] = acc[k];
        }
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                double a = red[0][k];
                for (int ww = 1; ww < WAVES_PER_WG; ++ww) a += red[ww][k];
                sums[3 * i + k] = a;
            }
        }
        __syncthreads();
    }
}

// Per leaf (one thread each): the f32 cosine, the new score and the masked
// factor (magma.py:98-122); scores[i] goes from s_prev to s_new.
__global__ void k_magma_factor(const rf_magma_leaf* __restrict__ leaves, int32_t n, const double* __restrict__ sums,
                               float* __restrict__ scores, float* __restrict__ factor, float p, float tau,
                               uint32_t k0, uint32_t k1)
{
    const int32_t i = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= n) return;
    const float dot = (float)sums[3 * i];
    const float ng = (float)sums[3 * i + 1];
    const float nm = (float)sums[3 * i + 2];
    const float prod = sqrtf(ng) * sqrtf(nm);
    const float denom = prod != prod ? prod : fmaxf(prod, 1e-12f);  // jnp.maximum keeps a NaN
    float cs = dot / denom;
    if (cs != cs) cs = 0.0f;                       // jnp.nan_to_num(nan=0.0)
    cs = cs < -1.0f ? -1.0f : (cs > 1.0f ? 1.0f : cs);  // jnp.clip (an infinity lands on +-1)
    const float s_tilde = 1.0f / (1.0f + expf(-(cs / tau)));  // jax.nn.sigmoid
    const float a = 0.9f * scores[i];
    const float b = 0.1f * s_tilde;
    const float s_new = a + b;
    // jax.random.bernoulli(split(key, n_keys)[key_index], p): uniform < p
    uint32_t b0, b1;
    jax_split(k0, k1, (uint32_t)leaves[i].key_index, b0, b1);
    const bool keep = uniform_from_bits(jax_bits(b0, b1, 0)) < p;
    scores[i] = s_new;
    factor[i] = (keep ? 1.0f : 0.0f) * s_new;
}

// updates = neg_lr * (factor[leaf] * updates) over the same units.
__global__ __launch_bounds__(WG) void k_magma_apply(const rf_magma_leaf* __restrict__ leaves,
                                                    const Seg* __restrict__ segs, int64_t nunits,
                                                    const float* __restrict__ factor, float neg_lr)
{
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t wave = (int64_t)blockIdx.x * WAVES_PER_WG + uniform_u32(threadIdx.x / WAVE);
    const int64_t nwaves = (int64_t)gridDim.x * WAVES_PER_WG;
    int32_t s = 0;
    const int32_t nseg = segs[0].nseg;
    for (int64_t u = wave; u < nunits; u += nwaves) {
        s = seek_seg(segs, nseg, s, u);
        const Seg sg = segs[s];
        RF_GLOBAL float* up = gstore_ptr<float>(leaves[sg.leaf].updates, 0);
        const float f = factor[sg.leaf];
        const int64_t e_begin = (u - sg.unit_start) * NORM_UNIT;
        const int64_t e_end = min(leaves[sg.leaf].size, e_begin + NORM_UNIT);
        if (e_end - e_begin == NORM_UNIT && ((uintptr_t)up & 15u) == 0) {
            for (int64_t e0 = e_begin + lane * 4; e0 < e_end; e0 += 256) {
                float4 v = *(const RF_GLOBAL float4*)(up + e0);
                v.x = neg_lr * (f * v.x);
                v.y = neg_lr * (f * v.y);
                v.z = neg_lr * (f * v.z);
                v.w = neg_lr * (f * v.w);
                *(RF_GLOBAL float4*)(up + e0) = v;
            }
        } else {
            for (int64_t e = e_begin + lane; e < e_end; e += WAVE) up[e] = neg_lr * (f * up[e]);
        }
    }
}

// Standalone clip_by_global_norm: out = grad * scale per leaf (blockIdx.y =
// leaf), with the leaf-dtype semantics of the fused path.
__global__ __launch_bounds__(WG) void k_clip_scale(const rf_clip_leaf* __restrict__ leaves,
                                                   const float* __restrict__ clip)
{
    const rf_clip_leaf L = leaves[blockIdx.y];
    const float cs = clip[0];
    const float cs16 = round_to_bf16(cs);
    const float csh = round_to_f16(cs);
    const int64_t tid = (int64_t)blockIdx.x * WG + threadIdx.x;
    const int64_t nthreads = (int64_t)gridDim.x * WG;
    const bool bf16 = L.dtype == RF_BF16;
    const bool vec = ((uintptr_t)L.grad % 16 == 0) && ((uintptr_t)L.out % 16 == 0);
    const int64_t ngroups = vec ? L.size / 8 : 0;
    for (int64_t gi = tid; gi < ngroups; gi += nthreads) {
        const int64_t e0 = gi * 8;
        float x[8];
        if (L.dtype == RF_F16) {
            load8<_Float16>(L.grad, e0, x);
            uint32_t hb[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) hb[t] = f32_to_f16_rne(x[t] * csh);
            store8_bf16(L.out, e0, hb);
        } else if (bf16) {
            load8<uint16_t>(L.grad, e0, x);
            uint32_t hb[8];
#pragma unroll
            for (int t = 0; t < 8; t += 2) {
                const uint32_t w2 = pack_bf16x2_rne(x[t] * cs16, x[t + 1] * cs16);
                hb[t] = w2 & 0xFFFFu;
                hb[t + 1] = w2 >> 16;
            }
            store8_bf16(L.out, e0, hb);
        } else {
            load8<float>(L.grad, e0, x);
#pragma unroll
            for (int t = 0; t < 8; ++t) x[t] = x[t] * cs;
            store8_f32(L.out, e0, x);
        }
    }
    for (int64_t e = ngroups * 8 + tid; e < L.size; e += nthreads) {
        if (L.dtype == RF_F16) {
            gst<uint16_t>(L.out, e, (uint16_t)f32_to_f16_rne(f16_bits_to_f32(gld<uint16_t>(L.grad, e)) * csh));
        } else if (bf16) {
            gst<uint16_t>(L.out, e, (uint16_t)f32_to_bf16_rne(bf16_bits_to_f32(gld<uint16_t>(L.grad, e)) * cs16));
        } else {
            gst<float>(L.out, e, gld<float>(L.grad, e) * cs);
        }
    }
}

// =================================================================== host ==
namespace {

// ---- codebooks and lookup tables (rollfast optim/adam8.py:461-503) ----
void build_codebook(bool is_signed, float out[256])
{
    std::vector<double> data;
    const int total_bits = 8, max_exponent_bits = 7;
    const int non_sign_bits = total_bits - 1;
    for (int index = 0; index < max_exponent_bits; ++index) {
        const int e = -(max_exponent_bits - 1) + index;
        const double exponent_scale = e == 0 ? 1.0 : std::pow(10.0, (double)e);
        const int items = is_signed ? (1 << (index + non_sign_bits - max_exponent_bits)) + 1
                                    : (1 << (index + non_sign_bits - max_exponent_bits + 1)) + 1;
        const double step = (1.0 - 0.1) / (double)(items - 1);
        for (int i = 0; i + 1 < items; ++i) {
            volatile double left = 0.1 + step * (double)i;
            volatile double right = 0.1 + step * (double)(i + 1);
            const double mean = (left + right) / 2.0;
            data.push_back(exponent_scale * mean);
            if (is_signed) data.push_back(-exponent_scale * mean);
        }
    }
    data.push_back(0.0);
    data.push_back(1.0);
    std::sort(data.begin(), data.end());
    for (int i = 0; i < 256; ++i) out[i] = (float)data[i];
}

inline uint32_t fbits(float f)
{
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
inline float bitsf(uint32_t u)
{
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
// Monotone key of an f32 (value order, -0 before +0).
inline uint32_t fkey(float f)
{
    const uint32_t u = fbits(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
inline float unkey(uint32_t k) { return bitsf((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }

// The reference's choice between neighbours lo < hi for lo < n <= hi.
inline bool picks_upper(float lo, float hi, volatile float n)
{
    volatile float du = hi - n;
    volatile float dl = n - lo;
    return std::fabs((float)du) < std::fabs((float)dl);
}

// Smallest f32 n in (lo, hi] for which the upper neighbour wins.
float upper_threshold(float lo, float hi)
{
    uint32_t a = fkey(lo) + 1u, b = fkey(hi);
    while (a < b) {
        const uint32_t mid = a + (b - a) / 2u;
        if (picks_upper(lo, hi, unkey(mid))) b = mid;
        else a = mid + 1u;
    }
    return unkey(a);
}

inline uint32_t count_le(const float* t, float a)
{
    uint32_t c = 0;
    for (int i = 0; i < 256; ++i) c += (t[i] <= a) ? 1u : 0u;
    return c;
}

struct HostTables {
    std::vector<uint8_t> bytes;
    std::string error;
};

// Candidate of each magnitude cell for one sign: the number of thresholds at
// or below the cell's low end in value space; a cell may hold at most one
// threshold.  CELL_LO also stands for every magnitude below it.
bool fill_cells(const float* thr, bool negative, uint8_t* cand, std::string& err)
{
    for (uint32_t cell = CELL_LO; cell <= CELL_HI; ++cell) {
        const float mlo = cell == CELL_LO ? 0.0f : bitsf(cell << CELL_SHIFT);
        const float mhi = bitsf((cell << CELL_SHIFT) | ((1u << CELL_SHIFT) - 1u));
        const float lo = negative ? -mhi : mlo;
        const float hi = negative ? -mlo : mhi;
        const uint32_t c0 = count_le(thr, lo);
        const uint32_t c1 = count_le(thr, hi);
        if (c1 > c0 + 1u) {
            err = "lookup cell " + std::to_string(cell) + " holds more than one threshold";
            return false;
        }
        if (c0 > 255u || thr[c0] <= lo) {
            err = "threshold table is not ascending";
            return false;
        }
        cand[cell - CELL_LO] = (uint8_t)c0;
    }
    return true;
}

// Searchsorted candidate of each magnitude cell for one sign: the number of
// codebook entries below the cell's low end in value space, so that for n in
// the cell searchsorted_left(cb, n) = cand + (cb[cand] < n).  A cell may hold
// at most one codebook entry.
bool fill_search_cells(const float* cb, bool negative, uint8_t* cand, std::string& err)
{
    for (uint32_t cell = CELL_LO; cell <= CELL_HI; ++cell) {
        const float mlo = cell == CELL_LO ? 0.0f : bitsf(cell << CELL_SHIFT);
        const float mhi = bitsf((cell << CELL_SHIFT) | ((1u << CELL_SHIFT) - 1u));
        const float lo = negative ? -mhi : mlo;
        const float hi = negative ? -mlo : mhi;
        uint32_t below = 0, upto = 0;
        for (int i = 0; i < 256; ++i) {
            below += cb[i] < lo ? 1u : 0u;
            upto += cb[i] <= hi ? 1u : 0u;
        }
        if (upto > below + 1u) {
            err = "search cell " + std::to_string(cell) + " holds more than one codebook entry";
            return false;
        }
        if (below > 255u) {
            err = "search cell above the codebook";
            return false;
        }
        cand[cell - CELL_LO] = (uint8_t)below;
    }
    return true;
}

HostTables build_tables()
{
    HostTables ht;
    ht.bytes.assign(TABLE_BYTES, 0);
    uint8_t* b = ht.bytes.data();
    float cbs[256], cbu[256];
    build_codebook(true, cbs);
    build_codebook(false, cbu);
    std::memcpy(b + L_CBS, cbs, 1024);
    std::memcpy(b + L_CBU, cbu, 1024);
    for (int i = 0; i < 255; ++i) {
        if (!(cbs[i] < cbs[i + 1]) || !(cbu[i] < cbu[i + 1])) {
            ht.error = "codebook is not strictly increasing";
            return ht;
        }
    }
    // Value-space thresholds t_i between cb[i] and cb[i+1]; t[255] = +inf.
    float ts[256], tu[256];
    for (int i = 0; i < 255; ++i) {
        ts[i] = upper_threshold(cbs[i], cbs[i + 1]);
        tu[i] = upper_threshold(cbu[i], cbu[i + 1]);
    }
    ts[255] = INFINITY;
    tu[255] = INFINITY;
    std::memcpy(b + L_TS, ts, 1024);
    std::memcpy(b + L_TU, tu, 1024);
    if (!fill_cells(ts, false, b + L_CANDS, ht.error)) return ht;
    if (!fill_cells(ts, true, b + L_CANDS + CANDS_SIGN_STRIDE, ht.error)) return ht;
    if (!fill_cells(tu, false, b + L_CANDU, ht.error)) return ht;
    return ht;
}

const HostTables& host_tables()
{
    static HostTables t = build_tables();
    return t;
}

// The f32 nearest to 1/d (ties to even) for a positive finite f32 d: y*d is
// exact in double, so |y*d - 1| = d*|y - 1/d| ranks the candidates exactly.
float rcp_rn(float d)
{
    float best = (float)(1.0 / (double)d);
    double err = std::fabs((double)best * (double)d - 1.0);
    const float around[2] = {std::nextafter(best, 0.0f), std::nextafter(best, INFINITY)};
    for (float c : around) {
        const double e = std::fabs((double)c * (double)d - 1.0);
        if (e < err || (e == err && (fbits(c) & 1u) == 0u)) {
            best = c;
            err = e;
        }
    }
    return best;
}

// Neighbour records of the moment-SR code choice for one codebook: per
// ui >= 1, {cb[ui - 1], (cb[ui] - cb[ui - 1]) 2^-16, RN(1 / that gap) 2^16
// (0 for an empty gap), 0}, the quotient's operands scaled so that it comes
// out as 65536 p; for ui = 0, {-2, 0, 65536, 0}, whose quotient exceeds
// every draw (the kernel's sr_upper).  The gaps (f32 differences of codebook
// values in [-1, 1]) and their reciprocals stay normal under the scaling.
void fill_sr_records(const float* cb, float* rec)
{
    rec[0] = -2.0f;
    rec[1] = 0.0f;
    rec[2] = 65536.0f;
    rec[3] = 0.0f;
    for (int ui = 1; ui < 256; ++ui) {
        const float lv = cb[ui - 1];
        const float d = cb[ui] - lv;
        rec[4 * ui + 0] = lv;
        rec[4 * ui + 1] = d * 0x1p-16f;
        rec[4 * ui + 2] = d > 0.0f ? rcp_rn(d) * 65536.0f : 0.0f;
        rec[4 * ui + 3] = 0.0f;
    }
}

// The image moment-SR launches stage instead: the same layout, with search
// candidates in the candidate regions (the threshold regions are unused),
// followed by the neighbour records.
HostTables build_search_tables()
{
    HostTables ht = build_tables();
    if (!ht.error.empty()) return ht;
    ht.bytes.resize(SEARCH_BYTES, 0);
    uint8_t* b = ht.bytes.data();
    const float* cbs = (const float*)(b + L_CBS);
    const float* cbu = (const float*)(b + L_CBU);
    std::memset(b + L_TS, 0, 1024);
    std::memset(b + L_TU, 0, 1024);
    if (!fill_search_cells(cbs, false, b + L_CANDS, ht.error)) return ht;
    if (!fill_search_cells(cbs, true, b + L_CANDS + CANDS_SIGN_STRIDE, ht.error)) return ht;
    if (!fill_search_cells(cbu, false, b + L_CANDU, ht.error)) return ht;
    fill_sr_records(cbs, (float*)(b + L_SRS));
    fill_sr_records(cbu, (float*)(b + L_SRU));
    return ht;
}

const HostTables& host_search_tables()
{
    static HostTables t = build_search_tables();
    return t;
}

// Host emulation of the moment-SR kernels' searchsorted index of a
// normalised n: the reference's ui = clip(searchsorted_left(cb, n), 0, 255)
// with n clipped to [cb[0], cb[255]].  The kernels' table path sees only
// finite n in [-1, 1] (signed) or [0, 1] (unsigned) and needs no clip there,
// since a value in [-1, cb[0]) counts no entry either; NaN sorts last.
uint32_t host_search_index(const uint8_t* tb, int32_t quantizer, float n)
{
    const bool uns = quantizer == RF_Q_DYNAMIC_UNSIGNED;
    const float* cb = (const float*)(tb + (uns ? L_CBU : L_CBS));
    if (n != n) return 255u;
    n = n < cb[0] ? cb[0] : n;
    n = n > cb[255] ? cb[255] : n;
    const uint32_t nb = fbits(n);
    const uint32_t cell = (nb >> CELL_SHIFT) & 0xFFFFu;
    const uint32_t idx = cell > CELL_LO ? cell - CELL_LO : 0u;
    const uint32_t cand = uns ? tb[L_CANDU + idx] : tb[L_CANDS + (nb >> 31) * CANDS_SIGN_STRIDE + idx];
    return cand + (cb[cand] < n ? 1u : 0u);
}

// Host emulation of the kernels' table lookup on a normalised n (NaN and the
// clip to [cb[0], cb[255]] as in the literal path).
uint32_t host_table_code(const uint8_t* tb, int32_t quantizer, float n)
{
    const bool uns = quantizer == RF_Q_DYNAMIC_UNSIGNED;
    const float* cb = (const float*)(tb + (uns ? L_CBU : L_CBS));
    if (n != n) return 254u;
    n = n < cb[0] ? cb[0] : n;
    n = n > cb[255] ? cb[255] : n;
    const uint32_t nb = fbits(n);
    const uint32_t cell = (nb >> CELL_SHIFT) & 0xFFFFu;
    const uint32_t idx = cell > CELL_LO ? cell - CELL_LO : 0u;
    uint32_t cand;
    float t;
    if (uns) {
        cand = tb[L_CANDU + idx];
        std::memcpy(&t, tb + L_TU + cand * 4u, 4);
    } else {
        cand = tb[L_CANDS + (nb >> 31) * CANDS_SIGN_STRIDE + idx];
        std::memcpy(&t, tb + L_TS + cand * 4u, 4);
    }
    return cand + (n >= t ? 1u : 0u);
}

}  // namespace

// ---- device-scope arrays (one copy per GPU, held until the process ends) ----
// The codebooks and requantization lookup tables every step kernel stages.
static __device__ __align__(256) uint4 lookup_tables[TABLE_BYTES / 16];
// The same for moment stochastic rounding: search candidates (searchsorted
// indices) instead of nearest-code thresholds.
static __device__ __align__(256) uint4 search_tables[SEARCH_BYTES / 16];
// rf_adam8_step_noalloc's working memory: the leaf and group tables, the work
// lists and the norm pre-pass's partial sums of one call.  Every call on a
// GPU shares that GPU's copy and leaves its contents behind; nothing in it
// needs to start at zero (each kernel writes every slot it later reads).
// Calls that overlap on one GPU (different streams, or threads racing to
// enqueue) race on it.
static __device__ __align__(256) uint8_t scratch[RF_NOALLOC_SCRATCH_BYTES];

namespace {

// ---- per-device state ----
// Staging of the standalone entry points (clip, Magma, apply, accumulate):
// a call's leaf table and work list go through a pinned host buffer and a
// device buffer that also holds its scratch (partial sums).  A ring of
// STAGE_RING slots per device: a slot grows (allocates) only when a call
// needs more than any earlier one, otherwise it is reused; the event
// recorded after the call's last launch guards its next use, and a slot is
// held by one call at a time.  Steady-state calls allocate nothing.
constexpr int STAGE_RING = 4;
// Events that only order work -- the host waits on them before it reuses a
// table buffer, or another stream waits on them -- and guard no data the
// host reads: no timing and no system-scope release (no cache writeback
// between steps).  The pre-pass event, which guards the finite flag's copy
// to host memory, keeps the default fences.
constexpr unsigned ORDER_EVENT_FLAGS = hipEventDisableTiming | hipEventDisableSystemFence;
struct StageSlot {
    std::mutex mu;  // held from acquire to release
    uint8_t* host = nullptr;
    size_t host_cap = 0;
    uint8_t* dev = nullptr;
    size_t dev_cap = 0;
    hipEvent_t ev = nullptr;
    bool pending = false;
};

constexpr int MAX_DEV = 64;
struct DevState {
    bool ready = false;
    uint4* tables = nullptr;     // this device's lookup_tables
    uint4* search = nullptr;     // this device's search_tables
    uint8_t* scratch_ptr = nullptr;  // this device's scratch
    // rf_adam8_step_noalloc's ordering of calls on this device: each call
    // makes its stream wait for the previous call's last launch (recorded
    // here) before it overwrites the scratch, under noalloc_mu so that the
    // wait-copy-launch-record sequences of racing threads do not interleave.
    hipEvent_t noalloc_ev = nullptr;
    std::mutex noalloc_mu;
    int num_cus = 0;
    StageSlot stage[STAGE_RING];
    std::atomic<uint32_t> stage_next{0};
};
std::mutex g_mu;
DevState g_dev[MAX_DEV];

// One call's hold on a staging slot: host() is pinned memory for the
// tables, dev() their device copy followed by the call's scratch.
class Staged {
public:
    ~Staged() { release(); }

    rf_status acquire(DevState* ds, size_t host_bytes, size_t dev_bytes)
    {
        slot_ = &ds->stage[ds->stage_next.fetch_add(1) % STAGE_RING];
        slot_->mu.lock();
        locked_ = true;
        if (slot_->pending) {
            HIP_TRY(hipEventSynchronize(slot_->ev));
            slot_->pending = false;
        }
        if (!slot_->ev) HIP_TRY(hipEventCreateWithFlags(&slot_->ev, ORDER_EVENT_FLAGS));
        host_bytes = std::max<size_t>(host_bytes, 256);
        dev_bytes = std::max<size_t>(dev_bytes, host_bytes);
        if (slot_->host_cap < host_bytes) {
            if (slot_->host) HIP_TRY(hipHostFree(slot_->host));
            slot_->host = nullptr;
            slot_->host_cap = 0;
            HIP_TRY(hipHostMalloc((void**)&slot_->host, host_bytes, hipHostMallocDefault));
            slot_->host_cap = host_bytes;
        }
        if (slot_->dev_cap < dev_bytes) {
            if (slot_->dev) HIP_TRY(hipFree(slot_->dev));
            slot_->dev = nullptr;
            slot_->dev_cap = 0;
            HIP_TRY(hipMalloc((void**)&slot_->dev, dev_bytes));
            slot_->dev_cap = dev_bytes;
        }
        return RF_OK;
    }

    uint8_t* host() const { return slot_->host; }
    uint8_t* dev() const { return slot_->dev; }

    // Copies the first `bytes` of host() to dev() on the stream.
    rf_status upload(size_t bytes, hipStream_t s)
    {
        if (bytes) HIP_TRY(hipMemcpyAsync(slot_->dev, slot_->host, bytes, hipMemcpyHostToDevice, s));
        return RF_OK;
    }

    // After the call's last launch: the slot is reusable once the stream
    // has passed this point.
    rf_status finish(hipStream_t s)
    {
        HIP_TRY(hipEventRecord(slot_->ev, s));
        slot_->pending = true;
        release();
        return RF_OK;
    }

private:
    void release()
    {
        if (locked_) slot_->mu.unlock();
        locked_ = false;
    }
    StageSlot* slot_ = nullptr;
    bool locked_ = false;
};

inline size_t up16(size_t x) { return (x + 15) & ~(size_t)15; }

// First use of a device: its arrays' addresses (with the device current,
// since each GPU holds its own copy at its own address) and the table upload
// (one synchronous copy; no allocation).
rf_status device_state(DevState** out)
{
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEV) return fail(RF_ERR_INVALID, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    DevState& d = g_dev[dev];
    if (!d.ready) {
        const HostTables& ht = host_tables();
        if (!ht.error.empty()) return fail(RF_ERR_INVALID, "table construction failed: " + ht.error);
        const HostTables& hs = host_search_tables();
        if (!hs.error.empty()) return fail(RF_ERR_INVALID, "search table construction failed: " + hs.error);
        HIP_TRY(hipDeviceGetAttribute(&d.num_cus, hipDeviceAttributeMultiprocessorCount, dev));
        HIP_TRY(hipGetSymbolAddress((void**)&d.tables, HIP_SYMBOL(lookup_tables)));
        HIP_TRY(hipGetSymbolAddress((void**)&d.search, HIP_SYMBOL(search_tables)));
        HIP_TRY(hipGetSymbolAddress((void**)&d.scratch_ptr, HIP_SYMBOL(scratch)));
        if (!d.tables || !d.search || !d.scratch_ptr)
            return fail(RF_ERR_HIP, "hipGetSymbolAddress returned a null address");
        HIP_TRY(hipEventCreateWithFlags(&d.noalloc_ev, ORDER_EVENT_FLAGS));
        HIP_TRY(hipMemcpy(d.tables, ht.bytes.data(), TABLE_BYTES, hipMemcpyHostToDevice));
        HIP_TRY(hipMemcpy(d.search, hs.bytes.data(), SEARCH_BYTES, hipMemcpyHostToDevice));
        d.ready = true;
    }
    *out = &d;
    return RF_OK;
}

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

inline bool valid_dtype(int32_t d) { return d == RF_F32 || d == RF_BF16 || d == RF_F16; }

// ---- kernel selection ----
// The fast kernel's instances: dtype_combo = 2*(param is bf16) + (grad is bf16)
// for f32/bf16 params and grads, COMBO_F16 for f16 params and grads; -1 (the
// generic kernel) for the other mixes, VEC_COMBO (its instance without the
// element-wise and quantized unit code) for a generic list that holds
// full-chunk fallback units only.
constexpr int COMBO_F16 = 4;
constexpr int GEN_LIST = 5;    // the generic kernel's work list
constexpr int GEN_TAIL = 6;    // build space: its fallback units, appended after its quantized ones
constexpr int64_t GEN_WAVE_PER_UNIT_MAX_ROUNDS = 8;  // mixed generic lists up to 8 chip-fulls: one unit per wave
constexpr int VEC_COMBO = -2;  // a generic list of full-chunk fallback units only

adam_kernel_t pick_adam_kernel(bool apply, bool msr, bool psr, bool nest, bool exact, int combo)
{
    if (combo == VEC_COMBO) msr = false;  // fallback units have no codes to round
    if (apply) {
        if (msr) return exact ? rf_pick_adam8_a1_m1_e1(combo, psr, nest) : rf_pick_adam8_a1_m1_e0(combo, psr, nest);
        return exact ? rf_pick_adam8_a1_m0_e1(combo, psr, nest) : rf_pick_adam8_a1_m0_e0(combo, psr, nest);
    }
    if (msr) return exact ? rf_pick_adam8_a0_m1_e1(combo, false, nest) : rf_pick_adam8_a0_m1_e0(combo, false, nest);
    return exact ? rf_pick_adam8_a0_m0_e1(combo, false, nest) : rf_pick_adam8_a0_m0_e0(combo, false, nest);
}


inline int dtype_combo(const rf_adam8_leaf& L)
{
    if (L.param_dtype == RF_F16 || L.grad_dtype == RF_F16)
        return L.param_dtype == RF_F16 && L.grad_dtype == RF_F16 ? COMBO_F16 : -1;
    return 2 * (L.param_dtype == RF_BF16 ? 1 : 0) + (L.grad_dtype == RF_BF16 ? 1 : 0);
}

struct OccKey {
    const void* fn;
    int dev;
    int blocks;
};
std::vector<OccKey> g_occ;

rf_status occupancy(const void* fn, int* blocks)
{
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    {
        std::lock_guard<std::mutex> lock(g_mu);
        for (const OccKey& k : g_occ)
            if (k.fn == fn && k.dev == dev) {
                *blocks = k.blocks;
                return RF_OK;
            }
    }
    int nb = 0;
    HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, WG, 0));
    if (nb < 1) nb = 1;
    std::lock_guard<std::mutex> lock(g_mu);
    g_occ.push_back({fn, dev, nb});
    *blocks = nb;
    return RF_OK;
}

int64_t nblocks_of(int64_t size, int64_t bs) { return size > 0 ? (size + bs - 1) / bs : 1; }

// Grid of a work-list kernel that walks `nunits` units, one per wave at a
// time: about `per_wave` units per wave, never fewer workgroups
// than fit on the chip at once, rounded to whole chip-fulls (the kernel's
// own occupancy), so that no last, mostly idle round of workgroups runs.
rf_status worklist_grid(const void* fn, const DevState* ds, int64_t nunits, unsigned* grid,
                        int64_t per_wave = STEP_UNITS_PER_WAVE)
{
    int occ = 1;
    const rf_status st = occupancy(fn, &occ);
    if (st != RF_OK) return st;
    const int64_t wg_needed = std::max<int64_t>(1, (nunits + WAVES_PER_WG - 1) / WAVES_PER_WG);
    const int64_t resident = (int64_t)ds->num_cus * occ;
    const int64_t spread = (nunits + (int64_t)WAVES_PER_WG * per_wave - 1) / ((int64_t)WAVES_PER_WG * per_wave);
    int64_t g = std::min(wg_needed, std::max(resident, spread));
    if (g > resident) g = std::min(wg_needed, std::max<int64_t>(1, (g + resident / 2) / resident) * resident);
    *grid = (unsigned)std::max<int64_t>(1, g);
    return RF_OK;
}

}  // namespace

// ---- plan ----
// Pointer tables for rf_adam8_plan_run_leaves, kept as a small cache of
// device copies.  A run whose leaf table (and group table) equals, byte for
// byte, one already uploaded launches on that copy: no validation pass (the
// same bytes passed it), no host copy and no upload between the previous
// step's last kernel and this step's first.  A training loop that cycles a
// few gradient buffers (the caching allocator hands the same ones back)
// hits every step.  Otherwise the least recently used slot takes the table:
// written into its pinned host buffer and copied to its device table on the
// stream.  The slot's event, recorded after every launch that used it,
// guards that overwrite, so a run waits for the device only when RING runs
// with distinct tables are still in flight.
constexpr int RING = 4;
struct RingSlot {
    rf_adam8_leaf* host = nullptr;  // leaf table, then (at group_off) the group table
    rf_adam8_leaf* dev = nullptr;
    hipEvent_t ev = nullptr;
    bool pending = false;
    bool valid = false;             // host and dev hold the same `span` bytes
    size_t span = 0;
    hipStream_t stream = nullptr;   // stream of the last launch that used the slot
    uint64_t last_use = 0;
};

// One launch per (param, grad) dtype combination present in the tree; each
// group has its own work list (ending in a sentinel) inside d_segs.
// Fed random bits present for every leaf that would read them: param bits
// (param SR), moment bits of quantized leaves (moment SR), moment bits of bf16
// fallback leaves stored with SR.  A leaf missing bits its flags require
// would make the kernel read through a null pointer, so runs refuse it.
struct BitsCover {
    bool pb = true, mb_quant = true, mb_store = true;
};

static BitsCover bits_cover(const rf_adam8_leaf* leaves, int32_t n)
{
    BitsCover c;
    for (int32_t i = 0; i < n; ++i) {
        const rf_adam8_leaf& L = leaves[i];
        if (L.size == 0) continue;
        const bool mb = L.mu_bits != nullptr && L.nu_bits != nullptr;
        if (!L.param_bits && L.param_dtype == RF_BF16) c.pb = false;  // SR rounds bf16 params only
        if (L.moment_kind == RF_MOMENT_QUANTIZED && !mb) c.mb_quant = false;
        if (L.moment_kind == RF_MOMENT_BF16 && (L.flags & RF_LEAF_STORE_SR) && !mb) c.mb_store = false;
    }
    return c;
}

struct PlanGroup {
    int combo;
    int64_t seg_offset;
    int64_t units;
    bool tables;   // the list holds quantized units (the kernel stages the LDS tables)
    int64_t lead;  // generic list: leading quantized units, a workgroup each
};

struct rf_adam8_plan {
    int device = 0;
    int32_t apply = 1;
    int32_t n_leaves = 0;
    int32_t group_cap = 1;    // group count of a grouped run: 1 + the largest leaf.group at creation
    size_t group_off = 0;     // byte offset of the group table in a ring slot
    int64_t total_units = 0;
    int64_t n_segs = 0;
    std::vector<PlanGroup> groups;
    rf_adam8_leaf* d_leaves = nullptr;  // creation-time pointer table
    Seg* d_segs = nullptr;
    // Global-norm clipping (allocated with the plan): one Seg per non-empty
    // leaf over NORM_UNIT-element units, per-unit f64 partial sums of squares,
    // per-leaf f32 sums and the (scale, norm) pair the step reads.
    Seg* d_nsegs = nullptr;
    int32_t n_nsegs = 0;
    int64_t n_norm_units = 0;
    double* d_npart = nullptr;
    double* d_leafsum = nullptr;
    float* d_clip = nullptr;  // (scale, norm, finite as f32, finite as int32 bits)
    // Magma sums written by the step (plans whose every leaf has unquantized
    // moments): one Seg per leaf whose unit_start is the leaf's first
    // 2048-element chunk slot, and an f64 triple per chunk (24 B per 2048
    // elements).  n_mchunks < 0: the plan cannot produce them.
    Seg* d_msegs = nullptr;
    int64_t n_mchunks = -1;
    double* d_mpart = nullptr;
    hipEvent_t ev_prepass = nullptr;  // recorded after the finite flag's copy to finite_host
    std::vector<rf_adam8_leaf> shape;   // creation-time table: the structure runs must match
    std::vector<uint8_t> vec;           // leaf has vectorised (16-byte aligned) work units
    BitsCover cover;  // which fed-bits arrays the creation-time table carries
    RingSlot ring[RING];
    uint32_t next = 0;
    std::mutex mu;
};

namespace {

bool release_plan(rf_adam8_plan* plan);

rf_status validate_leaf(const rf_adam8_leaf& L, int32_t i, int32_t apply)
{
    const std::string at = "leaf " + std::to_string(i) + ": ";
    if (L.size < 0) return fail(RF_ERR_INVALID, at + "negative size");
    if (!valid_dtype(L.param_dtype)) return fail(RF_ERR_UNSUPPORTED, at + "param dtype must be f32, bf16 or f16");
    if (!valid_dtype(L.grad_dtype)) return fail(RF_ERR_UNSUPPORTED, at + "grad dtype must be f32, bf16 or f16");
    if (L.moment_kind < RF_MOMENT_QUANTIZED || L.moment_kind > RF_MOMENT_F16) return fail(RF_ERR_INVALID, at + "bad moment kind");
    if ((L.flags & RF_LEAF_SCALE_BF16) && (L.flags & RF_LEAF_SCALE_F16))
        return fail(RF_ERR_INVALID, at + "RF_LEAF_SCALE_BF16 and RF_LEAF_SCALE_F16 together");
    if ((L.flags & (RF_LEAF_SCALE_BF16 | RF_LEAF_SCALE_F16)) && L.moment_kind != RF_MOMENT_QUANTIZED)
        return fail(RF_ERR_INVALID, at + "a scale dtype flag on unquantized moments");
    if (L.size > 0 && !L.grad) return fail(RF_ERR_INVALID, at + "null grad");
    if (L.size > 0 && !L.param && (apply || (L.flags & (RF_LEAF_DECAY | RF_LEAF_ZERO_DECAY))))
        return fail(RF_ERR_INVALID, at + "null param");
    if ((L.flags & RF_LEAF_ZERO_DECAY) && L.moment_kind == RF_MOMENT_QUANTIZED)
        return fail(RF_ERR_UNSUPPORTED, at + "RF_LEAF_ZERO_DECAY with quantized moments (scale_by_adam8 has no such term)");
    if (L.size > 0 && !apply && !L.updates) return fail(RF_ERR_INVALID, at + "null updates in update-only mode");
    // An empty unquantized-moment leaf has no work units (its buffers are
    // never read); a quantized one may still own a padded block.
    if ((L.size > 0 || L.moment_kind == RF_MOMENT_QUANTIZED) && (!L.mu || !L.nu))
        return fail(RF_ERR_INVALID, at + "null moment buffer");
    if (L.moment_kind == RF_MOMENT_QUANTIZED) {
        if (L.block_size <= 0) return fail(RF_ERR_INVALID, at + "block_size must be positive");
        if (!L.mu_scales || !L.nu_scales) return fail(RF_ERR_INVALID, at + "null scales");
    }
    if (L.state_index < 0 || L.param_index < 0) return fail(RF_ERR_INVALID, at + "negative key index");
    if (L.group < 0) return fail(RF_ERR_INVALID, at + "negative group index");
    return RF_OK;
}

// Stores the sentinel's index (the list's last record) in every record of a
// work list, for the kernels' segment search, and the generic list's count
// of leading quantized units (0 for the other lists).
void mark_list(std::vector<Seg>& list, int32_t lead = 0)
{
    const int32_t n = (int32_t)list.size() - 1;
    for (Seg& sg : list) {
        sg.nseg = n;
        sg.lead = lead;
    }
}

bool leaf_vec_ok(const rf_adam8_leaf& L, int32_t apply)
{
    const uintptr_t a = 16;
    if (!aligned(L.grad, a)) return false;
    if ((apply || (L.flags & RF_LEAF_DECAY)) && !aligned(L.param, a)) return false;
    if (!apply && !aligned(L.updates, a)) return false;
    if (L.moment_kind == RF_MOMENT_QUANTIZED) {
        if (!aligned(L.mu, 8) || !aligned(L.nu, 8)) return false;
        if (L.mu_bits && !aligned(L.mu_bits, a)) return false;
        if (L.nu_bits && !aligned(L.nu_bits, a)) return false;
    } else if (!aligned(L.mu, a) || !aligned(L.nu, a)) {
        return false;
    }
    if (L.param_bits && !aligned(L.param_bits, a)) return false;
    return true;
}

// Host-side work lists of a launch over a leaf table (validated here): the
// step's per-dtype lists, the norm pre-pass's units and Magma's chunk slots.
struct WorkLists {
    std::vector<Seg> segs;           // every launch's list, each ending in a sentinel
    std::vector<PlanGroup> groups;   // one launch per list
    int64_t units = 0;
    std::vector<Seg> nsegs;          // norm units (NORM_UNIT elements) of the non-empty leaves
    int32_t n_nsegs = 0;
    int64_t nunits = 0;
    std::vector<Seg> msegs;          // Magma chunk slots (every leaf unquantized), else empty
    int64_t mchunks = -1;
    std::vector<uint8_t> vecs;       // leaf has 16-byte aligned (vectorised) units
    std::vector<Seg> gsegs[7];       // build space: the lists of each dtype combination, the generic one and its tail
};

rf_status build_work_lists(const rf_adam8_leaf* leaves, int32_t n_leaves, int32_t apply, WorkLists& w)
{
    rf_status st = RF_OK;
    std::vector<Seg>* gsegs = w.gsegs;
    for (int c = 0; c <= GEN_TAIL; ++c) gsegs[c].clear();
    int64_t gunits[GEN_TAIL + 1] = {0, 0, 0, 0, 0, 0, 0};
    auto add = [&](int32_t leaf, int combo, int32_t kind, int64_t first, int64_t count) {
        if (count <= 0) return;
        Seg sg{};
        sg.unit_start = gunits[combo];
        sg.first = first;
        sg.leaf = leaf;
        sg.kind = kind;
        gsegs[combo].push_back(sg);
        gunits[combo] += count;
    };
    std::vector<uint8_t>& vecs = w.vecs;
    vecs.clear();
    for (int32_t i = 0; i < n_leaves; ++i) {
        const rf_adam8_leaf& L = leaves[i];
        st = validate_leaf(L, i, apply);
        if (st != RF_OK) return st;
        const bool vec = leaf_vec_ok(L, apply);
        vecs.push_back(vec ? 1 : 0);
        // Full aligned 2048-blocks go to the fast kernel of their dtype
        // combination; everything else to the generic kernel (GEN_LIST).
        const int combo = dtype_combo(L);
        if (L.moment_kind == RF_MOMENT_QUANTIZED) {
            const int64_t bs = L.block_size;
            const int64_t nb = nblocks_of(L.size, bs);
            if (bs == FAST_BS && vec && combo >= 0) {
                const int64_t nfull = L.size / bs;
                add(i, combo, KIND_QFAST, 0, nfull);
                add(i, GEN_LIST, KIND_QGEN, nfull, nb - nfull);
            } else {
                add(i, GEN_LIST, KIND_QGEN, 0, nb);
            }
        } else {
            // Full chunks of aligned leaves take the vectorised unit, the
            // tail element-wise units of EW_UNIT<apply> elements.
            const int64_t nfull = vec ? L.size / CHUNK : 0;
            const int64_t ew = apply ? EW_UNIT<true> : EW_UNIT<false>;
            add(i, GEN_TAIL, KIND_FALLBACK_VEC, 0, nfull);
            add(i, GEN_TAIL, KIND_FALLBACK, nfull * CHUNK / ew, (L.size - nfull * CHUNK + ew - 1) / ew);
        }
    }
    // The generic list holds the quantized units (the long ones: two passes
    // over a block) first, a workgroup each, then the fallback units, a wave
    // each.
    if (gunits[GEN_LIST] > INT32_MAX)
        return fail(RF_ERR_UNSUPPORTED, "more than 2^31 - 1 partial or odd-sized quantized blocks in one launch");
    const int64_t gen_lead = gunits[GEN_LIST];
    for (Seg sg : gsegs[GEN_TAIL]) {
        sg.unit_start += gunits[GEN_LIST];
        gsegs[GEN_LIST].push_back(sg);
    }
    gunits[GEN_LIST] += gunits[GEN_TAIL];
    std::vector<Seg>& segs = w.segs;
    std::vector<PlanGroup>& groups = w.groups;
    segs.clear();
    groups.clear();
    int64_t units = 0;
    for (int combo = GEN_LIST; combo >= 0; --combo) {
        if (gunits[combo] == 0) continue;
        bool quant = combo != GEN_LIST, vec_only = combo == GEN_LIST;
        for (const Seg& sg : gsegs[combo]) {
            quant |= sg.kind == KIND_QGEN;
            vec_only &= sg.kind == KIND_FALLBACK_VEC;
        }
        const int kc = combo != GEN_LIST ? combo : (vec_only ? VEC_COMBO : -1);
        const int64_t lead = kc == -1 ? gen_lead : 0;
        groups.push_back({kc, (int64_t)segs.size(), gunits[combo], quant, lead});
        Seg sentinel{};
        sentinel.unit_start = gunits[combo];
        sentinel.leaf = -1;
        sentinel.kind = -1;
        gsegs[combo].push_back(sentinel);
        mark_list(gsegs[combo], (int32_t)lead);
        segs.insert(segs.end(), gsegs[combo].begin(), gsegs[combo].end());
        units += gunits[combo];
    }
    if (segs.empty()) {
        Seg sentinel{};
        sentinel.leaf = -1;
        sentinel.kind = -1;
        segs.push_back(sentinel);
    }

    // Norm units for global-norm clipping: every non-empty leaf, in order.
    std::vector<Seg>& nsegs = w.nsegs;
    nsegs.clear();
    int64_t nunits = 0;
    for (int32_t i = 0; i < n_leaves; ++i) {
        if (leaves[i].size <= 0) continue;
        Seg sg{};
        sg.unit_start = nunits;
        sg.leaf = i;
        nsegs.push_back(sg);
        nunits += (leaves[i].size + NORM_UNIT - 1) / NORM_UNIT;
    }
    const int32_t n_nsegs = (int32_t)nsegs.size();
    {
        Seg sentinel{};
        sentinel.unit_start = nunits;
        sentinel.leaf = -1;
        sentinel.kind = -1;
        nsegs.push_back(sentinel);
        mark_list(nsegs);
    }

    // Magma chunk slots: leaf i's chunks c (its fallback work units'
    // indices) sum into slot msegs[i].unit_start + c.
    std::vector<Seg>& msegs = w.msegs;
    msegs.clear();
    int64_t mchunks = -1;
    if (n_leaves > 0 && std::all_of(leaves, leaves + n_leaves,
                                    [](const rf_adam8_leaf& L) { return L.moment_kind != RF_MOMENT_QUANTIZED; })) {
        mchunks = 0;
        for (int32_t i = 0; i < n_leaves; ++i) {
            Seg sg{};
            sg.unit_start = mchunks;
            sg.leaf = i;
            sg.kind = -1;
            msegs.push_back(sg);
            mchunks += (leaves[i].size + CHUNK - 1) / CHUNK;
        }
        Seg sentinel{};
        sentinel.unit_start = mchunks;
        sentinel.leaf = -1;
        sentinel.kind = -1;
        msegs.push_back(sentinel);
        mark_list(msegs);
    }

    w.units = units;
    w.n_nsegs = n_nsegs;
    w.nunits = nunits;
    w.mchunks = mchunks;
    return RF_OK;
}

int64_t step_grid(const DevState* ds, int occ, const PlanGroup& g, int32_t run, int64_t per_wave);
void find_carrier(const std::vector<PlanGroup>& groups, bool msr, const PlanGroup** gen, const PlanGroup** carrier);

}  // namespace

extern "C" {

const char* rf_version(void) { return RF_VERSION; }

int32_t rf_abi_version(void) { return RF_ABI_VERSION; }

const char* rf_last_error(void) { return g_err.c_str(); }

rf_status rf_codebook(int32_t quantizer, float* out256)
{
    if (!out256) return fail(RF_ERR_INVALID, "null output");
    if (quantizer != RF_Q_DYNAMIC_SIGNED && quantizer != RF_Q_DYNAMIC_UNSIGNED)
        return fail(RF_ERR_INVALID, "symmetric_int8 does not use a lookup codebook");
    build_codebook(quantizer == RF_Q_DYNAMIC_SIGNED, out256);
    return RF_OK;
}

rf_status rf_host_table_codes(int32_t quantizer, uint32_t first_bits, int64_t count, uint8_t* out)
{
    if (!out || count < 0) return fail(RF_ERR_INVALID, "bad arguments");
    if (quantizer != RF_Q_DYNAMIC_SIGNED && quantizer != RF_Q_DYNAMIC_UNSIGNED)
        return fail(RF_ERR_INVALID, "quantizer must be dynamic signed or unsigned");
    const HostTables& ht = host_tables();
    if (!ht.error.empty()) return fail(RF_ERR_INVALID, ht.error);
    for (int64_t i = 0; i < count; ++i)
        out[i] = (uint8_t)host_table_code(ht.bytes.data(), quantizer, bitsf(first_bits + (uint32_t)i));
    return RF_OK;
}

rf_status rf_host_sr_records(int32_t quantizer, float* out1024)
{
    if (!out1024) return fail(RF_ERR_INVALID, "null output");
    if (quantizer != RF_Q_DYNAMIC_SIGNED && quantizer != RF_Q_DYNAMIC_UNSIGNED)
        return fail(RF_ERR_INVALID, "quantizer must be dynamic signed or unsigned");
    const HostTables& hs = host_search_tables();
    if (!hs.error.empty()) return fail(RF_ERR_INVALID, hs.error);
    std::memcpy(out1024, hs.bytes.data() + (quantizer == RF_Q_DYNAMIC_SIGNED ? L_SRS : L_SRU), 4096);
    return RF_OK;
}

rf_status rf_host_search_index(int32_t quantizer, uint32_t first_bits, int64_t count, uint16_t* out)
{
    if (!out || count < 0) return fail(RF_ERR_INVALID, "bad arguments");
    if (quantizer != RF_Q_DYNAMIC_SIGNED && quantizer != RF_Q_DYNAMIC_UNSIGNED)
        return fail(RF_ERR_INVALID, "quantizer must be dynamic signed or unsigned");
    const HostTables& hs = host_search_tables();
    if (!hs.error.empty()) return fail(RF_ERR_INVALID, hs.error);
    for (int64_t i = 0; i < count; ++i)
        out[i] = (uint16_t)host_search_index(hs.bytes.data(), quantizer, bitsf(first_bits + (uint32_t)i));
    return RF_OK;
}

rf_status rf_adam8_plan_create(const rf_adam8_leaf* leaves, int32_t n_leaves, int32_t apply, rf_adam8_plan** out_plan)
{
    if (!out_plan) return fail(RF_ERR_INVALID, "null plan output");
    *out_plan = nullptr;
    if (n_leaves < 0 || (n_leaves > 0 && !leaves)) return fail(RF_ERR_INVALID, "bad leaf table");
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    WorkLists w;
    st = build_work_lists(leaves, n_leaves, apply, w);
    if (st != RF_OK) return st;
    std::vector<Seg>& segs = w.segs;
    std::vector<Seg>& nsegs = w.nsegs;
    std::vector<Seg>& msegs = w.msegs;
    const int64_t units = w.units, nunits = w.nunits, mchunks = w.mchunks;
    const int32_t n_nsegs = w.n_nsegs;
    int device = 0;
    HIP_TRY(hipGetDevice(&device));
    rf_adam8_plan* p = new rf_adam8_plan();
    p->n_mchunks = mchunks;
    p->device = device;
    p->n_nsegs = n_nsegs;
    p->n_norm_units = nunits;
    p->apply = apply ? 1 : 0;
    p->n_leaves = n_leaves;
    p->total_units = units;
    p->n_segs = (int64_t)segs.size();
    p->groups = w.groups;
    p->cover = bits_cover(leaves, n_leaves);
    p->shape.assign(leaves, leaves + n_leaves);
    p->vec = w.vecs;
    // Every buffer a run needs is allocated here, so runs never allocate
    // (pinned-host and device allocation synchronise the device).
    const size_t table_bytes = sizeof(rf_adam8_leaf) * (size_t)std::max(n_leaves, 1);
    for (int32_t i = 0; i < n_leaves; ++i) p->group_cap = std::max(p->group_cap, leaves[i].group + 1);
    p->group_off = (table_bytes + 15) & ~(size_t)15;
    const size_t slot_bytes = p->group_off + sizeof(rf_adam8_group) * (size_t)p->group_cap;
    hipError_t e = hipMalloc(&p->d_leaves, table_bytes);
    if (e == hipSuccess) e = hipMalloc(&p->d_segs, sizeof(Seg) * segs.size());
    for (RingSlot& slot : p->ring) {
        if (e == hipSuccess) e = hipHostMalloc((void**)&slot.host, slot_bytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc((void**)&slot.dev, slot_bytes);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&slot.ev, ORDER_EVENT_FLAGS);
    }
    if (e == hipSuccess) e = hipMalloc(&p->d_nsegs, sizeof(Seg) * nsegs.size());
    if (e == hipSuccess) e = hipMalloc(&p->d_npart, sizeof(double) * (size_t)std::max<int64_t>(nunits, 1));
    if (e == hipSuccess) e = hipMalloc(&p->d_leafsum, sizeof(double) * (size_t)std::max(n_nsegs, 1));
    if (e == hipSuccess) e = hipMalloc(&p->d_clip, sizeof(float) * 4);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&p->ev_prepass, hipEventDisableTiming);
    if (e == hipSuccess) e = hipMemcpy(p->d_nsegs, nsegs.data(), sizeof(Seg) * nsegs.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && n_leaves > 0)
        e = hipMemcpy(p->d_leaves, leaves, sizeof(rf_adam8_leaf) * (size_t)n_leaves, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->d_segs, segs.data(), sizeof(Seg) * segs.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && mchunks >= 0) {
        e = hipMalloc(&p->d_msegs, sizeof(Seg) * msegs.size());
        if (e == hipSuccess) e = hipMalloc(&p->d_mpart, sizeof(double) * 3 * (size_t)std::max<int64_t>(mchunks, 1));
        if (e == hipSuccess)
            e = hipMemcpy(p->d_msegs, msegs.data(), sizeof(Seg) * msegs.size(), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        release_plan(p);
        return fail(RF_ERR_HIP, std::string("plan allocation: ") + hipGetErrorString(e));
    }
    *out_plan = p;
    return RF_OK;
}

rf_status rf_adam8_plan_info(const rf_adam8_plan* plan, int64_t* launches, int64_t* leaves, int64_t* units)
{
    if (!plan) return fail(RF_ERR_INVALID, "null plan");
    if (launches) {
        // the generic list rides along with a bf16/bf16 fast launch (plan_launch)
        const PlanGroup *gen = nullptr, *carrier = nullptr;
        find_carrier(plan->groups, false, &gen, &carrier);
        *launches = (int64_t)plan->groups.size() - (carrier ? 1 : 0);
    }
    if (leaves) *leaves = plan->n_leaves;
    if (units) *units = plan->total_units;
    return RF_OK;
}

rf_status rf_adam8_plan_stream_probe(const rf_adam8_plan* plan, void* stream, int64_t* blocks_out)
{
    if (!plan) return fail(RF_ERR_INVALID, "null plan");
    if (!plan->apply) return fail(RF_ERR_UNSUPPORTED, "the stream probe moves the fused step's bytes: apply = 1 plans");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != plan->device) return fail(RF_ERR_INVALID, "the plan belongs to another device");
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    int64_t blocks = 0;
    for (const PlanGroup& g : plan->groups) {
        if (g.combo < 0) continue;  // generic units: not the fast kernel's traffic
        // the grid of the step kernel this list runs on (the default instance)
        const adam_kernel_t fn = pick_adam_kernel(true, false, false, false, false, g.combo);
        int occ = 1;
        st = occupancy((const void*)fn, &occ);
        if (st != RF_OK) return st;
        // the shape of the default (fused, nearest, hardware direction) step
        const int32_t run = STEP_SHAPE_STREAM.run;
        const int64_t grid = step_grid(ds, occ, g, run, STEP_SHAPE_STREAM.per_wave);
        const Seg* segs = plan->d_segs + g.seg_offset;
        const hipStream_t s = (hipStream_t)stream;
        switch (g.combo) {
            case COMBO_F16:
                hipLaunchKernelGGL((k_stream_probe<_Float16, _Float16>), dim3((unsigned)grid), dim3(WG), 0, s,
                                   plan->d_leaves, segs, g.units, run);
                break;
            case 3:
                hipLaunchKernelGGL((k_stream_probe<uint16_t, uint16_t>), dim3((unsigned)grid), dim3(WG), 0, s,
                                   plan->d_leaves, segs, g.units, run);
                break;
            case 2:
                hipLaunchKernelGGL((k_stream_probe<uint16_t, float>), dim3((unsigned)grid), dim3(WG), 0, s,
                                   plan->d_leaves, segs, g.units, run);
                break;
            case 1:
                hipLaunchKernelGGL((k_stream_probe<float, uint16_t>), dim3((unsigned)grid), dim3(WG), 0, s,
                                   plan->d_leaves, segs, g.units, run);
                break;
            default:
                hipLaunchKernelGGL((k_stream_probe<float, float>), dim3((unsigned)grid), dim3(WG), 0, s,
                                   plan->d_leaves, segs, g.units, run);
                break;
        }
        HIP_TRY(hipGetLastError());
        blocks += g.units;
    }
    if (blocks_out) *blocks_out = blocks;
    return RF_OK;
}

}  // extern "C"

namespace {

// The Magma sums of a run that asked for them: every leaf's chunk triples
// summed in a fixed order (a leaf without elements sums to zero).
rf_status magma_sums_finish(const rf_adam8_plan* plan, const rf_adam8_hparams* hp, void* stream)
{
    if (!hp->magma_sums) return RF_OK;
    DevState* ds = nullptr;
    const rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    const int64_t lw = std::max<int64_t>(1, std::min<int64_t>(plan->n_leaves, (int64_t)ds->num_cus * 8));
    hipLaunchKernelGGL(k_magma_leaf, dim3((unsigned)lw), dim3(WG), 0, (hipStream_t)stream, plan->d_msegs,
                       plan->n_leaves, plan->d_mpart, hp->magma_sums);
    HIP_TRY(hipGetLastError());
    return RF_OK;
}

// The generic list and the fast list it rides along with (the bf16/bf16
// one; not in moment-SR launches), or null carrier when the two launch
// apart.
void find_carrier(const std::vector<PlanGroup>& groups, bool msr, const PlanGroup** gen, const PlanGroup** carrier)
{
    *gen = *carrier = nullptr;
    for (const PlanGroup& g : groups) {
        if (g.combo == -1) *gen = &g;
        if (g.combo == 3) *carrier = &g;
    }
    if (!*gen || msr) *carrier = nullptr;
}

// Workgroups of one step launch over list g with `run` consecutive units per
// wave turn, for a kernel of `occ` workgroups per CU.
int64_t step_grid(const DevState* ds, int occ, const PlanGroup& g, int32_t run, int64_t per_wave)
{
    const int64_t runs = (g.units + run - 1) / run;
    const int64_t wg_needed = (runs + WAVES_PER_WG - 1) / WAVES_PER_WG;
    const int64_t wg_resident = (int64_t)ds->num_cus * occ;
    const int64_t wg_spread =
        std::min(wg_needed, (g.units + (int64_t)WAVES_PER_WG * per_wave - 1) / ((int64_t)WAVES_PER_WG * per_wave));
    int64_t grid = std::max<int64_t>(1, std::max(std::min(wg_needed, wg_resident), wg_spread));
    const int64_t wg_each = g.lead + (g.units - g.lead + WAVES_PER_WG - 1) / WAVES_PER_WG;
    if (g.combo == -1 && wg_each <= GEN_WAVE_PER_UNIT_MAX_ROUNDS * wg_resident) {
        // Mixed generic lists: a workgroup per leading quantized unit, then
        // a wave per unit.  These units are latency-bound (a partial block,
        // a leaf's tail), so the workgroups beyond a chip-full queue behind
        // the first ones' short units instead of stacking a second unit
        // behind a wave's partial block.
        grid = wg_each;
    } else if (STEP_GRID_ROUNDS && grid > wg_resident) {
        // a whole number of chip-fulls of workgroups: no last partial round
        const int64_t rounds = std::max<int64_t>(1, (grid + wg_resident / 2) / wg_resident);
        grid = std::min(wg_needed, rounds * wg_resident);
    }
    return grid;
}

rf_status plan_launch(const rf_adam8_plan* plan, const rf_adam8_leaf* d_leaves, const rf_adam8_group* d_groups,
                      const BitsCover& cover, const rf_adam8_hparams* hp, void* stream)
{
    const uint32_t f = hp->flags;
    if (hp->magma_sums) {
        if (plan->n_mchunks < 0)
            return fail(RF_ERR_UNSUPPORTED, "magma_sums needs a plan whose every leaf has unquantized moments");
        if (plan->apply) return fail(RF_ERR_UNSUPPORTED, "magma_sums needs an update-only plan (apply = 0)");
        if (f & RF_SKIP_NONFINITE) return fail(RF_ERR_UNSUPPORTED, "magma_sums with RF_SKIP_NONFINITE");
    }
    if (plan->total_units == 0) return magma_sums_finish(plan, hp, stream);

    const bool msr = (f & RF_MOMENT_SR) != 0;
    const bool psr = (f & RF_PARAM_SR) != 0 && plan->apply;
    if ((f & RF_FED_BITS) && (f & RF_PACKED_BITS))
        return fail(RF_ERR_INVALID, "RF_FED_BITS and RF_PACKED_BITS are exclusive bit sources");
    if (f & RF_FED_BITS) {
        if (psr && !cover.pb) return fail(RF_ERR_INVALID, "RF_FED_BITS with param SR: a leaf has no param_bits");
        if (msr && !cover.mb_quant)
            return fail(RF_ERR_INVALID, "RF_FED_BITS with moment SR: a quantized leaf has no mu_bits/nu_bits");
        if (!cover.mb_store)
            return fail(RF_ERR_INVALID, "RF_FED_BITS: a leaf with RF_LEAF_STORE_SR has no mu_bits/nu_bits");
    }
    const float max_norm = hp->clip_max_norm;
    if (!(max_norm >= 0.0f) || std::isinf(max_norm))
        return fail(RF_ERR_INVALID, "clip_max_norm must be a finite non-negative number (0: no clipping)");
    const bool skip = (f & RF_SKIP_NONFINITE) != 0;
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;

    // One read of the grads gives the clipping norm and the finite flag.
    if (max_norm > 0.0f || skip || hp->finite_out || hp->finite_host) {
        const int64_t pw = std::max<int64_t>(1, std::min<int64_t>((plan->n_norm_units + WAVES_PER_WG - 1) / WAVES_PER_WG,
                                                                  (int64_t)ds->num_cus * 8));
        hipLaunchKernelGGL(k_gnorm_partial, dim3((unsigned)pw), dim3(WG), 0, (hipStream_t)stream, d_leaves,
                           plan->d_nsegs, plan->n_norm_units, plan->d_npart);
        HIP_TRY(hipGetLastError());
        const int64_t lw = std::max<int64_t>(1, std::min<int64_t>((plan->n_nsegs + WAVES_PER_WG - 1) / WAVES_PER_WG,
                                                                  (int64_t)ds->num_cus * 8));
        hipLaunchKernelGGL(k_gnorm_leaf, dim3((unsigned)lw), dim3(WG), 0, (hipStream_t)stream, plan->d_nsegs,
                           plan->n_nsegs, plan->d_npart, plan->d_leafsum);
        HIP_TRY(hipGetLastError());
        hipLaunchKernelGGL(k_gnorm_finish, dim3(1), dim3(WAVE), 0, (hipStream_t)stream, plan->d_leafsum,
                           plan->n_nsegs, max_norm, plan->d_clip, max_norm > 0.0f ? hp->clip_out : nullptr,
                           hp->finite_out);
        HIP_TRY(hipGetLastError());
        if (hp->finite_host) {
            HIP_TRY(hipMemcpyAsync(hp->finite_host, plan->d_clip + 3, sizeof(int32_t), hipMemcpyDeviceToHost,
                                   (hipStream_t)stream));
            if (plan->ev_prepass) HIP_TRY(hipEventRecord(plan->ev_prepass, (hipStream_t)stream));
        }
    }

    KHp k{};
    k.groups = hp->n_groups > 0 ? d_groups : nullptr;
    k.clip = max_norm > 0.0f ? plan->d_clip : nullptr;
    k.gate = skip ? plan->d_clip + 2 : nullptr;
    k.b1 = hp->b1;
    k.omb1 = hp->one_minus_b1;
    k.b2 = hp->b2;
    k.omb2 = hp->one_minus_b2;
    k.bc1 = hp->bc1;
    k.bc2 = hp->bc2;
    k.bc1n = hp->bc1_next;
    {
        const double bc1 = hp->bc1, bc2 = hp->bc2, bc1n = hp->bc1_next;
        k.k1 = (float)(bc1 / std::sqrt(bc2));
        k.k2 = (float)((double)hp->eps * bc1);
        k.er2 = (float)((double)hp->eps_root * bc2);
        k.nb1 = (float)((double)hp->b1 / bc1n);
        k.nomb1 = (float)((double)hp->nesterov_one_minus_b1 / bc1);
        k.rsbc2 = (float)(1.0 / std::sqrt(bc2));
    }
    k.nomb1x = hp->nesterov_one_minus_b1;
    k.eps = hp->eps;
    k.eps_root = hp->eps_root;
    k.wd = hp->weight_decay;
    {
        // bf16(wd), round to nearest even (JAX weak typing of a Python scalar).
        uint32_t u = fbits(hp->weight_decay);
        if (std::isnan(hp->weight_decay)) u = (u & 0x80000000u) | 0x7FC00000u;
        else u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
        k.wd16 = bitsf(u);
        // f16(wd), round to nearest even: the weak-typed decay of f16 params
        k.wdh = (float)(_Float16)hp->weight_decay;
    }
    k.neg_lr = (f & RF_LR) ? hp->neg_lr : 1.0f;
    k.flags = f;
    k.kmu0 = hp->key_mu[0];
    k.kmu1 = hp->key_mu[1];
    k.knu0 = hp->key_nu[0];
    k.knu1 = hp->key_nu[1];
    k.kp0 = hp->key_param[0];
    k.kp1 = hp->key_param[1];
    k.mpart = hp->magma_sums ? plan->d_mpart : nullptr;
    k.msegs = plan->d_msegs;

    // The generic list (partial blocks, small leaves) rides along with the
    // bf16/bf16 fast launch when the step has one and no moment SR: its
    // workgroups lead that grid (k_adam8's KHp.gsegs, CARRIES_GEN), one
    // launch instead of two.
    const PlanGroup* gen = nullptr;
    const PlanGroup* carrier = nullptr;
    find_carrier(plan->groups, msr, &gen, &carrier);
    k.gsegs = nullptr;
    k.gunits = 0;
    k.gwgs = 0;
    for (const PlanGroup& g : plan->groups) {
        if (carrier && &g == gen) continue;
        adam_kernel_t fn =
            pick_adam_kernel(plan->apply != 0, msr, psr, (f & RF_NESTEROV) != 0, (f & RF_EXACT) != 0, g.combo);
        if (!fn) return fail(RF_ERR_HIP, "no step kernel instance for this launch");
        int occ = 1;
        st = occupancy((const void*)fn, &occ);
        if (st != RF_OK) return st;
        // About shape.per_wave units per wave, never fewer workgroups than
        // fit on the chip at once.  On the Llama-7B tree this measured 3-5 %
        // faster than one persistent grid; one unit per wave is 26 % slower
        // (the lookup tables are staged per workgroup).  Rounding the grid
        // to whole chip-fulls removes a last, mostly idle round of
        // workgroups (the ragged tree's 1,570 workgroups on 768 slots become
        // 1,536, GPT-2-small's 943 become 768).
        const bool streaming = plan->apply && !msr && !psr && !(f & RF_EXACT);
        const StepShape shape = streaming ? STEP_SHAPE_STREAM : STEP_SHAPE_HEAVY;
        k.run = g.combo < 0 ? 1 : shape.run;
        // f32 updates (update-only launches) and f32 params are stored on
        // whole cache lines; nontemporally from UPD_NT_MIN_BLOCKS_PER_CU
        // blocks per CU on.  Three store forms on one GPU (old half-line
        // plain / whole-line nontemporal / whole-line plain): the Llama-7B
        // update-only step 13.98-14.77 / 13.17-13.22 / 13.50-13.56 ms,
        // GPT-2-small's launch 265 / 294 / 256 us.
        k.upd_nt = (g.combo >= 0 && g.units >= UPD_NT_MIN_BLOCKS_PER_CU * (int64_t)ds->num_cus) ? 1 : 0;
        int64_t grid = step_grid(ds, occ, g, k.run, shape.per_wave);
        KHp kg = k;
        if (&g == carrier) {
            const int64_t ggrid = step_grid(ds, occ, *gen, 1, shape.per_wave);
            if (ggrid > INT32_MAX || grid + ggrid > (int64_t)UINT32_MAX)
                return fail(RF_ERR_UNSUPPORTED, "step grid beyond 2^32 - 1 workgroups");
            kg.gsegs = plan->d_segs + gen->seg_offset;
            kg.gunits = gen->units;
            kg.gwgs = (int32_t)ggrid;
            grid += ggrid;
        }
        hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3(WG), 0, (hipStream_t)stream, d_leaves,
                           plan->d_segs + g.seg_offset, g.units, kg,
                           !g.tables ? nullptr : (msr ? ds->search : ds->tables));
        HIP_TRY(hipGetLastError());
    }
    HIP_TRY(hipGetLastError());
    return magma_sums_finish(plan, hp, stream);
}

// Frees everything a plan owns (waiting for runs still in flight) and the
// plan itself; true when every free succeeded.  Current device = plan's.
bool release_plan(rf_adam8_plan* plan)
{
    bool ok = true;
    for (RingSlot& slot : plan->ring) {
        if (slot.ev) {
            if (slot.pending) (void)hipEventSynchronize(slot.ev);
            (void)hipEventDestroy(slot.ev);
        }
        if (slot.dev) ok &= hipFree(slot.dev) == hipSuccess;
        if (slot.host) ok &= hipHostFree(slot.host) == hipSuccess;
    }
    if (plan->d_leaves) ok &= hipFree(plan->d_leaves) == hipSuccess;
    if (plan->d_segs) ok &= hipFree(plan->d_segs) == hipSuccess;
    for (void* q : {(void*)plan->d_nsegs, (void*)plan->d_npart, (void*)plan->d_leafsum, (void*)plan->d_clip,
                    (void*)plan->d_msegs, (void*)plan->d_mpart})
        if (q) ok &= hipFree(q) == hipSuccess;
    if (plan->ev_prepass) {
        (void)hipEventSynchronize(plan->ev_prepass);
        ok &= hipEventDestroy(plan->ev_prepass) == hipSuccess;
    }
    delete plan;
    return ok;
}

bool same_structure(const rf_adam8_leaf& a, const rf_adam8_leaf& b)
{
    return a.size == b.size && a.block_size == b.block_size && a.param_dtype == b.param_dtype &&
           a.grad_dtype == b.grad_dtype && a.moment_kind == b.moment_kind && a.state_index == b.state_index &&
           a.param_index == b.param_index && a.flags == b.flags && a.group == b.group;
}

rf_status check_groups(const rf_adam8_plan* plan, const rf_adam8_hparams* hp)
{
    if (hp->n_groups < 0) return fail(RF_ERR_INVALID, "negative n_groups");
    if (hp->n_groups == 0) return RF_OK;
    if (!hp->groups) return fail(RF_ERR_INVALID, "n_groups > 0 with a null group table");
    // Every leaf's group index is below group_cap (leaf structure is fixed by the plan).
    if (hp->n_groups != plan->group_cap)
        return fail(RF_ERR_INVALID, "n_groups must be 0 or the plan's group count (1 + the largest leaf.group at creation)");
    return RF_OK;
}

// Stages the leaf table (and the group table) in the next pinned ring slot,
// copies it to the slot's device twin on `stream` and launches.
// Validation of a run's leaf table against the plan (rf_adam8_plan_run_leaves).
rf_status check_run_leaves(const rf_adam8_plan* plan, const rf_adam8_leaf* leaves, int32_t n_leaves)
{
    for (int32_t i = 0; i < n_leaves; ++i) {
        const rf_adam8_leaf& L = leaves[i];
        if (!same_structure(L, plan->shape[i]))
            return fail(RF_ERR_INVALID, "leaf " + std::to_string(i) + " differs in structure from the plan");
        rf_status st = validate_leaf(L, i, plan->apply);
        if (st != RF_OK) return st;
        if (plan->vec[i] && !leaf_vec_ok(L, plan->apply))
            return fail(RF_ERR_INVALID, "leaf " + std::to_string(i) + " lost the 16-byte alignment the plan relies on");
    }
    return RF_OK;
}

// `validate`: check the leaf table before its first upload (a table found in
// the cache passed that check when it was uploaded).
rf_status run_staged(rf_adam8_plan* plan, const rf_adam8_leaf* leaves, int32_t n_leaves, const rf_adam8_hparams* hp,
                     void* stream, bool validate)
{
    std::lock_guard<std::mutex> lock(plan->mu);
    const size_t bytes = sizeof(rf_adam8_leaf) * (size_t)n_leaves;
    const size_t gbytes = sizeof(rf_adam8_group) * (size_t)std::max(hp->n_groups, 0);
    const size_t span = gbytes ? plan->group_off + gbytes : bytes;
    const hipStream_t s = (hipStream_t)stream;
    RingSlot* slot = nullptr;
    for (RingSlot& c : plan->ring) {
        if (!c.valid || c.span != span || std::memcmp(c.host, leaves, bytes) != 0) continue;
        if (gbytes && std::memcmp((const uint8_t*)c.host + plan->group_off, hp->groups, gbytes) != 0) continue;
        slot = &c;
        break;
    }
    if (slot) {
        // uploaded (and last used) on another stream: this stream waits for it
        if (slot->pending && slot->stream != s) HIP_TRY(hipStreamWaitEvent(s, slot->ev, 0));
    } else {
        if (validate) {
            rf_status st = check_run_leaves(plan, leaves, n_leaves);
            if (st != RF_OK) return st;
        }
        slot = &plan->ring[0];
        for (RingSlot& c : plan->ring)
            if (c.last_use < slot->last_use) slot = &c;
        if (slot->pending) HIP_TRY(hipEventSynchronize(slot->ev));
        slot->pending = false;
        slot->valid = false;
        std::memcpy(slot->host, leaves, bytes);
        if (gbytes) std::memcpy((uint8_t*)slot->host + plan->group_off, hp->groups, gbytes);
        HIP_TRY(hipMemcpyAsync(slot->dev, slot->host, span, hipMemcpyHostToDevice, s));
        slot->valid = true;
        slot->span = span;
    }
    slot->last_use = ++plan->next;
    const rf_adam8_group* d_groups = (const rf_adam8_group*)((uint8_t*)slot->dev + plan->group_off);
    rf_status st = plan_launch(plan, slot->dev, d_groups, bits_cover(leaves, n_leaves), hp, stream);
    HIP_TRY(hipEventRecord(slot->ev, s));
    slot->pending = true;
    slot->stream = s;
    return st;
}

}  // namespace

extern "C" {

rf_status rf_adam8_plan_run(const rf_adam8_plan* plan, const rf_adam8_hparams* hp, void* stream)
{
    if (!plan || !hp) return fail(RF_ERR_INVALID, "null plan or hparams");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != plan->device) return fail(RF_ERR_INVALID, "plan was created on another device");
    rf_status st = check_groups(plan, hp);
    if (st != RF_OK) return st;
    if (hp->n_groups == 0) return plan_launch(plan, plan->d_leaves, nullptr, plan->cover, hp, stream);
    // The group table travels through the staging ring with the creation-time leaf table.
    if (plan->total_units == 0) return plan_launch(plan, plan->d_leaves, nullptr, plan->cover, hp, stream);
    rf_adam8_plan* mp = const_cast<rf_adam8_plan*>(plan);
    return run_staged(mp, plan->shape.data(), plan->n_leaves, hp, stream, false);
}

rf_status rf_adam8_plan_run_leaves(rf_adam8_plan* plan, const rf_adam8_leaf* leaves, int32_t n_leaves,
                                   const rf_adam8_hparams* hp, void* stream)
{
    if (!plan || !hp) return fail(RF_ERR_INVALID, "null plan or hparams");
    if (n_leaves != plan->n_leaves || (n_leaves > 0 && !leaves))
        return fail(RF_ERR_INVALID, "leaf table does not match the plan");
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev != plan->device) return fail(RF_ERR_INVALID, "plan was created on another device");
    rf_status st = check_groups(plan, hp);
    if (st != RF_OK) return st;
    // No work units: nothing to stage (plan_launch still writes zero Magma sums).
    if (plan->total_units == 0) {
        st = check_run_leaves(plan, leaves, n_leaves);
        if (st != RF_OK) return st;
        return plan_launch(plan, plan->d_leaves, nullptr, plan->cover, hp, stream);
    }
    return run_staged(plan, leaves, n_leaves, hp, stream, true);
}

rf_status rf_adam8_plan_wait_prepass(const rf_adam8_plan* plan)
{
    if (!plan) return fail(RF_ERR_INVALID, "null plan");
    HIP_TRY(hipEventSynchronize(plan->ev_prepass));
    return RF_OK;
}

rf_status rf_adam8_plan_destroy(rf_adam8_plan* plan)
{
    if (!plan) return RF_OK;
    int cur = 0;
    HIP_TRY(hipGetDevice(&cur));
    const int dev = plan->device;
    if (cur != dev) HIP_TRY(hipSetDevice(dev));
    const bool ok = release_plan(plan);
    if (cur != dev) (void)hipSetDevice(cur);
    if (!ok) return fail(RF_ERR_HIP, "hipFree of the plan tables failed");
    return RF_OK;
}

rf_status rf_adam8_step(const rf_adam8_leaf* leaves, int32_t n_leaves, int32_t apply, const rf_adam8_hparams* hp,
                        void* stream)
{
    rf_adam8_plan* plan = nullptr;
    rf_status st = rf_adam8_plan_create(leaves, n_leaves, apply, &plan);
    if (st != RF_OK) return st;
    st = rf_adam8_plan_run(plan, hp, stream);
    if (st == RF_OK) {
        hipError_t e = hipStreamSynchronize((hipStream_t)stream);
        if (e != hipSuccess) st = fail(RF_ERR_HIP, std::string("hipStreamSynchronize: ") + hipGetErrorString(e));
    }
    rf_status st2 = rf_adam8_plan_destroy(plan);
    return st != RF_OK ? st : st2;
}

rf_status rf_adam8_step_noalloc(const rf_adam8_leaf* leaves, int32_t n_leaves, int32_t apply,
                                const rf_adam8_hparams* hp, void* stream)
{
    if (!hp) return fail(RF_ERR_INVALID, "null hparams");
    if (n_leaves < 0 || (n_leaves > 0 && !leaves)) return fail(RF_ERR_INVALID, "bad leaf table");
    if (hp->magma_sums) return fail(RF_ERR_UNSUPPORTED, "rf_adam8_step_noalloc does not write Magma sums");
    int32_t group_cap = 1;
    for (int32_t i = 0; i < n_leaves; ++i) group_cap = std::max(group_cap, leaves[i].group + 1);
    if (hp->n_groups < 0) return fail(RF_ERR_INVALID, "negative n_groups");
    if (hp->n_groups > 0 && !hp->groups) return fail(RF_ERR_INVALID, "n_groups > 0 with a null group table");
    if (hp->n_groups > 0 && hp->n_groups != group_cap)
        return fail(RF_ERR_INVALID, "n_groups must be 0 or 1 + the largest leaf.group");
    // Under stream capture the table copy below would either fail to be
    // captured or be recorded with a host source that a later call
    // overwrites before the graph replays; refused before anything is
    // enqueued.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing((hipStream_t)stream, &capture));
    if (capture != hipStreamCaptureStatusNone)
        return fail(RF_ERR_UNSUPPORTED, "rf_adam8_step_noalloc cannot be captured into a graph (its leaf tables "
                                        "are copied from host memory at each call)");
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    std::lock_guard<std::mutex> order(ds->noalloc_mu);
    // Host-side lists in per-thread buffers that keep their capacity.
    thread_local WorkLists w;
    st = build_work_lists(leaves, n_leaves, apply, w);
    if (st != RF_OK) return st;

    // Scratch layout: what the host stages (leaf table, group table, step and
    // norm work lists), then what the kernels write (norm partial sums per
    // unit and per leaf, the clipping scalars).
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t n_groups = (size_t)hp->n_groups;
    const size_t o_groups = up(sizeof(rf_adam8_leaf) * (size_t)n_leaves);
    const size_t o_segs = up(o_groups + sizeof(rf_adam8_group) * n_groups);
    const size_t o_nsegs = up(o_segs + sizeof(Seg) * w.segs.size());
    // The norm sums exist only when the pre-pass runs (clipping or the finite flag).
    const bool prepass = hp->clip_max_norm > 0.0f || (hp->flags & RF_SKIP_NONFINITE) || hp->finite_out ||
                         hp->finite_host;
    const size_t o_npart = up(o_nsegs + sizeof(Seg) * w.nsegs.size());
    const size_t o_leafsum = up(o_npart + sizeof(double) * (size_t)(prepass ? std::max<int64_t>(w.nunits, 1) : 1));
    const size_t o_clip = up(o_leafsum + sizeof(double) * (size_t)(prepass ? std::max(w.n_nsegs, 1) : 1));
    const size_t need = o_clip + 4 * sizeof(float);
    if (need > (size_t)RF_NOALLOC_SCRATCH_BYTES)
        return fail(RF_ERR_INVALID, "rf_adam8_step_noalloc: this tree needs " + std::to_string(need) +
                                        " bytes of scratch (leaf and group tables, work lists, norm sums); "
                                        "the maximum is " + std::to_string((size_t)RF_NOALLOC_SCRATCH_BYTES) +
                                        ": use a plan");
    thread_local std::vector<uint8_t> host;
    host.assign(o_npart, 0);
    if (n_leaves > 0) std::memcpy(host.data(), leaves, sizeof(rf_adam8_leaf) * (size_t)n_leaves);
    if (n_groups) std::memcpy(host.data() + o_groups, hp->groups, sizeof(rf_adam8_group) * n_groups);
    std::memcpy(host.data() + o_segs, w.segs.data(), sizeof(Seg) * w.segs.size());
    std::memcpy(host.data() + o_nsegs, w.nsegs.data(), sizeof(Seg) * w.nsegs.size());
    uint8_t* const base = ds->scratch_ptr;
    // After the previous call's launches on this device, whatever its stream;
    // from pageable memory the copy returns once its source is consumed.
    HIP_TRY(hipStreamWaitEvent((hipStream_t)stream, ds->noalloc_ev, 0));
    HIP_TRY(hipMemcpyAsync(base, host.data(), o_npart, hipMemcpyHostToDevice, (hipStream_t)stream));

    // The launch description of plan_launch, over the scratch (owns nothing).
    rf_adam8_plan plan;
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    plan.device = dev;
    plan.apply = apply ? 1 : 0;
    plan.n_leaves = n_leaves;
    plan.group_cap = group_cap;
    plan.total_units = w.units;
    plan.n_segs = (int64_t)w.segs.size();
    plan.groups.swap(w.groups);  // lent for the launch, then handed back with its capacity
    plan.d_leaves = (rf_adam8_leaf*)base;
    plan.d_segs = (Seg*)(base + o_segs);
    plan.d_nsegs = (Seg*)(base + o_nsegs);
    plan.n_nsegs = w.n_nsegs;
    plan.n_norm_units = w.nunits;
    plan.d_npart = (double*)(base + o_npart);
    plan.d_leafsum = (double*)(base + o_leafsum);
    plan.d_clip = (float*)(base + o_clip);
    plan.n_mchunks = -1;
    const rf_adam8_group* d_groups = n_groups ? (const rf_adam8_group*)(base + o_groups) : nullptr;
    st = plan_launch(&plan, plan.d_leaves, d_groups, bits_cover(leaves, n_leaves), hp, stream);
    w.groups.swap(plan.groups);
    // The next call (any stream) waits for these launches; recorded even
    // after a failed launch, so that whatever was enqueued is covered.
    const hipError_t rec = hipEventRecord(ds->noalloc_ev, (hipStream_t)stream);
    if (st == RF_OK && rec != hipSuccess) return fail(RF_ERR_HIP, std::string("hipEventRecord: ") + hipGetErrorString(rec));
    return st;
}

rf_status rf_blockwise_quantize(int32_t quantizer, const void* x, int32_t x_dtype, int64_t size, int32_t block_size,
                                int32_t sr, uint32_t key0, uint32_t key1, const uint32_t* bits, void* values,
                                void* scales, int32_t scale_dtype, void* stream)
{
    if (quantizer < RF_Q_DYNAMIC_SIGNED || quantizer > RF_Q_SYMMETRIC_INT8) return fail(RF_ERR_INVALID, "unknown quantizer");
    if (block_size <= 0) return fail(RF_ERR_INVALID, "block_size must be positive.");
    if (!valid_dtype(x_dtype) || !valid_dtype(scale_dtype))
        return fail(RF_ERR_UNSUPPORTED, "input and scale dtypes must be f32, bf16 or f16");
    if (size < 0) return fail(RF_ERR_INVALID, "negative size");
    if ((size > 0 && !x) || !values || !scales) return fail(RF_ERR_INVALID, "null buffer");
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    const int64_t nb = nblocks_of(size, block_size);
    // One wave per block at a time, about 4 blocks per wave: on 2^30 f32
    // elements 0.968 ms, against 1.047 ms at 16 blocks per wave with ordinary
    // code stores and 1.023-1.027 ms with nontemporal ones; 2 per wave 0.971,
    // 1 per wave 0.986 (each workgroup stages its tables once).
    unsigned grid = 1;
    st = worklist_grid((const void*)&k_quantize, ds, nb, &grid, 4);
    if (st != RF_OK) return st;
    const int32_t vec_ok = aligned(x, 16) && aligned(values, 8) && (!bits || aligned(bits, 16));
    hipLaunchKernelGGL(k_quantize, dim3(grid), dim3(WG), 0, (hipStream_t)stream, quantizer, x, x_dtype, size,
                       (int64_t)block_size, nb, sr, key0, key1, bits, (uint8_t*)values, scales, scale_dtype,
                       ds->tables, vec_ok);
    HIP_TRY(hipGetLastError());
    return RF_OK;
}

rf_status rf_blockwise_dequantize(int32_t quantizer, const void* values, const void* scales, int32_t scale_dtype,
                                  int64_t size, int32_t block_size, int32_t out_dtype, void* out, void* stream)
{
    if (quantizer < RF_Q_DYNAMIC_SIGNED || quantizer > RF_Q_SYMMETRIC_INT8) return fail(RF_ERR_INVALID, "unknown quantizer");
    if (block_size <= 0) return fail(RF_ERR_INVALID, "block_size must be positive.");
    if (!valid_dtype(out_dtype) || !valid_dtype(scale_dtype))
        return fail(RF_ERR_UNSUPPORTED, "out and scale dtypes must be f32, bf16 or f16");
    if (size < 0) return fail(RF_ERR_INVALID, "negative size");
    if (size == 0) return RF_OK;
    if (!values || !scales || !out) return fail(RF_ERR_INVALID, "null buffer");
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    const bool pow2 = block_size >= 4 && (block_size & (block_size - 1)) == 0;
    int32_t bs_log2 = 0;
    while (pow2 && (1 << bs_log2) < block_size) ++bs_log2;
    const int32_t vec_ok = pow2 && aligned(values, 4) && aligned(out, out_dtype == RF_F32 ? 16 : 8);
    // Vector path: one wave per two 1024-element tiles, every pair its own
    // wave (the workgroup stages only the 1 KB codebook): on 2^30 elements
    // 0.963 ms against 1.056 ms for a grid of 8 workgroups per CU walking the
    // tiles, 0.934 ms with nontemporal stores.  The scalar tail needs few
    // threads.
    const int64_t tiles = vec_ok ? size / 1024 : 0;
    const int64_t wg_needed = std::max<int64_t>(1, (tiles + 2 * WAVES_PER_WG - 1) / (2 * WAVES_PER_WG));
    const int grid = (int)std::min<int64_t>(std::max<int64_t>(wg_needed, vec_ok ? 1 : (size + WG - 1) / WG),
                                            (int64_t)1 << 30);
    hipLaunchKernelGGL(k_dequantize, dim3(grid), dim3(WG), 0, (hipStream_t)stream, quantizer,
                       (const uint8_t*)values, scales, scale_dtype, size, (int64_t)block_size, bs_log2, out_dtype,
                       out, ds->tables, vec_ok);
    HIP_TRY(hipGetLastError());
    return RF_OK;
}

}  // extern "C"

namespace {

rf_status sr_bf16_launch(const float* x, int64_t size, uint32_t key0, uint32_t key1, const uint32_t* bits,
                         uint16_t* out, bool packed, void* stream)
{
    if (size < 0) return fail(RF_ERR_INVALID, "negative size");
    if (size == 0) return RF_OK;
    if (!x || !out) return fail(RF_ERR_INVALID, "null buffer");
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    const int32_t vec_ok = aligned(x, 16) && aligned(out, 16) && (!bits || aligned(bits, 16));
    // One wave per pair of 1024-element tiles (the dequantizer's shape); the
    // scalar tail (fewer than 1024 elements, or unaligned buffers) a thread
    // per element.
    const int64_t tiles = vec_ok ? size / 1024 : 0;
    const int64_t wg_needed = std::max<int64_t>(1, (tiles + 2 * WAVES_PER_WG - 1) / (2 * WAVES_PER_WG));
    const int64_t tail = size - tiles * 1024;
    const int64_t tail_wg = std::min<int64_t>((tail + WG - 1) / WG, (int64_t)ds->num_cus * 8);
    const int grid = (int)std::min<int64_t>(std::max<int64_t>(wg_needed, tail_wg), (int64_t)1 << 30);
    if (packed)
        hipLaunchKernelGGL(k_sr_bf16<true>, dim3(grid), dim3(WG), 0, (hipStream_t)stream, x, size, key0, key1,
                           nullptr, out, vec_ok);
    else
        hipLaunchKernelGGL(k_sr_bf16<false>, dim3(grid), dim3(WG), 0, (hipStream_t)stream, x, size, key0, key1,
                           bits, out, vec_ok);
    HIP_TRY(hipGetLastError());
    return RF_OK;
}

}  // namespace

extern "C" {

rf_status rf_sr_bf16(const float* x, int64_t size, uint32_t key0, uint32_t key1, const uint32_t* bits, uint16_t* out,
                     void* stream)
{
    return sr_bf16_launch(x, size, key0, key1, bits, out, false, stream);
}

rf_status rf_sr_bf16_packed(const float* x, int64_t size, uint32_t key0, uint32_t key1, uint16_t* out, void* stream)
{
    return sr_bf16_launch(x, size, key0, key1, nullptr, out, true, stream);
}

rf_status rf_clip_by_global_norm(const rf_clip_leaf* leaves, int32_t n_leaves, float max_norm, float* stats,
                                 void* stream)
{
    if (n_leaves < 0 || (n_leaves > 0 && !leaves)) return fail(RF_ERR_INVALID, "bad leaf table");
    if (!(max_norm > 0.0f) || std::isinf(max_norm)) return fail(RF_ERR_INVALID, "max_norm must be positive.");
    if (n_leaves > 65535) return fail(RF_ERR_UNSUPPORTED, "more than 65535 leaves in one clip call");
    // The norm pre-pass kernels read rf_adam8_leaf records: only grad, size
    // and grad_dtype are used.
    std::vector<rf_adam8_leaf> gl((size_t)n_leaves);
    std::vector<Seg> nsegs;
    int64_t nunits = 0, maxsize = 0;
    for (int32_t i = 0; i < n_leaves; ++i) {
        const rf_clip_leaf& L = leaves[i];
        if (L.size < 0) return fail(RF_ERR_INVALID, "negative size");
        if (!valid_dtype(L.dtype)) return fail(RF_ERR_UNSUPPORTED, "dtype must be f32, bf16 or f16");
        if (L.size > 0 && (!L.grad || !L.out)) return fail(RF_ERR_INVALID, "null buffer");
        gl[i] = rf_adam8_leaf{};
        gl[i].grad = L.grad;
        gl[i].size = L.size;
        gl[i].grad_dtype = L.dtype;
        maxsize = std::max(maxsize, L.size);
        if (L.size == 0) continue;
        Seg sg{};
        sg.unit_start = nunits;
        sg.leaf = i;
        nsegs.push_back(sg);
        nunits += (L.size + NORM_UNIT - 1) / NORM_UNIT;
    }
    const int32_t nseg = (int32_t)nsegs.size();
    Seg sentinel{};
    sentinel.unit_start = nunits;
    sentinel.leaf = -1;
    sentinel.kind = -1;
    nsegs.push_back(sentinel);
    mark_list(nsegs);
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    // One staging slot: leaf tables and segments (copied), then the partials,
    // leaf sums and (scale, norm, finite, 0) the kernels write.
    const size_t o_gl = 0;
    const size_t o_cl = o_gl + sizeof(rf_adam8_leaf) * (size_t)std::max(n_leaves, 1);
    const size_t o_sg = up16(o_cl + sizeof(rf_clip_leaf) * (size_t)std::max(n_leaves, 1));
    const size_t o_pt = up16(o_sg + sizeof(Seg) * nsegs.size());
    const size_t o_ls = o_pt + sizeof(double) * (size_t)std::max<int64_t>(nunits, 1);
    const size_t o_cp = up16(o_ls + sizeof(double) * (size_t)std::max(nseg, 1));
    const size_t total = o_cp + 4 * sizeof(float);
    Staged stg;
    st = stg.acquire(ds, o_pt, total);
    if (st != RF_OK) return st;
    uint8_t* const host = stg.host();
    if (n_leaves > 0) {
        std::memcpy(host + o_gl, gl.data(), sizeof(rf_adam8_leaf) * (size_t)n_leaves);
        std::memcpy(host + o_cl, leaves, sizeof(rf_clip_leaf) * (size_t)n_leaves);
    }
    std::memcpy(host + o_sg, nsegs.data(), sizeof(Seg) * nsegs.size());
    st = stg.upload(o_pt, s);
    if (st != RF_OK) return st;
    uint8_t* const buf = stg.dev();
    hipError_t e = hipSuccess;
    const rf_adam8_leaf* d_gl = (const rf_adam8_leaf*)(buf + o_gl);
    const rf_clip_leaf* d_cl = (const rf_clip_leaf*)(buf + o_cl);
    const Seg* d_sg = (const Seg*)(buf + o_sg);
    double* d_pt = (double*)(buf + o_pt);
    double* d_ls = (double*)(buf + o_ls);
    float* d_cp = (float*)(buf + o_cp);
    if (e == hipSuccess && nunits > 0) {
        const int64_t pw = std::max<int64_t>(1, std::min<int64_t>((nunits + WAVES_PER_WG - 1) / WAVES_PER_WG,
                                                                  (int64_t)ds->num_cus * 8));
        hipLaunchKernelGGL(k_gnorm_partial, dim3((unsigned)pw), dim3(WG), 0, s, d_gl, d_sg, nunits, d_pt);
        e = hipGetLastError();
        if (e == hipSuccess) {
            const int64_t lw = std::max<int64_t>(1, std::min<int64_t>((nseg + WAVES_PER_WG - 1) / WAVES_PER_WG,
                                                                      (int64_t)ds->num_cus * 8));
            hipLaunchKernelGGL(k_gnorm_leaf, dim3((unsigned)lw), dim3(WG), 0, s, d_sg, nseg, d_pt, d_ls);
            e = hipGetLastError();
        }
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_gnorm_finish, dim3(1), dim3(WAVE), 0, s, d_ls, nseg, max_norm, d_cp, stats, nullptr);
        e = hipGetLastError();
    }
    if (e == hipSuccess && maxsize > 0) {
        const int gx = (int)std::max<int64_t>(1, std::min<int64_t>((maxsize / 8 + WG - 1) / WG,
                                                                   (int64_t)ds->num_cus * 4));
        hipLaunchKernelGGL(k_clip_scale, dim3(gx, n_leaves), dim3(WG), 0, s, d_cl, d_cp);
        e = hipGetLastError();
    }
    st = stg.finish(s);
    if (e != hipSuccess) return fail(RF_ERR_HIP, std::string("rf_clip_by_global_norm: ") + hipGetErrorString(e));
    return st;
}

}  // extern "C"

namespace {

rf_status apply_launch(const rf_apply_leaf* leaves, int32_t n_leaves, int32_t stochastic, uint32_t key0,
                       uint32_t key1, const float* factor, float neg_lr, void* stream, bool packed = false);

// Validates a Magma leaf table and builds its work list (segment i = leaf i).
rf_status magma_list(const rf_magma_leaf* leaves, int32_t n_leaves, bool need_updates, std::vector<Seg>& segs,
                     int64_t& nunits)
{
    if (n_leaves < 0 || (n_leaves > 0 && !leaves)) return fail(RF_ERR_INVALID, "bad leaf table");
    nunits = 0;
    segs.clear();
    for (int32_t i = 0; i < n_leaves; ++i) {
        const rf_magma_leaf& L = leaves[i];
        if (L.size < 0) return fail(RF_ERR_INVALID, "negative size");
        if (!valid_dtype(L.grad_dtype) || !valid_dtype(L.mu_dtype))
            return fail(RF_ERR_UNSUPPORTED, "grad and moment dtypes must be f32, bf16 or f16");
        if (L.size > 0 && (!L.grad || !L.mu || (need_updates && !L.updates)))
            return fail(RF_ERR_INVALID, "null buffer");
        Seg sg{};
        sg.unit_start = nunits;
        sg.leaf = i;
        segs.push_back(sg);
        nunits += (L.size + NORM_UNIT - 1) / NORM_UNIT;
    }
    Seg sentinel{};
    sentinel.unit_start = nunits;
    sentinel.leaf = -1;
    sentinel.kind = -1;
    segs.push_back(sentinel);
    mark_list(segs);
    return RF_OK;
}

// Stages the leaf table and the work list in a staging slot with `extra`
// more device bytes after them (returned at `*tail`).
rf_status magma_stage(Staged& stg, DevState* ds, const rf_magma_leaf* leaves, int32_t n_leaves,
                      const std::vector<Seg>& segs, size_t extra, hipStream_t s, uint8_t** buf, uint8_t** tail)
{
    const size_t o_sg = up16(sizeof(rf_magma_leaf) * (size_t)std::max(n_leaves, 1));
    const size_t o_tail = up16(o_sg + sizeof(Seg) * segs.size());
    rf_status st = stg.acquire(ds, o_tail, o_tail + std::max<size_t>(extra, 16));
    if (st != RF_OK) return st;
    if (n_leaves > 0) std::memcpy(stg.host(), leaves, sizeof(rf_magma_leaf) * (size_t)n_leaves);
    std::memcpy(stg.host() + o_sg, segs.data(), sizeof(Seg) * segs.size());
    st = stg.upload(o_tail, s);
    if (st != RF_OK) return st;
    *buf = stg.dev();
    *tail = stg.dev() + o_tail;
    return RF_OK;
}

}  // namespace

extern "C" {

rf_status rf_magma_reduce(const rf_magma_leaf* leaves, int32_t n_leaves, float b1, float one_minus_b1, double* sums,
                          void* stream)
{
    std::vector<Seg> segs;
    int64_t nunits = 0;
    rf_status st = magma_list(leaves, n_leaves, false, segs, nunits);
    if (st != RF_OK) return st;
    if (n_leaves == 0) return RF_OK;
    if (!sums) return fail(RF_ERR_INVALID, "null sums");
    DevState* ds = nullptr;
    st = device_state(&ds);
    if (st != RF_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    uint8_t *buf = nullptr, *tail = nullptr;
    Staged stg;
    st = magma_stage(stg, ds, leaves, n_leaves, segs, sizeof(double) * 3 * (size_t)std::max<int64_t>(nunits, 1), s,
                     &buf, &tail);
    if (st != RF_OK) return st;
    const rf_magma_leaf* d_leaves = (const rf_magma_leaf*)buf;
    const Seg* d_segs = (const Seg*)(buf + ((sizeof(rf_magma_leaf) * (size_t)n_leaves + 15) & ~(size_t)15));
    double* d_part = (double*)tail;
    hipError_t e = hipSuccess;
    if (nunits > 0) {
        const int64_t pw = std::max<int64_t>(1, std::min<int64_t>((nunits + WAVES_PER_WG - 1) / WAVES_PER_WG,
                                                                  (int64_t)ds->num_cus * 8));
        hipLaunchKernelGGL(k_magma_partial, dim3((unsigned)pw), dim3(WG), 0, s, d_leaves, d_segs, nunits, b1,
                           one_minus_b1, d_part);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        const int64_t lw = std::max<int64_t>(1, std::min<int64_t>(n_leaves, (int64_t)ds->num_cus * 8));
        hipLaunchKernelGGL(k_magma_leaf, dim3((unsigned)lw), dim3(WG), 0, s, d_segs, n_leaves, d_part, sums);
        e = hipGetLastError();
    }
    st = stg.finish(s);
    if (e != hipSuccess) return fail(RF_ERR_HIP, std::string("rf_magma_reduce: ") + hipGetErrorString(e));
    return st;
}

rf_status rf_magma_scale(const rf_magma_leaf* leaves, int32_t n_leaves, const double* sums, float* scores, float p,
                         float tau, uint32_t key0, uint32_t key1, int32_t n_keys, float neg_lr, float* factor_out,
                         void* stream)
{
    // magma.py:8-13 validate_magma_args
    if (!(p >= 0.0f && p <= 1.0f)) return fail(RF_ERR_INVALID, "magma_p must be in [0, 1].");
    if (!(tau > 0.0f)) return fail(RF_ERR_INVALID, "magma_tau must be positive.");
    std::vector<Seg> segs;
    int64_t nunits = 0;
    rf_status st = magma_list(leaves, n_leaves, factor_out == nullptr, segs, nunits);
    if (st != RF_OK) return st;
    if (n_leaves == 0) return RF_OK;
    if (!sums || !scores) return fail(RF_ERR_INVALID, "null sums or scores");
    for (int32_t i = 0; i < n_leaves; ++i)
        if (leaves[i].key_index < 0 || leaves[i].key_index >= n_keys)
            return fail(RF_ERR_INVALID, "key_index outside [0, n_keys)");
    DevState* ds = nullptr;
    st = device_state(&ds);
    if (st != RF_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    uint8_t *buf = nullptr, *tail = nullptr;
    Staged stg;
    st = magma_stage(stg, ds, leaves, n_leaves, segs, sizeof(float) * (size_t)n_leaves, s, &buf, &tail);
    if (st != RF_OK) return st;
    const rf_magma_leaf* d_leaves = (const rf_magma_leaf*)buf;
    const Seg* d_segs = (const Seg*)(buf + ((sizeof(rf_magma_leaf) * (size_t)n_leaves + 15) & ~(size_t)15));
    float* d_factor = factor_out ? factor_out : (float*)tail;
    hipLaunchKernelGGL(k_magma_factor, dim3((unsigned)((n_leaves + WG - 1) / WG)), dim3(WG), 0, s, d_leaves,
                       n_leaves, sums, scores, d_factor, p, tau, key0, key1);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && nunits > 0 && !factor_out) {
        const int64_t aw = std::max<int64_t>(1, std::min<int64_t>((nunits + WAVES_PER_WG - 1) / WAVES_PER_WG,
                                                                  (int64_t)ds->num_cus * 8));
        hipLaunchKernelGGL(k_magma_apply, dim3((unsigned)aw), dim3(WG), 0, s, d_leaves, d_segs, nunits, d_factor,
                           neg_lr);
        e = hipGetLastError();
    }
    st = stg.finish(s);
    if (e != hipSuccess) return fail(RF_ERR_HIP, std::string("rf_magma_scale: ") + hipGetErrorString(e));
    return st;
}

rf_status rf_apply_updates(const rf_apply_leaf* leaves, int32_t n_leaves, int32_t stochastic, uint32_t key0,
                           uint32_t key1, void* stream)
{
    return apply_launch(leaves, n_leaves, stochastic, key0, key1, nullptr, 1.0f, stream);
}

rf_status rf_apply_updates_packed(const rf_apply_leaf* leaves, int32_t n_leaves, uint32_t key0, uint32_t key1,
                                  void* stream)
{
    for (int32_t i = 0; leaves && i < n_leaves; ++i)
        if (leaves[i].bits) return fail(RF_ERR_INVALID, "rf_apply_updates_packed draws its own bits: leaf bits must be NULL");
    return apply_launch(leaves, n_leaves, 1, key0, key1, nullptr, 1.0f, stream, true);
}

rf_status rf_magma_apply_updates(const rf_apply_leaf* leaves, int32_t n_leaves, const float* factor, float neg_lr,
                                 int32_t stochastic, uint32_t key0, uint32_t key1, void* stream)
{
    if (n_leaves > 0 && !factor) return fail(RF_ERR_INVALID, "null factor");
    return apply_launch(leaves, n_leaves, stochastic, key0, key1, factor, neg_lr, stream);
}

rf_status rf_accumulate(const rf_accum_leaf* leaves, int32_t n_leaves, int32_t mode, int32_t n_acc, void* stream)
{
    if (n_leaves < 0 || (n_leaves > 0 && !leaves)) return fail(RF_ERR_INVALID, "bad leaf table");
    if (mode != RF_ACC_SUM && mode != RF_ACC_MEAN && mode != RF_ACC_ZERO) return fail(RF_ERR_INVALID, "unknown mode");
    if (n_acc < 0) return fail(RF_ERR_INVALID, "negative n_acc");
    thread_local std::vector<Seg> segs;
    segs.clear();
    int64_t nunits = 0;
    for (int32_t i = 0; i < n_leaves; ++i) {
        const rf_accum_leaf& L = leaves[i];
        if (L.size < 0) return fail(RF_ERR_INVALID, "negative size");
        if (!valid_dtype(L.grad_dtype) || !valid_dtype(L.acc_dtype))
            return fail(RF_ERR_UNSUPPORTED, "grad and accumulator dtypes must be f32, bf16 or f16");
        if (L.size == 0) continue;
        if (!L.acc || (mode != RF_ACC_ZERO && !L.grad)) return fail(RF_ERR_INVALID, "null buffer");
        Seg sg{};
        sg.unit_start = nunits;
        sg.leaf = i;
        segs.push_back(sg);
        nunits += (L.size + APPLY_UNIT - 1) / APPLY_UNIT;
    }
    if (nunits == 0) return RF_OK;
    Seg sentinel{};
    sentinel.unit_start = nunits;
    sentinel.leaf = -1;
    sentinel.kind = -1;
    segs.push_back(sentinel);
    mark_list(segs);
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    hipStream_t s = (hipStream_t)stream;
    unsigned aw = 1;  // before the staging slot: an error here leaves nothing in flight
    st = worklist_grid((const void*)&k_accumulate, ds, nunits, &aw);
    if (st != RF_OK) return st;
    const size_t o_sg = up16(sizeof(rf_accum_leaf) * (size_t)n_leaves);
    const size_t bytes = o_sg + sizeof(Seg) * segs.size();
    Staged stg;
    st = stg.acquire(ds, bytes, bytes);
    if (st != RF_OK) return st;
    std::memcpy(stg.host(), leaves, sizeof(rf_accum_leaf) * (size_t)n_leaves);
    std::memcpy(stg.host() + o_sg, segs.data(), sizeof(Seg) * segs.size());
    st = stg.upload(bytes, s);
    if (st != RF_OK) return st;
    hipLaunchKernelGGL(k_accumulate, dim3(aw), dim3(WG), 0, s, (const rf_accum_leaf*)stg.dev(),
                       (const Seg*)(stg.dev() + o_sg), nunits, mode, n_acc);
    const hipError_t le = hipGetLastError();
    st = stg.finish(s);
    if (le != hipSuccess) return fail(RF_ERR_HIP, std::string("k_accumulate launch: ") + hipGetErrorString(le));
    return st;
}

}  // extern "C"

namespace {

rf_status apply_launch(const rf_apply_leaf* leaves, int32_t n_leaves, int32_t stochastic, uint32_t key0,
                       uint32_t key1, const float* factor, float neg_lr, void* stream, bool packed)
{
    if (n_leaves < 0 || (n_leaves > 0 && !leaves)) return fail(RF_ERR_INVALID, "bad leaf table");
    if (n_leaves == 0) return RF_OK;
    int64_t maxsize = 0;
    for (int32_t i = 0; i < n_leaves; ++i) {
        const rf_apply_leaf& L = leaves[i];
        if (L.size < 0) return fail(RF_ERR_INVALID, "negative size");
        if (!valid_dtype(L.param_dtype)) return fail(RF_ERR_UNSUPPORTED, "param dtype must be f32, bf16 or f16");
        if (L.size > 0 && (!L.param || !L.updates)) return fail(RF_ERR_INVALID, "null buffer");
        if (L.param_index < 0) return fail(RF_ERR_INVALID, "negative key index");
        maxsize = std::max(maxsize, L.size);
    }
    if (maxsize == 0) return RF_OK;
    DevState* ds = nullptr;
    rf_status st = device_state(&ds);
    if (st != RF_OK) return st;
    // Work list: APPLY_UNIT-element units of every non-empty leaf.
    thread_local std::vector<Seg> segs;
    segs.clear();
    int64_t nunits = 0;
    for (int32_t i = 0; i < n_leaves; ++i) {
        if (leaves[i].size == 0) continue;
        Seg sg{};
        sg.unit_start = nunits;
        sg.leaf = i;
        segs.push_back(sg);
        nunits += (leaves[i].size + APPLY_UNIT - 1) / APPLY_UNIT;
    }
    Seg sentinel{};
    sentinel.unit_start = nunits;
    sentinel.leaf = -1;
    sentinel.kind = -1;
    segs.push_back(sentinel);
    mark_list(segs);
    hipStream_t s = (hipStream_t)stream;
    const void* fn = !stochastic ? (const void*)&k_apply<false, false>
                     : packed    ? (const void*)&k_apply<true, true>
                                 : (const void*)&k_apply<true, false>;
    unsigned aw = 1;  // before the staging slot: an error here leaves nothing in flight
    st = worklist_grid(fn, ds, nunits, &aw);
    if (st != RF_OK) return st;
    const size_t o_sg = up16(sizeof(rf_apply_leaf) * (size_t)n_leaves);
    const size_t bytes = o_sg + sizeof(Seg) * segs.size();
    Staged stg;
    st = stg.acquire(ds, bytes, bytes);
    if (st != RF_OK) return st;
    std::memcpy(stg.host(), leaves, sizeof(rf_apply_leaf) * (size_t)n_leaves);
    std::memcpy(stg.host() + o_sg, segs.data(), sizeof(Seg) * segs.size());
    st = stg.upload(bytes, s);
    if (st != RF_OK) return st;
    if (stochastic && packed)
        hipLaunchKernelGGL((k_apply<true, true>), dim3(aw), dim3(WG), 0, s, (const rf_apply_leaf*)stg.dev(),
                           (const Seg*)(stg.dev() + o_sg), nunits, key0, key1, factor, neg_lr);
    else if (stochastic)
        hipLaunchKernelGGL((k_apply<true, false>), dim3(aw), dim3(WG), 0, s, (const rf_apply_leaf*)stg.dev(),
                           (const Seg*)(stg.dev() + o_sg), nunits, key0, key1, factor, neg_lr);
    else
        hipLaunchKernelGGL((k_apply<false, false>), dim3(aw), dim3(WG), 0, s, (const rf_apply_leaf*)stg.dev(),
                           (const Seg*)(stg.dev() + o_sg), nunits, key0, key1, factor, neg_lr);
    const hipError_t le = hipGetLastError();
    st = stg.finish(s);
    if (le != hipSuccess) return fail(RF_ERR_HIP, std::string("k_apply launch: ") + hipGetErrorString(le));
    return st;
}

}  // namespace
