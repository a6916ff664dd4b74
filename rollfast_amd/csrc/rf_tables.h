// rf_tables.h -- codebooks and requantization lookup tables shared by the
// gfx950 kernels (device side) and their host-side builder.
//
// Requantization identity.  For a dynamic codebook cb[0..255] (strictly
// increasing) the reference picks, for a normalised value n in
// [cb[0], cb[255]], ui = searchsorted_left(cb, n), li = ui - 1 (clipped) and
// the upper code iff fl(|cb[ui] - n|) < fl(|n - cb[li]|)
// (rollfast optim/adam8.py:542-569).  Inside each interval (cb[i], cb[i+1]]
// that choice is monotone in n, so there is a smallest f32 t_i from which the
// upper code wins, and code(n) = #{ i : n >= t_i } (values below cb[0] count
// zero thresholds, which is the reference's clip to code 0).  The kernels
// count thresholds instead of searching the codebook:
//
//   cell = (bits(n) >> 15) & 0xFFFF   (|n|: exponent + 8 mantissa bits)
//   cand = CAND[sign(n)][cell]        (thresholds <= the cell's low end)
//   code = cand + (n >= T[cand])      (T ascending, value space, T[255] = inf)
//
// The cells are narrow enough (relative width <= 2^-8, while consecutive
// thresholds are >= 0.53 % apart) that each holds at most one threshold; the
// builder checks this and refuses to produce tables otherwise.  Cells below
// CELL_LO all map to CELL_LO (no threshold lies below 2^-23 in magnitude).
//
// Moment stochastic rounding needs ui = searchsorted_left(cb, n) instead
// (adam8.py:549-564).  Its launches stage a second image of the same layout
// whose candidate regions hold, per cell, the number of codebook entries
// below the cell's low end; a cell holds at most one entry (checked), so
// ui = cand + (cb[cand] < n).  Its threshold regions are unused.  After the
// shared layout the search image holds, per codebook and per ui, the
// neighbour record {cb[li], cb[ui] - cb[li], y, 0} with li = max(ui - 1, 0)
// and y = RN(1 / (cb[ui] - cb[li])) (0 where the two coincide, ui = 0): the
// probability p = (n - cb[li]) / (cb[ui] - cb[li]) is then formed as
// q0 = a*y, r = fma(-d, q0, a), p = fma(r, y, q0), which equals the IEEE
// quotient wherever the Bernoulli draw can tell them apart (the host's
// tables test holds it to IEEE division over every gap), and is 0 for ui = 0
// without a branch.
//
// Byte layout (identical in global memory and in LDS).  The two sign halves
// of the signed candidates sit CANDS_SIGN_STRIDE (a power of two) apart, so
// a lookup forms its index as ((bits(n) >> 31) << 13) | cell with one
// shift-and-or; the threshold tables fill the gap between the halves.
//   [L_CANDS]    u8  signed candidates, n >= 0    [NCELL_PAD]
//   [L_TS]       f32 signed thresholds T[256]     (value space, +inf padded)
//   [L_TU]       f32 unsigned thresholds T[256]
//   [L_CANDS + CANDS_SIGN_STRIDE]  signed candidates, n < 0
//   [L_CBS]      f32 cb_signed[256]
//   [L_CBU]      f32 cb_unsigned[256]
//   [L_CANDU]    u8  unsigned candidates          [NCELL_PAD]
//   [L_SRS]      float4 signed neighbour records [256]    (search image only)
//   [L_SRU]      float4 unsigned neighbour records [256]  (search image only)
#pragma once
#include <stdint.h>

namespace rf {

constexpr uint32_t CELL_SHIFT = 15;
constexpr uint32_t CELL_LO = 0x6800;   // bits(2^-23) >> 15: every threshold lies above
constexpr uint32_t CELL_HI = 0x7F00;   // bits(1.0f) >> 15
constexpr uint32_t NCELL = CELL_HI - CELL_LO + 1;
constexpr uint32_t NCELL_PAD = (NCELL + 15u) & ~15u;

constexpr uint32_t CANDS_SIGN_SHIFT = 13;
constexpr uint32_t CANDS_SIGN_STRIDE = 1u << CANDS_SIGN_SHIFT;
constexpr uint32_t L_CANDS = 0;
constexpr uint32_t L_TS = L_CANDS + NCELL_PAD;
constexpr uint32_t L_TU = L_TS + 1024;
constexpr uint32_t L_CBS = L_CANDS + CANDS_SIGN_STRIDE + NCELL_PAD;
constexpr uint32_t L_CBU = L_CBS + 1024;
constexpr uint32_t L_CANDU = L_CBU + 1024;
constexpr uint32_t TABLE_BYTES = L_CANDU + NCELL_PAD;
static_assert(NCELL_PAD <= CANDS_SIGN_STRIDE, "a cell index fits below the sign bit");
static_assert(L_TU + 1024 <= L_CANDS + CANDS_SIGN_STRIDE, "thresholds fit between the sign halves");
static_assert(NCELL_PAD % 16 == 0 && TABLE_BYTES % 16 == 0, "tables are copied in 16-byte words");
constexpr uint32_t L_SRS = TABLE_BYTES;
constexpr uint32_t L_SRU = L_SRS + 256 * 16;
constexpr uint32_t SEARCH_BYTES = L_SRU + 256 * 16;

// Fast requantization is exact when the block scale s satisfies
// FAST_SCALE_MIN <= s < inf: the reciprocal-and-correct division
// q0 = x*rcp(s), r = fma(-s, q0, x), q = fma(r, rcp(s), q0) then equals the
// IEEE quotient for every |q| >= 2^-25, and all smaller quotients map to the
// zero code either way.  Other blocks (tiny, zero-free but subnormal-range,
// Inf or NaN scales) take the literal search path.
constexpr float FAST_SCALE_MIN = 0x1p-70f;

}  // namespace rf
