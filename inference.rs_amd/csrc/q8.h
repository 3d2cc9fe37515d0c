// Activation block quantizers shared by the standalone quantize kernels and the matvec that quantizes its
// own activations into LDS.  Bit-exact with the reference CPU quantizers:
//   Q8_K  BlockQ8K::from_float        crates/inference-tensor/src/quantized/k_quants.rs:2721-2760
//   Q8_0  quantize_block32 + f16 d    crates/inference-tensor/src/quantized/mod.rs:41-56, k_quants.rs:923-949
// Every step is a single IEEE operation (division, multiply, roundf: half away from zero), so contraction
// cannot merge them; it is switched off here regardless.
#pragma once

#include "common.h"

namespace qmm_q8 {

// Output addressing of one 256-value Q8_K block:
//   decode   the 292-byte qmm_block_q8k (int16 bsums of 16), the one-launch matvec's LDS copy
//   tc       the tensor-core entries' {f32 d; int8 qs[256]} of 260 bytes (no sums)
//   slot     the 288-byte qmm_block_q8ks of the reference-named decode entries: int16 sums of each 32, 12 zero bytes
//   tile     the prefill layout of one channel: qs[nsb][rows][256], d[nsb][rows] f32, s32[nsb][rows][8] int16 sums of
//            each 32 (276 bytes per 256 values)
//   tile16   the same with h16[nsb][rows][16], the sums of each 16 as f16 (exact: |sum| <= 2032), for the
//            `_q8k` prefill entries (292 bytes per 256 values)
struct q8k_dst {
  uint8_t *qs;
  float *d;
  uint16_t *bsums;  // int16 sums of 16 values
  int16_t *s32;     // int16 sums of 32 values
  uint32_t *pad;    // three dwords set to zero
  uint16_t *h16;    // f16 sums of 16 values
};

__device__ __forceinline__ q8k_dst q8k_decode_dst(uint8_t *vy, int64_t block) {
  uint8_t *b = vy + block * (int64_t)sizeof(qmm_block_q8k);
  return {b + 4, (float *)b, (uint16_t *)(b + 260), nullptr, nullptr, nullptr};
}

__device__ __forceinline__ q8k_dst q8k_tc_dst(uint8_t *vy, int64_t block) {
  uint8_t *b = vy + block * 260;
  return {b + 4, (float *)b, nullptr, nullptr, nullptr, nullptr};
}

__device__ __forceinline__ q8k_dst q8k_slot_dst(uint8_t *vy, int64_t block) {
  uint8_t *b = vy + block * (int64_t)sizeof(qmm_block_q8ks);
  return {b + 4, (float *)b, nullptr, (int16_t *)(b + 260), (uint32_t *)(b + 276), nullptr};
}

__device__ __forceinline__ q8k_dst q8k_tile_dst(uint8_t *chan, int64_t rows, int64_t nsb, int64_t sb, int64_t r) {
  const int64_t i = sb * rows + r;
  uint8_t *qs = chan + i * 256;
  float *d = (float *)(chan + nsb * rows * 256) + i;
  int16_t *s32 = (int16_t *)(chan + nsb * rows * 260) + i * 8;
  return {qs, d, nullptr, s32, nullptr, nullptr};
}

__device__ __forceinline__ q8k_dst q8k_tile16_dst(uint8_t *chan, int64_t rows, int64_t nsb, int64_t sb, int64_t r) {
  const int64_t i = sb * rows + r;
  uint8_t *qs = chan + i * 256;
  float *d = (float *)(chan + nsb * rows * 256) + i;
  uint16_t *h16 = (uint16_t *)(chan + nsb * rows * 260) + i * 16;
  return {qs, d, nullptr, nullptr, nullptr, h16};
}

// One wave quantizes G blocks: v[t][0..3] of lanes 0..63 are values 4*lane .. 4*lane+3 of block t, written to
// dst[t] when store[t] (uniform over the wave).  The value of largest magnitude is the first one in index order,
// as the reference's sequential scan with a strict '>' finds it: the wave maximum of |x| (DPP), then the first
// lane holding it (ballot), then that lane's first such value.  NaNs are never the maximum (fmaxf drops them, as
// the scan's comparison does).  A block whose maximum is 0 (or that holds no number) is written as zeros
// (k_quants.rs:2740-2743), through selects rather than a branch, and each step runs for all G blocks before the
// next, so their DPP chains interleave.
template <int G>
__device__ __forceinline__ void q8k_waves(const float (&v)[G][4], int lane, const q8k_dst (&dst)[G],
                                          const bool (&store)[G]) {
#pragma clang fp contract(off)
  // The wave maximum runs on the bit patterns: for non-negative floats their unsigned order is the numeric one, a
  // lane whose four values are all NaN takes part as 0 (fmaxf drops NaNs), and one max per DPP step needs no
  // canonicalizing of its operands.
  float am[G];
  uint32_t mx[G];
#pragma unroll
  for (int t = 0; t < G; t++) {
    am[t] = fmaxf(fmaxf(fabsf(v[t][0]), fabsf(v[t][1])), fmaxf(fabsf(v[t][2]), fabsf(v[t][3])));
    mx[t] = am[t] == am[t] ? __builtin_bit_cast(uint32_t, am[t]) : 0u;
  }
#pragma unroll
  for (int t = 0; t < G; t++) mx[t] = dpp_max_u32<0xb1, 0xf>(mx[t]);
#pragma unroll
  for (int t = 0; t < G; t++) mx[t] = dpp_max_u32<0x4e, 0xf>(mx[t]);
#pragma unroll
  for (int t = 0; t < G; t++) mx[t] = dpp_max_u32<0x141, 0xf>(mx[t]);
#pragma unroll
  for (int t = 0; t < G; t++) mx[t] = dpp_max_u32<0x140, 0xf>(mx[t]);
#pragma unroll
  for (int t = 0; t < G; t++) mx[t] = dpp_max_u32<0x142, 0xa>(mx[t]);
#pragma unroll
  for (int t = 0; t < G; t++) mx[t] = dpp_max_u32<0x143, 0xc>(mx[t]);
#pragma unroll
  for (int t = 0; t < G; t++) {
    const float amax = __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)mx[t], 63));
    const bool nz = amax > 0.0f;
    const float *x = v[t];
    float first = x[3];  // this lane's first value of magnitude amax (selects, latest index first)
    first = fabsf(x[2]) == amax ? x[2] : first;
    first = fabsf(x[1]) == amax ? x[1] : first;
    first = fabsf(x[0]) == amax ? x[0] : first;
    // the first lane holding it (lane 63's bit keeps the count defined for a block with no number)
    const int holder = __builtin_ctzll(__ballot(am[t] == amax) | (1ull << 63));
    const float m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, first), holder));
    const float iscale = nz ? -127.0f / m : 0.0f;
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = round_sat_i8(iscale * x[i]);  // (iscale 0: every q is 0)
    const int s = quad_sum(q[0] + q[1] + q[2] + q[3]);  // values 16 (lane / 4) .. +16
    // row_shr:4: lane 8i + 4 adds the sum of the quad before it, values 32 i .. +32
    const int s32 = s + __builtin_amdgcn_update_dpp(0, s, 0x114, 0xf, 0xf, false);
    if (!store[t]) continue;
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    *(uint32_t *)(dst[t].qs + 4 * lane) = packed;
    if ((lane & 3) == 0 && dst[t].bsums) dst[t].bsums[lane >> 2] = (uint16_t)(int16_t)s;  // +0 for a zero block
    if ((lane & 3) == 0 && dst[t].h16) dst[t].h16[lane >> 2] = f32_to_f16_bits((float)s);
    if ((lane & 7) == 4 && dst[t].s32) dst[t].s32[lane >> 3] = (int16_t)s32;
    if (lane < 3 && dst[t].pad) dst[t].pad[lane] = 0u;
    if (lane == 0) *dst[t].d = nz ? 1.0f / iscale : 0.0f;
  }
}

__device__ __forceinline__ void q8k_wave(const float v[4], int lane, q8k_dst dst) {
  const float (&vv)[1][4] = *reinterpret_cast<const float(*)[1][4]>(v);
  const q8k_dst d[1] = {dst};
  const bool st[1] = {true};
  q8k_waves<1>(vv, lane, d, st);
}

// Eight lanes quantize one 32-value Q8_0 block (4 values each); writes qs (4 bytes/lane) and the f16 scale when
// `store`.  Every lane of the wave takes part (the 8-lane maximum goes through DPP within each group of 8).
__device__ __forceinline__ void q8_0_group(const float v[4], int sub, int8_t *qs, uint16_t *d_out, bool store) {
#pragma clang fp contract(off)
  // from 0, as the reference's fold(0, max(|v|)) starts: a block of NaNs has d = 0
  const float am = fmaxf(0.0f, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  // (on the bit patterns of these non-negative, NaN-free values, as in q8k_waves)
  uint32_t mb = __builtin_bit_cast(uint32_t, am);
  mb = dpp_max_u32<0xb1, 0xf>(mb);
  mb = dpp_max_u32<0x4e, 0xf>(mb);
  mb = dpp_max_u32<0x141, 0xf>(mb);  // row_half_mirror: the other quad of the group of 8
  const float amax = __builtin_bit_cast(float, mb);
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  int q[4];
#pragma unroll
  for (int i = 0; i < 4; i++) q[i] = round_sat_i8(v[i] * id);
  if (!store) return;
  // qs may be only 2-byte aligned (34-byte blocks): two 16-bit stores
  uint16_t *q16 = (uint16_t *)(qs + 4 * sub);
  q16[0] = (uint16_t)((q[0] & 0xff) | ((q[1] & 0xff) << 8));
  q16[1] = (uint16_t)((q[2] & 0xff) | ((q[3] & 0xff) << 8));
  if (sub == 0) *d_out = f32_to_f16_bits(d);
}

// values k0 .. k0 + 3 of a row of kx values, zero past its end: one vector load where all four are in the row and
// aligned (every row of an aligned, padded activation), else four element loads
template <class In>
__device__ __forceinline__ void load4(const typename In::T *row, int64_t k0, int64_t kx, float v[4]) {
  const typename In::T *p = row + k0;
  if (k0 + 4 <= kx && ((uintptr_t)p & (4 * sizeof(typename In::T) - 1)) == 0) {
    In::load4(p, v);
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) v[i] = (k0 + i < kx) ? In::load(row, k0 + i) : 0.0f;
}

}  // namespace qmm_q8
