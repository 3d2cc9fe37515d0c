// Prefill matmul for GGUF Q4_K / Q6_K / Q8_0 weights against activations quantized to Q8_K / Q8_0 blocks,
// on CDNA4 int8 MFMA (v_mfma_i32_32x32x32_i8), plus its expert-grouped MoE form.
//
// Replaces the llama.cpp-derived MMQ of crates/inference-quant/kernels/cuda/mmq_gguf (mmq_instance.cuh:8-268,
// mmq_gguf.cuh:3533-3875, 4020-4061).  Exactness: the reference CPU QMatMul sums integer block dots and scales
// each by f32 factors per 256 values (Q4_K, Q6_K) or per 32 (Q8_0).  The int8 MFMA reproduces the integer
// dots exactly; the per-32 / per-16 integer scales of the K-quants are folded into the weight operand, which
// then needs more than 8 bits, so it is split into two int8 planes:
//   Q4_K  sc (6 bit) = 8 sh + sl:   sc*q4 = 8 (sh*q4) + (sl*q4), both planes <= 105
//         min term  sum_j m_j * S_j  through one f16 MFMA (S_j, the activation sum of sub-block j, split as
//         64 h + l so both parts are exact in f16; planes.h min_frag)
//   Q6_K  w = sc * (q6 - 32) in [-4096, 4064] = 64 wh + wl, wl in [0, 63], wh in [-64, 63]
//   Q8_0  one plane; the f32 scales apply per 32-value block (so this one is VALU-bound by design)
// Each superblock's integer result is exact in int32; the f32 epilogue per superblock mirrors the
// reference's d * dy * integer (k_quants.rs:1848-1928, 2518-2575).
//
// Tiling: a 256-thread workgroup owns BN = 128 weight rows x 32 TM activation rows (TM = 1, 2 or 4); wave w takes
// weight rows [32w, 32w+32) against all of them (TM MFMA tiles of 32x32).  Per 256-value K step the workgroup
// moves the activation superblock (int8 qs, f32 d, int16 sums of 32) global -> registers -> one of three LDS slots, and
// each wave loads its weight rows straight from HBM into registers two superblocks ahead and builds the B
// operands there.  A and B fragments use the same lane/byte -> k assignment, so the hardware's k order inside an
// MFMA does not matter.  The Q8_0 kernel keeps a simpler single-buffered loop.
#include "common.h"
#include "inferencequant.h"
#include "planes.h"
#include "skinny.h"
#include "units.h"

// 1: the expert-grouped matmul takes 32-row tiles when the average expert has at most 32 rows (0: the largest).
// MI355X, 8 x Q4_K 14336x4096 / 4096x14336 experts, 64 tokens top-2 (16 rows per expert on average, more than 32
// in the largest): MoE step 303 -> 227 us; a grouped 14336x4096 projection with 64 rows in one expert and 16 on
// average: Q8_0 222 -> 185 us, Q4_0 166 -> 120 us.
#ifndef QMM_MOE_SMALL_AVG
#define QMM_MOE_SMALL_AVG 1
#endif
// 1: the K-quant kernel's 32-row activation tiles (small batches, the expert-grouped matmul) take Q4_K weights
// from LDS too
#ifndef QMM_KQ_LW_TM1
#define QMM_KQ_LW_TM1 1
#endif

namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int TM = BM / 32;
constexpr int QS_STRIDE = 272;  // LDS row stride of the activation tile: 256 + 16 (bank spread)

struct ActTile {
  // global views of one channel of a prefill activation layout (include/inferencequant.h)
  const uint8_t *qs;     // [nsb][rows][256]
  const uint16_t *d8;    // Q8_0 blocks: [nsb][rows][8] f16
  const float *d32;      // Q8_K tiles: [nsb][rows] f32 (the int16 sums of 32, [nsb][rows][8], follow and are
                         //             addressed from qs)
  int64_t rows, nsb;
};

// ------------------------------------------------------------------------------------------ K-quant kernel

// One superblock of the activation tile (BMt rows x 256 values: int8 qs, int16 sums of 32, f32 d) in registers on its
// way from global memory to an LDS slot.  The prefill layout keeps a superblock's rows contiguous, so thread t
// moves 16-byte chunks t, t + NT, ... of each section (NT threads); every address is a per-thread constant plus a
// scalar.
// SB: bytes of sums per row and superblock, 16 (int16 sums of 32) or 32 (the `_q8k` tiles' f16 sums of 16).
template <int BMt, bool MIN, int NT, int SB = 16>
struct ActStage {
  static_assert(BMt * 16 % NT == 0, "whole qs chunks per thread");
  static constexpr int NQ = BMt * 16 / NT;  // qs chunks per thread
  static constexpr int QS = BMt * 256;       // LDS bytes: qs, row r's chunk c at chunk slot c ^ (r % 16)
  // the sums of row r at QS + 16 r (the second half of the area is the DMA form's overrun: ActDma)
  static constexpr int BSB = MIN ? BMt * 32 : 0;
  static constexpr int STAGE = QS + BSB + BMt * 4;
  u32x4 q[NQ];
  u32x4 bs;  // MIN, threads < BMt: one row's 8 sums
  u32x4 d;   // threads < BMt / 4: 4 scales

  // voff: per-thread byte offsets (qs, bsums, d) of row m0; s_*: offsets of superblock sb.  The whole offset
  // goes in the vector operand, where the buffer range check applies: rows past the channel read as zero.
  __device__ __forceinline__ void load(rsrc_t r, const uint32_t voff[3], uint32_t s_qs, uint32_t s_bs,
                                       uint32_t s_d) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NQ; i++) q[i] = __builtin_amdgcn_raw_buffer_load_b128(r, voff[0] + s_qs + 16 * NT * i, 0, 0);
    if (MIN && tid < BMt * SB / 16) bs = __builtin_amdgcn_raw_buffer_load_b128(r, voff[1] + s_bs, 0, 0);
    if (tid < BMt / 4) d = __builtin_amdgcn_raw_buffer_load_b128(r, voff[2] + s_d, 0, 0);
  }
  __device__ __forceinline__ void store(uint8_t *slot) const {
    const int tid = threadIdx.x;
    const int swz = (tid & 15) ^ ((tid >> 4) & 15);
#pragma unroll
    for (int i = 0; i < NQ; i++) *(u32x4 *)(slot + 16 * NT * i + 256 * (tid >> 4) + 16 * swz) = q[i];
    if (MIN && tid < BMt * SB / 16) *(u32x4 *)(slot + QS + 16 * tid) = bs;
    if (tid < BMt / 4) *(u32x4 *)(slot + QS + BSB + 16 * tid) = d;
  }
};

// The same superblock loaded by DMA straight into an LDS slot (buffer loads with the LDS flag): no registers hold
// it on the way, so the ring can be deep without spilling.  Wave w's lane l writes LDS byte 16 l (4 l for the
// 4-byte sections) of each 1 KB (256 B) piece it loads; it fetches the global bytes that belong at that place of
// the swizzled layout.  Every one of the NW waves issues kLoads loads per superblock (the same count: the tile loop's
// wait counts on it).  The compiler does not order LDS reads after these writes: the tile loop waits for them with an
// explicit vmcnt before its barrier.
template <int BMt, bool MIN, int NW, int SB = 16>
struct ActDma {
  static_assert(BMt % (4 * NW) == 0 && (!MIN || BMt % (8 * NW) == 0), "the same load count in every wave");
  static constexpr int QS = BMt * 256;
  static constexpr int BSB = MIN ? BMt * 32 : 0;
  static constexpr int STAGE = QS + BSB + BMt * 4;
  static constexpr int NQ = BMt / (4 * NW);            // 1 KB qs pieces per wave
  // 256 B pieces of sums per wave: twice the 16 BMt bytes of the tile's rows, so that every wave issues the same
  // number of loads; the second half reads the rows after the tile into the second half of the area, unused
  static constexpr int NB = MIN ? BMt / (8 * NW) : 0;
  static constexpr int ND = BMt / NW;                  // lanes of each wave that load one f32 scale
  static constexpr int kLoads = NQ + NB + 1;
  uint32_t oq[NQ], ob[NB > 0 ? NB : 1], od;

  // per-lane byte offsets of row block m0 in superblock 0 (the superblock's part is added at issue, in the
  // vector operand too, so the buffer range check covers the whole offset)
  __device__ __forceinline__ void init(int wave, int lane, int64_t m0, int64_t rows, int64_t nsb) {
#pragma unroll
    for (int i = 0; i < NQ; i++) {
      const int L = 64 * (NW * i + wave) + lane, r = L >> 4, c = (L & 15) ^ (r & 15);
      oq[i] = (uint32_t)((m0 + r) * 256 + 16 * c);
    }
#pragma unroll
    for (int i = 0; i < NB; i++) {
      const int D = 64 * (NW * i + wave) + lane, r = SB == 32 ? D >> 3 : D >> 2, k = SB == 32 ? D & 7 : D & 3;
      ob[i] = (uint32_t)(nsb * rows * 260 + (m0 + r) * SB + 4 * k);
    }
    od = (uint32_t)(nsb * rows * 256 + (m0 + ND * wave + lane) * 4);
  }
  // (device pass only: the host pass rejects the gfx950 16-byte LDS load inside this template)
  __device__ __forceinline__ void issue(rsrc_t r, uint8_t *slot, int wave, int lane, uint32_t sb_rows) const {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
    for (int i = 0; i < NQ; i++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(slot + 1024 * (NW * i + wave)),
                                               16, oq[i] + 256 * sb_rows, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NB; i++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void *)(slot + QS + 256 * (NW * i + wave)), 4, ob[i] + SB * sb_rows, 0,
          0, 0);
    if (lane < ND)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void *)(slot + QS + BSB + 4 * ND * wave), 4, od + 4 * sb_rows, 0, 0,
          0);
#endif
  }
};

// Workgroup barrier for the DMA ring: first this wave's loads but the newest N have landed (they complete in
// order) and its LDS reads have returned, then s_barrier.  No fence: the LDS is written only by DMA, which the
// compiler does not track (its own fence would wait for every DMA in flight); the asm's memory clobber keeps
// LDS reads from moving across.
template <int N>
__device__ __forceinline__ void dma_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(N) : "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// LDS-only workgroup barrier: orders LDS accesses (lgkmcnt) but leaves global loads in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One workgroup: NW (4 or 8) waves x 32 weight rows (32 NW of them) against BMt = 32 TM activation rows; wave w's lanes
// hold weight row n0 + 32w + (lane % 32) as the MFMA B column and TM 32x32 output tiles.  The activation tile in LDS
// serves all NW waves, so 8 waves halve the activation bytes read per weight row.  Three LDS slots and three
// register sets rotate: during superblock s the workgroup computes from slot s, writes the activations of s + 1
// (loaded one step earlier) into slot s + 1, and has the activations and weights of s + 2 in flight, so global
// latency is covered by two steps of MFMA work.  One LDS barrier per superblock.
// S16: the activations are `_q8k` tiles (f16 sums of 16, the min term's A operand as it is), else the reference-named
// tiles (int16 sums of 32, split for the f16 MFMA here: planes.h min_frag).
template <class WT, class Out, int TM, int NW, bool S16 = false>
__device__ __forceinline__ void mmq_kq_tile(const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes,
                                            const ActTile &a, int64_t m0, int64_t mrows, int64_t n0, int64_t sb0,
                                            int64_t sb1, typename Out::T *__restrict__ dst, int64_t ldd,
                                            const int32_t *__restrict__ dst_rows, float *__restrict__ part) {
  constexpr int BMt = 32 * TM;
  constexpr int BNt = 32 * NW;
  // kLw: the weight superblocks go by DMA into LDS too, as the tile's rows' contiguous 16-byte pieces, and each wave
  // reads its B-operand bytes from there.  Loaded straight into registers, one 16-byte load per lane covers 32 weight
  // rows, 32 bytes of each, and the texture addresser's per-cache-line work for those loads bounds the kernel; as
  // contiguous pieces the same bytes take a quarter of the cache-line accesses.  Two stages of activations, so the
  // next superblock's loads are in flight during one step (the LDS does not hold three).  Q4_K takes this path at
  // 64-row activation tiles and (QMM_KQ_LW_TM1) at 32-row ones (MI355X, 14336x4096 at M = 32: 21.2 -> 16.8 us).
  constexpr bool kLw = WT::kLdsWeights && (TM == WT::kLwTM || (QMM_KQ_LW_TM1 && TM == 1 && WT::kMin));
  // Without kLw, Q4_K stages its activations by DMA (its register budget at two waves per SIMD has no room for a
  // register ring); Q6_K, at one wave per SIMD, through registers.  Both write the same LDS layout.
  constexpr bool kDma = WT::kDma || kLw;
  constexpr int SB = S16 ? 32 : 16;
  typedef ActStage<BMt, WT::kMin, 64 * NW, SB> AS;
  typedef ActDma<BMt, WT::kMin, NW, SB> AD;
  static_assert(AS::STAGE == AD::STAGE, "one LDS layout");
  // Superblocks of a multiple of 16 bytes (Q4_K: 16-byte aligned) are copied as their own pieces and kept row after
  // row.  Others (Q6_K: 210 bytes, 2-byte aligned) are copied as the 16-byte pieces of a window that starts at the
  // dword holding their first byte, and kept piece-major: piece k of tile row r at 16 (BNt k + r).  Then each DMA
  // round of the workgroup (64 NW lanes = 2 BNt) takes pieces 2i and 2i + 1 of every row, so a lane's global offset
  // is one row's window plus a constant, and the reads of a piece by consecutive rows are consecutive 16 bytes.
  constexpr bool kRowMajor = WT::kBytes % 16 == 0;
  constexpr int kPieces = kRowMajor ? WT::kBytes / 16 : (WT::kBytes + 3 + 15) / 16;  // pieces per superblock
  constexpr int kWI = kLw ? (BNt * kPieces + 64 * NW - 1) / (64 * NW) : 0;  // weight DMA loads per wave
  // weight bytes per stage: every lane of every load writes its 16 bytes, the padding lanes past the slab included
  constexpr int WST = kWI * 64 * NW * 16;
  constexpr int STG = AS::STAGE + WST;
  // weight stages: two where two workgroups still fit the 160 KB of a CU, else one, reloaded once every wave has
  // read it (a second barrier per superblock).  (Three to five stages for 32-row activation tiles, at one workgroup
  // per CU, measured slower than two at two workgroups.)
  constexpr int kWS = 2 * STG <= (TM == 2 ? 80 : 160) * 1024 ? 2 : 1;
  constexpr int kPS = kRowMajor ? 16 : 16 * BNt;  // LDS bytes from one piece of a row to its next
  // (only where two workgroups share each SIMD: at one wave per SIMD it measured no gain.  On 32-row tiles for the
  // two-plane Q4_K: M = 32, 14336x4096 18.3 -> 16.7 us, the 64-token MoE step 260 -> 252 us; Q5_K's three planes at
  // 32-row tiles measured slower with it, M = 512 135.8 -> 141.5 us)
  constexpr bool kPrio = kLw && (TM == 2 || (TM == 1 && WT::kPlanes == 2));
  static_assert(!kLw || AS::STAGE % 16 == 0, "16-byte aligned stages");
  static_assert(!kLw || kRowMajor || 64 * NW == 2 * BNt, "two pieces of every row per DMA round");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLw ? 2 * AS::STAGE + kWS * WST : 3 * AS::STAGE];
  // kLw stage u: activations and weights (two weight stages: as STG-byte stages, activations first)
  auto act_slot = [&](int u) { return lds + u * (kWS == 2 ? STG : AS::STAGE); };
  auto w_slot = [&](int u) { return kWS == 2 ? lds + u * STG + AS::STAGE : lds + 2 * AS::STAGE; };

  // (the wave index as a scalar: the LDS addresses of the DMA loads, which go through M0, are then scalar arithmetic)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 5,
            li = lane & 31;
  const int64_t n = n0 + 32 * wave + li;
  const int64_t nlast = (nrows_w - n0 < BNt ? nrows_w - n0 : BNt) - 1;
  const int64_t nl = 32 * wave + li < nlast ? 32 * wave + li : nlast;  // row within the tile, clamped

  // activations: one resource over the channel; the scalar part of each address moves with the superblock
  const int64_t rows = a.rows, nsb = a.nsb;
  const rsrc_t ra = make_rsrc(a.qs, nsb * rows * (260 + SB));
  const uint32_t voff[3] = {(uint32_t)(m0 * 256 + 16 * tid),
                            (uint32_t)(nsb * rows * 260 + m0 * SB + 16 * tid),
                            (uint32_t)(nsb * rows * 256 + m0 * 4 + 16 * tid)};
  // weights: one resource over the tile's rows, from the dword that holds the tile's first byte (wdelta bytes
  // before it), so offsets that are multiples of 4 from the resource are dword aligned in memory, to the end of the
  // dword that holds its last byte: the range check passes or zeroes whole dwords, and a superblock that ends inside
  // a dword (Q6_K) has its last bytes there
  const uintptr_t wt = (uintptr_t)(W + n0 * w_row_bytes);
  const uint32_t wdelta = (uint32_t)(wt & 3);
  const rsrc_t rw = make_rsrc((const uint8_t *)(wt - wdelta), ((nlast + 1) * w_row_bytes + wdelta + 3) & ~(int64_t)3);
  const uint32_t wrow = (uint32_t)(nl * w_row_bytes) + wdelta;

  // LDS read offsets of this lane's A fragments: row 32t + li, chunk WT::chunk(j, g) (2j + g but for IQ4_XS),
  // swizzled
  uint32_t qoff[8];
#pragma unroll
  for (int j = 0; j < 8; j++) qoff[j] = 256 * li + 16 * (WT::chunk(j, g) ^ (li & 15));

  v16f fa[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) fa[t] = (v16f){};

  AS st[kDma ? 1 : 3];
  AD dma;
  if (kDma) dma.init(wave, lane, m0, rows, nsb);
  typename WT::Raw raw[kLw ? 1 : 3];
  // kLw: lane's weight piece C = 64 (NW i + wave) + lane of the stage's slab goes to LDS byte 16 C of the stage's
  // weight part.  Row-major: row C / kPieces, piece C % kPieces, and pieces past the slab read past the resource (no
  // memory traffic).  Piece-major: row C % BNt = 64 wave + lane - BNt (wave >= NW / 2), piece C / BNt = 2i + (wave >=
  // NW / 2); a piece index past the window is not loaded.
  constexpr int kWO = kRowMajor ? (kWI > 0 ? kWI : 1) : 1;
  uint32_t woff[kWO];
  const int whalf = wave >= NW / 2 ? 1 : 0;
  if constexpr (kRowMajor) {
#pragma unroll
    for (int i = 0; i < kWI; i++) {
      const int C = 64 * (NW * i + wave) + lane, r = C / kPieces, pc = C - r * kPieces;
      woff[i] = C < BNt * kPieces ? (uint32_t)(r * w_row_bytes + 16 * pc) : 0x80000000u;
    }
  } else {
    woff[0] = (uint32_t)((64 * wave + lane - BNt * whalf) * w_row_bytes) + wdelta + 16 * whalf;
  }
  auto issue_lw = [&](int64_t sb, int u) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_sched_barrier(0);
    dma.issue(ra, act_slot(u), wave, lane, (uint32_t)(sb * rows));
    // (piece-major: the window starts at the dword of the superblock's first byte; whalf's 16 bytes are a multiple
    // of 4, so they survive the rounding)
    const uint32_t wv = kRowMajor ? 0u : (woff[0] + (uint32_t)sb * WT::kBytes) & ~3u;
#pragma unroll
    for (int i = 0; i < kWI; i++) {
      if (kRowMajor || 2 * i + 1 < kPieces || whalf == 0)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rw, (__attribute__((address_space(3))) void *)(w_slot(u) + 1024 * (NW * i + wave)), 16,
            kRowMajor ? woff[i] + (uint32_t)sb * WT::kBytes : wv + 32 * i, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
#endif
  };
  // DMA first, then the weights (WT::kLoads 16-byte loads, which cannot merge): the explicit wait in step()
  // counts on that order
  auto issue = [&](int64_t sb, int u, AS &as, typename WT::Raw &rr) {
    if constexpr (kDma) {
      __builtin_amdgcn_sched_barrier(0);
      dma.issue(ra, lds + u * AS::STAGE, wave, lane, (uint32_t)(sb * rows));
      WT::load(rw, wrow, (uint32_t)sb, g, rr);
      __builtin_amdgcn_sched_barrier(0);
    } else {
      as.load(ra, voff, (uint32_t)(sb * rows * 256), (uint32_t)(sb * rows * SB), (uint32_t)(sb * rows * 4));
      WT::load(rw, wrow, (uint32_t)sb, g, rr);
    }
  };

  // The A-fragment LDS reads run one sub-block ahead of the MFMAs that consume them, so LDS latency overlaps
  // matrix work.
  auto compute = [&](const uint8_t *slot, const typename WT::Raw &rr) {
    typename WT::Prep p;
    if constexpr (WT::kMin)
      WT::template prepare<S16>(rr, g, p);
    else
      WT::prepare(rr, g, p);
    v16i acc1[TM], acc2[TM], acc3[TM];  // acc3: Q5_K's fifth-bit plane
#pragma unroll
    for (int t = 0; t < TM; t++) acc1[t] = acc2[t] = acc3[t] = (v16i){};
    // (Q4_K at TM = 2 runs at 2 waves per SIMD, where the extra registers would spill: it reads just in time)
    constexpr bool kAhead = !(WT::kMin && TM == 2);
    v4i av[2][TM];
#pragma unroll
    for (int t = 0; t < TM; t++) av[0][t] = *(const v4i *)(slot + 8192 * t + qoff[0]);
    // The two waves on a SIMD come from two workgroups and drift apart: a wave in its MFMA chain gets the issue slots
    // first, so the other's VALU epilogue fills the matrix core's cycles instead of the two taking turns (MI355X,
    // Q4_K at M = 512: 90 -> 83 us)
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(3);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (kAhead && j < 7) {
#pragma unroll
        for (int t = 0; t < TM; t++) av[(j + 1) & 1][t] = *(const v4i *)(slot + 8192 * t + qoff[j + 1]);
      }
      v4i b1, b2, b3;
      if constexpr (WT::kPlanes == 3)
        WT::planes(rr, p, j, b1, b2, b3);
      else
        WT::planes(rr, p, j, b1, b2);
#pragma unroll
      for (int t = 0; t < TM; t++) {
        const v4i a = kAhead ? av[j & 1][t] : *(const v4i *)(slot + 8192 * t + qoff[j]);
        acc1[t] = mfma_i8(a, b1, acc1[t]);
        acc2[t] = mfma_i8(a, b2, acc2[t]);
        if constexpr (WT::kPlanes == 3) acc3[t] = mfma_i8(a, b3, acc3[t]);
      }
    }
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      v16f fmin = (v16f){};
      if (WT::kMin && S16) {  // the f16 sums of 16 of sub-blocks 4g .. 4g + 3 of row 32t + li
        const v8h bs = *(const v8h *)(slot + AS::QS + (32 * t + li) * 32 + 16 * g);
        fmin = mfma_f16(bs, p.bmin, fmin);
      } else if (WT::kMin) {  // the sums of 32 of sub-blocks 4g .. 4g + 3 of row 32t + li
        const u32x2 sm = *(const u32x2 *)(slot + AS::QS + (32 * t + li) * 16 + 8 * g);
        fmin = mfma_f16(min_frag(sm.x, sm.y), p.bmin, fmin);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const v4f dy4 = *(const v4f *)(slot + AS::QS + AS::BSB + 4 * (32 * t + 8 * q + 4 * g));  // rows 8q + 4g + i
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int r = 4 * q + i;
          int iv = (acc1[t][r] << WT::kShift) + acc2[t][r];
          if constexpr (WT::kPlanes == 3) iv += acc3[t][r] << 4;
          float v = p.d * (float)iv;
          if (WT::kMin) v -= p.dmin * fmin[r];
          fa[t][r] += dy4[i] * v;
        }
      }
    }
  };

  // Every step issues the loads of s + 2 (past the end: the last superblock again, into a slot and registers
  // that are never read), so each step starts with the same loads outstanding and the wait counts stay exact.
  auto step = [&](int64_t s, int u) {
    // u = (s - sb0) % 3 is a constant after unrolling: slot u, register sets u, u + 1, u + 2
    if constexpr (kDma) {
      // this wave's DMA into slot u (issued two steps ago) has landed once at most the loads issued after it are
      // outstanding: the weights of s, then the DMA and weights of s + 1 (counted as if the weights came
      // first, which can only wait longer)
      __builtin_amdgcn_sched_barrier(0);
      dma_barrier<AD::kLoads + WT::kLoads>();
    } else {
      __builtin_amdgcn_sched_barrier(0);
      lds_barrier();
    }
    const int64_t sn = s + 2 < sb1 ? s + 2 : sb1 - 1;
    if constexpr (kDma) {
      issue(sn, (u + 2) % 3, st[0], raw[(u + 2) % 3]);
      if (s < sb1) compute(lds + u * AS::STAGE, raw[u]);  // (no memory loads inside: the load pattern is uniform)
    } else {
      issue(sn, (u + 2) % 3, st[(u + 2) % 3], raw[(u + 2) % 3]);
      if (s < sb1) compute(lds + u * AS::STAGE, raw[u]);
      st[(u + 1) % 3].store(lds + ((u + 1) % 3) * AS::STAGE);
    }
    __builtin_amdgcn_sched_barrier(0);  // steps do not interleave: each one's registers die at its end
  };

  if constexpr (kLw) {
    // two stages: after the barrier of step s every wave is done with stage (s + 1) % 2, so the loads of s + 1 go
    // there while s is computed from stage s % 2.  With one weight stage, the weights of s go to registers first
    // and a second barrier waits until every wave has read them before the loads of s + 1 overwrite them.
    const uint32_t wl = kRowMajor ? (uint32_t)(nl * WT::kBytes) : (uint32_t)(16 * nl);  // the lane's row in a stage
    issue_lw(sb0, 0);
    for (int64_t sb = sb0; sb < sb1; sb += 2) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int64_t s = sb + u;
        if (s < sb1) {  // (uniform over the workgroup)
          __builtin_amdgcn_sched_barrier(0);
          dma_barrier<0>();
          const uint32_t off = kRowMajor ? 0u : (wrow + (uint32_t)s * WT::kBytes) & 3u;
          if constexpr (kWS == 1) WT::template load_lds<kPS>(w_slot(u) + wl, off, g, raw[0]);
          if (s + 1 < sb1) {
            if constexpr (kWS == 1) dma_barrier<0>();
            issue_lw(s + 1, u ^ 1);
          }
          if constexpr (kWS == 2) WT::template load_lds<kPS>(w_slot(u) + wl, off, g, raw[0]);
          compute(act_slot(u), raw[0]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  } else {
  issue(sb0, 0, st[0], raw[0]);
  issue(sb0 + 1 < sb1 ? sb0 + 1 : sb1 - 1, 1, st[kDma ? 0 : 1], raw[1]);
  if constexpr (!kDma) st[0].store(lds);
  // every step runs its barrier and loads; steps past sb1 (at most two) skip only the math
  for (int64_t sb = sb0; sb < sb1; sb += 3) {
    step(sb, 0);
    step(sb + 1, 1);
    step(sb + 2, 2);
  }
  }

  if (n < nrows_w) {
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int64_t m = m0 + 32 * t + out_row(r, g);
        if (m < mrows) {
          if (part)  // split K: this split's partial sum, row m of the activation order (summed by k_split_sum)
            part[m * nrows_w + n] = fa[t][r];
          else
            Out::store(dst, (dst_rows ? dst_rows[m] : m) * ldd + n, fa[t][r]);
        }
      }
  }
}

// Split K: split s of a tile writes its partial sums to plane s of the caller's fixup buffer (planes of rows x cols
// f32, row m of the activation order); this kernel adds the planes in split order, so the result does not depend on
// which split finished first, and stores them in the output type (dst row rows_map ? rows_map[m] : m).  Workgroup
// (x, y) takes 1024 columns of rows y, y + gridDim.y, ...; 4 columns per thread.  A kernel, so that the launch
// sequence can sit in a HIP graph.
template <class Out>
__global__ __launch_bounds__(256) void k_split_sum(const float *__restrict__ part, int64_t splits, int64_t rows,
                                                   int64_t cols, typename Out::T *__restrict__ dst, int64_t ldd,
                                                   const int32_t *__restrict__ rows_map) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= cols) return;
  const int64_t plane = rows * cols;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float *p = part + r * cols + c;
    const int64_t o = (rows_map ? rows_map[r] : r) * ldd + c;
    if (c + 4 <= cols && cols % 4 == 0) {
      v4f v = *(const v4f *)p;
      for (int64_t sp = 1; sp < splits; sp++) v += *(const v4f *)(p + sp * plane);
#pragma unroll
      for (int i = 0; i < 4; i++) Out::store(dst, o + i, v[i]);
    } else {
      for (int64_t i = 0; i < 4 && c + i < cols; i++) {
        float v = p[i];
        for (int64_t sp = 1; sp < splits; sp++) v += p[sp * plane + i];
        Out::store(dst, o + i, v);
      }
    }
  }
}

template <class Out>
void split_sum(const float *part, int64_t splits, int64_t rows, int64_t cols, typename Out::T *dst, int64_t ldd,
               const int32_t *rows_map, hipStream_t s) {
  const dim3 grid((unsigned)qmm_ceil_div(cols, 1024), (unsigned)(rows < 64 ? rows : 64));
  k_split_sum<Out><<<grid, 256, 0, s>>>(part, splits, rows, cols, dst, ldd, rows_map);
}

// ------------------------------------------------------------------------------------------ Q8_0 kernel

// Q8_0 weights against Q8_0 activations: one MFMA per 32-value block, scaled in f32 per block as
// k_quants.rs:982-999 does ((sum as f32 * d_w) * d_a, summed over blocks).
// The 32-value weight blocks of the Q8_0-layout prefill: lane half g of a weight row takes values 16g .. 16g + 15 of
// each block as 16 signed bytes, and the block's f32 scale.
//   Q8_0  34 B {f16 d; i8 q[32]}                      (k_quants.rs:152-157)
//   Q4_0  18 B {f16 d; u8 qs[16]}, value q - 8         (k_quants.rs:116-120): half g = nibble g of qs[0..15]
//   Q5_0  22 B {f16 d; u8 qh[4]; u8 qs[16]}, q - 16    (k_quants.rs:133-138): fifth bit of value v = bit v of qh
// q - 8 is the 4-bit two's complement of q ^ 8, and q - 16 the 5-bit one of q ^ 16; their sign bits spread to the
// byte's top bits by one multiply per dword (no carry crosses a byte).
struct wb_q8_0 {
  static constexpr int kBytes = 34;
  static __device__ __forceinline__ void load(const uint8_t *p, int g, uint32_t (&wq)[4], float &d) {
    d = f16_bits_to_f32(ld16(p));
    const uint8_t *q = p + 2 + 16 * g;
    const uint32_t off = (uint32_t)((uintptr_t)q & 3);
    unit_q6k::realign(ld_a4(q - off), ld32(q - off + 16), off, wq);
  }
};
struct wb_q4_0 {
  static constexpr int kBytes = 18;
  static __device__ __forceinline__ void load(const uint8_t *p, int g, uint32_t (&wq)[4], float &d) {
    d = f16_bits_to_f32(ld16(p));
    const uint8_t *q = p + 2;
    const uint32_t off = (uint32_t)((uintptr_t)q & 3);
    uint32_t raw[4];
    unit_q6k::realign(ld_a4(q - off), ld32(q - off + 16), off, raw);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t v = ((raw[i] >> (4 * g)) & 0x0f0f0f0fu) ^ 0x08080808u;
      wq[i] = v | ((v & 0x08080808u) * 0x1eu);
    }
  }
};
struct wb_q5_0 {
  static constexpr int kBytes = 22;
  static __device__ __forceinline__ void load(const uint8_t *p, int g, uint32_t (&wq)[4], float &d) {
    d = f16_bits_to_f32(ld16(p));
    const uint32_t qh = ld16(p + 2) | (ld16(p + 4) << 16);
    const uint8_t *q = p + 6;
    const uint32_t off = (uint32_t)((uintptr_t)q & 3);
    uint32_t raw[4];
    unit_q6k::realign(ld_a4(q - off), ld32(q - off + 16), off, raw);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t hb = (((qh >> (16 * g + 4 * i)) & 15u) * 0x00204081u & 0x01010101u) << 4;
      const uint32_t v = (((raw[i] >> (4 * g)) & 0x0f0f0f0fu) | hb) ^ 0x10101010u;
      wq[i] = v | ((v & 0x10101010u) * 0x0fu);
    }
  }
};

template <class WB, class Out, bool F32D>
__device__ __forceinline__ void mmq_q8_0_tile(const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes,
                                              int64_t nblk_w, const ActTile &a, int64_t m0, int64_t mrows, int64_t n0,
                                              int64_t nsb, typename Out::T *__restrict__ dst, int64_t ldd,
                                              const int32_t *__restrict__ dst_rows) {
  __shared__ __attribute__((aligned(16))) uint8_t s_qs[BM * QS_STRIDE];
  __shared__ float s_da[BM * 9];  // 8 block scales per row (stride 9 against bank conflicts)

  // (the wave index as a scalar: the LDS addresses of the DMA loads, which go through M0, are then scalar arithmetic)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 5,
            li = lane & 31;
  const int64_t n = n0 + 32 * wave + li;
  const int64_t n_ld = n < nrows_w ? n : nrows_w - 1;
  const uint8_t *wrow = W + n_ld * w_row_bytes;

  v16f fa[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) fa[t] = (v16f){};

  for (int64_t sb = 0; sb < nsb; sb++) {
    uint32_t wq[8][4];
    float dw[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int64_t blk = sb * 8 + j;
      if (blk < nblk_w) {
        WB::load(wrow + blk * WB::kBytes, g, wq[j], dw[j]);
      } else {
        dw[j] = 0.0f;
        wq[j][0] = wq[j][1] = wq[j][2] = wq[j][3] = 0;
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < BM * 16 / 256; it++) {
      const int i = it * 256 + tid;
      const int row = i >> 4, c = i & 15;
      const int64_t m = m0 + row;
      u32x4 v = {0, 0, 0, 0};
      if (m < mrows) v = ld_a16(a.qs + (sb * a.rows + m) * 256 + 16 * c);
      *(u32x4 *)(s_qs + row * QS_STRIDE + 16 * c) = v;
    }
#pragma unroll
    for (int it = 0; it < BM * 8 / 256; it++) {
      const int i = it * 256 + tid;
      const int row = i >> 3, j = i & 7;
      const int64_t m = m0 + row;
      s_da[row * 9 + j] = m >= mrows ? 0.0f : F32D ? a.d32[sb * a.rows + m] : f16_bits_to_f32(a.d8[(sb * a.rows + m) * 8 + j]);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const v4i b = {(int)wq[j][0], (int)wq[j][1], (int)wq[j][2], (int)wq[j][3]};
#pragma unroll
      for (int t = 0; t < TM; t++) {
        const v4i av = *(const v4i *)(s_qs + (32 * t + li) * QS_STRIDE + 32 * j + 16 * g);
        const v16i acc = mfma_i8(av, b, (v16i){});
#pragma unroll
        for (int r = 0; r < 16; r++) fa[t][r] += ((float)acc[r] * dw[j]) * s_da[(32 * t + out_row(r, g)) * 9 + j];
      }
    }
  }
  if (n >= nrows_w) return;
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int64_t m = m0 + 32 * t + out_row(r, g);
      if (m < mrows) {
        const int64_t drow = dst_rows ? dst_rows[m] : m;
        Out::store(dst, drow * ldd + n, fa[t][r]);
      }
    }
}

// ------------------------------------------------------------------------------------------ 32-value blocks, runs

// The pipelined kernel for Q8_0 / Q4_0 / Q5_0 weights (rows a whole number of superblocks, dword-aligned).  Each
// superblock of a weight row is read as two dword-aligned runs of four blocks: lane half g of the row's lane pair
// loads blocks 4g .. 4g + 3 with 16-byte loads, decodes both 16-value halves of each, and one v_permlane32_swap per
// dword trades halves with the partner lane, so that half g of all eight blocks ends in lane half g (the MFMA B
// layout used by the Q8_0 kernel above).  Per block, the scale products da * dw (exact in f32: two f16 factors)
// come from an outer-product MFMA in the accumulator layout, leaving one convert and one FMA per output: an f16 MFMA
// on the scales' f16 bits (half the matrix-core cycles of the f32 one; the f16 MFMA keeps subnormal inputs, so the
// products are the same bits) over Q8_0 activation tiles, the f32 MFMA over Q8_K tiles (an f32 activation scale).
__device__ __forceinline__ uint32_t run_dw(const uint32_t *R, int o) {  // dword at byte offset o of the run
  return o % 4 == 0 ? R[o / 4] : __builtin_amdgcn_alignbyte(R[o / 4 + 1], R[o / 4], (uint32_t)(o % 4));
}
__device__ __forceinline__ uint32_t run_u16(const uint32_t *R, int o) { return (R[o / 4] >> (8 * (o % 4))) & 0xffffu; }

// decode(R, i, d, h0, h1): block i of the run: f16 scale bits d, values 0..15 (h0) and 16..31 (h1) as signed bytes
// kSets: weight register sets (two: the weights of s + 2 are in flight while s is computed; one: those of s + 1).
// Q8_0's 34-dword runs take one, which leaves room for the f16 scale MFMA's operands: with two sets and the f16 MFMA
// the kernel spilled (172.7 us at M = 512, 14336x4096), with two and the f32 MFMA it took 152.9 us, with one and the
// f16 MFMA 137.1 us.  Q4_0 / Q5_0 keep two (one: 114.4 -> 122.5 us, 127.5 -> 138.1 us).
struct wr_q8_0 {
  static constexpr int kBytes = 34, kDwords = 34;  // run: 136 bytes
  static constexpr int kSets = 1;
  static __device__ __forceinline__ void decode(const uint32_t *R, int i, uint32_t &d, uint32_t (&h0)[4],
                                                uint32_t (&h1)[4]) {
    const int o = 34 * i;
    d = run_u16(R, o);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      h0[q] = run_dw(R, o + 2 + 4 * q);
      h1[q] = run_dw(R, o + 18 + 4 * q);
    }
  }
};
struct wr_q4_0 {
  static constexpr int kBytes = 18, kDwords = 18;  // run: 72 bytes
  static constexpr int kSets = 2;
  static __device__ __forceinline__ void decode(const uint32_t *R, int i, uint32_t &d, uint32_t (&h0)[4],
                                                uint32_t (&h1)[4]) {
    const int o = 18 * i;
    d = run_u16(R, o);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t Q = run_dw(R, o + 2 + 4 * q);
      const uint32_t v0 = (Q & 0x0f0f0f0fu) ^ 0x08080808u, v1 = ((Q >> 4) & 0x0f0f0f0fu) ^ 0x08080808u;
      h0[q] = v0 | ((v0 & 0x08080808u) * 0x1eu);
      h1[q] = v1 | ((v1 & 0x08080808u) * 0x1eu);
    }
  }
};
struct wr_q5_0 {
  static constexpr int kBytes = 22, kDwords = 22;  // run: 88 bytes
  static constexpr int kSets = 2;
  static __device__ __forceinline__ void decode(const uint32_t *R, int i, uint32_t &d, uint32_t (&h0)[4],
                                                uint32_t (&h1)[4]) {
    const int o = 22 * i;
    d = run_u16(R, o);
    const uint32_t qh = run_dw(R, o + 2);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t Q = run_dw(R, o + 6 + 4 * q);
      const uint32_t b0 = ((((qh >> (4 * q)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
      const uint32_t b1 = ((((qh >> (16 + 4 * q)) & 15u) * 0x00204081u) & 0x01010101u) << 4;
      const uint32_t v0 = ((Q & 0x0f0f0f0fu) | b0) ^ 0x10101010u, v1 = (((Q >> 4) & 0x0f0f0f0fu) | b1) ^ 0x10101010u;
      h0[q] = v0 | ((v0 & 0x10101010u) * 0x0fu);
      h1[q] = v1 | ((v1 & 0x10101010u) * 0x0fu);
    }
  }
};

// The lane's run of superblock sb: kDwords / 4 16-byte loads and one 8-byte load (every run is 4k + 2 dwords).
template <class WR>
struct RunLoad {
  static_assert(WR::kDwords % 4 == 2, "run of 4k + 2 dwords");
  static constexpr int kLoads = WR::kDwords / 4 + 1;
  static __device__ __forceinline__ void load(rsrc_t rs, uint32_t off, uint32_t (&R)[WR::kDwords]) {
#pragma unroll
    for (int k = 0; k < WR::kDwords / 4; k++) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * k, 0, 0);
      R[4 * k] = v[0], R[4 * k + 1] = v[1], R[4 * k + 2] = v[2], R[4 * k + 3] = v[3];
    }
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, off + 16 * (WR::kDwords / 4), 0, 0);
    R[WR::kDwords - 2] = v[0], R[WR::kDwords - 1] = v[1];
  }
};

// Activation superblock of a prefill layout by DMA into an LDS slot: qs as in ActDma (swizzled 256-byte rows), then
// the scales.  Q8_0 blocks (F32D false): the rows' 16-byte groups of eight f16 (one per 32 values) in row order.
// Q8_K tiles (F32D): one f32 per row and superblock; every wave loads 64 rows' (row 64 w + l at byte 4 (64 w + l) of
// a 1 KB area), so every wave issues the same loads, and the rows past the tile land in the area's unused part.
template <int BMt, bool F32D = false>
struct ActDma8 {
  static constexpr int QS = BMt * 256;
  static constexpr int STAGE = QS + (F32D ? 1024 : BMt * 16);
  static constexpr int NQ = BMt / 16;  // 1 KB qs pieces per wave
  static constexpr int ND = BMt / 4;   // (Q8_0 blocks) lanes of each wave that load one row's 16 bytes of scales
  static constexpr int kLoads = NQ + 1;
  uint32_t oq[NQ], od;

  __device__ __forceinline__ void init(int wave, int lane, int64_t m0, int64_t rows, int64_t nsb) {
#pragma unroll
    for (int i = 0; i < NQ; i++) {
      const int L = 64 * (4 * i + wave) + lane, r = L >> 4, c = (L & 15) ^ (r & 15);
      oq[i] = (uint32_t)((m0 + r) * 256 + 16 * c);
    }
    od = F32D ? (uint32_t)(nsb * rows * 256 + (m0 + 64 * wave + lane) * 4)
              : (uint32_t)(nsb * rows * 256 + (m0 + ND * wave + lane) * 16);
  }
  // (device pass only: the host pass rejects the gfx950 16-byte LDS load inside this template)
  __device__ __forceinline__ void issue(rsrc_t r, uint8_t *slot, int wave, int lane, uint32_t sb_rows) const {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
    for (int i = 0; i < NQ; i++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(slot + 1024 * (4 * i + wave)),
                                               16, oq[i] + 256 * sb_rows, 0, 0, 0);
    if (F32D)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)(slot + QS + 256 * wave), 4,
                                               od + 4 * sb_rows, 0, 0, 0);
    else if (lane < ND)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void *)(slot + QS + 16 * ND * wave), 16, od + 16 * sb_rows, 0, 0, 0);
#endif
  }
};

// An empty volatile asm statement on v: the compiler keeps such statements in order, and v's producers before it
// (device pass only: the host pass has no VGPR constraint and never runs this code)
template <class T>
__device__ __forceinline__ void order_point(T &v) {
#if defined(__HIP_DEVICE_COMPILE__)
  __asm__ volatile("" : "+v"(v));
#endif
}

__device__ __forceinline__ v16f mfma_f32x2(float a, float b) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, (v16f){}, 0, 0, 0);
}

// Group k = (tile k / 8, block j = k % 8): the integer block dot and the scale outer product on A fragment av.
// Block j's scales live in lane half j / 4; the other half contributes zeros.  F32S: the scales as f32 (da, dw) and
// the f32 MFMA (k = g); else their f16 bits, two to a dword (blocks 2p and 2p + 1 of the half in dword p of dah, dwh),
// and the f16 MFMA (k = 4g, the rest of each half zero).
template <bool F32S>
__device__ __forceinline__ void b32_group(v4i av, const v4i (&b)[8], const float (&da)[4], const uint32_t (&dah)[2],
                                          const float (&dw)[4], const uint32_t (&dwh)[2], int g, int k, v16i &acc,
                                          v16f &sc) {
  const int j = k & 7, i = j & 3;
  const bool mine = g == (j >> 2);
  order_point(av);
  acc = mfma_i8(av, b[j], (v16i){});
  if constexpr (F32S) {
    sc = mfma_f32x2(mine ? da[i] : 0.0f, mine ? dw[i] : 0.0f);
  } else {
    const uint32_t a = (i & 1) ? dah[i >> 1] >> 16 : dah[i >> 1] & 0xffffu;
    const uint32_t w = (i & 1) ? dwh[i >> 1] >> 16 : dwh[i >> 1] & 0xffffu;
    const u32x2 A = {mine ? a : 0u, 0u}, B = {mine ? w : 0u, 0u};
    sc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, A), __builtin_bit_cast(v4h, B), (v16f){}, 0, 0,
                                              0);
  }
}

// One workgroup: 4 waves x 32 weight rows (BN = 128) against BMt = 32 TM activation rows, superblocks [sb0, sb1).
// Three LDS slots and three weight register sets rotate as in mmq_kq_tile: the activations and weights of s + 2 are
// in flight while s is computed.
template <class WR, class Out, int TM, bool F32D>
__device__ __forceinline__ void mmq_b32_tile(const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes,
                                             const ActTile &a, int64_t m0, int64_t mrows, int64_t n0, int64_t sb0,
                                             int64_t sb1, typename Out::T *__restrict__ dst, int64_t ldd,
                                             const int32_t *__restrict__ dst_rows, float *__restrict__ part) {
  constexpr int BMt = 32 * TM;
  typedef ActDma8<BMt, F32D> AD;
  typedef RunLoad<WR> RL;
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * AD::STAGE];

  // (the wave index as a scalar: the LDS addresses of the DMA loads, which go through M0, are then scalar arithmetic)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, g = lane >> 5,
            li = lane & 31;
  const int64_t n = n0 + 32 * wave + li;
  const int64_t nlast = (nrows_w - n0 < BN ? nrows_w - n0 : BN) - 1;
  const int64_t nl = 32 * wave + li < nlast ? 32 * wave + li : nlast;

  const int64_t rows = a.rows, nsb = a.nsb;
  const rsrc_t ra = make_rsrc(a.qs, nsb * rows * (F32D ? 276 : 272));
  const rsrc_t rw = make_rsrc(W + n0 * w_row_bytes, (nlast + 1) * w_row_bytes);
  const uint32_t wrun = (uint32_t)(nl * w_row_bytes + 4 * WR::kBytes * g);

  uint32_t qoff[8];
#pragma unroll
  for (int j = 0; j < 8; j++) qoff[j] = 256 * li + 16 * ((2 * j + g) ^ (li & 15));

  v16f fa[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) fa[t] = (v16f){};

  AD dma;
  dma.init(wave, lane, m0, rows, nsb);
  // WR::kSets weight register sets: with two, step s decodes set s % 2 into B operands, then reloads it with
  // superblock s + 2; with one, it reloads the set with superblock s + 1
  constexpr int kSets = WR::kSets;
  static_assert(kSets == 1 || kSets == 2, "one or two weight sets");
  uint32_t raw[kSets][WR::kDwords];
  auto issue_a = [&](int64_t sb, int u) {
    __builtin_amdgcn_sched_barrier(0);
    dma.issue(ra, lds + u * AD::STAGE, wave, lane, (uint32_t)(sb * rows));
    __builtin_amdgcn_sched_barrier(0);
  };
  auto issue_w = [&](int64_t sb, int v) {
    __builtin_amdgcn_sched_barrier(0);
    RL::load(rw, wrun + (uint32_t)(sb * 8 * WR::kBytes), raw[v % kSets]);
    __builtin_amdgcn_sched_barrier(0);
  };

  // the scales take the f32 MFMA with Q8_K tiles (an f32 da), else the f16 one
  constexpr bool F32S = F32D;
  v4i b[8];
  float dw[4];
  uint32_t dwh[2];
  auto decode = [&](const uint32_t (&R)[WR::kDwords]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t d, h0[4], h1[4];
      WR::decode(R, i, d, h0, h1);
      if constexpr (F32S)
        dw[i] = f16_bits_to_f32(d);
      else if (i & 1)
        dwh[i >> 1] |= d << 16;
      else
        dwh[i >> 1] = d;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        swap_lane_halves(h0[q], h1[q]);
        b[i][q] = (int)h0[q];
        b[4 + i][q] = (int)h1[q];
      }
    }
  };

  // Groups (t, j) = activation tile t x block j run in order, software-pipelined: the two MFMAs of group k + 1
  // (integer dot, scale outer product) are issued before the 16 converts and 16 FMAs of group k, and the A fragment
  // of group k + 2 is read from LDS meanwhile.  Empty volatile asm statements (which keep their order) pin that
  // sequence: group k + 2's A fragment passes one after group k's accumulator update, so no MFMA is hoisted further
  // ahead (the compiler would otherwise issue every group's MFMAs first and spill their results), and by then the
  // fragment has arrived.
  auto compute = [&](const uint8_t *slot) {
    // this lane's activation rows 32t + li: scales of blocks 4g .. 4g + 3 (Q8_K tiles: the row's one scale)
    float da[TM][4];
    uint32_t dah[TM][2];
#pragma unroll
    for (int t = 0; t < TM; t++) {
      if constexpr (F32D) {
        const float d = *(const float *)(slot + AD::QS + 4 * (32 * t + li));
        da[t][0] = da[t][1] = da[t][2] = da[t][3] = d;
      } else {
        const uint2 d4 = *(const uint2 *)(slot + AD::QS + 16 * (32 * t + li) + 8 * g);
        if constexpr (F32S) {
          da[t][0] = f16_bits_to_f32(d4.x & 0xffffu), da[t][1] = f16_bits_to_f32(d4.x >> 16);
          da[t][2] = f16_bits_to_f32(d4.y & 0xffffu), da[t][3] = f16_bits_to_f32(d4.y >> 16);
        } else {
          dah[t][0] = d4.x, dah[t][1] = d4.y;
        }
      }
    }
    auto frag = [&](int k) { return *(const v4i *)(slot + 8192 * (k >> 3) + qoff[k & 7]); };
    v16i acc[2];
    v16f sc[2];
    v4i av[2];
    av[0] = frag(0);
    av[1] = frag(1);
    b32_group<F32S>(av[0], b, da[0], dah[0], dw, dwh, g, 0, acc[0], sc[0]);
#pragma unroll
    for (int k = 0; k < 8 * TM; k++) {
      // (read before group k + 1's MFMAs: the fragment then has registers of its own, apart from group k's results,
      // and a whole group's work to arrive; read after them, it took group k's accumulator registers once their
      // converts were done and was waited for right away -- same bits, 1-2% slower)
      if (k + 2 < 8 * TM) av[k & 1] = frag(k + 2);
      if (k + 1 < 8 * TM)
        b32_group<F32S>(av[(k + 1) & 1], b, da[(k + 1) >> 3], dah[(k + 1) >> 3], dw, dwh, g, k + 1, acc[(k + 1) & 1],
                        sc[(k + 1) & 1]);
      const int t = k >> 3;
#pragma unroll
      for (int r = 0; r < 16; r++) fa[t][r] = __builtin_fmaf((float)acc[k & 1][r], sc[k & 1][r], fa[t][r]);
      order_point(fa[t]);
    }
  };

  // u = (s - sb0) % 3 selects the LDS slot, v = (s - sb0) % 2 the weight set; both constant after unrolling.  Two
  // sets: step s waits for the activations and weights of s (issued together two steps earlier; those of s + 1 may
  // still be in flight), decodes, and issues both for s + 2.  One set: step s waits for its weights (issued in step
  // s - 1) and activations (step s - 2), decodes, then issues the weights of s + 1 and the activations of s + 2, in
  // that order, so that only the newest activations may still be in flight at the next step's wait.  Past the end
  // the last superblock is loaded again, into places that are not read, so every wait count stays exact.
  auto step = [&](int64_t s, int u, int v) {
    __builtin_amdgcn_sched_barrier(0);
    dma_barrier<kSets == 2 ? AD::kLoads + RL::kLoads : AD::kLoads>();
    decode(raw[v % kSets]);
    if constexpr (kSets == 2) {
      const int64_t sn = s + 2 < sb1 ? s + 2 : sb1 - 1;
      issue_a(sn, (u + 2) % 3);
      issue_w(sn, v);
    } else {
      issue_w(s + 1 < sb1 ? s + 1 : sb1 - 1, 0);
      issue_a(s + 2 < sb1 ? s + 2 : sb1 - 1, (u + 2) % 3);
    }
    if (s < sb1) compute(lds + u * AD::STAGE);
    __builtin_amdgcn_sched_barrier(0);
  };

  if constexpr (kSets == 2) {
    issue_a(sb0, 0);
    issue_w(sb0, 0);
    issue_a(sb0 + 1 < sb1 ? sb0 + 1 : sb1 - 1, 1);
    issue_w(sb0 + 1 < sb1 ? sb0 + 1 : sb1 - 1, 1);
  } else {
    issue_w(sb0, 0);
    issue_a(sb0, 0);
    issue_a(sb0 + 1 < sb1 ? sb0 + 1 : sb1 - 1, 1);
  }
  for (int64_t sb = sb0; sb < sb1; sb += 6) {
    step(sb, 0, 0);
    step(sb + 1, 1, 1);
    step(sb + 2, 2, 0);
    step(sb + 3, 0, 1);
    step(sb + 4, 1, 0);
    step(sb + 5, 2, 1);
  }

  if (n >= nrows_w) return;
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int64_t m = m0 + 32 * t + out_row(r, g);
      if (m < mrows) {
        if (part)
          part[m * nrows_w + n] = fa[t][r];
        else
          Out::store(dst, (dst_rows ? dst_rows[m] : m) * ldd + n, fa[t][r]);
      }
    }
}

// ------------------------------------------------------------------------------------------ kernels

// Workgroups are numbered so that the BM-row tiles sharing one weight tile are consecutive, then spread over
// the 8 XCDs (dispatch assigns workgroup i to XCD i % 8): each XCD's L2 sees whole weight tiles.
__device__ __forceinline__ void tile_of(int64_t mtiles, int64_t ntiles, int64_t splits, int64_t &mt, int64_t &nt,
                                        int64_t &split) {
  const int64_t total = mtiles * ntiles * splits;
  const int64_t b = blockIdx.x;
  int64_t id = b;
  if (total % 8 == 0) id = (b % 8) * (total / 8) + b / 8;
  split = id % splits;
  const int64_t tile = id / splits;
  mt = tile % mtiles;
  nt = tile / mtiles;
}

ActTile act_tile(const void *y, int64_t rows, int64_t nsb) {
  ActTile a;
  a.qs = (const uint8_t *)y;
  a.rows = rows;
  a.nsb = nsb;
  a.d8 = (const uint16_t *)((const uint8_t *)y + nsb * rows * 256);
  a.d32 = (const float *)((const uint8_t *)y + nsb * rows * 256);
  return a;
}

// Q4_K (measured on MI355X): 64 activation rows per wave at 2 waves per SIMD beats 128 rows at 1 wave; Q6_K, whose
// plane building needs more registers, runs 1 wave per SIMD and takes 128 rows.
template <class WT>
constexpr int kq_tm_max() { return WT::kPlanes == 3 ? 1 : WT::kMin ? 2 : WT::kLdsWeights && WT::kLwTM ? WT::kLwTM : 4; }
template <class WT, int TMv>
constexpr int kq_waves() {
  return (WT::kMin || (WT::kLdsWeights && WT::kLwTM == 2)) && TMv <= (WT::kPlanes == 3 ? 1 : 2) ? 2 : 1;
}

// grid: tiles x splits; split s of a tile sums superblocks [s * per, min((s + 1) * per, nsb)) into dst, or with more
// than one split into plane s of `part` (mrows x nrows_w f32 per plane)
template <class WT, class Out, int TMv, int NW, bool S16 = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(kq_waves<WT, TMv>()))) void k_mmq_kq(
    const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes, ActTile a, int64_t mrows, int64_t nsb,
    int64_t splits, typename Out::T *__restrict__ dst, int64_t ldd, float *__restrict__ part) {
  constexpr int BMt = 32 * TMv, BNt = 32 * NW;
  int64_t mt, nt, split;
  tile_of((mrows + BMt - 1) / BMt, (nrows_w + BNt - 1) / BNt, splits, mt, nt, split);
  const int64_t per = (nsb + splits - 1) / splits;
  const int64_t sb0 = split * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  if (sb0 >= sb1) return;
  mmq_kq_tile<WT, Out, TMv, NW, S16>(W, nrows_w, w_row_bytes, a, mt * BMt, mrows, nt * BNt, sb0, sb1, dst, ldd,
                                     nullptr, part ? part + split * mrows * nrows_w : nullptr);
}

template <class WB, class Out, bool F32D>
__global__ __launch_bounds__(256) void k_mmq_q8_0(const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes,
                                                  int64_t nblk_w, ActTile a, int64_t mrows, int64_t nsb,
                                                  typename Out::T *__restrict__ dst, int64_t ldd) {
  int64_t mt, nt, split;
  tile_of((mrows + BM - 1) / BM, (nrows_w + BN - 1) / BN, 1, mt, nt, split);
  mmq_q8_0_tile<WB, Out, F32D>(W, nrows_w, w_row_bytes, nblk_w, a, mt * BM, mrows, nt * BN, nsb, dst, ldd, nullptr);
}

// Expert-grouped: grid (n tiles, m tiles of the largest expert, experts).  Expert e's rows of `a` are
// [bounds[e], bounds[e+1]); its weights start at W + e * expert_bytes; row m is written to dst row ids_dst[m].
// S16: `_q8k` activation tiles.
template <class WT, int TMv, bool S16 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kq_waves<WT, TMv>()))) void k_mmq_kq_moe(const uint8_t *__restrict__ W, int64_t expert_bytes,
                                                    int64_t nrows_w, int64_t w_row_bytes, ActTile a,
                                                    const int32_t *__restrict__ bounds,
                                                    const int32_t *__restrict__ ids_dst, int64_t nsb, int64_t splits,
                                                    float *__restrict__ dst, int64_t ldd, float *__restrict__ part,
                                                    int64_t ncols_dst) {
  const int64_t e = blockIdx.z;
  const int64_t m0 = bounds[e] + (int64_t)blockIdx.y * (32 * TMv), m1 = bounds[e + 1];
  if (m0 >= m1) return;  // uniform over the workgroup
  const int64_t split = blockIdx.x % splits, per = (nsb + splits - 1) / splits;
  const int64_t sb0 = split * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  if (sb0 >= sb1) return;
  mmq_kq_tile<WT, out_f32, TMv, 4, S16>(W + e * expert_bytes, nrows_w, w_row_bytes, a, m0, m1,
                                (int64_t)(blockIdx.x / splits) * BN, sb0, sb1, dst, ldd, ids_dst,
                                part ? part + split * ncols_dst * nrows_w : nullptr);
}

template <class WB, bool F32D>
__global__ __launch_bounds__(256) void k_mmq_q8_0_moe(const uint8_t *__restrict__ W, int64_t expert_bytes,
                                                      int64_t nrows_w, int64_t w_row_bytes, int64_t nblk_w, ActTile a,
                                                      const int32_t *__restrict__ bounds,
                                                      const int32_t *__restrict__ ids_dst, int64_t nsb,
                                                      float *__restrict__ dst, int64_t ldd) {
  const int64_t e = blockIdx.z;
  const int64_t m0 = bounds[e] + (int64_t)blockIdx.y * BM, m1 = bounds[e + 1];
  if (m0 >= m1) return;
  mmq_q8_0_tile<WB, out_f32, F32D>(W + e * expert_bytes, nrows_w, w_row_bytes, nblk_w, a, m0, m1, (int64_t)blockIdx.x * BN,
                             nsb, dst, ldd, ids_dst);
}

// The pipelined 32-value-block kernels: 32 or 64 activation rows per workgroup, two waves per SIMD.
template <int TMv>
constexpr int b32_waves() { return 2; }

template <class WR, class Out, int TMv, bool F32D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(b32_waves<TMv>()))) void k_mmq_b32(
    const uint8_t *__restrict__ W, int64_t nrows_w, int64_t w_row_bytes, ActTile a, int64_t mrows, int64_t nsb,
    int64_t splits, typename Out::T *__restrict__ dst, int64_t ldd, float *__restrict__ part) {
  constexpr int BMt = 32 * TMv;
  int64_t mt, nt, split;
  tile_of((mrows + BMt - 1) / BMt, (nrows_w + BN - 1) / BN, splits, mt, nt, split);
  const int64_t per = (nsb + splits - 1) / splits;
  const int64_t sb0 = split * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  if (sb0 >= sb1) return;
  mmq_b32_tile<WR, Out, TMv, F32D>(W, nrows_w, w_row_bytes, a, mt * BMt, mrows, nt * BN, sb0, sb1, dst, ldd, nullptr,
                             part ? part + split * mrows * nrows_w : nullptr);
}

template <class WR, int TMv, bool F32D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(b32_waves<TMv>()))) void k_mmq_b32_moe(
    const uint8_t *__restrict__ W, int64_t expert_bytes, int64_t nrows_w, int64_t w_row_bytes, ActTile a,
    const int32_t *__restrict__ bounds, const int32_t *__restrict__ ids_dst, int64_t nsb, int64_t splits,
    float *__restrict__ dst, int64_t ldd, float *__restrict__ part, int64_t ncols_dst) {
  const int64_t e = blockIdx.z;
  const int64_t m0 = bounds[e] + (int64_t)blockIdx.y * (32 * TMv), m1 = bounds[e + 1];
  if (m0 >= m1) return;  // uniform over the workgroup
  const int64_t split = blockIdx.x % splits, per = (nsb + splits - 1) / splits;
  const int64_t sb0 = split * per, sb1 = sb0 + per < nsb ? sb0 + per : nsb;
  if (sb0 >= sb1) return;
  mmq_b32_tile<WR, out_f32, TMv, F32D>(W + e * expert_bytes, nrows_w, w_row_bytes, a, m0, m1,
                                 (int64_t)(blockIdx.x / splits) * BN, sb0, sb1, dst, ldd, ids_dst,
                                 part ? part + split * ncols_dst * nrows_w : nullptr);
}

bool check_mmq(const char *who, int type, const void *x, int64_t ncols_x, int64_t nrows_x, int64_t stride_row_x) {
  const int64_t bs = (int64_t)qmm_block_size(type);
  if (ncols_x <= 0 || nrows_x <= 0 || ncols_x % bs != 0 || stride_row_x < ncols_x / bs) {
    qmm_set_error("%s: ncols_x=%lld nrows_x=%lld stride_row_x=%lld", who, (long long)ncols_x, (long long)nrows_x,
                  (long long)stride_row_x);
    return false;
  }
  if ((type == QMM_TYPE_Q4K || type == QMM_TYPE_Q5K) && ((uintptr_t)x % 16 != 0)) {
    qmm_set_error("%s: Q4_K / Q5_K weights must be 16-byte aligned", who);
    return false;
  }
  if (type == QMM_TYPE_IQ4_XS && ((uintptr_t)x % 4 != 0)) {
    qmm_set_error("%s: IQ4_XS weights must be 4-byte aligned", who);
    return false;
  }
  if ((uintptr_t)x % 2 != 0) {
    qmm_set_error("%s: weights must be 2-byte aligned", who);
    return false;
  }
  return true;
}

// K splits so that tiles x splits fills every CU once over, each split keeping at least 4 superblocks, as long as the
// caller's fixup buffer holds one rows x cols f32 plane per split.  The reference sizes that buffer (tmp_fixup) as
// nsm * 128 * 128 f32 (fast_mmq.rs:442-444); without one there is no split.  Every split gets at least one
// superblock, since each writes its whole plane.
int64_t k_splits(int64_t tiles, int64_t nsb, int64_t rows, int64_t cols, const void *fixup, int nsm) {
  if (!fixup || (uintptr_t)fixup % 16 != 0) return 1;
  const int64_t cap = (int64_t)(nsm > 0 ? nsm : qmm_device_cus()) * 128 * 128 * 4;
  const int64_t want = qmm_device_cus();
  int64_t s = 1;
  while (tiles * s < want && nsb / (s * 2) >= 4 && 2 * s * rows * cols * 4 <= cap) s *= 2;
  while (s > 1 && (s - 1) * ((nsb + s - 1) / s) >= nsb) s--;
  return s;
}

// Waves (weight rows / 32) per workgroup of the plain K-quant prefill from 64 activation rows per wave on (32-row
// tiles keep 4: their per-wave DMA share would not be uniform over 8).  Measured on MI355X for Q4_K at M = 512 with
// the weights staged in LDS: 8 waves 95.6 us, 4 waves 90.9 us -- a workgroup's waves run in lockstep between its
// barriers, and two 4-wave workgroups per CU let one's VALU epilogue overlap the other's MFMAs.
#ifndef QMM_KQ_WAVES
#define QMM_KQ_WAVES 4
#endif

template <class WT, class Out, bool S16 = false>
void launch_kq(const uint8_t *w, int64_t nrows_x, int64_t w_row_bytes, const ActTile &a, int64_t ncols_y, int64_t nsb,
               typename Out::T *d, int64_t ldd, void *fixup, int nsm, hipStream_t s) {
  // activation rows per wave: the smallest of 32, 64, 128 that covers the batch
  const int tm = ncols_y <= 32 || kq_tm_max<WT>() < 2 ? 1 : ncols_y <= 64 || kq_tm_max<WT>() < 4 ? 2 : 4;
  // (8 waves per workgroup fit where one wave needs at most 256 registers: Q4_K at 64 rows; Q6_K / IQ4_XS take 128
  // rows at one wave per SIMD and keep 4)
  constexpr int NW = WT::kMin && kq_tm_max<WT>() == 2 ? QMM_KQ_WAVES : 4;
  const int nw = tm == 1 ? 4 : NW;
  const int64_t ntiles = (nrows_x + 32 * nw - 1) / (32 * nw);
  const int64_t tiles = ((ncols_y + 32 * tm - 1) / (32 * tm)) * ntiles;
  const int64_t splits = k_splits(tiles, nsb, ncols_y, nrows_x, fixup, nsm);
  float *part = splits > 1 ? (float *)fixup : nullptr;
  const dim3 grid((unsigned)(tiles * splits));
  if (tm == 1) {
    k_mmq_kq<WT, Out, 1, 4, S16><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, splits, d, ldd, part);
  } else if (tm == 2) {
    k_mmq_kq<WT, Out, 2, NW, S16><<<grid, 64 * NW, 0, s>>>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, splits, d, ldd,
                                                          part);
  } else if constexpr (kq_tm_max<WT>() >= 4) {  // (not instantiated where it cannot be chosen)
    k_mmq_kq<WT, Out, 4, NW, S16><<<grid, 64 * NW, 0, s>>>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, splits, d, ldd,
                                                          part);
  }
  if (part) split_sum<Out>(part, splits, ncols_y, nrows_x, d, ldd, nullptr, s);
}

// The pipelined 32-value-block kernel takes rows of whole superblocks that start on dword boundaries; other
// shapes take the Q8_0 kernel.
bool b32_runs(const void *x, int64_t ncols_x, int64_t w_row_bytes) {
  return ncols_x % 256 == 0 && w_row_bytes % 4 == 0 && (uintptr_t)x % 4 == 0;
}

template <class WR, class Out, bool F32D>
void launch_b32(const uint8_t *w, int64_t nrows_x, int64_t w_row_bytes, const ActTile &a, int64_t ncols_y,
                int64_t nsb, typename Out::T *d, int64_t ldd, void *fixup, int nsm, hipStream_t s) {
  const int64_t ntiles = (nrows_x + BN - 1) / BN;
  const int tm = ncols_y <= 32 ? 1 : 2;
  const int64_t tiles = ((ncols_y + 32 * tm - 1) / (32 * tm)) * ntiles;
  const int64_t splits = k_splits(tiles, nsb, ncols_y, nrows_x, fixup, nsm);
  float *part = splits > 1 ? (float *)fixup : nullptr;
  const dim3 grid((unsigned)(tiles * splits));
  if (tm == 1)
    k_mmq_b32<WR, Out, 1, F32D><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, splits, d, ldd, part);
  else
    k_mmq_b32<WR, Out, 2, F32D><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, splits, d, ldd, part);
  if (part) split_sum<Out>(part, splits, ncols_y, nrows_x, d, ldd, nullptr, s);
}

template <class WR, bool F32D>
void launch_b32_moe(const uint8_t *w, int64_t expert_bytes, int64_t nrows_x, int64_t w_row_bytes, const ActTile &a,
                    const int32_t *bounds, const int32_t *ids_dst, int64_t nsb, float *d, int64_t ldd,
                    int64_t ncols_dst, int64_t ncols_max, int64_t num_experts, void *fixup, int nsm, hipStream_t s) {
  const int64_t ntiles = (nrows_x + BN - 1) / BN;
  // 32-row tiles where the experts' rows are few on average (an expert with more takes several)
  const int tm = (QMM_MOE_SMALL_AVG ? (ncols_dst + num_experts - 1) / num_experts : ncols_max) <= 32 ? 1 : 2;
  const int64_t bm = 32 * tm;
  // expected work: about ncols_dst / bm row tiles per n tile over all experts
  const int64_t splits = k_splits(ntiles * ((ncols_dst + bm - 1) / bm), nsb, ncols_dst, nrows_x, fixup, nsm);
  float *part = splits > 1 ? (float *)fixup : nullptr;
  const dim3 grid((unsigned)(ntiles * splits), (unsigned)((ncols_max + bm - 1) / bm), (unsigned)num_experts);
  if (tm == 1)
    k_mmq_b32_moe<WR, 1, F32D><<<grid, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb,
                                               splits, d, ldd, part, ncols_dst);
  else
    k_mmq_b32_moe<WR, 2, F32D><<<grid, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb,
                                               splits, d, ldd, part, ncols_dst);
  if (part) split_sum<out_f32>(part, splits, ncols_dst, nrows_x, d, ldd, ids_dst, s);
}

// F32D: the Q8_K tile layout (every type; the reference-named entries); else Q8_0 blocks (the 32-value types' _q8_0
// entries)
template <class Out, bool F32D>
void mmq_plain(int type, const void *x, const void *y, void *dst, int64_t ncols_x, int64_t nrows_x, int64_t ncols_y,
               int64_t stride_row_x, int64_t ldd, void *fixup, int nsm, hipStream_t s) {
  const int64_t nsb = (ncols_x + 255) / 256;
  const int64_t w_row_bytes = stride_row_x * (int64_t)qmm_type_size(type);
  const ActTile a = act_tile(y, ncols_y, nsb);
  typename Out::T *d = (typename Out::T *)dst;
  const uint8_t *w = (const uint8_t *)x;
  switch (F32D ? type : QMM_TYPE_Q8_0) {
    case QMM_TYPE_Q4K: launch_kq<wq4k, Out>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, fixup, nsm, s); break;
    case QMM_TYPE_Q6K: launch_kq<wq6k, Out>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, fixup, nsm, s); break;
    case QMM_TYPE_Q5K: launch_kq<wq5k, Out>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, fixup, nsm, s); break;
    case QMM_TYPE_IQ4_XS: launch_kq<wiq4xs, Out>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, fixup, nsm, s); break;
    default: {
      if (b32_runs(w, ncols_x, w_row_bytes)) {
        if (type == QMM_TYPE_Q4_0)
          launch_b32<wr_q4_0, Out, F32D>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, fixup, nsm, s);
        else if (type == QMM_TYPE_Q5_0)
          launch_b32<wr_q5_0, Out, F32D>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, fixup, nsm, s);
        else
          launch_b32<wr_q8_0, Out, F32D>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, d, ldd, fixup, nsm, s);
        break;
      }
      const dim3 grid((unsigned)(((ncols_y + BM - 1) / BM) * ((nrows_x + BN - 1) / BN)));
      if (type == QMM_TYPE_Q4_0)
        k_mmq_q8_0<wb_q4_0, Out, F32D><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, ncols_x / 32, a, ncols_y, nsb, d, ldd);
      else if (type == QMM_TYPE_Q5_0)
        k_mmq_q8_0<wb_q5_0, Out, F32D><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, ncols_x / 32, a, ncols_y, nsb, d, ldd);
      else
        k_mmq_q8_0<wb_q8_0, Out, F32D><<<grid, 256, 0, s>>>(w, nrows_x, w_row_bytes, ncols_x / 32, a, ncols_y, nsb, d, ldd);
    }
  }
}

// The kernels address one activation channel with 32-bit offsets.
bool check_act_bytes(const char *who, int64_t ncols_x, int64_t rows, int bytes_per_256 = 276) {
  if ((ncols_x + 255) / 256 * rows * bytes_per_256 > 0x7ffffff0) {
    qmm_set_error("%s: activation channel of %lld x %lld values exceeds 2 GiB", who, (long long)rows,
                  (long long)ncols_x);
    return false;
  }
  return true;
}

// q8_0: the activations are Q8_0 blocks (the 32-value types' _q8_0 entries), else Q8_K tiles
void mmq(int type, bool q8_0, void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,
         int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, int nsm, int type_dst,
         void *stream, const char *who) {
  if (!check_mmq(who, type, x, ncols_x, nrows_x, stride_row_x) || !check_act_bytes(who, ncols_x, ncols_y)) return;
  if (ncols_y < 0 || stride_col_dst < nrows_x) {
    qmm_set_error("%s: ncols_y=%lld stride_col_dst=%lld", who, (long long)ncols_y, (long long)stride_col_dst);
    return;
  }
  if (ncols_y == 0) return;
  hipStream_t s = (hipStream_t)stream;
#define QMM_MMQ_P(Out)                                                                                            \
  (q8_0 ? mmq_plain<Out, false>(type, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, tmp_fixup,  \
                                nsm, s)                                                                             \
        : mmq_plain<Out, true>(type, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, tmp_fixup,   \
                               nsm, s))
  switch (type_dst) {
    case QMM_TYPE_F32: QMM_MMQ_P(out_f32); break;
    case QMM_TYPE_F16: QMM_MMQ_P(out_f16); break;
    case QMM_TYPE_BF16: QMM_MMQ_P(out_bf16); break;
    default: qmm_set_error("%s: type_dst=%d (0 f32, 1 f16, 30 bf16)", who, type_dst);
  }
#undef QMM_MMQ_P
}

// launch_mmq_gguf_{q4_k,q5_k}_q8k: the plain prefill over `_q8k` tiles (f16 sums of 16)
void mmq_q8k(int type, void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x, int64_t nrows_x,
             int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst, int nsm, int type_dst, void *stream,
             const char *who) {
  if (!check_mmq(who, type, x, ncols_x, nrows_x, stride_row_x) || !check_act_bytes(who, ncols_x, ncols_y, 292)) return;
  if (ncols_y < 0 || stride_col_dst < nrows_x) {
    qmm_set_error("%s: ncols_y=%lld stride_col_dst=%lld", who, (long long)ncols_y, (long long)stride_col_dst);
    return;
  }
  if (ncols_y == 0) return;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nsb = (ncols_x + 255) / 256;
  const int64_t w_row_bytes = stride_row_x * (int64_t)qmm_type_size(type);
  const ActTile a = act_tile(y, ncols_y, nsb);
  const uint8_t *w = (const uint8_t *)x;
#define QMM_Q8K(Out)                                                                                                 \
  (type == QMM_TYPE_Q4K ? launch_kq<wq4k, Out, true>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, (Out::T *)dst,       \
                                                     stride_col_dst, tmp_fixup, nsm, s)                              \
                        : launch_kq<wq5k, Out, true>(w, nrows_x, w_row_bytes, a, ncols_y, nsb, (Out::T *)dst,       \
                                                     stride_col_dst, tmp_fixup, nsm, s))
  switch (type_dst) {
    case QMM_TYPE_F32: QMM_Q8K(out_f32); break;
    case QMM_TYPE_F16: QMM_Q8K(out_f16); break;
    case QMM_TYPE_BF16: QMM_Q8K(out_bf16); break;
    default: qmm_set_error("%s: type_dst=%d (0 f32, 1 f16, 30 bf16)", who, type_dst);
  }
#undef QMM_Q8K
}

template <class WT, int TMv, bool S16 = false>
void kq_moe(dim3 grid, hipStream_t s, const uint8_t *w, int64_t expert_bytes, int64_t nrows_x, int64_t w_row_bytes,
            const ActTile &a, const int32_t *bounds, const int32_t *ids_dst, int64_t nsb, int64_t splits, float *d,
            int64_t ldd, float *part, int64_t ncols_dst) {
  k_mmq_kq_moe<WT, TMv, S16><<<grid, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb,
                                                  splits, d, ldd, part, ncols_dst);
}

template <bool F32D>
void mmq_moe_t(int type, void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst, const int32_t *bounds,
               void *dst, int64_t ncols_x, int64_t nrows_x, int64_t ncols_dst, int64_t stride_row_x,
               int64_t stride_col_dst, int64_t num_experts, int64_t ncols_max, int nsm, void *stream,
               const char *who) {
  if (!check_mmq(who, type, x, ncols_x, nrows_x, stride_row_x) || !check_act_bytes(who, ncols_x, ncols_dst)) return;
  if (num_experts <= 0 || ncols_max < 0 || ncols_dst < 0 || stride_col_dst < nrows_x || num_experts > 65535) {
    qmm_set_error("%s: num_experts=%lld ncols_max=%lld ncols_dst=%lld stride_col_dst=%lld", who,
                  (long long)num_experts, (long long)ncols_max, (long long)ncols_dst, (long long)stride_col_dst);
    return;
  }
  if (ncols_max == 0 || ncols_dst == 0) return;
  const int64_t nsb = (ncols_x + 255) / 256;
  const int64_t w_row_bytes = stride_row_x * (int64_t)qmm_type_size(type);
  const int64_t expert_bytes = nrows_x * w_row_bytes;
  const ActTile a = act_tile(y, ncols_dst, nsb);
  const dim3 grid((unsigned)((nrows_x + BN - 1) / BN), (unsigned)((ncols_max + BM - 1) / BM), (unsigned)num_experts);
  hipStream_t s = (hipStream_t)stream;
  // a few rows per expert: the few-row kernel streams each expert's weights once, without 64-row tiles of padding
  const bool b32 = qmm_block_size(type) == 32;  // Q8_0, Q4_0, Q5_0: the Q8_0-layout kernel
  if (!b32 && F32D && qmm_skinny_moe(type, x, y, ids_dst, bounds, (float *)dst, ncols_x, nrows_x, w_row_bytes,
                                              ncols_dst, stride_col_dst, num_experts, s))
    return;
  const uint8_t *w = (const uint8_t *)x;
  float *d = (float *)dst;
  if (b32 && b32_runs(w, ncols_x, w_row_bytes)) {
    if (type == QMM_TYPE_Q4_0)
      launch_b32_moe<wr_q4_0, F32D>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, d, stride_col_dst,
                              ncols_dst, ncols_max, num_experts, tmp_fixup, nsm, s);
    else if (type == QMM_TYPE_Q5_0)
      launch_b32_moe<wr_q5_0, F32D>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, d, stride_col_dst,
                              ncols_dst, ncols_max, num_experts, tmp_fixup, nsm, s);
    else
      launch_b32_moe<wr_q8_0, F32D>(w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, d, stride_col_dst,
                              ncols_dst, ncols_max, num_experts, tmp_fixup, nsm, s);
    return;
  }
  // 32-row tiles for a few rows per expert, and always for Q5_K (its third plane does not fit two waves per SIMD at
  // 64 rows, the form the plain prefill measured slower)
  // 32-row tiles where the experts' rows are few on average (an expert with more takes several)
  const bool small = (QMM_MOE_SMALL_AVG ? (ncols_dst + num_experts - 1) / num_experts : ncols_max) <= 32 ||
                     type == QMM_TYPE_Q5K;
  const int64_t ntiles = (nrows_x + BN - 1) / BN;
  const int64_t mt = small ? (ncols_max + 31) / 32 : (ncols_max + 63) / 64;
  // expected work: about ncols_dst / (32 tm) row tiles per n tile over all experts
  const int64_t busy = ntiles * (small ? (ncols_dst + 31) / 32 : (ncols_dst + 63) / 64);
  const int64_t splits = b32 ? 1 : k_splits(busy, nsb, ncols_dst, nrows_x, tmp_fixup, nsm);
  float *part = splits > 1 ? (float *)tmp_fixup : nullptr;
  const dim3 gridk((unsigned)(ntiles * splits), (unsigned)mt, (unsigned)num_experts);
  switch (F32D ? type : QMM_TYPE_Q8_0) {
    case QMM_TYPE_Q4K:
      if (small)
        kq_moe<wq4k, 1>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                        stride_col_dst, part, ncols_dst);
      else
        kq_moe<wq4k, 2>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                        stride_col_dst, part, ncols_dst);
      break;
    case QMM_TYPE_Q5K:  // always 32-row tiles (small)
      kq_moe<wq5k, 1>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                        stride_col_dst, part, ncols_dst);
      break;
    case QMM_TYPE_Q6K:
      if (small)
        kq_moe<wq6k, 1>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                        stride_col_dst, part, ncols_dst);
      else
        kq_moe<wq6k, 2>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                        stride_col_dst, part, ncols_dst);
      break;
    case QMM_TYPE_IQ4_XS:
      if (small)
        kq_moe<wiq4xs, 1>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                        stride_col_dst, part, ncols_dst);
      else
        kq_moe<wiq4xs, 2>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                        stride_col_dst, part, ncols_dst);
      break;
    case QMM_TYPE_Q4_0:
      k_mmq_q8_0_moe<wb_q4_0, F32D><<<grid, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, ncols_x / 32, a, bounds,
                                                   ids_dst, nsb, d, stride_col_dst);
      break;
    case QMM_TYPE_Q5_0:
      k_mmq_q8_0_moe<wb_q5_0, F32D><<<grid, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, ncols_x / 32, a, bounds,
                                                   ids_dst, nsb, d, stride_col_dst);
      break;
    default:
      k_mmq_q8_0_moe<wb_q8_0, F32D><<<grid, 256, 0, s>>>(w, expert_bytes, nrows_x, w_row_bytes, ncols_x / 32, a, bounds,
                                                   ids_dst, nsb, d, stride_col_dst);
  }
  if (part) split_sum<out_f32>(part, splits, ncols_dst, nrows_x, d, stride_col_dst, ids_dst, s);
}

// q8_0: the activations are Q8_0 blocks (the 32-value types' _q8_0 entries), else Q8_K tiles
void mmq_moe(int type, bool q8_0, void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,
             const int32_t *bounds, void *dst, int64_t ncols_x, int64_t nrows_x, int64_t ncols_dst,
             int64_t stride_row_x, int64_t stride_col_dst, int64_t num_experts, int64_t ncols_max, int nsm,
             void *stream, const char *who) {
  if (q8_0)
    mmq_moe_t<false>(type, tmp_fixup, x, y, ids_dst, bounds, dst, ncols_x, nrows_x, ncols_dst, stride_row_x,
                     stride_col_dst, num_experts, ncols_max, nsm, stream, who);
  else
    mmq_moe_t<true>(type, tmp_fixup, x, y, ids_dst, bounds, dst, ncols_x, nrows_x, ncols_dst, stride_row_x,
                    stride_col_dst, num_experts, ncols_max, nsm, stream, who);
}

// launch_mmq_gguf_{q4_k,q5_k}_moe_q8k: the grouped prefill over `_q8k` tiles, with mmq_moe_t's tile and split choice
void mmq_moe_q8k(int type, void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,
                 const int32_t *bounds, void *dst, int64_t ncols_x, int64_t nrows_x, int64_t ncols_dst,
                 int64_t stride_row_x, int64_t stride_col_dst, int64_t num_experts, int64_t ncols_max, int nsm,
                 void *stream, const char *who) {
  if (!check_mmq(who, type, x, ncols_x, nrows_x, stride_row_x) || !check_act_bytes(who, ncols_x, ncols_dst, 292))
    return;
  if (num_experts <= 0 || ncols_max < 0 || ncols_dst < 0 || stride_col_dst < nrows_x || num_experts > 65535) {
    qmm_set_error("%s: num_experts=%lld ncols_max=%lld ncols_dst=%lld stride_col_dst=%lld", who,
                  (long long)num_experts, (long long)ncols_max, (long long)ncols_dst, (long long)stride_col_dst);
    return;
  }
  if (ncols_max == 0 || ncols_dst == 0) return;
  const int64_t nsb = (ncols_x + 255) / 256;
  const int64_t w_row_bytes = stride_row_x * (int64_t)qmm_type_size(type);
  const int64_t expert_bytes = nrows_x * w_row_bytes;
  const ActTile a = act_tile(y, ncols_dst, nsb);
  hipStream_t s = (hipStream_t)stream;
  const uint8_t *w = (const uint8_t *)x;
  float *d = (float *)dst;
  const bool small = (QMM_MOE_SMALL_AVG ? (ncols_dst + num_experts - 1) / num_experts : ncols_max) <= 32 ||
                     type == QMM_TYPE_Q5K;
  const int64_t ntiles = (nrows_x + BN - 1) / BN;
  const int64_t mt = small ? (ncols_max + 31) / 32 : (ncols_max + 63) / 64;
  const int64_t busy = ntiles * (small ? (ncols_dst + 31) / 32 : (ncols_dst + 63) / 64);
  const int64_t splits = k_splits(busy, nsb, ncols_dst, nrows_x, tmp_fixup, nsm);
  float *part = splits > 1 ? (float *)tmp_fixup : nullptr;
  const dim3 gridk((unsigned)(ntiles * splits), (unsigned)mt, (unsigned)num_experts);
  if (type == QMM_TYPE_Q5K)
    kq_moe<wq5k, 1, true>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                          stride_col_dst, part, ncols_dst);
  else if (small)
    kq_moe<wq4k, 1, true>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                          stride_col_dst, part, ncols_dst);
  else
    kq_moe<wq4k, 2, true>(gridk, s, w, expert_bytes, nrows_x, w_row_bytes, a, bounds, ids_dst, nsb, splits, d,
                          stride_col_dst, part, ncols_dst);
  if (part) split_sum<out_f32>(part, splits, ncols_dst, nrows_x, d, stride_col_dst, ids_dst, s);
}

}  // namespace

// launch_mmq_gguf_<t><sfx> and launch_mmq_gguf_<t>_moe<sfx> (sfx _q8_0: Q8_0-block activations)
#define QMM_DEFINE_MMQ_ENTRIES(t, TYPE, Q8_0, sfx)                                                                 \
  void launch_mmq_gguf_##t##sfx(void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,        \
                                int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst,   \
                                int cc, int nsm, int64_t smpbo, int warp_size, int type_dst, void *stream) {      \
    (void)cc, (void)smpbo, (void)warp_size;                                                                        \
    mmq(TYPE, Q8_0, tmp_fixup, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, nsm, type_dst,  \
        stream, "mmq_" #t #sfx);                                                                                   \
  }                                                                                                                \
  void launch_mmq_gguf_##t##_moe##sfx(void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,      \
                                      const int32_t *expert_bounds, void *dst, int64_t ncols_x, int64_t nrows_x,   \
                                      int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst,             \
                                      int64_t num_experts, int64_t ncols_max, int cc, int nsm, int64_t smpbo,      \
                                      int warp_size, void *stream) {                                               \
    (void)cc, (void)smpbo, (void)warp_size;                                                                        \
    mmq_moe(TYPE, Q8_0, tmp_fixup, x, y, ids_dst, expert_bounds, dst, ncols_x, nrows_x, ncols_dst, stride_row_x,   \
            stride_col_dst, num_experts, ncols_max, nsm, stream, "mmq_" #t "_moe" #sfx);                           \
  }
#define QMM_DEFINE_MMQ(t, TYPE) QMM_DEFINE_MMQ_ENTRIES(t, TYPE, false, )

extern "C" {
QMM_DEFINE_MMQ(q8_0, QMM_TYPE_Q8_0)
QMM_DEFINE_MMQ(q4_k, QMM_TYPE_Q4K)
QMM_DEFINE_MMQ(q6_k, QMM_TYPE_Q6K)
QMM_DEFINE_MMQ(q5_k, QMM_TYPE_Q5K)
QMM_DEFINE_MMQ(q4_0, QMM_TYPE_Q4_0)
QMM_DEFINE_MMQ(q5_0, QMM_TYPE_Q5_0)
QMM_DEFINE_MMQ(iq4_xs, QMM_TYPE_IQ4_XS)
QMM_DEFINE_MMQ_ENTRIES(q8_0, QMM_TYPE_Q8_0, true, _q8_0)
QMM_DEFINE_MMQ_ENTRIES(q4_0, QMM_TYPE_Q4_0, true, _q8_0)
QMM_DEFINE_MMQ_ENTRIES(q5_0, QMM_TYPE_Q5_0, true, _q8_0)

#define QMM_DEFINE_MMQ_Q8K(t, TYPE)                                                                                \
  void launch_mmq_gguf_##t##_q8k(void *tmp_fixup, const void *x, const void *y, void *dst, int64_t ncols_x,       \
                                 int64_t nrows_x, int64_t ncols_y, int64_t stride_row_x, int64_t stride_col_dst,  \
                                 int cc, int nsm, int64_t smpbo, int warp_size, int type_dst, void *stream) {     \
    (void)cc, (void)smpbo, (void)warp_size;                                                                        \
    mmq_q8k(TYPE, tmp_fixup, x, y, dst, ncols_x, nrows_x, ncols_y, stride_row_x, stride_col_dst, nsm, type_dst,     \
            stream, "mmq_" #t "_q8k");                                                                             \
  }                                                                                                                \
  void launch_mmq_gguf_##t##_moe_q8k(void *tmp_fixup, const void *x, const void *y, const int32_t *ids_dst,       \
                                     const int32_t *expert_bounds, void *dst, int64_t ncols_x, int64_t nrows_x,    \
                                     int64_t ncols_dst, int64_t stride_row_x, int64_t stride_col_dst,              \
                                     int64_t num_experts, int64_t ncols_max, int cc, int nsm, int64_t smpbo,       \
                                     int warp_size, void *stream) {                                                \
    (void)cc, (void)smpbo, (void)warp_size;                                                                        \
    mmq_moe_q8k(TYPE, tmp_fixup, x, y, ids_dst, expert_bounds, dst, ncols_x, nrows_x, ncols_dst, stride_row_x,     \
                stride_col_dst, num_experts, ncols_max, nsm, stream, "mmq_" #t "_moe_q8k");                        \
  }
QMM_DEFINE_MMQ_Q8K(q4_k, QMM_TYPE_Q4K)
QMM_DEFINE_MMQ_Q8K(q5_k, QMM_TYPE_Q5K)
#undef QMM_DEFINE_MMQ_Q8K
}
