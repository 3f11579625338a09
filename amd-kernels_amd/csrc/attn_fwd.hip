// bf16 flash-attention forward for MI355X (gfx950), head_dim 128, no mask.
//
//   O = softmax(Q K^T / sqrt(128)) V,  bf16 in / bf16 out, fp32 accumulate.
//
// Replaces the reference's gfx942 kernel family (moonmath reference
// csrc/attention_kernel.hip:454-1127 forward, :1137-1217 V transpose,
// :1221-1279 merge, :1286-1393 tail planner) with a gfx950-native design:
//
//  * MFMA v_mfma_f32_32x32x16_bf16. Scores are computed transposed,
//    S^T = K Q^T (A = K fragment, B = Q fragment), so each lane owns one query
//    column and 16 kv rows per 32x32 tile; P^T then feeds O^T = V^T P^T as the
//    B operand straight from registers (no shuffle).
//  * K and the pre-transposed V_t are staged through LDS with 16-byte
//    global->LDS DMA (global_load_lds_dwordx4) in 4-slot rings, two blocks of
//    lead. Every DMA is inline asm, waited for by explicit vmcnt waits: with
//    one the compiler can see in flight, its wait counting turns every LDS
//    fragment wait into lgkmcnt(0) instead of the partial count the
//    in-order reads allow. K slots are chunk-major in 16-row groups and V_t
//    slots hold whole MFMA fragments in lane order, so every operand read is
//    a conflict-free ds_read_b128.
//  * Online softmax in base 2 with the running max kept on the integer grid:
//    m = ceil(max(s) * log2(e)/sqrt(128)). Every rescale is an exact power of
//    two, so the bf16 rounding of P (done with the output round mode, as in
//    the reference :438-449) does not depend on the KV blocking, on the
//    KV-split factor or on the merge order. The denominator sums unrounded
//    fp32 p (reference :445-451).
//  * Output: (O * rcp(l)) rounded per mode with every NaN -> 0x7FFF; l == 0
//    gives inv = 0 (reference :1114-1117). Staged through idle LDS so each
//    store writes whole 256-byte rows, with non-temporal stores.
//  * At most two KV blocks (short cross-attention): a persistent kernel keeps
//    a head's K / V_t in LDS across its q-blocks and gathers each item's Q
//    into a per-wave LDS stage during the previous item.
//  * KV split: the CTAs of the last, partially filled round of the grid
//    (the "tail") can be split over KV into G contiguous block ranges; each
//    part writes unnormalised fp32 (O, m, l) and a merge kernel combines them
//    (reference :1094-1112, :1239-1279).
//  * LiteAttention (reference :629-716, :1296-1347, :1497-1542, :1599-1681):
//    the same kernel walks only the KV blocks its CTA's read list (an int16
//    run-length row) names; each wave votes per block whether any of its 32
//    rows came within `threshold` (log2) of the row's running max and, if
//    none did, adds nothing for that block (per-wave soft skip); the CTA
//    writes the next step's list from the votes, and a planning kernel
//    orders the CTAs heaviest first (LPT).

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

#include <type_traits>

#include "mm_common.hpp"

namespace mm {
namespace attn {

constexpr int kD = 128;            // head_dim
constexpr int kKvBlock = 64;       // kv rows per main-loop block
constexpr int kWaves = 8;          // waves per CTA (two per SIMD; one CTA per CU)
constexpr int kThreads = 64 * kWaves;
constexpr int kQRowsPerTile = 32;  // q rows per wave = one 32x32 MFMA tile
constexpr int kRowsPerCta = kWaves * kQRowsPerTile;  // 256
constexpr int kFragBytes = 1024;   // one 32x16 bf16 MFMA operand fragment (64 lanes x 16 B)
constexpr int kKBytes = kKvBlock * kD * 2;   // 16 KB per K block
constexpr int kVBytes = kKvBlock * kD * 2;   // 16 KB per V_t block
constexpr int kVtBlockElems = kKvBlock * kD; // 8192 bf16 per V_t block
constexpr int kRing = 4;           // K / V_t ring slots: block j lives in slot j % kRing
constexpr int kLdsBytes = kRing * (kKBytes + kVBytes);  // K ring + V_t ring
// A row's running max m stays fixed while every p = 2^(s*c - m) of a block
// stays <= kGrowLimit (tested on the lane's sums of 8 p, which bound each p).
// A larger p makes the wave raise m and rescale (see rebase in run_tile), so O
// and l never hold a p above 2^20 (no fp32 overflow of O for |v| < 2^90).
constexpr float kGrowLimit = 1048576.0f;     // 2^20

// Split-KV limits: partial records are laid out for CTAs of kMaxRows q rows
// and up to kMaxParts parts.
constexpr int kMaxRows = kRowsPerCta;
constexpr int kMaxParts = 1024;
constexpr size_t kPartOFloats = (size_t)kMaxRows * kD;
constexpr size_t kWorkspaceBytes = (size_t)kMaxParts * kMaxRows * (kD + 2) * sizeof(float);

// LiteAttention: a CTA's processed block list (int16 ids, bit 15 marks the
// last block of a read-list range) and per-block vote bytes follow the rings.
constexpr int kMaxLiteBlocks = 8192;  // kv blocks per head (Skv <= 524288)
constexpr int kLiteListOff = kLdsBytes;
constexpr int kLiteVoteOff = kLiteListOff + kMaxLiteBlocks * 2;
constexpr int kLiteMiscOff = kLiteVoteOff + kMaxLiteBlocks;
constexpr int kLdsLiteBytes = kLiteMiscOff + 64;
static_assert(kLdsLiteBytes <= 160 * 1024, "lite LDS fits a CU");

// Short KV (at most kShortMaxBlocks blocks per head): persistent CTAs keep the
// head's K / V_t blocks resident in 2-slot rings and stage the next q-block's
// Q (256 rows x 256 B) in LDS while computing the current one.
constexpr int kShortMaxBlocks = 2;
constexpr int kShortOStageOff = 2 * kShortMaxBlocks * kKBytes;         // 64 KB: output staging
constexpr int kShortQStageOff = kShortOStageOff + kWaves * 16 * 256;    // 96 KB: Q stage
constexpr int kShortQStageBytes = kRowsPerCta * kD * 2;                // 64 KB
constexpr int kLdsShortBytes = kShortQStageOff + kShortQStageBytes;     // 160 KB
static_assert(kLdsShortBytes <= 160 * 1024, "short-KV LDS fits a CU");

// Item state of a persistent short-KV CTA across run_tile calls.
struct ShortCtx {
  int item;      // items this CTA has run
  int resident;  // (b, h) whose K / V_t blocks are in the slots, or -1
  int next_bh;   // the next item's (b, h) and q-block, whose Q is prefetched
  int next_qb;   //   into the stage during this item (next_bh < 0: none)
  bool first;    // the stage does not hold this item's Q yet
};

struct Params {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  uint16_t* out;
  float* ws;         // split partials (null unless split)
  int B, H, Sq, Skv;
  int bshd;          // 1 = [B,S,H,D], 0 = [B,H,S,D]
  int nqb, nkb;      // q-blocks per head, kv blocks per head
  int prefix_wgs;    // CTAs that run the whole KV stream
  int split_ways;    // G (parts per tail q-block)
  float scale_log2e; // log2(e) / sqrt(128), rounded to fp32 on the host
  // LiteAttention only.
  const int16_t* read_list;   // [B*H][nqb][nkb + 2]
  int16_t* write_list;        // same shape
  const int16_t* must_do;     // [len, s0, e0, ...] or null
  const int* order;           // LPT permutation of the CTAs, or null
  float threshold;            // log2 units, < 0
  int phase;                  // 1: ranges ascend, 0: descend
};

// Element offset of (b, h, s=0, d=0) and the stride between seq positions.
__device__ __forceinline__ long long head_base(int b, int h, int S, int H, int bshd) {
  return bshd ? ((long long)b * S * H + h) * kD : ((long long)b * H + h) * (long long)S * kD;
}

// ---------------------------------------------------------------------------
// LiteAttention write list of one CTA, by wave 0 after the main loop: the
// run-length row of the next step (reference record(), :685-716), in the
// processing order of this step. Block i is skipped iff no wave voted to keep
// it and no must_do range [s, e) holds it. A marker (the block id) is written
// at every change of the skip state, which starts as "skip" at the first
// block and again after the last block of each read-list range; after a kept
// range-end block the marker block + lstep closes its range. Lanes take one
// block each and place their 0..2 markers by a prefix sum over the wave.
// Markers past the row's nkb + 1 slots are dropped (possible only for read
// rows no writer produces) and the count keeps whole pairs.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_excl_sum(int x, int lane) {
  int incl = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  return incl - x;
}

__device__ __forceinline__ void lite_emit(const Params& p, long long row, int n, int lstep, const int16_t* list,
                                          uint8_t* vote, int lane) {
  int16_t* out = p.write_list + row;
  int md_len = p.must_do ? (int)p.must_do[0] : 0;
  md_len = md_len < 0 ? 0 : md_len;
  // Pass 1: vote byte -> skip flag (1 = skip).
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int i = i0 + lane;
    if (i < n) {
      const int blk = list[i] & 0x7FFF;
      bool keep = vote[i] != 0;
      for (int m = 1; m + 1 <= md_len && !keep; m += 2) keep = blk >= p.must_do[m] && blk < p.must_do[m + 1];
      vote[i] = keep ? 0 : 1;
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // Pass 2: markers.
  const int cap = p.nkb + 1;
  int base = 0;
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int i = i0 + lane;
    int blk = 0, cntm = 0;
    bool skip = true, rend = false, flip = false;
    if (i < n) {
      const int e = list[i];
      blk = e & 0x7FFF;
      rend = (e & 0x8000) != 0 || i == n - 1;
      skip = vote[i] != 0;
      const bool before = (i == 0 || (list[i - 1] & 0x8000) != 0) ? true : (vote[i - 1] != 0);
      flip = skip != before;
      cntm = (int)flip + (int)(rend && !skip);
    }
    const int ex = wave_excl_sum(cntm, lane);
    int pos = 1 + base + ex;
    if (flip) {
      if (pos <= cap) out[pos] = (int16_t)blk;
      ++pos;
    }
    if (rend && !skip && pos <= cap) out[pos] = (int16_t)(blk + lstep);
    base += __shfl(ex + cntm, 63, 64);
  }
  if (lane == 0) {
    const int len = base <= cap ? base : (cap & ~1);
    out[0] = (int16_t)len;
  }
}

// One CTA = 8 waves (two per SIMD) = 256 q rows of one (b, h), one CTA per CU,
// so every K / V_t block is gathered once per CU. Wave w owns rows
// [32w, 32w+32). Per 64-row kv block j:
//     QK(j+1) MFMAs || softmax(j) VALU      then      PV(j) MFMAs
// with the last 4 PV(j) MFMAs run after the next block barrier, ahead of
// QK(j+2), whose first K fragment reads they cover. K and V_t stream through 4-slot LDS rings (128 KB): block j+3 is gathered
// while block j is processed, so each DMA has two blocks of lead (measured at
// the headline shape: 1.485 ms vs 1.621 ms for two 128-row CTAs per CU with
// 2-slot rings and one block of lead).
//
// Max policy: each row's running max m is an integer (log2 units), set from
// the first block (m = ceil(max(s) * c)) and kept while the block's p stay
// <= kGrowLimit, so O and l are not rescaled in the common case. A block with
// a larger p makes its wave (a wave owns its rows, so no other wave takes
// part) raise m to the integer ceiling of the block's max, scale O and l by
// the exact power of two 2^(m_old - m_new) and recompute the block's p before
// they reach PV. Since m is always an integer, bf16(P) under any such m is
// bf16(P) under the final max times an exact power of two (up to the last
// fp32 bit of the exp2 argument): the output does not depend on where the
// rebases happen, on the KV blocking or on the split.
template <int MODE, bool LITE, bool SHORT = false>
__device__ __forceinline__ void run_tile(const Params& p, int bh, int qb, int kb_begin, int kb_end, int part,
                                         char* lds, ShortCtx* sc = nullptr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31;  // query column owned by this lane
  const int g = lane >> 5;  // lane half
  // Short KV (no barrier between items): the two waves of a SIMD (w and
  // w + 4) take turns at the higher priority level item by item; otherwise
  // the older wave wins every tie and the younger one falls behind, and the
  // CTA ends with the younger waves running alone.
  bool boost = false;
  if constexpr (SHORT) boost = ((sc->item + (wave >> 2)) & 1) != 0;

  const int b = bh / p.H, h = bh % p.H;
  const long long row_stride = p.bshd ? (long long)p.H * kD : kD;
  const uint16_t* qh = p.q + head_base(b, h, p.Sq, p.H, p.bshd);
  const char* kh = reinterpret_cast<const char*>(p.k + head_base(b, h, p.Skv, p.H, p.bshd));
  const char* vth = reinterpret_cast<const char*>(p.vt + (long long)bh * p.nkb * kVtBlockElems);
  const float c = p.scale_log2e;
  const int kv_end = p.Skv < kb_end * kKvBlock ? p.Skv : kb_end * kKvBlock;

  // LDS: K ring [kRing] | V_t ring [kRing].
  // K slot: 4 groups of 16 rows, chunk-major inside a group: the 16-byte chunk
  // c of row k at byte (k / 16) * 4096 + c * 256 + (k % 16) * 16. One DMA
  // instruction (1 KB) moves chunks 4j..4j+3 of 16 rows (64 contiguous bytes
  // per row); an MFMA fragment read (chunk 2ds+g of 32 rows) touches 16
  // consecutive 16-byte cells per 16 lanes (conflict free), and the 8 reads of
  // a row tile differ only by the immediate offset 512 * ds.
  // V_t slot: fragments [t(2)][s(2)][dt(4)], 1 KB each in lane order.
  // Short KV: K slots 0..1, V_t slots 0..1, the output stage, the Q stage.
  char* kring = lds;
  char* vring = lds + (SHORT ? kShortMaxBlocks : kRing) * kKBytes;
  auto kslot_off = [](int k, int c) { return (k >> 4) * 4096 + c * 256 + (k & 15) * 16; };
  // This lane's MFMA fragment cell for row tile t, k-step ds: kfrag_lane +
  // 8192 t + 512 ds (rows t*32 + r, chunk 2 ds + g), constants the LDS reads
  // carry as immediate offsets.
  const int kfrag_lane = kslot_off(r, g);
  // Lane source row / chunk of this wave's 2 K-DMA instructions (instruction
  // j = 2 wave + i fills slot bytes 1024 j .. 1024 j + 1023).
  auto kdma_row = [&](int i) { return 16 * ((wave * 2 + i) >> 2) + (lane & 15); };
  auto kdma_chunk = [&](int i) { return 4 * ((wave * 2 + i) & 3) + (lane >> 4); };
  uint32_t koff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) koff[i] = (uint32_t)(kdma_row(i) * row_stride * 2) + (uint32_t)(kdma_chunk(i) * 16);
  const long long kblk_bytes = (long long)kKvBlock * row_stride * 2;
  auto issue_k = [&](int kb, int slot) {
    char* st = kring + slot * kKBytes;
    if ((kb + 1) * kKvBlock <= p.Skv) {
      const char* base = kh + kb * kblk_bytes;
#pragma unroll
      for (int i = 0; i < 2; ++i) dma16_sbase(base, koff[i], st + (wave * 2 + i) * kFragBytes);
    } else {
      // Last partial block: clamp rows past Skv (they are masked in softmax).
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        int kv = kb * kKvBlock + kdma_row(i);
        kv = kv < p.Skv ? kv : p.Skv - 1;
        dma16_opaque(kh + (long long)kv * row_stride * 2 + kdma_chunk(i) * 16, st + (wave * 2 + i) * kFragBytes);
      }
    }
  };
  const uint32_t voff = (uint32_t)(wave * 2 * kFragBytes + lane * 16);
  auto issue_v = [&](int kb, int slot) {
    char* st = vring + slot * kVBytes;
    const char* base = vth + (long long)kb * kVBytes;
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16_sbase(base, voff + i * kFragBytes, st + (wave * 2 + i) * kFragBytes);
  };

  // ---- Q fragments (B operand of S^T = K Q^T), kept in registers --------------
  bf16x8 qf[8];
  const int q_row0 = qb * kRowsPerCta + wave * kQRowsPerTile;
  // A wave whose 32 query rows all lie past Sq (in the last q-block of a
  // ragged Sq; dense, unsplit tiles) issues its share of every block's DMAs
  // and meets every block barrier in the same order as its CTA's other waves,
  // and computes and stores nothing, so the CTA finishes sooner.
  if constexpr (!LITE && !SHORT) {
    if (part < 0 && q_row0 >= p.Sq && kb_end > kb_begin) {
      const int nb = kb_end - kb_begin;
      for (int j = 0; j < 3 && j < nb; ++j) {
        issue_k(kb_begin + j, j);
        issue_v(kb_begin + j, j);
      }
      if (nb > 2) {
        wait_vmem_barrier<8>();
      } else if (nb > 1) {
        wait_vmem_barrier<4>();
      } else {
        wait_vmem_barrier<0>();
      }
      for (int i = 0; i < nb; ++i) {
        if (i + 2 < nb) {
          asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        if (i + 3 < nb) {
          issue_k(kb_begin + i + 3, (i + 3) % kRing);
          issue_v(kb_begin + i + 3, (i + 3) % kRing);
        }
      }
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      return;
    }
  }
  // Short KV: Q staged in LDS, row rr's 16-byte chunk cc at
  // rr * 256 + 16 * (cc ^ (rr & 15)); wave w's 8 DMAs fill rows 32w .. 32w+31
  // (instruction i: rows 4i .. 4i+3, lane l -> row 4i + l/16, slot l % 16).
  char* qstage = lds + kShortQStageOff;
  auto issue_q_stage = [&](int sbh, int sqb) {
    const uint16_t* sq = p.q + head_base(sbh / p.H, sbh % p.H, p.Sq, p.H, p.bshd);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int ins = wave * 8 + k;
      const int rr = 4 * ins + (lane >> 4);
      const int cc = (lane & 15) ^ (rr & 15);
      int qr = sqb * kRowsPerCta + rr;
      qr = qr < p.Sq ? qr : p.Sq - 1;
      dma16_opaque(sq + (long long)qr * row_stride + cc * 8, qstage + ins * kFragBytes);
    }
  };
  if constexpr (SHORT) {
    // This item's Q: prefetched during the previous item (each wave waited for
    // its own DMAs before that item's output stores), or gathered now. A wave
    // gathers and reads only its own 32 rows of the stage, so no barrier:
    // the waves of a CTA meet only where the K/V slots change hands.
    if (sc->first) {
      issue_q_stage(bh, qb);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    const int rr = wave * kQRowsPerTile + r;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
      qf[ds] = *reinterpret_cast<const bf16x8*>(qstage + rr * 256 + 16 * ((2 * ds + g) ^ (rr & 15)));
    // The wave's stage rows are read before its next prefetch refills them.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  } else {
    int qr = q_row0 + r;
    qr = qr < p.Sq ? qr : p.Sq - 1;
    const uint16_t* src = qh + (long long)qr * row_stride + g * 8;
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) qf[ds] = *reinterpret_cast<const bf16x8*>(src + ds * 16);
  }

  // ---- the processed block sequence ---------------------------------------------
  // Dense: kb_begin .. kb_end-1. Lite: the blocks the CTA's read-list row names,
  // decoded into LDS in processing order (reference cursor :629-668): ranges are
  // taken from the end of the row; range (s, e) yields s+d, s+2d, ... while
  // strictly before e+d, at least one block (d = +1 in phase 1, -1 in phase 0).
  // Ids outside [0, nkb) are dropped and the list is capped at kMaxLiteBlocks,
  // so no row content makes the kernel read or write out of bounds.
  int16_t* lite_list = reinterpret_cast<int16_t*>(lds + kLiteListOff);
  uint8_t* lite_vote = reinterpret_cast<uint8_t*>(lds + kLiteVoteOff);
  int* lite_misc = reinterpret_cast<int*>(lds + kLiteMiscOff);
  const long long lite_row = ((long long)bh * p.nqb + qb) * (p.nkb + 2);
  const int lstep = p.phase ? 1 : -1;
  int nblk = kb_end - kb_begin;
  if constexpr (LITE) {
    // Stage the row (nkb + 2 int16) in the K ring, then wave 0 expands it.
    int16_t* stage = reinterpret_cast<int16_t*>(lds);
    const int row_len = p.nkb + 2;
    for (int e = tid; e < row_len; e += kThreads) stage[e] = p.read_list[lite_row + e];
    for (int e = tid; e < kMaxLiteBlocks / 4; e += kThreads) reinterpret_cast<uint32_t*>(lite_vote)[e] = 0u;
    lds_reads_done_barrier();
    if (wave == 0) {
      int len = stage[0];
      len = len < 0 ? 0 : (len > p.nkb + 1 ? p.nkb + 1 : len);
      int n = 0;
      for (int idx = len; idx >= 2 && n < kMaxLiteBlocks; idx -= 2) {
        const int start = stage[idx] + lstep;
        const int stop = stage[idx - 1] + lstep;
        const int span = (stop - start) * lstep;
        const int cnt = span > 1 ? span : 1;  // blocks start + j * lstep, j < cnt
        // j range whose block lies in [0, nkb)
        int jlo, jhi;
        if (lstep > 0) {
          jlo = start < 0 ? -start : 0;
          jhi = p.nkb - start;
        } else {
          jlo = start >= p.nkb ? start - p.nkb + 1 : 0;
          jhi = start + 1;
        }
        jhi = jhi < cnt ? jhi : cnt;
        if (jhi - jlo > kMaxLiteBlocks - n) jhi = jlo + (kMaxLiteBlocks - n);
        if (jhi <= jlo) continue;
        for (int j0 = jlo; j0 < jhi; j0 += 64) {
          const int j = j0 + lane;
          if (j < jhi) {
            const int blk = start + j * lstep;
            lite_list[n + (j - jlo)] = (int16_t)(blk | (j == jhi - 1 ? 0x8000 : 0));
          }
        }
        n += jhi - jlo;
      }
      if (lane == 0) lite_misc[0] = n;
    }
    lds_reads_done_barrier();
    nblk = __builtin_amdgcn_readfirstlane(lite_misc[0]);
  }
  auto blk_of = [&](int i) -> int {
    if constexpr (LITE) {
      return __builtin_amdgcn_readfirstlane(lite_list[i] & 0x7FFF);
    } else {
      return kb_begin + i;
    }
  };

  // Short KV: a block with at most 32 valid keys leaves its second row tile
  // out of QK and PV (its scores are masked to -inf, so p = 0, and V_t rows
  // past Skv are zero: the skipped MFMAs would add exact zeros).
  auto half_block = [&](int kbk) { return SHORT && kbk * kKvBlock + 32 >= kv_end; };
  auto qk = [&](const char* kst, f32x16 (&s)[2], bool half) {
#pragma unroll
    for (int t = 0; t < 2; ++t) s[t] = f32x16{};
#pragma unroll
    for (int ds = 0; ds < 8; ++ds) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (t == 1 && half) continue;
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kst + kfrag_lane + 8192 * t + 512 * ds);
        s[t] = mfma32(kf, qf[ds], s[t]);
      }
    }
  };
  f32x16 oacc[4];
  // Rows past kv_end get -inf scores (p = 0). Uniform branch: last block only.
  auto mask = [&](f32x16 (&s)[2], int kb) {
    const int kv0 = kb * kKvBlock;
    if (kv0 + kKvBlock > kv_end) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kv = kv0 + t * 32 + (e >> 2) * 8 + g * 4 + (e & 3);
          if (kv >= kv_end) s[t][e] = -__builtin_inff();
        }
    }
  };
  // Integer-grid max of row tiles t0..1 of a block: ceil(max(s) * c), NaN
  // ignored (fmaxf), -inf when every score is -inf or NaN.
  auto block_max = [&](const f32x16 (&s)[2], int t0) {
    float bm = -__builtin_inff();
#pragma unroll
    for (int t = t0; t < 2; ++t)
#pragma unroll
      for (int e = 0; e < 16; ++e) bm = fmaxf(bm, s[t][e]);
    return __builtin_ceilf(xor32_max(bm) * c);
  };
  float row_m = kNegFltMax, row_l = 0.f;

  // Lite vote state: each row's exact running max of s*c (log2 units) over the
  // blocks this wave kept so far (reference softmax_update's row_max,
  // :398-436, which a dropped block never reaches).
  float run_mx = -__builtin_inff();
  const bool row_valid = q_row0 + r < p.Sq;

  f32x16 sA[2], sB[2];
  bf16x8 pf[2][2];
  // Operands of the last 4 PV MFMAs of the previous block (row tile 1, k-step
  // 1: V^T fragments 12..15 and P^T), which run after the next block barrier.
  // Zero before the first block, so those MFMAs then add exact zeros.
  bf16x8 vtail[4] = {};
  bf16x8 ptail = {};
  // Lite: whether the previous block's deferred MFMAs carry a kept block
  // (wave-uniform; a dropped block leaves nothing to add).
  bool tail_on = false;
  // Short KV: the previous block skipped its second row tile, so its deferred
  // MFMAs (row tile 1, k-step 1) are skipped too.
  bool tail_half = false;
  if (nblk > 0) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) oacc[dt] = f32x16{};
    // Blocks 0..2 in flight; block j lives in slot j % kRing.
    auto issue_kv = [&](int kb, int slot) {
      issue_k(kb, slot);
      issue_v(kb, slot);
    };
    if constexpr (SHORT) {
      // The head's blocks stay in the slots across its q-blocks; then the next
      // item's Q goes out (8 DMAs per wave), which the block wait leaves in
      // flight.
      const bool kv_new = sc->resident != bh;  // CTA-uniform
      if (kv_new) {
        // Every wave is done with the previous head's blocks.
        lds_reads_done_barrier();
        for (int j = 0; j < nblk; ++j) issue_kv(blk_of(j), j);
      }
      const bool prefetch = sc->next_bh >= 0;
      if (prefetch) issue_q_stage(sc->next_bh, sc->next_qb);
      if (kv_new) {
        if (prefetch) {
          wait_vmem_barrier<8>();
        } else {
          wait_vmem_barrier<0>();
        }
      }
      sc->resident = bh;
    } else {
      issue_kv(blk_of(0), 0);
      if (nblk > 1) issue_kv(blk_of(1), 1);
      if (nblk > 2) issue_kv(blk_of(2), 2);
      // 4 DMAs per wave per block: block 0 has landed, blocks 1 and 2 stay in flight.
      if (nblk > 2) {
        wait_vmem_barrier<8>();
      } else if (nblk > 1) {
        wait_vmem_barrier<4>();
      } else {
        wait_vmem_barrier<0>();
      }
    }
    qk(kring, sA, half_block(blk_of(0)));
    mask(sA, blk_of(0));
    row_m = fmaxf(block_max(sA, 0), kNegFltMax);

    // LAST: the tile's last step, with no next block to score (its QK MFMAs
    // and K fragment reads are left out).
    auto step = [&](int i, f32x16 (&scur)[2], f32x16 (&snext)[2], auto last) {
      constexpr bool LAST = decltype(last)::value;
      // Lite: the list entries of blocks i and i+3 are read before the barrier,
      // whose lgkmcnt(0) covers their latency.
      int kb_raw = 0, kb3_raw = 0;
      if constexpr (LITE) {
        kb_raw = lite_list[i];
        kb3_raw = lite_list[i + 3 < nblk ? i + 3 : i];
      }
      // Block i+1 has landed (block i+2 stays in flight, 4 DMAs per wave); every
      // wave is done with step i-1, so the slot of block i-1 is free.
      sched_fence();
      if constexpr (SHORT) {
        // Every block is resident and no slot is refilled: no barrier, and no
        // wait for the Q prefetch in flight.
      } else if (i + 2 < nblk) {
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
      sched_fence();
      const int kb = LITE ? __builtin_amdgcn_readfirstlane(kb_raw & 0x7FFF) : kb_begin + i;
      const bool half_cur = half_block(kb);
      const bool half_next = !LAST && half_block(kb + 1);
      // Block kb+3: a full block's 4 DMAs go out one per odd QK step below (all
      // 8 waves issuing theirs back to back after the barrier stall their QK);
      // a partial last block is gathered here.
      const bool dma3 = i + 3 < nblk;
      const int kb3 = !dma3 ? kb : LITE ? __builtin_amdgcn_readfirstlane(kb3_raw & 0x7FFF) : kb_begin + i + 3;
      const bool dma3_full = dma3 && (kb3 + 1) * kKvBlock <= p.Skv;
      if (dma3 && !dma3_full) issue_kv(kb3, (i + 3) % kRing);
      const int pd3 = __builtin_amdgcn_readfirstlane((int)dma3_full);
      const char* kbase3 = kh + (long long)kb3 * kblk_bytes;
      const char* vbase3 = vth + (long long)kb3 * kVBytes;
      const char* kst3 = kring + ((i + 3) % kRing) * kKBytes;
      const char* vst3 = vring + ((i + 3) % kRing) * kVBytes;
      auto dma3_step = [&](int d) {  // d = 0, 1: K instructions; 2, 3: V instructions
        // Global address = SGPR base + 32-bit lane offset (no 64-bit VALU add).
        const char* base = d < 2 ? kbase3 : vbase3;
        const uint32_t off = d < 2 ? koff[d] : voff + (uint32_t)((d - 2) * kFragBytes);
        const char* dst = d < 2 ? kst3 + (wave * 2 + d) * kFragBytes : vst3 + (wave * 2 + d - 2) * kFragBytes;
        const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)dst;
        asm volatile("s_cmp_eq_u32 %3, 0\n\ts_cbranch_scc1 1f\n\tglobal_load_lds_dwordx4 %0, %1\n1:" ::"v"(off),
                     "s"(base), "{m0}"(m0v), "s"(pd3)
                     : "memory", "scc");
      };
      mask(scur, kb);
      // Sliced pipeline: QK(i+1) (16 MFMAs) carries softmax(i) of row tile 0
      // and the first half of row tile 1; PV(i) of row tile 0 (8 MFMAs) carries
      // the rest; PV(i) of row tile 1 follows, its second k-step after the next
      // barrier. Per-accumulator orders (S, O and each lpart sum) are those of
      // an unsliced softmax.
      const char* kst = kring + ((i + 1) % kRing) * kKBytes;  // last block: stale slot, unused
      const char* vst = vring + (i % kRing) * kVBytes;
      const float neg_m0 = -row_m;
      float lpart[4] = {0.f, 0.f, 0.f, 0.f};
      uint32_t w[2][2][4];
      // p of score pair pi (0..7) of row tile t, under the running max -neg_m.
      auto sm_pair = [&](int t, int pi, float neg_m) {
        const int ss = pi >> 2, e2 = pi & 3;
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(scur[t][8 * ss + 2 * e2], c, neg_m));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(scur[t][8 * ss + 2 * e2 + 1], c, neg_m));
        // The first pair starts the half's sum (0 + x is not folded: -0 + 0
        // is +0; a sum of p is never -0, so the result is the same).
        if (e2 == 0) {
          lpart[t * 2 + ss] = p0 + p1;
        } else {
          lpart[t * 2 + ss] += p0 + p1;
        }
        w[t][ss][e2] = pack2_bf16<MODE>(p0, p1);
      };
      auto pack_pf = [&](int t) {
#pragma unroll
        for (int ss = 0; ss < 2; ++ss) {
          const u32x4 wv = {w[t][ss][0], w[t][ss][1], w[t][ss][2], w[t][ss][3]};
          pf[t][ss] = __builtin_bit_cast(bf16x8, wv);
        }
      };
      // Some lane of the wave has a p above kGrowLimit in score halves
      // [h0, h1) (half hh = row tile hh / 2, pairs 4 (hh % 2) .. +3; halves below
      // h0 are accepted, and those of earlier blocks are in O): raise each row's
      // max to cover halves [h0, h1), rescale O, l and the accepted half sums
      // by the exact power of two 2^(m_old - m_new), and recompute the p of
      // halves [h0, h1).
      auto rebase = [&](int h0, int h1) {
        float bm = -__builtin_inff();
#pragma unroll
        for (int hh = h0; hh < h1; ++hh)
#pragma unroll
          for (int e = 0; e < 8; ++e) bm = fmaxf(bm, scur[hh >> 1][8 * (hh & 1) + e]);
        const float m_new = fmaxf(row_m, __builtin_ceilf(xor32_max(bm) * c));
        const float diff = row_m - m_new;  // integer-valued <= 0, -inf or NaN (both +inf)
        float sc = __builtin_ldexpf(1.0f, (int)fmaxf(diff, -127.f));
        sc = (diff >= -126.f) ? sc : 0.f;
        sc = (m_new > row_m) ? sc : 1.f;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) oacc[dt] *= sc;
        row_l *= sc;
#pragma unroll
        for (int hh = 0; hh < h0; ++hh) lpart[hh] *= sc;
        row_m = m_new;
#pragma unroll
        for (int hh = h0; hh < h1; ++hh) {
          lpart[hh] = 0.f;
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) sm_pair(hh >> 1, 4 * (hh & 1) + e2, -m_new);
        }
      };
      auto kfrag = [&](int t, int ds) {
        return *reinterpret_cast<const bf16x8*>(kst + kfrag_lane + 8192 * t + 512 * ds);
      };
      // V^T fragments in a 4-deep rolling buffer, 4 MFMAs ahead: PV MFMA n (0..15)
      // = row tile n/8, k-step (n/4)%2, d-tile n%4.
      auto vfrag_n = [&](int nn) {
        return *reinterpret_cast<const bf16x8*>(vst + (((nn >> 2) & 3) * 4 + (nn & 3)) * kFragBytes + lane * 16);
      };
      // Raised wave priority over the QK + softmax phase: the wave in this phase
      // wins issue slots over its SIMD partner when both are ready (measured
      // -0.7% to -2.8% at the headline shape).
      if (boost) {
        __builtin_amdgcn_s_setprio(2);
      } else {
        __builtin_amdgcn_s_setprio(1);
      }
      bf16x8 kf0, kf1;
      if constexpr (!LAST) {
        snext[0] = f32x16{};
        snext[1] = f32x16{};
        kf0 = kfrag(0, 0);
        kf1 = kfrag(1, 0);
      }
      // The previous block's last 4 PV MFMAs (operands in registers since
      // before the barrier) cover the latency of these first K reads:
      // 1.435 -> 1.411 ms at the headline shape (RTNA, one box). The first
      // step has no previous block.
      if (i > 0 && (!LITE || tail_on) && !tail_half) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          oacc[dt] = mfma32(vtail[dt], ptail, oacc[dt]);
          sched_fence();
        }
      }
      bf16x8 vb[4];
      // Lite: the block max of the vote, folded over the QK steps (4 scores
      // per step).
      float vmx = -__builtin_inff();
#pragma unroll
      for (int ds = 0; ds < 8; ++ds) {
        bf16x8 nk0, nk1;
        if (!LAST && ds + 1 < 8) {
          nk0 = kfrag(0, ds + 1);
          nk1 = kfrag(1, ds + 1);
        }
        if (ds == 7) {
#pragma unroll
          for (int k = 0; k < 4; ++k) vb[k] = vfrag_n(k);
        }
        if constexpr (!LAST) snext[0] = mfma32(kf0, qf[ds], snext[0]);
        sm_pair(0, ds, neg_m0);
        if constexpr (LITE) {
          const int t = ds >> 2, e0 = 4 * (ds & 3);
          vmx = fmaxf(fmaxf(vmx, scur[t][e0]), scur[t][e0 + 1]);
          vmx = fmaxf(fmaxf(vmx, scur[t][e0 + 2]), scur[t][e0 + 3]);
        }
        if (ds & 1) dma3_step(ds >> 1);
        if constexpr (!LAST) {
          if (!half_next) snext[1] = mfma32(kf1, qf[ds], snext[1]);
        }
        if ((ds & 1) && !half_cur) sm_pair(1, ds >> 1, neg_m0);
        if (!LAST && ds + 1 < 8) {
          kf0 = nk0;
          kf1 = nk1;
        }
        sched_fence();
      }
      pack_pf(0);
      if (boost) {
        __builtin_amdgcn_s_setprio(1);
      } else {
        __builtin_amdgcn_s_setprio(0);
      }
      // Lite vote, decided before any PV, rebase or sum of this block (per-wave
      // soft skip, reference :983-1001 and :891-898): the wave keeps the block
      // if some valid row's block max came within `threshold` of the row's
      // running max over the blocks this wave kept before it; the first
      // processed block is always kept. bm and bm - run_mx are each rounded to
      // fp32 (no fused multiply-subtract). A block the wave drops adds nothing
      // to its rows: no PV MFMAs (its deferred tail included), no l, no max
      // change. The wave's bit in the block's LDS vote byte feeds the next
      // step's list.
      // A lane holds half of its row's scores. With c > 0, rounding to fp32 is
      // monotone, so fl(fl(max(a, b) c) - run) > threshold holds exactly when it
      // holds for a or for b: each lane tests its own half, and the row's full
      // max (for run_mx) is formed off the critical path, after the PV.
      bool wkeep = true;
      float bmh = 0.f;
      if constexpr (LITE) {
#pragma clang fp contract(off)
        bmh = vmx * c;
        const bool keep = row_valid && (bmh - run_mx > p.threshold);
        wkeep = __builtin_amdgcn_ballot_w64(keep) != 0 || i == 0;
        if (wkeep) {
          if (lane == 0) {
            // Inline asm: the compiler would put a vmcnt(0) wait (for the
            // in-flight K/V DMAs, which also write LDS) before an atomic it
            // can see. The DMAs never touch the vote bytes; lite_emit reads
            // them after lgkmcnt(0) and a barrier.
            const uint32_t va = (uint32_t)(uintptr_t)(MM_LDS uint8_t*)(lite_vote + ((i >> 2) << 2));
            const uint32_t vbits = (1u << wave) << ((i & 3) * 8);
            asm volatile("ds_or_b32 %0, %1" ::"v"(va), "v"(vbits) : "memory");
          }
        }
        tail_on = wkeep;
      }
      if (wkeep) {
        // Wave-uniform growth tests: row tile 0 and the first half of row tile
        // 1 before any PV of this block, the second half of row tile 1 before
        // its PV.
        if (__builtin_amdgcn_ballot_w64(fmaxf(lpart[0] + lpart[1], lpart[2]) > kGrowLimit) != 0) {
          rebase(0, 3);
          pack_pf(0);
        }
        const float neg_m1 = -row_m;
        // PV of row tile 0 (k-step ss, d-tile dt) with softmax pairs 4..7 of tile 1.
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const int ss = m >> 2, dt = m & 3;
          const bf16x8 a = vb[m & 3];
          vb[m & 3] = vfrag_n(m + 4);
          oacc[dt] = mfma32(a, pf[0][ss], oacc[dt]);
          if (m < 4 && !half_cur) sm_pair(1, 4 + m, neg_m1);
          sched_fence();
        }
        if (__builtin_amdgcn_ballot_w64(lpart[3] > kGrowLimit) != 0) rebase(2, 4);
        pack_pf(1);
        // PV of row tile 1, k-step 0 (k-step 1 runs after the next barrier,
        // from vtail / ptail).
        if (!half_cur) {
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const bf16x8 a = vb[m];
            vb[m] = vfrag_n(12 + m);
            oacc[m] = mfma32(a, pf[1][0], oacc[m]);
            sched_fence();
          }
#pragma unroll
          for (int m = 0; m < 4; ++m) vtail[m] = vb[m];
          ptail = pf[1][1];
        }
        if constexpr (SHORT) tail_half = half_cur;
        row_l += (lpart[0] + lpart[1]) + (lpart[2] + lpart[3]);
        if constexpr (LITE) run_mx = fmaxf(run_mx, xor32_max(bmh));
      }
    };
    int i = 0;
    if constexpr (!SHORT) {  // short KV: at most two blocks
      for (; i + 2 < nblk; i += 2) {
        step(i, sA, sB, std::false_type{});
        step(i + 1, sB, sA, std::false_type{});
      }
    }
    if (i + 1 < nblk) {
      step(i, sA, sB, std::false_type{});
      ++i;
      sA[0] = sB[0];  // the last block's scores, where the last step reads them
      sA[1] = sB[1];
    }
    step(i, sA, sB, std::true_type{});
    // The last block's deferred PV MFMAs.
    if ((!LITE || tail_on) && !tail_half) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) oacc[dt] = mfma32(vtail[dt], ptail, oacc[dt]);
    }
  }
  sched_fence();
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  if constexpr (LITE) {
    lds_reads_done_barrier();  // every wave's votes are in
    if (wave == 0) lite_emit(p, lite_row, nblk, lstep, lite_list, lite_vote, lane);
  }

  // ---- epilogue -----------------------------------------------------------------
  row_l = xor32_sum(row_l);
  if (part >= 0) {
    // Split part: unnormalised fp32 partials. Record layout per part:
    // O [kMaxRows][128] fp32 then (m, l) [kMaxRows][2] fp32.
    float* po = p.ws + (size_t)part * kPartOFloats;
    float* pml = p.ws + (size_t)kMaxParts * kPartOFloats + (size_t)part * kMaxRows * 2;
    const int row = wave * kQRowsPerTile + r;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = dt * 32 + j * 8 + g * 4;
        f32x4 v = {oacc[dt][4 * j], oacc[dt][4 * j + 1], oacc[dt][4 * j + 2], oacc[dt][4 * j + 3]};
        *reinterpret_cast<f32x4*>(po + (size_t)row * kD + d) = v;
      }
    if (g == 0) {
      pml[row * 2] = row_m;
      pml[row * 2 + 1] = row_l;
    }
    return;
  }

  // The wave's 32 output rows go through LDS so that every store instruction
  // writes whole 256-byte rows (16 lanes per row, 4 rows per instruction):
  // stored straight from the accumulator layout, each instruction would write
  // 16 bytes into each of 32 rows' cache lines. Staging: row rr's 16-byte
  // chunk cc at rr * 256 + 16 * (cc ^ (rr & 15)) (conflict-free writes and
  // reads). The area is wave-private and idle: dense and lite use K and V_t
  // ring slots (nblk + 1) % 4 and (nblk + 2) % 4, which the last step neither
  // reads nor fills (8 KB per wave, all 32 rows at once); the short-KV kernel
  // its 32 KB output stage (4 KB per wave, 16 rows per round).
  const float inv = (row_l == 0.f) ? 0.f : __builtin_amdgcn_rcpf(row_l);
  uint16_t* ohead = p.out + head_base(b, h, p.Sq, p.H, p.bshd);
  constexpr int kRoundRows = SHORT ? 16 : kQRowsPerTile;
  char* ost;
  if constexpr (SHORT) {
    ost = lds + kShortOStageOff + wave * (kRoundRows * 256);
  } else {
    const int slot = ((wave & 2) ? nblk + 2 : nblk + 1) & (kRing - 1);
    ost = ((wave & 4) ? vring : kring) + slot * kKBytes + (wave & 1) * (kQRowsPerTile * 256);
  }
  u32x2 ow[4][4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ow[dt][j][0] = pack2_bf16_canon<MODE>(oacc[dt][4 * j] * inv, oacc[dt][4 * j + 1] * inv);
      ow[dt][j][1] = pack2_bf16_canon<MODE>(oacc[dt][4 * j + 2] * inv, oacc[dt][4 * j + 3] * inv);
    }
#pragma unroll
  for (int rd = 0; rd < kQRowsPerTile / kRoundRows; ++rd) {
    if (r / kRoundRows == rd) {
      char* wrow = ost + (r % kRoundRows) * 256 + g * 8;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x2*>(wrow + 16 * ((dt * 4 + j) ^ (r & 15))) = ow[dt][j];
    }
#pragma unroll
    for (int k = 0; k < kRoundRows / 4; ++k) {
      const int rr = 4 * k + (lane >> 4);  // row within the round
      const int row = rd * kRoundRows + rr;
      const int cs = lane & 15;
      const u32x4 v = *reinterpret_cast<const u32x4*>(ost + rr * 256 + 16 * cs);
      const int orow = q_row0 + row;
      // Non-temporal: the output is written once and not read back by this
      // launch (8192 x 77: 51.7 -> 49.6 us, 8192 x 512: -1.6%).
      if (orow < p.Sq)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(ohead + (long long)orow * row_stride +
                                                                8 * (cs ^ (row & 15))));
    }
  }
}

template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  const int idx = blockIdx.x;
  if (idx < p.prefix_wgs) {
    const int w = xcd_remap(idx, p.prefix_wgs);
    run_tile<MODE, false>(p, w / p.nqb, w % p.nqb, 0, p.nkb, -1, lds);
  } else {
    // Split part: tail q-block t, part j of G, contiguous kv-block range.
    const int part = idx - p.prefix_wgs;
    const int t = part / p.split_ways, j = part % p.split_ways;
    const int w = p.prefix_wgs + t;
    const int kb0 = (int)((long long)p.nkb * j / p.split_ways);
    const int kb1 = (int)((long long)p.nkb * (j + 1) / p.split_ways);
    run_tile<MODE, false>(p, w / p.nqb, w % p.nqb, kb0, kb1, part, lds);
  }
}

// Short-KV forward (at most kShortMaxBlocks KV blocks): persistent CTAs, CTA c
// runs items [c * per_cta, (c + 1) * per_cta) in order (item = (b, h) * nqb +
// q-block, so consecutive items share a head and its resident blocks). While
// an item computes, the next item's Q is gathered into the LDS stage and the
// previous item's output stores drain, so the q-blocks' HBM traffic overlaps
// the MFMA work instead of alternating with it in lockstep rounds.
template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void attn_short_kernel(Params p, int per_cta) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsShortBytes];
  const int total = p.nqb * p.B * p.H;
  const int w0 = blockIdx.x * per_cta;
  const int w1 = w0 + per_cta < total ? w0 + per_cta : total;
  ShortCtx sc{0, -1, -1, 0, true};
  for (int w = w0; w < w1; ++w) {
    const int wn = w + 1 < w1 ? w + 1 : -1;
    sc.next_bh = wn >= 0 ? wn / p.nqb : -1;
    sc.next_qb = wn >= 0 ? wn % p.nqb : 0;
    run_tile<MODE, false, true>(p, w / p.nqb, w % p.nqb, 0, p.nkb, -1, lds, &sc);
    sc.first = false;
    ++sc.item;
  }
}

// Grid slot -> position in the LPT order. Slot s runs on XCD s % 8, and each
// XCD starts its slots in order, one per CU (32 at a time). Round r of the
// grid (slots 256r .. 256r + 255) takes order positions [256r, 256r + 256):
// XCD x takes the contiguous run x of 32 positions (run 7 - x in odd rounds,
// so no XCD always draws the heaviest run of a round). CTAs that run together
// on one XCD are neighbours in the order -- the q-blocks of one head when
// their kept counts share a bucket, every q-block of the head in a
// compute-all step -- and read the same K/V through that XCD's L2. A partial
// last round is dealt as the dense mapping deals a grid.
constexpr int kCusPerXcd = 32;
__device__ __forceinline__ int lpt_position(int s, int total) {
  constexpr int kRound = kNumXcds * kCusPerXcd;
  const int base = s - s % kRound;
  const int idx = s - base;
  if (total - base < kRound) return base + xcd_remap(idx, total - base);
  const int x = idx % kNumXcds;
  const int run = ((base / kRound) & 1) ? kNumXcds - 1 - x : x;
  return base + run * kCusPerXcd + idx / kNumXcds;
}

// LiteAttention forward: one CTA per (b, h, q-block); grid slot s runs CTA
// order[lpt_position(s)] (LPT order) or, without an order, the XCD-grouped
// dense mapping.
template <int MODE>
__global__ __launch_bounds__(kThreads, 1) void attn_lite_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsLiteBytes];
  const int total = p.nqb * p.B * p.H;
  const int w = p.order ? p.order[lpt_position(blockIdx.x, total)] : xcd_remap(blockIdx.x, total);
  if (w < 0 || w >= total) return;
  run_tile<MODE, true>(p, w / p.nqb, w % p.nqb, 0, p.nkb, -1, lds);
}

// ---------------------------------------------------------------------------
// LPT order of the lite CTAs (reference plan_lite_order, :1296-1347): CTAs
// sorted by the number of blocks their read-list row keeps, heaviest first, in
// 64 buckets of kept/(nkb+1); a stable counting sort (thread t owns the
// contiguous CTA range [t*C, (t+1)*C)), so the order is deterministic. Two
// launches: lite_count_kernel buckets the rows, one thread per row over many
// CUs (a row's entries are scattered relative to its neighbours', so one CU
// doing every row is bound by its memory pipeline's rate of distinct cache
// lines: ~36 us at 1536 rows of ~25 ranges, against ~3 us spread out); then
// lite_order_kernel (one CTA of 256 threads) sorts the buckets, up to
// kLptMaxCtas CTAs. Workspace: the order (int per CTA), then the buckets
// (byte per CTA).
// ---------------------------------------------------------------------------
constexpr int kLptThreads = 256;
constexpr int kLptCountThreads = 64;  // rows per counting CTA
constexpr int kLptBuckets = 64;
constexpr int kLptMaxCtas = 65536;
constexpr int kLptPairBatch = 16;     // pairs whose entries are loaded together

// Kept blocks of a read-list row: the sum of |row[i] - row[i - 1]| over
// i = len, len - 2, ... >= 2, len = row[0] clamped to [0, nkb + 1]. The two
// entries of kLptPairBatch pairs are loaded before any is used, so a row of
// up to 16 ranges costs one round of memory latency. Reads stay inside the
// row. The sum stays below 2^28 ((nkb + 1) / 2 <= 4096 pairs of int16 ids).
__device__ __forceinline__ int lite_kept(const int16_t* row, int nkb) {
  int len = row[0];
  len = len < 0 ? 0 : (len > nkb + 1 ? nkb + 1 : len);
  int kept = 0;
  for (int i0 = len; i0 >= 2; i0 -= 2 * kLptPairBatch) {
    int hi[kLptPairBatch], lo[kLptPairBatch];
#pragma unroll
    for (int k = 0; k < kLptPairBatch; ++k) {
      const int i = i0 - 2 * k;
      hi[k] = i >= 2 ? (int)row[i] : 0;
      lo[k] = i >= 2 ? (int)row[i - 1] : 0;
    }
#pragma unroll
    for (int k = 0; k < kLptPairBatch; ++k) {
      const int d = hi[k] - lo[k];
      kept += d < 0 ? -d : d;
    }
  }
  return kept;
}

// Bucket of every CTA's row. A count past nkb lands in the top bucket either
// way; clamping it first keeps the product in range for any row content.
__global__ __launch_bounds__(kLptCountThreads) void lite_count_kernel(const int16_t* __restrict__ read_list,
                                                                     uint8_t* __restrict__ bucket, int nctas,
                                                                     int nkb) {
  const int w = blockIdx.x * kLptCountThreads + threadIdx.x;
  if (w >= nctas) return;
  int kept = lite_kept(read_list + (long long)w * (nkb + 2), nkb);
  kept = kept < nkb + 1 ? kept : nkb + 1;
  const int bk = kept * kLptBuckets / (nkb + 1);
  bucket[w] = (uint8_t)(bk < kLptBuckets ? bk : kLptBuckets - 1);
}

__global__ __launch_bounds__(kLptThreads) void lite_order_kernel(const uint8_t* __restrict__ bucket,
                                                                int* __restrict__ order, int nctas) {
  static_assert(kLptThreads == 256 && kLptBuckets == 64, "4 threads' counts per lane, one bucket per lane");
  __shared__ __attribute__((aligned(16))) int hist[kLptBuckets][kLptThreads];
  __shared__ int bucket_base[kLptBuckets];
  __shared__ uint8_t bk_of[kLptMaxCtas];
  const int t = threadIdx.x;
  const int chunk = (nctas + kLptThreads - 1) / kLptThreads;
  const int w0 = t * chunk;
  const int w1 = w0 + chunk < nctas ? w0 + chunk : nctas;
  for (int b = 0; b < kLptBuckets; ++b) hist[b][t] = 0;
  for (int w = t; w < nctas; w += kLptThreads) bk_of[w] = bucket[w];
  __syncthreads();
  for (int w = w0; w < w1; ++w) ++hist[bk_of[w]][t];
  __syncthreads();
  // Exclusive prefix of each bucket's counts over the threads: wave v takes
  // buckets v, v+4, ...; lane l holds threads 4l..4l+3 (one conflict-free
  // 16-byte LDS access each way).
  const int wv = t >> 6, ln = t & 63;
  for (int b = wv; b < kLptBuckets; b += kLptThreads / 64) {
    int4* cell = reinterpret_cast<int4*>(&hist[b][4 * ln]);
    const int4 c = *cell;
    const int s1 = c.x + c.y, s2 = s1 + c.z, s3 = s2 + c.w;
    const int incl = wave_incl_scan(s3);
    const int excl = incl - s3;
    *cell = make_int4(excl, excl + c.x, excl + s1, excl + s2);
    if (ln == 63) bucket_base[b] = incl;  // bucket total, turned into a base below
  }
  __syncthreads();
  // Bucket bases, heaviest first: exclusive scan of the totals in descending
  // bucket order (lane l holds bucket 63 - l).
  if (wv == 0) {
    const int c = bucket_base[kLptBuckets - 1 - ln];
    bucket_base[kLptBuckets - 1 - ln] = wave_incl_scan(c) - c;
  }
  __syncthreads();
  for (int w = w0; w < w1; ++w) {
    const int bk = bk_of[w];
    order[bucket_base[bk] + hist[bk][t]] = w;
    ++hist[bk][t];
  }
}

// ---------------------------------------------------------------------------
// Merge of split partials. One thread = 4 consecutive d of one row.
// M = max_p m_p; w_p = 2^(m_p - M) (exact, m_p integer-valued);
// out = mode(sum_p w_p O_p * rcp(sum_p w_p l_p)), inv = 0 when the sum is 0.
// ---------------------------------------------------------------------------
constexpr int kMergeThreads = 256;

__device__ __forceinline__ float pow2_weight(float m_p, float M) {
  if (m_p == M) return 1.f;  // also covers M == +inf with m_p == +inf
  const float diff = m_p - M;  // < 0
  const float w = __builtin_ldexpf(1.0f, (int)fmaxf(diff, -127.f));
  return diff >= -126.f ? w : 0.f;
}

template <int MODE>
__global__ __launch_bounds__(kMergeThreads) void attn_merge_kernel(Params p, int rows) {
  const int per_qb = rows * kD / 4 / kMergeThreads;
  const int t = blockIdx.x / per_qb;
  const int cell = ((blockIdx.x % per_qb) * kMergeThreads + threadIdx.x) * 4;
  const int row = cell / kD, d = cell % kD;
  const int w = p.prefix_wgs + t;
  const int bh = w / p.nqb, qb = w % p.nqb;
  const int qr = qb * rows + row;
  if (qr >= p.Sq) return;
  const int G = p.split_ways;
  const int part0 = t * G;
  const float* pml = p.ws + (size_t)kMaxParts * kPartOFloats;
  float M = kNegFltMax;
  for (int j = 0; j < G; ++j) M = fmaxf(M, pml[(size_t)(part0 + j) * kMaxRows * 2 + row * 2]);
  float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f, L = 0.f;
  for (int j = 0; j < G; ++j) {
    const float m_p = pml[(size_t)(part0 + j) * kMaxRows * 2 + row * 2];
    const float l_p = pml[(size_t)(part0 + j) * kMaxRows * 2 + row * 2 + 1];
    const f32x4 o = *reinterpret_cast<const f32x4*>(p.ws + (size_t)(part0 + j) * kPartOFloats + (size_t)row * kD + d);
    const float wt = pow2_weight(m_p, M);
    o0 = __builtin_fmaf(wt, o[0], o0);
    o1 = __builtin_fmaf(wt, o[1], o1);
    o2 = __builtin_fmaf(wt, o[2], o2);
    o3 = __builtin_fmaf(wt, o[3], o3);
    L = __builtin_fmaf(wt, l_p, L);
  }
  const float inv = (L == 0.f) ? 0.f : __builtin_amdgcn_rcpf(L);
  const int b = bh / p.H, h = bh % p.H;
  const long long row_stride = p.bshd ? (long long)p.H * kD : kD;
  uint16_t* dst = p.out + head_base(b, h, p.Sq, p.H, p.bshd) + (long long)qr * row_stride + d;
  u32x2 wv;
  wv[0] = pack2_bf16_canon<MODE>(o0 * inv, o1 * inv);
  wv[1] = pack2_bf16_canon<MODE>(o2 * inv, o3 * inv);
  *reinterpret_cast<u32x2*>(dst) = wv;
}

// ---------------------------------------------------------------------------
// V -> V_t: per (b, h, 64-row kv block), 16 fragments of 64 lanes x 8 bf16:
//   V_t[bh][kb][(t*2+s)*4+dt][lane][e] = V[kb*64 + 32t + 16s + 8(e/4) + 4(lane/32) + e%4][32dt + lane%32]
// which is the A-operand order of O^T = V^T P^T. Rows >= Skv are zero.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void v_transpose_kernel(const uint16_t* __restrict__ v, uint16_t* __restrict__ vt,
                                                          int H, int Skv, int nkb, int bshd) {
  // Row-major tile of the block's 64 rows, 288-byte row pitch (256 B + 32 B of
  // padding: the four rows of one transposing read start 8 banks apart).
  constexpr int kPitch = 288;
  __shared__ __attribute__((aligned(16))) char tile[kKvBlock * kPitch];
  const int kb = blockIdx.x % nkb;
  const int bh = blockIdx.x / nkb;
  const int b = bh / H, h = bh % H;
  const long long row_stride = bshd ? (long long)H * kD : kD;
  const uint16_t* vh = v + head_base(b, h, Skv, H, bshd);
  const int tid = threadIdx.x;
  // Load 64 rows x 256 B: 1024 16-byte pieces, 4 per thread, one LDS write each.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int piece = tid + i * 256;
    const int row = piece >> 4, c16 = piece & 15;
    const int kv = kb * kKvBlock + row;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (kv < Skv) val = *reinterpret_cast<const u32x4*>(vh + (long long)kv * row_stride + c16 * 8);
    *reinterpret_cast<u32x4*>(tile + row * kPitch + c16 * 16) = val;
  }
  __syncthreads();
  // Output unit (fragment f, lane l): 8 bf16 of column d = 32dt + l%32, rows
  // base + {0..3, 8..11} with base = 32t + 16s + 4(l/32). A 16-lane group holds
  // 16 consecutive columns d0 .. d0+15 of one base, so two ds_read_b64_tr_b16
  // (within a 16-lane group out[i][e] = in[4e + i/4][i%4]) deliver them: member
  // m supplies 4 bf16 of row base(+8) + m/4 at columns d0 + 4(m%4), and lane i
  // receives column d0 + i of those 4 rows.
  uint16_t* dst = vt + ((long long)bh * nkb + kb) * kVtBlockElems;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int unit = tid + i * 256;
    const int f = unit >> 6, lane = unit & 63;
    const int t = f >> 3, s = (f >> 2) & 1, dt = f & 3;
    const int base = t * 32 + s * 16 + (lane >> 5) * 4;
    const int d0 = dt * 32 + ((lane >> 4) & 1) * 16;
    const int m = lane & 15;
    const char* a = tile + (base + (m >> 2)) * kPitch + (d0 + 4 * (m & 3)) * 2;
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((MM_LDS i16x4*)a);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((MM_LDS i16x4*)(a + 8 * kPitch));
    const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
    const u32x4 out = {lo2[0], lo2[1], hi2[0], hi2[1]};
    *reinterpret_cast<u32x4*>(dst + (size_t)unit * 8) = out;
  }
}

// Test hook kernel: the output packing of the epilogue and the merge applied
// to arbitrary fp32 pairs.
template <int MODE>
__global__ __launch_bounds__(256) void pack_bf16_kernel(const float* __restrict__ in, uint32_t* __restrict__ out,
                                                        int npairs) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < npairs) out[i] = pack2_bf16_canon<MODE>(in[2 * i], in[2 * i + 1]);
}

}  // namespace attn
}  // namespace mm

// ===========================================================================
// Host side: planner + C ABI
// ===========================================================================
namespace {
using namespace mm::attn;

constexpr int kNumCUs = 256;
// Kernel variant used by the launchers: QT q-tiles of 32 rows per wave and
// MINB CTAs resident per CU.
constexpr int kMinBlocks = 1;  // CTAs resident per CU
constexpr int kSlots = kNumCUs * kMinBlocks;

// Tail KV-split cost model, in KV blocks of the last round (after reference
// csrc/attention_kernel.hip:1349-1393, whose span is rounds x blocks per part
// + 3 for the merge; re-derived on MI355X with 256 CUs x 1 CTA of 256 rows):
//   unsplit: nkb + kCtaCostBlocks
//   G parts: rounds x (ceil(nkb / G) + kCtaCostBlocks) + kMergeCostBlocks
//            + ceil(tail x G / kPartsPerRecordBlock)
// kCtaCostBlocks: a CTA's prologue and epilogue (~7 us at ~1.7 us per block);
// the last term: each part's 133 KB fp32 record is written and read back by
// the merge (~64 records per block of time). Measured on (2,24,4097) with a
// 48-CTA tail: Skv 8192 779 us with the reference's choice (16 parts, three
// rounds) against 752 us with 5 parts (this model's choice), Skv 4096 417 ->
// 386 us (5 parts), Skv 2048 226 -> 212 us; Skv 512 (8 blocks) loses with any
// split (77 -> 80 us), hence no split below 16 blocks (the reference: 48).
constexpr int kMinKvBlocksToSplit = 16;
constexpr int kMinBlocksPerPart = 4;
constexpr int kMergeCostBlocks = 3;
constexpr int kCtaCostBlocks = 4;
constexpr int kPartsPerRecordBlock = 64;

struct TailPlan {
  int prefix_wgs, tail, split_ways, parts;
};

// The persistent short-KV kernel serves shapes of at most kShortMaxBlocks KV
// blocks unless MOONMATH_NO_SHORT_KV is set (a switch for comparing it with
// the one-CTA-per-q-block kernel on the same shape).
bool short_kv_enabled() {
  const char* v = getenv("MOONMATH_NO_SHORT_KV");
  return !(v && *v && *v != '0');
}

TailPlan plan_tail(int nqb, int nbh, int nkb, int slots, bool enable, int force_ways) {
  const int wgs = nqb * nbh;
  const TailPlan none{wgs, 0, 1, 0};
  if (!enable) return none;
  int tail = wgs % slots;
  if (force_ways > 1) {
    // Test hook: split the last `tail` CTAs (the whole grid if it tiles evenly).
    if (tail == 0) tail = wgs < slots ? wgs : slots;
    int G = force_ways;
    if (G > nkb) G = nkb;
    while (tail * G > kMaxParts) --G;
    if (G < 2) return none;
    return TailPlan{wgs - tail, tail, G, tail * G};
  }
  if (tail == 0 || tail > slots * 19 / 20 || nkb < kMinKvBlocksToSplit) return none;
  int G = 1;
  long long best = (long long)nkb + kCtaCostBlocks;
  for (int gw = 2; gw <= kMaxParts / tail && nkb / gw >= kMinBlocksPerPart; ++gw) {
    const long long rounds = ((long long)tail * gw + slots - 1) / slots;
    const long long per_part = (nkb + gw - 1) / gw;
    const long long records = ((long long)tail * gw + kPartsPerRecordBlock - 1) / kPartsPerRecordBlock;
    const long long span = rounds * (per_part + kCtaCostBlocks) + kMergeCostBlocks + records;
    if (span < best) {
      best = span;
      G = gw;
    }
  }
  if (G == 1) return none;
  return TailPlan{wgs - tail, tail, G, tail * G};
}

template <int MODE>
int launch_fwd(const void* q, const void* k, const void* v_t, void* out, int batch, int heads, int seq_len,
               int seq_len_kv, int head_dim, int layout, void* workspace, int force_ways, void* stream) {
  if (batch <= 0 || heads <= 0) return 1;
  if (seq_len <= 0) return 2;
  if (head_dim != kD) return 3;
  if (seq_len_kv <= 0) return 5;
  if (layout != 0 && layout != 1) return 7;
  if (!q || !k || !v_t || !out) return 8;
  Params p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.vt = static_cast<const uint16_t*>(v_t);
  p.out = static_cast<uint16_t*>(out);
  p.ws = static_cast<float*>(workspace);
  p.B = batch;
  p.H = heads;
  p.Sq = seq_len;
  p.Skv = seq_len_kv;
  p.bshd = layout;
  p.nqb = (seq_len + kRowsPerCta - 1) / kRowsPerCta;
  p.nkb = (seq_len_kv + kKvBlock - 1) / kKvBlock;
  p.scale_log2e = (float)(1.4426950408889634 / 11.313708498984761);
  const long long nbh = (long long)batch * heads;
  if ((long long)p.nqb * nbh > 0x7FFFFFFFLL) return 9;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const long long items = (long long)p.nqb * nbh;
  if (p.nkb <= kShortMaxBlocks && items > kSlots && force_ways <= 1 && short_kv_enabled()) {
    // Short KV: one persistent CTA per CU (no tail split: nkb is far below the
    // planner's minimum).
    const int per_cta = (int)((items + kSlots - 1) / kSlots);
    const int grid = (int)((items + per_cta - 1) / per_cta);
    hipLaunchKernelGGL((attn_short_kernel<MODE>), dim3(grid), dim3(kThreads), 0, st, p, per_cta);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
  }
  const TailPlan tp = plan_tail(p.nqb, (int)nbh, p.nkb, kSlots, workspace != nullptr, force_ways);
  p.prefix_wgs = tp.prefix_wgs;
  p.split_ways = tp.split_ways;
  const int grid = tp.prefix_wgs + tp.parts;
  hipLaunchKernelGGL((attn_fwd_kernel<MODE>), dim3(grid), dim3(kThreads), 0, st, p);
  if (tp.parts > 0) {
    const int per_qb = kRowsPerCta * kD / 4 / kMergeThreads;
    hipLaunchKernelGGL((attn_merge_kernel<MODE>), dim3(tp.tail * per_qb), dim3(kMergeThreads), 0, st, p,
                       kRowsPerCta);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

// LiteAttention launcher (reference launch_attention_forward_lite,
// attention_kernel.hip:1599-1681). workspace: lite_workspace_bytes bytes for
// the LPT order and buckets (null = plain order); LPT runs when the kv range
// is long enough to amortise its planning launches (48 blocks, as the
// reference).
constexpr int kLiteMinKvBlocksForLpt = 48;

template <int MODE>
int launch_lite(const void* q, const void* k, const void* v_t, void* out, int batch, int heads, int seq_len,
                int seq_len_kv, int head_dim, const void* read_list, void* write_list, const void* must_do,
                float threshold, int phase, int layout, void* workspace, void* stream) {
  if (batch <= 0 || heads <= 0) return 1;
  if (seq_len <= 0) return 2;
  if (head_dim != kD) return 3;
  if (!read_list || !write_list) return 4;
  if (seq_len_kv <= 0) return 5;
  if (layout != 0 && layout != 1) return 7;
  if (!q || !k || !v_t || !out) return 8;
  Params p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.vt = static_cast<const uint16_t*>(v_t);
  p.out = static_cast<uint16_t*>(out);
  p.B = batch;
  p.H = heads;
  p.Sq = seq_len;
  p.Skv = seq_len_kv;
  p.bshd = layout;
  p.nqb = (seq_len + kRowsPerCta - 1) / kRowsPerCta;
  p.nkb = (seq_len_kv + kKvBlock - 1) / kKvBlock;
  if (p.nkb > kMaxLiteBlocks) return 6;
  p.scale_log2e = (float)(1.4426950408889634 / 11.313708498984761);
  p.read_list = static_cast<const int16_t*>(read_list);
  p.write_list = static_cast<int16_t*>(write_list);
  p.must_do = static_cast<const int16_t*>(must_do);
  p.threshold = threshold;
  p.phase = phase ? 1 : 0;
  const long long total = (long long)p.nqb * batch * heads;
  if (total > 0x7FFFFFFFLL) return 9;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (workspace && p.nkb >= kLiteMinKvBlocksForLpt && total <= kLptMaxCtas) {
    p.order = static_cast<const int*>(workspace);
    uint8_t* bucket = static_cast<uint8_t*>(workspace) + total * sizeof(int);
    hipLaunchKernelGGL(lite_count_kernel, dim3((unsigned)((total + kLptCountThreads - 1) / kLptCountThreads)),
                       dim3(kLptCountThreads), 0, st, p.read_list, bucket, (int)total, p.nkb);
    hipLaunchKernelGGL(lite_order_kernel, dim3(1), dim3(kLptThreads), 0, st, bucket, static_cast<int*>(workspace),
                       (int)total);
  }
  hipLaunchKernelGGL((attn_lite_kernel<MODE>), dim3((unsigned)total), dim3(kThreads), 0, st, p);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

int launch_vt(const void* v, void* v_t, int n_rows, int seq_len_per_head, int heads, int layout, void* stream) {
  if (heads <= 0 || seq_len_per_head <= 0 || n_rows <= 0) return 1;
  if (n_rows % ((long long)heads * seq_len_per_head) != 0) return 2;
  if (layout != 0 && layout != 1) return 7;
  if (!v || !v_t) return 8;
  const int batch = (int)(n_rows / ((long long)heads * seq_len_per_head));
  const int nkb = (seq_len_per_head + kKvBlock - 1) / kKvBlock;
  const long long grid = (long long)batch * heads * nkb;
  if (grid > 0x7FFFFFFFLL) return 9;
  hipLaunchKernelGGL(v_transpose_kernel, dim3((unsigned)grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(v), static_cast<uint16_t*>(v_t), heads, seq_len_per_head, nkb,
                     layout);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // namespace

extern "C" {

#define MM_ATTN_MODE_SYMBOLS(NAME, MODE)                                                                      \
  int launch_v_transpose_##NAME(const void* v, void* v_t, int n_rows, int seq_len_per_head, int heads,       \
                                int layout, void* stream) {                                                  \
    return launch_vt(v, v_t, n_rows, seq_len_per_head, heads, layout, stream);                               \
  }                                                                                                          \
  int launch_attention_forward_##NAME(const void* q, const void* k, const void* v_t, void* out, int batch,   \
                                      int heads, int seq_len, int seq_len_kv, int head_dim, int layout,      \
                                      void* workspace, void* stream) {                                       \
    return launch_fwd<MODE>(q, k, v_t, out, batch, heads, seq_len, seq_len_kv, head_dim, layout, workspace, \
                            0, stream);                                                                      \
  }                                                                                                          \
  size_t tail_workspace_bytes_##NAME(void) { return kWorkspaceBytes; }                                     \
  int launch_attention_forward_lite_##NAME(const void* q, const void* k, const void* v_t, void* out, int batch, \
                                           int heads, int seq_len, int seq_len_kv, int head_dim,              \
                                           const void* read_list, void* write_list, const void* must_do_list, \
                                           float threshold, int phase, int layout, void* workspace,           \
                                           void* stream) {                                                    \
    return launch_lite<MODE>(q, k, v_t, out, batch, heads, seq_len, seq_len_kv, head_dim, read_list,          \
                             write_list, must_do_list, threshold, phase, layout, workspace, stream);          \
  }                                                                                                          \
  size_t lite_workspace_bytes_##NAME(int batch, int heads, int seq_len) {                                    \
    if (batch <= 0 || heads <= 0 || seq_len <= 0) return 0;                                                  \
    return (size_t)batch * heads * ((seq_len + kRowsPerCta - 1) / kRowsPerCta) * (sizeof(int) + 1);          \
  }

MM_ATTN_MODE_SYMBOLS(rtne, mm::kRTNE)
MM_ATTN_MODE_SYMBOLS(rtna, mm::kRTNA)
MM_ATTN_MODE_SYMBOLS(rtz, mm::kRTZ)

int moonmath_attention_forward_ex(const void* q, const void* k, const void* v_t, void* out, int batch, int heads,
                                  int seq_len, int seq_len_kv, int head_dim, int layout, int round_mode,
                                  void* workspace, int force_split_ways, void* stream) {
  switch (round_mode) {
    case 0:
      return launch_fwd<mm::kRTNE>(q, k, v_t, out, batch, heads, seq_len, seq_len_kv, head_dim, layout, workspace,
                                   force_split_ways, stream);
    case 1:
      return launch_fwd<mm::kRTNA>(q, k, v_t, out, batch, heads, seq_len, seq_len_kv, head_dim, layout, workspace,
                                   force_split_ways, stream);
    case 2:
      return launch_fwd<mm::kRTZ>(q, k, v_t, out, batch, heads, seq_len, seq_len_kv, head_dim, layout, workspace,
                                  force_split_ways, stream);
    default:
      return 10;
  }
}

int moonmath_attention_plan_tail(int batch, int heads, int seq_len, int seq_len_kv, int enable, int force_split_ways,
                                 int* out4) {
  if (!out4 || batch <= 0 || heads <= 0 || seq_len <= 0 || seq_len_kv <= 0) return 1;
  const int nqb = (seq_len + kRowsPerCta - 1) / kRowsPerCta;
  const int nkb = (seq_len_kv + kKvBlock - 1) / kKvBlock;
  const TailPlan tp = plan_tail(nqb, batch * heads, nkb, kSlots, enable != 0, force_split_ways);
  out4[0] = tp.prefix_wgs;
  out4[1] = tp.tail;
  out4[2] = tp.split_ways;
  out4[3] = tp.parts;
  return 0;
}

int moonmath_attention_geometry(int* out4) {
  if (!out4) return 1;
  out4[0] = kRowsPerCta;
  out4[1] = kKvBlock;
  out4[2] = kSlots;
  out4[3] = kMaxParts;
  return 0;
}

size_t moonmath_attention_vt_bytes(int batch, int heads, int seq_len_kv) {
  if (batch <= 0 || heads <= 0 || seq_len_kv <= 0) return 0;
  const size_t nkb = (size_t)(seq_len_kv + kKvBlock - 1) / kKvBlock;
  return (size_t)batch * heads * nkb * kVtBlockElems * 2;
}

int moonmath_pack_bf16(const void* in, void* out, int n, int round_mode, void* stream) {
  if (!in || !out || n < 0 || (n & 1)) return -6;
  if (round_mode < 0 || round_mode > 2) return 10;
  if (n == 0) return 0;
  const int npairs = n / 2;
  const dim3 grid((npairs + 255) / 256), block(256);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const float* src = static_cast<const float*>(in);
  uint32_t* dst = static_cast<uint32_t*>(out);
  if (round_mode == 0)
    hipLaunchKernelGGL(pack_bf16_kernel<mm::kRTNE>, grid, block, 0, s, src, dst, npairs);
  else if (round_mode == 1)
    hipLaunchKernelGGL(pack_bf16_kernel<mm::kRTNA>, grid, block, 0, s, src, dst, npairs);
  else
    hipLaunchKernelGGL(pack_bf16_kernel<mm::kRTZ>, grid, block, 0, s, src, dst, npairs);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // extern "C"
