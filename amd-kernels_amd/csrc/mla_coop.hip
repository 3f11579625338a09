// Absorbed-MLA decode for small query blocks (H * q_len <= 16, e.g. DeepSeek-V3's
// 128 heads split over 8 GPUs) on MI355X (gfx950). Same contract, split plan,
// records and numerics as mla_decode_kernel (reference csrc/mla_decode_a16w8.hip
// :183-754, csrc/mla_decode_a16w8_multiq.hip:282-856). With at most 16 query
// rows the decode is bound by HBM: besides streaming the KV, the time goes to
// per-CTA set-up and, in a kernel whose waves split the tokens, to merging the
// waves' 512-wide outputs at the end. This kernel has no such merge:
//
//  * One CTA = the <= 16 query rows of one request part, 4 waves. The part's
//    fp8 rows are gathered in 64-token tiles into a shared 4-slot LDS ring;
//    wave w gathers (9 of the 36 16-byte DMAs per tile) and scores tokens
//    16w .. 16w+15 of every tile.
//    The gathers are non-temporal: each token is read by one CTA, once
//    (44.4 -> 40.8 us per call at the bench's H=16 batch).
//  * S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (16 tokens x 16 rows; all of Q
//    lives in VGPRs). Softmax in base 2 on the integer grid: each row's max m
//    is fixed for the whole CTA at the part's first tile, p = exp2(s c - m)
//    (<= 2^64 later, else the exact-max fallback), P rounded to bf16 RTNE and
//    published in LDS as the P^T operand.
//  * O^T = V^T P^T is split by output dims: wave w accumulates latent dims
//    128w .. 128w+127 of the rows over all 64 tokens of each tile (8 d-blocks x
//    2 token k-steps), so no wave holds another wave's dims and only the rows'
//    l sums cross waves at the end.
//  * One CTA barrier per tile publishes P^T (double-buffered by tile parity) and
//    frees the ring slot that the tile three ahead is gathered into.
//  * The split plan also returns the request's length and slot offset, and the
//    first slot-index batch and Q are loaded in one round of memory latency, so
//    the first tile is requested after three dependent round trips.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "mla_common.hpp"

namespace mm {
namespace mla {

constexpr int kCRows = 16;                              // query rows per CTA (one 16-wide MFMA block)
constexpr int kCWaves = 4;
constexpr int kCThreads = 64 * kCWaves;
constexpr int kCTileTok = 64;                           // tokens per tile
constexpr int kCSubTok = kCTileTok / kCWaves;           // 16 tokens per wave and tile
constexpr int kCTileBytes = kCTileTok * kQK;            // 36864
constexpr int kCSubBytes = kCSubTok * kQK;              // 9216
constexpr int kCDmaPerSub = kCSubBytes / 1024;          // 9 wave-DMA instructions
constexpr int kCSlots = 4;                              // tile ring depth
constexpr int kCQPairs = kQK / 64;                      // 9 pairs of 32-dim k-steps

// LDS map (bytes). Ring slot 3 receives its first tile only after the first
// tile barrier; before that it holds the plan scratch (wave 0), then each
// wave's staged slot indices (9 KB per wave: 144 tiles, which bounds a segment).
constexpr int kCRingBytes = kCSlots * kCTileBytes;              // 147456
constexpr int kCScratchOff = 3 * kCTileBytes;                   // slot 3
constexpr int kCStageBytes = kCTileBytes / kCWaves;             // 9216 per wave
constexpr int kCTabTiles = kCStageBytes / (kCSubTok * 4);       // 144 tiles per segment (9216 tokens)
constexpr int kCPOff = kCRingBytes;                             // P^T of a tile: [16 rows][64 tokens] bf16
constexpr int kCPBytes = kCRows * kCTileTok * 2;                // 2048
constexpr int kCTabOff = kCPOff + 2 * kCPBytes;                 // 151552: [wave][kCTabTiles] first slots
constexpr int kCMaxOff = kCTabOff + kCWaves * kCTabTiles * 4;   // 153856: [wave][16 rows] row max
constexpr int kCLOff = kCMaxOff + kCWaves * kCRows * 4;         // 154112: [wave][16 rows] row l
constexpr int kCMiscOff = kCLOff + kCWaves * kCRows * 4;        // 154368: unit broadcast, fallback flags
constexpr int kCLdsBytes = kCMiscOff + 64;                      // 154432
static_assert(12 * kMaxPagedB <= kCTileBytes, "plan scratch fits ring slot 3");
static_assert(kCLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kCSubBytes % 1024 == 0, "a wave's share of a tile is whole DMA instructions");

template <bool PAGED>
__global__ __launch_bounds__(kCThreads, 1) void mla_coop_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) char lds[kCLdsBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15;  // MFMA column (query row); row of A (token for QK, dim for PV)
  const int G = lane >> 4;  // 16-lane group: k-slice of the operands, 4-row slice of the result
  char* stg = lds + kCScratchOff + wave * kCStageBytes;  // this wave's staged slot indices
  int* tab = reinterpret_cast<int*>(lds + kCTabOff) + wave * kCTabTiles;
  float* red_m = reinterpret_cast<float*>(lds + kCMaxOff);
  float* red_l = reinterpret_cast<float*>(lds + kCLOff);
  int* misc = reinterpret_cast<int*>(lds + kCMiscOff);

  // ---- work item: unit u dealt over the XCDs in snake order (as the 32-row kernel) -------
  const int xcd = blockIdx.x % kNumXcds;
  const int uslot = blockIdx.x / kNumXcds;
  const int u = 16 * (uslot >> 1) + ((uslot & 1) ? 15 - xcd : xcd);
  Unit un;
  if constexpr (PAGED) {
    // Wave 0 plans in ring slot 3 and broadcasts the unit.
    if (wave == 0) {
      const Unit w0 =
          plan_unit_paged(p.seq_lens, p.kv_indptr, p.B, p.parts, p.unit_cap, u, lane,
                          reinterpret_cast<int*>(lds + kCScratchOff));
      if (lane == 0) {
        misc[0] = w0.b;
        misc[1] = w0.part;
        misc[2] = w0.nparts;
        misc[3] = w0.rec0;
        misc[4] = w0.ptok;
        misc[5] = w0.units;
        misc[6] = w0.len;
        misc[7] = w0.slot0;
      }
    }
    lds_reads_done_barrier();
    un = Unit{__builtin_amdgcn_readfirstlane(misc[0]), __builtin_amdgcn_readfirstlane(misc[1]),
              __builtin_amdgcn_readfirstlane(misc[2]), __builtin_amdgcn_readfirstlane(misc[3]),
              __builtin_amdgcn_readfirstlane(misc[4]), __builtin_amdgcn_readfirstlane(misc[5]),
              __builtin_amdgcn_readfirstlane(misc[6]), __builtin_amdgcn_readfirstlane(misc[7])};
  } else {
    un = plan_unit_contig(p.S_fixed, p.B, p.parts, p.unit_cap, u);
  }
  if (u >= un.units) return;  // padding CTA: every wave leaves together
  const int b = un.b;
  const int part = un.part;
  int qb = b;
  if (p.rows) {
    qb = p.rows[b];
    qb = qb < 0 ? 0 : (qb >= p.B ? p.B - 1 : qb);
  }
  const int S = un.len;
  const int slot0 = un.slot0;
  const long long lo64 = (long long)part * un.ptok;
  const int kv_lo = lo64 < S ? (int)lo64 : S;
  const int kv_hi = (lo64 + un.ptok < S) ? (int)(lo64 + un.ptok) : S;

  // ---- the query row of this lane's MFMA column -------------------------------------
  const bool row_ok = i < p.qrows;
  const int qr = row_ok ? i : p.qrows - 1;  // padding columns repeat the last row
  const int t_pos = qr / p.H;
  const int lim = S - (p.q_len - 1 - t_pos);  // tokens >= lim are masked for this row
  const long long qoff = (long long)qb * p.qrows + qr;

  auto seg_end = [&](int seg_lo) {
    const long long e = (long long)seg_lo + kCTabTiles * kCTileTok;
    return e < kv_hi ? (int)e : kv_hi;
  };
  auto ntiles_of = [&](int seg_lo, int seg_hi) { return (seg_hi - seg_lo + kCTileTok - 1) / kCTileTok; };
  // Slot indices of this wave's 16 tokens of every tile of a segment, into its
  // staging area: one 4-byte DMA per 4 tiles (lane (G, i): tile 4q + G, token
  // i), 256 B per DMA. Tokens past the segment re-read its last index.
  auto stage = [&](int seg_lo, int seg_hi, int ntiles) {
    for (int q = 0; q < (ntiles + 3) / 4; ++q) {
      int tok = seg_lo + kCTileTok * (4 * q + G) + kCSubTok * wave + i;
      tok = tok < seg_hi ? tok : seg_hi - 1;
      dma4_opaque(p.kv_indices + slot0 + tok, stg + 256 * q);
    }
  };
  bool prestaged = false;
  if constexpr (PAGED) {
    if (kv_lo < kv_hi) {
      const int seg_hi = seg_end(kv_lo);
      stage(kv_lo, seg_hi, ntiles_of(kv_lo, seg_hi));
      prestaged = true;
    }
  }
  // Q, as the B operand of S^T = K Q^T: k-step pair s covers dims 64s .. 64s+63;
  // lane group G holds dims 64s + 16G .. +16 of its row, the first 8 for k-step
  // 2s and the next 8 for k-step 2s+1 (the K fragment holds the same dims).
  // Pair 8 is the rope part (q_pe).
  bf16x8 qf[2 * kCQPairs];
#pragma unroll
  for (int s = 0; s < kCQPairs; ++s) {
    const uint16_t* src = (s < kCQPairs - 1) ? p.q_lat + qoff * kLat + 64 * s + 16 * G : p.q_pe + qoff * kRope + 16 * G;
    qf[2 * s] = *reinterpret_cast<const bf16x8*>(src);
    qf[2 * s + 1] = *reinterpret_cast<const bf16x8*>(src + 8);
  }
  // Staged indices and Q in one round of latency; visible to the compiler, so
  // it adds no wait of its own for Q later (when tile gathers are in flight).
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); expcnt and lgkmcnt untouched

  // ---- per-lane constant offsets inside a staged tile --------------------------------
  // Staging layout (as the 32-row kernel): token t's 576-byte row at t*576, its
  // 16-byte piece c at piece slot c ^ swz(t).
  // K read of pair s: token 16w + i, piece 4s + G -> slot 4s + (G ^ swz(i)).
  const int koff = (kCSubTok * wave + i) * kQK + 16 * (G ^ swz(i));
  // V^T transpose read of d-block j (dims 128w + 16j ..), k-step kk (tokens
  // 32kk ..): in 16-lane group G, member i supplies 8 bytes of token
  // 32kk + 8G + i/2, dims 128w + 16j + 8(i&1) .. +8, so output lane i gets dim
  // 128w + 16j + i of tokens 32kk + 8G .. +8 (the A operand's k-slice G).
  // swz(token) = (2G + i/8) & 3 for every kk; piece 8w + j sits at slot
  // 8w + (j ^ swz) for j < 4 and 64 bytes further for j >= 4.
  const int vsw = (2 * G + (i >> 3)) & 3;
  const int vrow = (8 * G + (i >> 1)) * kQK + 8 * (i & 1) + 128 * wave;
  int voff[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) voff[jj] = vrow + 16 * (jj ^ vsw);
  // P^T of a tile: row r's 64 tokens as 8 units of 8 tokens (16 B), unit v of
  // row r at slot v ^ ((r >> 1) & 7) (the 16 lanes of a write or read hit
  // distinct banks). Write: this lane's 4 scores, tokens 16w + 4G .. +4 of row
  // i = half G&1 of unit 2w + G/2. Read (k-step kk): tokens 32kk + 8G .. +8 of
  // row i = unit 4kk + G.
  const int psw = (i >> 1) & 7;
  const int pw_off = i * (kCTileTok * 2) + 16 * ((2 * wave + (G >> 1)) ^ psw) + 8 * (G & 1);
  const int pr_off0 = i * (kCTileTok * 2) + 16 * (G ^ psw);
  const int pr_off1 = i * (kCTileTok * 2) + 16 * ((4 + G) ^ psw);
  // DMA: instruction k of this wave's share moves LDS pieces 64k .. 64k+63 of
  // its 16-row sub-tile (36 pieces per row): lane l fills piece slot
  // pc = 64k + l, i.e. token tg = pc / 36, slot cs = pc % 36, with global piece
  // cs ^ swz(tg). Offsets < 2^14, two per VGPR.
  uint32_t dma_pk[5];
#pragma unroll
  for (int k = 0; k < kCDmaPerSub; ++k) {
    const int pc = 64 * k + lane;
    const int tg = pc / 36, cs = pc % 36;
    const uint32_t off = tg * kQK + 16 * (cs ^ swz(tg));
    dma_pk[k / 2] = (k & 1) ? (dma_pk[k / 2] | (off << 16)) : off;
  }
  auto dma_off = [&](int k) -> int { return (int)((dma_pk[k / 2] >> (16 * (k & 1))) & 0xFFFFu); };
  auto dma_offv = [&](int k) { return u16_field(dma_pk[k / 2], k & 1); };

  f32x4 oacc[8];  // O^T, d-block j: lane (G, i) element e = dim 128w + 16j + 4G + e of row i
#pragma unroll
  for (int j = 0; j < 8; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float row_m = -__builtin_inff();  // CTA-wide max of row i (integer grid) once fixed
  float row_l = 0.f;                // this lane's share of row i's sum
  bool m_fixed = false;
  bool grew = false;                // a later tile exceeded row_m by more than kGrowLimit
  bool ring_used = false;           // a segment has run (the next one starts with a barrier)
  const float c = p.score_c;

  // One pass over the part. Accumulate mode: softmax + PV with each row's max
  // fixed at the part's first tile (or before the pass). Max-only mode: QK and
  // this lane's largest masked score (row_m).
  auto sweep = [&](auto max_only_tag) {
    constexpr bool kMaxOnly = decltype(max_only_tag)::value;
    for (int seg_lo = kv_lo; seg_lo < kv_hi; seg_lo += kCTabTiles * kCTileTok) {
      const int seg_hi = seg_end(seg_lo);
      const int ntiles = ntiles_of(seg_lo, seg_hi);
      // A later segment or pass: every wave is done with the ring and its
      // staging area. (The first segment of the first pass needs no barrier:
      // each wave gathers only its own sub-tiles, from its own table, into ring
      // slots 0..2, and slot 3 -- plan scratch, staging -- takes its first tile
      // only after the first tile barrier.)
      if (ring_used) lds_reads_done_barrier();
      ring_used = true;
      if constexpr (PAGED) {
        if (!prestaged) {
          stage(seg_lo, seg_hi, ntiles);
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        prestaged = false;
      }
      // Tile table of this wave: tab[j] = slot of the first of its 16 tokens of
      // tile j when its valid tokens occupy consecutive slots, else -1. Built in
      // batches of up to 8 staged dwords (4 tiles each), read before any table
      // write so their LDS latencies overlap; the first batch covers the first
      // gathers, the rest is built while they are in flight.
      const int nq = (ntiles + 3) / 4;
      auto build_tab = [&](int qa, int qb_end, auto batch_tag) {
        constexpr int kB = decltype(batch_tag)::value;
        for (int q0 = qa; q0 < qb_end; q0 += kB) {
          int vv[kB];
#pragma unroll
          for (int k = 0; k < kB; ++k)
            vv[k] = (q0 + k < qb_end) ? *reinterpret_cast<const int*>(stg + 256 * (q0 + k) + 4 * lane) : 0;
#pragma unroll
          for (int k = 0; k < kB; ++k) {
            if (q0 + k < qb_end) {
              const int v = vv[k];
              const int j = 4 * (q0 + k) + G;
              const int f0 = __builtin_amdgcn_readlane(v, 0), f1 = __builtin_amdgcn_readlane(v, 16);
              const int f2 = __builtin_amdgcn_readlane(v, 32), f3 = __builtin_amdgcn_readlane(v, 48);
              const int first = G == 0 ? f0 : (G == 1 ? f1 : (G == 2 ? f2 : f3));
              const int tok = seg_lo + kCTileTok * j + kCSubTok * wave + i;
              const unsigned long long bal = __builtin_amdgcn_ballot_w64(tok >= seg_hi || v == first + i);
              const bool contiguous = ((bal >> (16 * G)) & 0xFFFFull) == 0xFFFFull;
              if (i == 0 && j < ntiles) tab[j] = contiguous ? first : -1;
            }
          }
        }
      };
      if constexpr (PAGED) build_tab(0, 1, std::integral_constant<int, 1>{});  // tiles 0..3
      const int eff = lim < seg_hi ? lim : seg_hi;  // this row's token limit in the segment

      // This wave's share of the gather of tile j into ring slot j % 4. Fast
      // path: the 16 rows are consecutive slots (one SGPR base + lane offsets);
      // with `defer` its 9 DMAs are left pending (pend_base, pend_dst) and go out
      // one per step of the next body. Partial: rows past the valid ones re-read
      // the last valid row. Slow path: every lane looks its row up.
      const uint8_t* pend_base = nullptr;
      const char* pend_dst = nullptr;
      auto issue_tile = [&](int j, int tabv, bool defer) -> bool {
        const char* dst = lds + (j & (kCSlots - 1)) * kCTileBytes + wave * kCSubBytes;
        const int tok0 = seg_lo + j * kCTileTok + kCSubTok * wave;
        const int nvalid = seg_hi - tok0;  // <= 0: every row re-reads the segment's last token
        const uint8_t* base;
        bool fast = true;
        if constexpr (PAGED) {
          const int s0 = __builtin_amdgcn_readfirstlane(tabv);
          base = p.kv + (long long)s0 * kQK;
          fast = s0 >= 0;
        } else {
          base = p.kv + ((long long)b * p.S_fixed + (nvalid > 0 ? tok0 : seg_hi - 1)) * kQK;
        }
        if (fast && nvalid >= kCSubTok) {
          if (defer) {
            pend_base = base;
            pend_dst = dst;
            return true;
          }
#pragma unroll
          for (int k = 0; k < kCDmaPerSub; ++k) dma16_sbase_nt(base, dma_offv(k), dst + 1024 * k);
        } else if (fast) {
          const int nv = nvalid > 0 ? nvalid : 1;
#pragma unroll 1
          for (int k = 0; k < kCDmaPerSub; ++k) {
            const int o = dma_off(k);
            const int tg = (o * 7282) >> 22;  // o / 576 for o < 9216
            const int t = tg < nv ? tg : nv - 1;
            dma16_opaque_nt(base + t * kQK + (o - tg * kQK), dst + 1024 * k);
          }
        } else {
          int tk = tok0 + i;
          tk = tk < seg_hi ? tk : seg_hi - 1;
          const int myrow = p.kv_indices[slot0 + tk];  // lanes (G, i): slot of token tok0 + i
#pragma unroll 1
          for (int k = 0; k < kCDmaPerSub; ++k) {
            const int o = dma_off(k);
            const int tg = (o * 7282) >> 22;
            const int row = __shfl(myrow, tg);
            dma16_opaque_nt(p.kv + (long long)row * kQK + (o - tg * kQK), dst + 1024 * k);
          }
        }
        return false;
      };
      // DMA k of a deferred gather, skipped inside the asm when nothing is
      // pending (no branch for the compiler to split the step sequence at).
      auto dma_if = [&](int pending, int k) {
        const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)(pend_dst + 1024 * k);
        const int pu = __builtin_amdgcn_readfirstlane(pending);
        asm volatile("s_cmp_eq_u32 %3, 0\n\ts_cbranch_scc1 1f\n\tglobal_load_lds_dwordx4 %0, %1 nt\n1:" ::"v"(dma_offv(k)),
                     "s"(pend_base), "{m0}"(m0v), "s"(pu)
                     : "memory", "scc");
      };
      auto tab_at = [&](int j) -> int {
        if constexpr (PAGED) {
          return tab[j];
        } else {
          return 0;
        }
      };

      // Software pipeline over the tiles. body(t) waits for this wave's share
      // of tile t and computes its S^T; interleaved with those 18 MFMAs run the
      // 16 PV MFMAs of tile t-1 (whose P^T every wave published before the last
      // barrier) and the 9 deferred DMAs of tile t+2. finish(t) does the
      // softmax, publishes P^T(t), passes the tile barrier and schedules the
      // gather of tile t+3 into the slot of tile t-1. Wait rule: every DMA of
      // tile t+1 was issued before body(t), so vmcnt(9) (tile t+2 in flight, or
      // fewer) always retires tile t's share.
      auto body = [&](int t, int pending, int vm_left, auto with_pv) -> f32x4 {
        constexpr bool kPV = decltype(with_pv)::value;
        const char* sk = lds + (t & (kCSlots - 1)) * kCTileBytes + koff;  // K: tile t, this wave's tokens
        const char* sv = lds + ((t - 1) & (kCSlots - 1)) * kCTileBytes;    // V: tile t-1
        const char* pb = lds + kCPOff + ((t - 1) & 1) * kCPBytes;           // P^T of tile t-1
        bf16x8 pop[2];
        i32x2 vr[16];  // V^T fragment m: k-step m / 8, d-block m % 8
        if constexpr (kPV) {
          pop[0] = *reinterpret_cast<const bf16x8*>(pb + pr_off0);
          pop[1] = *reinterpret_cast<const bf16x8*>(pb + pr_off1);
#pragma unroll
          for (int m = 0; m < 16; ++m) {
            const int j = m & 7, kk = m >> 3;
            vr[m] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                (MM_LDS i32x2*)(sv + voff[j & 3] + 64 * (j >> 2) + kk * 32 * kQK));
          }
        }
        if (vm_left == 18) {
          asm volatile("s_waitcnt vmcnt(18)" ::: "memory");
        } else if (vm_left == 9) {
          asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        u32x4 kr[kCQPairs];
#pragma unroll
        for (int s = 0; s < kCQPairs; ++s) kr[s] = *reinterpret_cast<const u32x4*>(sk + 64 * s);
        f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kCQPairs; ++s) {
          dma_if(pending, s);
          if constexpr (kPV) {
            if (s < 8) {
              const int m = 2 * s;
              oacc[m & 7] = mfma16(fp8x8_bf16((uint32_t)vr[m][0], (uint32_t)vr[m][1]), pop[m >> 3], oacc[m & 7]);
            }
          }
          a0 = mfma16(fp8x8_bf16(kr[s][0], kr[s][1]), qf[2 * s], a0);
          if constexpr (kPV) {
            if (s < 8) {
              const int m = 2 * s + 1;
              oacc[m & 7] = mfma16(fp8x8_bf16((uint32_t)vr[m][0], (uint32_t)vr[m][1]), pop[m >> 3], oacc[m & 7]);
            }
          }
          a1 = mfma16(fp8x8_bf16(kr[s][2], kr[s][3]), qf[2 * s + 1], a1);
          sched_fence();
        }
        return a0 + a1;
      };
      // The 16 PV MFMAs of the last tile on their own.
      auto pv_last = [&](int t) {
        const char* sv = lds + (t & (kCSlots - 1)) * kCTileBytes;
        const char* pb = lds + kCPOff + (t & 1) * kCPBytes;
        const bf16x8 pop0 = *reinterpret_cast<const bf16x8*>(pb + pr_off0);
        const bf16x8 pop1 = *reinterpret_cast<const bf16x8*>(pb + pr_off1);
        i32x2 vr[16];
#pragma unroll
        for (int m = 0; m < 16; ++m) {
          const int j = m & 7, kk = m >> 3;
          vr[m] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MM_LDS i32x2*)(sv + voff[j & 3] + 64 * (j >> 2) + kk * 32 * kQK));
        }
#pragma unroll
        for (int m = 0; m < 16; ++m)
          oacc[m & 7] = mfma16(fp8x8_bf16((uint32_t)vr[m][0], (uint32_t)vr[m][1]), m < 8 ? pop0 : pop1, oacc[m & 7]);
      };

      bool pend = false;  // a deferred gather waits for the next body
      auto finish = [&](int t, const f32x4 sacc, int tab_next) {
        // Lane (G, i), element e: token seg_lo + 64t + 16w + 4G + e of row i.
        const int rel = eff - (seg_lo + t * kCTileTok + kCSubTok * wave + 4 * G);  // e valid iff e < rel
        float sv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) sv[e] = (e < rel) ? sacc[e] : -__builtin_inff();
        const float bm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        if constexpr (kMaxOnly) {
          row_m = fmaxf(row_m, bm);
        } else {
          if (!m_fixed) {
            // The part's first tile fixes each row's max for the whole CTA.
            float wm = fmaxf(bm, __shfl_xor(bm, 16));
            wm = fmaxf(wm, __shfl_xor(wm, 32));
            if (G == 0) red_m[wave * kCRows + i] = wm;
            lds_reads_done_barrier();
            const float M = fmaxf(fmaxf(red_m[i], red_m[kCRows + i]), fmaxf(red_m[2 * kCRows + i], red_m[3 * kCRows + i]));
            row_m = (M == -__builtin_inff()) ? M : __builtin_ceilf(M * c);
            m_fixed = true;
          } else {
            grew = grew || (__builtin_ceilf(bm * c) > row_m + kGrowLimit);
          }
          const float neg_m = (row_m == -__builtin_inff()) ? 0.f : -row_m;
          float pe[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) pe[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[e], c, neg_m));
          row_l += (pe[0] + pe[1]) + (pe[2] + pe[3]);
          const u32x2 w2 = {pack2_bf16<kRTNE>(pe[0], pe[1]), pack2_bf16<kRTNE>(pe[2], pe[3])};
          *reinterpret_cast<u32x2*>(lds + kCPOff + (t & 1) * kCPBytes + pw_off) = w2;
        }

        // ---- tile barrier: P^T(t) published, every wave's share of tile t landed,
        // every wave done with tile t-1 (its slot takes tile t+3) ----
        lds_reads_done_barrier();
        pend = (t + 3 < ntiles) ? issue_tile(t + 3, tab_next, true) : false;
      };

      // Tiles 0 and 1 now; a fast-path tile 2 goes out one DMA per step of
      // body(0) (108 back-to-back DMAs per CU stall the issuing waves for ~1 us).
      issue_tile(0, tab_at(0), false);
      if (ntiles > 1) issue_tile(1, tab_at(1), false);
      const bool pend0 = (ntiles > 2) ? issue_tile(2, tab_at(2), true) : false;
      if constexpr (PAGED) build_tab(1, nq, std::integral_constant<int, 8>{});
      // Tile 0 has no PV before it (peeled, so the accumulators stay put in the loop).
      finish(0, body(0, pend0, ntiles > 1 ? 9 : 0, std::false_type{}), ntiles > 3 ? tab_at(3) : 0);
      for (int t = 1; t < ntiles; ++t) {
        const int tab_next = (t + 3 < ntiles) ? tab_at(t + 3) : 0;
        const int pd = pend;
        const int vm_left = t + 1 < ntiles ? 9 : 0;
        if constexpr (kMaxOnly) {
          finish(t, body(t, pd, vm_left, std::false_type{}), tab_next);
        } else {
          finish(t, body(t, pd, vm_left, std::true_type{}), tab_next);
        }
      }
      if constexpr (!kMaxOnly) pv_last(ntiles - 1);
    }
  };

  // Each wave posts its rows' l sums and its fallback flag, then one barrier.
  auto post_l = [&]() {
    float l = row_l;
    l += __shfl_xor(l, 16);  // the four lanes of a row end with the same sum
    l += __shfl_xor(l, 32);
    if (G == 0) red_l[wave * kCRows + i] = l;
    const bool any = __builtin_amdgcn_ballot_w64(grew) != 0;
    if (lane == 0) misc[wave] = any;
    lds_reads_done_barrier_vm0();
  };
  sweep(std::false_type{});
  post_l();
  // Fallback (only when some row's scores rise more than 2^64 above the part's
  // first tile): redo the part with the exact row max. CTA-uniform: the flags
  // are read after a barrier.
  if ((misc[0] | misc[1] | misc[2] | misc[3]) != 0) {
    asm volatile("s_barrier" ::: "memory");  // every wave has read the flags
    row_m = -__builtin_inff();
    sweep(std::true_type{});
    float wm = fmaxf(row_m, __shfl_xor(row_m, 16));
    wm = fmaxf(wm, __shfl_xor(wm, 32));
    if (G == 0) red_m[wave * kCRows + i] = wm;
    lds_reads_done_barrier();
    const float M = fmaxf(fmaxf(red_m[i], red_m[kCRows + i]), fmaxf(red_m[2 * kCRows + i], red_m[3 * kCRows + i]));
    row_m = (M == -__builtin_inff()) ? M : __builtin_ceilf(M * c);
    m_fixed = true;
    row_l = 0.f;
    grew = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    sweep(std::false_type{});
    post_l();
  }

  // ---- epilogue: this wave's 128 dims of the rows ------------------------------------
  // Branch-free stores through buffer resources that span exactly the valid
  // query rows: lanes of padding rows fall outside and their stores are dropped.
  const float L = (red_l[i] + red_l[kCRows + i]) + (red_l[2 * kCRows + i] + red_l[3 * kCRows + i]);
  const bool split = un.nparts > 1;
  const size_t rec0 = (size_t)un.rec0 + part;
  constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer access, gfx9 family
  if (split) {
    // Unnormalised fp32 O of this part: record rec0 * qrows + row.
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(ws_rec_o(p, rec0), (short)0, p.qrows * kLat * 4, kRsrcWord3);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u32x4 v = __builtin_bit_cast(u32x4, oacc[j]);
      __builtin_amdgcn_raw_buffer_store_b128(v, rs, (i * kLat + 128 * wave + 16 * j + 4 * G) * 4, 0, 0);
    }
    if (row_ok && G == 0 && wave == 0) {
      float* pml = ws_ml(p) + (rec0 * p.qrows + i) * 2;
      pml[0] = row_m;
      pml[1] = L;
    }
  } else {
    const float inv = (L == 0.f) ? 0.f : p.kv_scale * __builtin_amdgcn_rcpf(L);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        p.o_lat + (long long)qb * p.qrows * kLat, (short)0, p.qrows * kLat * 2, kRsrcWord3);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x2 o;
      o[0] = pack2_bf16_canon<kRTNE>(oacc[j][0] * inv, oacc[j][1] * inv);
      o[1] = pack2_bf16_canon<kRTNE>(oacc[j][2] * inv, oacc[j][3] * inv);
      __builtin_amdgcn_raw_buffer_store_b64(o, rs, (i * kLat + 128 * wave + 16 * j + 4 * G) * 2, 0, 0);
    }
  }
  if (p.parts > 1 && part == 0 && tid == 0) {
    // Per-request (parts, first record) table for the merge kernel.
    int* tbl = ws_tbl(p);
    tbl[2 * b] = un.nparts;
    tbl[2 * b + 1] = un.rec0;
  }
}

int launch_coop_kernel(const Params& p, long long grid, hipStream_t st) {
  if (p.paged)
    hipLaunchKernelGGL(mla_coop_kernel<true>, dim3((unsigned)grid), dim3(kCThreads), 0, st, p);
  else
    hipLaunchKernelGGL(mla_coop_kernel<false>, dim3((unsigned)grid), dim3(kCThreads), 0, st, p);
  return 0;
}

}  // namespace mla
}  // namespace mm
