// Absorbed-MLA decode for wide query blocks (H * q_len >= 96, e.g. the
// DeepSeek-V3 shape H = 128) on MI355X (gfx950). Same contract, split plan,
// records and numerics as mla_decode_kernel (reference csrc/mla_decode_a16w8.hip
// :183-754, csrc/mla_decode_a16w8_multiq.hip:282-856); the work is cut
// differently:
//
//  * One CTA = 128 query rows (4 row tiles of 32) of one request part. The
//    part's fp8 tiles are gathered once per CTA into a shared 4-slot LDS ring
//    (each wave issues a quarter of every tile's 16-byte DMAs), not once per
//    32 rows.
//  * QK and softmax are split by rows: wave w computes S^T = K Q^T for row tile
//    w (K widened from the fp8 tile exactly as in the 32-row kernel) and
//    publishes its bf16 P^T operands in LDS.
//  * PV is split by output dims: wave w accumulates O^T for latent dims
//    128w .. 128w+127 of all 128 rows (4 d-tiles x 4 row tiles = 256 AGPRs),
//    reading every row tile's P^T from LDS. Each V^T fragment is widened once
//    and feeds four MFMAs, and no wave ever holds another wave's output dims,
//    so there is no O merge at the end: only the rows' (m, l) cross waves.
//  * One CTA barrier per tile publishes P^T, retires the next tile's DMAs and
//    frees the ring slot three tiles ahead; P^T is double-buffered by tile
//    parity so one barrier suffices.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "mla_common.hpp"

namespace mm {
namespace mla {

constexpr int kWRows = 128;                      // query rows per CTA
constexpr int kWWaves = 4;
constexpr int kWThreads = 64 * kWWaves;
constexpr int kWSlots = 4;                       // tile ring depth
constexpr int kWTabTiles = 2048;                 // tile-table entries (one segment = 64K tokens)
constexpr int kWStageTiles = 64;                 // tiles whose slot indices one wave stages per round

// LDS map (bytes).
constexpr int kWRingBytes = kWSlots * kTileBytes;                     // 73728
constexpr int kWQOff = kWRingBytes;                                   // Q dims [448, 576): [wave][32 rows][256 B]
constexpr int kWPOff = kWQOff + kWRows * kQLdsRowBytes;               // 106496
constexpr int kWPBytes = kWWaves * 2 * 1024;                          // P^T of one tile: [row tile][k-step][lane] x 16 B
constexpr int kWTabOff = kWPOff + 2 * kWPBytes;                       // 122880
constexpr int kWMlOff = kWTabOff + 4 * kWTabTiles;                    // 131072: (m, l) of the 128 rows
constexpr int kWMiscOff = kWMlOff + kWRows * 8;                       // 132096: unit broadcast, fallback flags
constexpr int kWLdsBytes = kWMiscOff + 64;                            // 132160
static_assert(12 * kMaxPagedB <= kWRingBytes, "plan scratch fits the ring");
static_assert(kWWaves * kWStageTiles * 128 <= kWRingBytes, "index staging fits the ring");
static_assert(kWLdsBytes <= 160 * 1024, "LDS budget");

template <bool PAGED>
__global__ __launch_bounds__(kWThreads, 1) void mla_wide_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) char lds[kWLdsBytes];
  char* ring = lds;
  int* tab = reinterpret_cast<int*>(lds + kWTabOff);
  float* mlb = reinterpret_cast<float*>(lds + kWMlOff);
  int* misc = reinterpret_cast<int*>(lds + kWMiscOff);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31;  // MFMA column: query row (S^T, O^T) / token or dim row of A
  const int g = lane >> 5;  // lane half
  char* qlds = lds + kWQOff + wave * (32 * kQLdsRowBytes);  // this wave's LDS-resident Q dims

  // ---- work item: unit (request part) x 128-row block, dealt as in the 32-row kernel ----
  const int xcd = blockIdx.x % kNumXcds;
  const int k_in_xcd = blockIdx.x / kNumXcds;
  const int uslot = k_in_xcd / p.ngroups;
  const int rb = k_in_xcd % p.ngroups;
  const int u = 16 * (uslot >> 1) + ((uslot & 1) ? 15 - xcd : xcd);
  Unit un;
  if constexpr (PAGED) {
    if (wave == 0) {
      const Unit w0 =
          plan_unit_paged(p.seq_lens, p.kv_indptr, p.B, p.parts, p.unit_cap, u, lane, reinterpret_cast<int*>(ring));
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

  // ---- this wave's query rows (row tile `wave` of the block) --------------------------
  const int qrow = rb * kWRows + 32 * wave + n;
  const bool row_ok = qrow < p.qrows;
  const int qr = row_ok ? qrow : p.qrows - 1;
  const int t_pos = qr / p.H;
  const int lim = S - (p.q_len - 1 - t_pos);  // tokens >= lim are masked for this row
  const long long qoff = (long long)qb * p.qrows + qr;

  // Slot indices of the first staging round of the first segment (paged), then
  // Q: the first table build waits only for the staged indices (older in the
  // in-order vmcnt), while Q, the table build and the first tiles' gathers
  // overlap. Staging layout: see the table build in sweep().
  char* stg = ring + wave * (kWStageTiles * 128);
  // Tile pairs this wave stages in the round of 256 tiles from r0: pairs
  // wave, wave + 4, ... (pair q of the wave = tiles r0 + 8q + 2 wave + {0, 1}).
  auto stage_pairs = [&](int ntiles, int r0) {
    const int np = (ntiles - r0 - 2 * wave + 7) / 8;
    return np < 0 ? 0 : (np > kWStageTiles / 2 ? kWStageTiles / 2 : np);
  };
  auto stage_round = [&](int seg_lo, int seg_hi, int ntiles, int r0) {
    const int np = stage_pairs(ntiles, r0);
    for (int q = 0; q < np; ++q) {
      int tok = seg_lo + kTileTok * (r0 + 8 * q + 2 * wave + g) + n;
      tok = tok < seg_hi ? tok : seg_hi - 1;
      dma4_opaque(p.kv_indices + slot0 + tok, stg + 256 * q);
    }
    return np;
  };
  auto seg_end = [&](int seg_lo) {
    return (long long)seg_lo + kWTabTiles * kTileTok < kv_hi ? seg_lo + kWTabTiles * kTileTok : kv_hi;
  };
  bool prestaged = false;
  if constexpr (PAGED) {
    if (kv_lo < kv_hi) {
      const int seg_hi = seg_end(kv_lo);
      stage_round(kv_lo, seg_hi, (seg_hi - kv_lo + kTileTok - 1) / kTileTok, 0);
      prestaged = true;
    }
  }
  bf16x8 qf[2 * kQRegPairs];
#pragma unroll
  for (int s = 0; s < kQRegPairs; ++s) {
    const uint16_t* src = p.q_lat + qoff * kLat + s * 32 + g * 16;
    qf[2 * s] = *reinterpret_cast<const bf16x8*>(src);
    qf[2 * s + 1] = *reinterpret_cast<const bf16x8*>(src + 8);
  }
  // Q dims [448, 576) of the wave's 32 rows, 16 chunks of 8 bf16 per row
  // (chunks 0..7 from q_lat, 8..15 = q_pe), chunk c of row r stored at slot
  // c ^ (r & 15): DMA'd straight into LDS, lane l filling slot (64 it + l) % 16
  // of row (64 it + l) / 16.
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int id = lane + 64 * it;
    const int r = id >> 4, c = (id & 15) ^ (r & 15);
    const int rr = rb * kWRows + 32 * wave + r;
    const long long ro = (long long)qb * p.qrows + (rr < p.qrows ? rr : p.qrows - 1);
    const uint16_t* src = (c < 8) ? p.q_lat + ro * kLat + kQLdsDim0 + c * 8 : p.q_pe + ro * kRope + (c - 8) * 8;
    dma16_opaque(src, qlds + 1024 * it);
  }
  constexpr int kQLoads = 2 * kQRegPairs + 8;  // vector memory ops per wave above

  // ---- per-lane constant offsets inside a staged tile (same layout as the 32-row kernel) ----
  const int koff0 = n * kQK + 16 * (g ^ swz(n));
  const int koff1 = n * kQK + 16 * ((2 + g) ^ swz(n));
  const int vj = lane & 15, vmh = (lane >> 4) & 1, ve = vj >> 1;
  const int vT = 8 * (ve >> 2) + 4 * g + (ve & 3);
  const int vsw = 2 * (ve >> 2) + g;
  const int voff0 = vT * kQK + 16 * (vmh ^ vsw) + 8 * (vj & 1);
  const int voff1 = vT * kQK + 16 * ((2 + vmh) ^ vsw) + 8 * (vj & 1);
  // This wave's DMAs of a tile: instructions k = wave + 4i (5, 5, 4, 4 of the
  // 18). Instruction k moves LDS pieces 64k .. 64k+63 (36 pieces per token
  // row); doff[i] = the byte offset, inside the tile's 32 consecutive rows, of
  // the piece this lane fills (token 16(k/9) + tg, piece cs at slot cs ^ swz).
  const bool five = wave < kDmaPerTile - 4 * 4;  // waves 0 and 1 own a fifth DMA
  uint32_t doff[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    int k = wave + 4 * i;
    k = k < kDmaPerTile ? k : kDmaPerTile - 1;
    const int pc = 64 * (k % 9) + lane;
    const int tg = pc / 36, cs = pc % 36;
    doff[i] = (uint32_t)((k / 9) * 16 * kQK + tg * kQK + 16 * (cs ^ swz(tg)));
  }
  auto dma_dst = [&](const char* slot, int i) { return slot + 1024 * (wave + 4 * i); };

  // O accumulators, [d-tile j of this wave][row tile], zeroed by an MFMA of zero
  // operands so that every definition of them is an AGPR write: a constant
  // zero-fill would let the register allocator stage them through VGPRs where
  // the fallback path merges back (and spill).
  // The s_nop covers the VALU write of the zero operand before the MFMA reads
  // it (a hazard the compiler cannot see through the asm).
  f32x16 oacc[16];
  auto zero_o = [&]() {
    const bf16x8 z = {};
#pragma unroll
    for (int i = 0; i < 16; ++i)
      asm volatile("s_nop 4\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=&a"(oacc[i]) : "v"(z));
  };
  zero_o();
  float row_m = -__builtin_inff(), row_l = 0.f;
  bool grew = false;
  const float c = p.score_c;

  auto sweep = [&](auto max_only_tag) {
    constexpr bool kMaxOnly = decltype(max_only_tag)::value;
    for (int seg_lo = kv_lo; seg_lo < kv_hi; seg_lo += kWTabTiles * kTileTok) {
      const int seg_hi = seg_end(seg_lo);
      const int ntiles = (seg_hi - seg_lo + kTileTok - 1) / kTileTok;
      // Every wave is done with the ring and the table (a segment's last
      // barrier already retired all of its tile DMAs).
      lds_reads_done_barrier();
      if constexpr (PAGED) {
        // Tile table: tab[j] = slot of tile j's first token when its valid
        // tokens occupy consecutive slots (one base + lane offsets), else -1.
        // Each wave stages the slot indices of every fourth tile pair of a
        // round of 256 tiles in its own 8 KB of the ring (two tiles per 4-byte
        // DMA) and builds their entries, so the 4 waves share the build.
        for (int r0 = 0; r0 < ntiles; r0 += kWWaves * kWStageTiles) {
          int np;
          if (prestaged) {
            // First round of the first segment, staged before the Q loads:
            // wait for it only.
            np = stage_pairs(ntiles, 0);
            static_assert(kQLoads == 36, "the vmcnt below counts the Q loads");
            asm volatile("s_waitcnt vmcnt(36)" ::: "memory");
            prestaged = false;
          } else {
            np = stage_round(seg_lo, seg_hi, ntiles, r0);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          }
          for (int q = 0; q < np; ++q) {
            const int j = r0 + 8 * q + 2 * wave + g;
            const int v = *reinterpret_cast<const int*>(stg + 256 * q + 4 * lane);
            const int f0 = __builtin_amdgcn_readlane(v, 0), f1 = __builtin_amdgcn_readlane(v, 32);
            const int first = g ? f1 : f0;
            const int tok = seg_lo + kTileTok * j + n;
            const unsigned long long bal = __builtin_amdgcn_ballot_w64(tok >= seg_hi || v == first + n);
            const bool contiguous = ((bal >> (32 * g)) & 0xffffffffull) == 0xffffffffull;
            if (n == 0 && j < ntiles) tab[j] = contiguous ? first : -1;
          }
        }
      }
      // Q is retired by the tile-0 wait below (it is older than the tiles); the
      // compiler, which does not count the DMAs, adds its own wait before the
      // first use of Q.
      if constexpr (PAGED) lds_reads_done_barrier();  // the table is complete; the staging area is free
      const int eff = lim < seg_hi ? lim : seg_hi;  // this row's token limit in the segment

      // Gather of tile j into ring slot j % 4 (this wave's share of the DMAs).
      // A full fast-path gather is returned as deferred (pend_base set) when
      // `defer`: its DMAs then go out one per step of the next body.
      const uint8_t* pend_base = nullptr;
      const char* pend_dst = nullptr;
      auto issue_tile = [&](int j, int tabv, bool defer) -> bool {
        const char* dst = ring + (j & (kWSlots - 1)) * kTileBytes;
        const int tok0 = seg_lo + j * kTileTok;
        const int nvalid = seg_hi - tok0;
        const uint8_t* base;
        bool fast = true;
        if constexpr (PAGED) {
          const int s0 = __builtin_amdgcn_readfirstlane(tabv);
          base = p.kv + (long long)s0 * kQK;
          fast = s0 >= 0;
        } else {
          base = p.kv + ((long long)b * p.S_fixed + tok0) * kQK;
        }
        if (fast && nvalid >= kTileTok) {
          if (defer) {
            pend_base = base;
            pend_dst = dst;
            return true;
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) dma16_sbase(base, doff[i], dma_dst(dst, i));
          if (five) dma16_sbase(base, doff[4], dma_dst(dst, 4));
        } else if (fast) {  // partial tile: rows past the valid ones re-read the last valid row
#pragma unroll 1
          for (int i = 0; i < (five ? 5 : 4); ++i) {
            const int o = (int)doff[i];
            const int t = o / kQK;  // token row of the piece
            const int tc = t < nvalid ? t : nvalid - 1;
            dma16_opaque(base + tc * kQK + (o - t * kQK), dma_dst(dst, i));
          }
        } else {  // rows in scattered slots: every lane looks its row up
          int tk = tok0 + n;
          tk = tk < seg_hi ? tk : seg_hi - 1;
          const int myrow = p.kv_indices[slot0 + tk];  // lane n: slot of token tok0 + n
#pragma unroll 1
          for (int i = 0; i < (five ? 5 : 4); ++i) {
            const int o = (int)doff[i];
            const int t = o / kQK;
            const int row = __shfl(myrow, t);
            dma16_opaque(p.kv + (long long)row * kQK + (o - t * kQK), dma_dst(dst, i));
          }
        }
        return false;
      };
      auto tab_at = [&](int j) -> int {
        if constexpr (PAGED) {
          return tab[j];
        } else {
          return 0;
        }
      };

      issue_tile(0, tab_at(0), false);
      if (ntiles > 1) issue_tile(1, tab_at(1), false);
      if (ntiles > 2) issue_tile(2, tab_at(2), false);
      // Tile 0 has landed in every wave (at most 5 DMAs per wave per tile; tiles
      // 1 and 2 stay in flight).
      if (ntiles > 2) {
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }

      // Software pipeline over the tiles. body(t) computes S^T of tile t for this
      // wave's rows and, interleaved into its 36 QK MFMAs, the 32 PV MFMAs of
      // tile t-1 (whose P^T every wave published before the last barrier). Then
      // softmax(t) publishes P^T(t); the barrier retires tile t+1's DMAs and frees
      // the slot of tile t-1, which tile t+3 is gathered into -- a full fast-path
      // gather one DMA per step of the next body.
      constexpr int kKAhead = 4;
      // One deferred DMA, skipped inside the asm when nothing is pending (no
      // branch for the compiler to split the step sequence at).
      auto dma_if = [&](int pending, int i) {
        const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)dma_dst(pend_dst, i);
        const int pu = __builtin_amdgcn_readfirstlane(pending);  // wave-uniform: keep it in an SGPR
        asm volatile("s_cmp_eq_u32 %3, 0\n\ts_cbranch_scc1 1f\n\tglobal_load_lds_dwordx4 %0, %1\n1:" ::"v"(doff[i]),
                     "s"(pend_base), "{m0}"(m0v), "s"(pu)
                     : "memory", "scc");
      };
      // Scores of tile t plus the PV MFMAs of tile t-1 the body carries; the
      // operands of the 8 it leaves (k-step 1, d-tiles 2 and 3) go to finish().
      struct Carry {
        f32x16 s;
        bf16x8 pop[4];
        i32x2 v2, v3;
      };
      auto body = [&](int t, int pending, auto with_pv) -> Carry {
        constexpr bool kPV = decltype(with_pv)::value;
        const char* st = ring + (t & (kWSlots - 1)) * kTileBytes;          // K: tile t
        const char* sp = ring + ((t - 1) & (kWSlots - 1)) * kTileBytes;    // V: tile t-1
        const char* pr = lds + kWPOff + ((t - 1) & 1) * kWPBytes + lane * 16;  // P^T of tile t-1
        auto kaddr = [&](int s) { return st + ((s & 1) ? koff1 : koff0) + 64 * (s >> 1); };
        auto vaddr = [&](int kk, int j) {
          return sp + ((j & 1) ? voff1 : voff0) + 128 * wave + 64 * (j >> 1) + kk * 16 * kQK;
        };
        auto paddr = [&](int kk, int rt) { return reinterpret_cast<const bf16x8*>(pr + (2 * rt + kk) * 1024); };
        u32x4 kraw[kKAhead];
#pragma unroll
        for (int s = 0; s < kKAhead; ++s) kraw[s] = *reinterpret_cast<const u32x4*>(kaddr(qk_pair_at(s)));
        bf16x8 pop[4];  // P^T operand of each row tile (k-step 0, then reloaded for k-step 1)
        i32x2 vraw[4];  // V^T fragment of each d-tile (k-step 0, then reloaded for k-step 1)
        bf16x8 va;
        if constexpr (kPV) {
#pragma unroll
          for (int rt = 0; rt < 4; ++rt) pop[rt] = *paddr(0, rt);
#pragma unroll
          for (int j = 0; j < 4; ++j) vraw[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MM_LDS i32x2*)vaddr(0, j));
        }
        bf16x8 qpa, qpb;  // LDS-resident Q of the next pair, read one step ahead
        // One accumulator chain: the PV MFMAs interleaved between consecutive QK
        // MFMAs cover the dependency.
        f32x16 s0 = f32x16{};
#pragma unroll
        for (int s = 0; s < kKPairs; ++s) {
          if (s < 4) dma_if(pending, s);
          if (s == 4) dma_if(pending && five, 4);
          const u32x4 raw = kraw[s % kKAhead];
          if (s + kKAhead < kKPairs)
            kraw[s % kKAhead] = *reinterpret_cast<const u32x4*>(kaddr(qk_pair_at(s + kKAhead)));
          const int pp = qk_pair_at(s);
          bf16x8 qa, qb2;
          if (pp >= kQRegPairs) {
            qa = qpa;
            qb2 = qpb;
          } else {
            qa = qf[2 * pp];
            qb2 = qf[2 * pp + 1];
          }
          const int pn = s + 1 < kKPairs ? qk_pair_at(s + 1) : 0;
          if (pn >= kQRegPairs) {
            const char* qrow_p = qlds + n * kQLdsRowBytes;
            const int c0 = 4 * (pn - kQRegPairs) + 2 * g;  // chunk of dims 32 pn + 16g
            qpa = *reinterpret_cast<const bf16x8*>(qrow_p + 16 * (c0 ^ (n & 15)));
            qpb = *reinterpret_cast<const bf16x8*>(qrow_p + 16 * ((c0 + 1) ^ (n & 15)));
          }
          const bf16x8 ka = fp8x8_bf16(raw[0], raw[1]);
          const bf16x8 kb = fp8x8_bf16(raw[2], raw[3]);
          s0 = mfma32(ka, qa, s0);
          if constexpr (kPV) {
            // PV MFMA i = 2s (and 2s+1 below): k-step i/16, d-tile (i/4)%4, row
            // tile i%4; i < 24 here, the last 8 run under the softmax.
            if (s < 12) {
              const int i = 2 * s, j = (i >> 2) & 3, rt = i & 3;
              if (rt == 0) {
                va = fp8x8_bf16((uint32_t)vraw[j][0], (uint32_t)vraw[j][1]);
                if (i < 16) vraw[j] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MM_LDS i32x2*)vaddr(1, j));
              }
              pv_mfma(oacc[4 * j + rt], va, pop[rt]);
              // The k-step 0 operand of row tile rt is done after d-tile 3.
              if (i >= 12 && i < 16) pop[rt] = *paddr(1, rt);
            }
          }
          s0 = mfma32(kb, qb2, s0);
          if constexpr (kPV) {
            if (s < 12) {
              const int i = 2 * s + 1, j = (i >> 2) & 3, rt = i & 3;
              pv_mfma(oacc[4 * j + rt], va, pop[rt]);
              if (i >= 12 && i < 16) pop[rt] = *paddr(1, rt);
            }
          }
          sched_fence();
        }
        Carry cr;
        cr.s = s0;
        if constexpr (kPV) {
#pragma unroll
          for (int rt = 0; rt < 4; ++rt) cr.pop[rt] = pop[rt];
          cr.v2 = vraw[2];
          cr.v3 = vraw[3];
        }
        return cr;
      };
      // The 32 PV MFMAs of the last tile on their own.
      auto pv_last = [&](int t) {
        const char* sp = ring + (t & (kWSlots - 1)) * kTileBytes;
        const char* pr = lds + kWPOff + (t & 1) * kWPBytes + lane * 16;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          bf16x8 pop[4];
#pragma unroll
          for (int rt = 0; rt < 4; ++rt) pop[rt] = *reinterpret_cast<const bf16x8*>(pr + (2 * rt + kk) * 1024);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const char* va = sp + ((j & 1) ? voff1 : voff0) + 128 * wave + 64 * (j >> 1) + kk * 16 * kQK;
            const i32x2 r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MM_LDS i32x2*)va);
            const bf16x8 a = fp8x8_bf16((uint32_t)r[0], (uint32_t)r[1]);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) pv_mfma(oacc[4 * j + rt], a, pop[rt]);
          }
        }
      };

      bool pend = false;  // a deferred gather waits for the next body
      // Softmax of tile t, the tile barrier and the gather of tile t+3 (slot
      // table entry read before the barrier).
      auto finish = [&](int t, const Carry& cr, int tab_next, auto with_pv) {
        constexpr bool kPV = decltype(with_pv)::value;
        // The 8 PV MFMAs of tile t-1 the body left (k-step 1, d-tiles 2 and 3),
        // one per softmax chunk below so the softmax VALU runs under them.
        bf16x8 a2, a3;
        if constexpr (kPV) {
          a2 = fp8x8_bf16((uint32_t)cr.v2[0], (uint32_t)cr.v2[1]);
          a3 = fp8x8_bf16((uint32_t)cr.v3[0], (uint32_t)cr.v3[1]);
        }
        auto pv_left = [&](int k) {  // k = 0..7: d-tile 2 + k/4, row tile k%4
          if constexpr (kPV) pv_mfma(oacc[8 + k], k < 4 ? a2 : a3, cr.pop[k & 3]);
          sched_fence();
        };
        const int tok0 = seg_lo + t * kTileTok;
        // Lane (n, g), register i: token tok0 + 8(i/4) + 4g + i%4 of query row n.
        float sv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] = cr.s[i];
        const int rel = eff - tok0 - 4 * g;  // register i is valid iff 8(i/4) + i%4 < rel
        if (__builtin_amdgcn_ballot_w64(rel < 32)) {
#pragma unroll
          for (int i = 0; i < 16; ++i) sv[i] = ((8 * (i >> 2) + (i & 3)) < rel) ? sv[i] : -__builtin_inff();
        }
        pv_left(0);
        float mx[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) mx[i] = fmaxf(sv[i], sv[i + 8]);
#pragma unroll
        for (int i = 0; i < 4; ++i) mx[i] = fmaxf(mx[i], mx[i + 4]);
        float bm = fmaxf(fmaxf(mx[0], mx[2]), fmaxf(mx[1], mx[3]));
        pv_left(1);
        bm = xor32_max(bm);
        if constexpr (kMaxOnly) {
          row_m = fmaxf(row_m, bm);
        } else {
          // ---- softmax on the integer grid, max fixed at the row's first non-empty tile ----
          const float mc = __builtin_ceilf(bm * c);
          if (row_m == -__builtin_inff()) {
            row_m = mc;
          } else {
            grew = grew || (mc > row_m + kGrowLimit);
          }
          const float neg_m = (row_m == -__builtin_inff()) ? 0.f : -row_m;
          pv_left(2);
          float pv[16];
          float lsum = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], c, neg_m));
            lsum += pv[i];
            if ((i & 3) == 3) pv_left(3 + (i >> 2));  // chunks 3..6
          }
          row_l += lsum;
          // P^T operands of this row tile for both token k-steps, as the MFMA B
          // operand lane layout: [row tile][k-step][lane] x 16 B.
          char* pw = lds + kWPOff + (t & 1) * kWPBytes + wave * 2048 + lane * 16;
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            const u32x4 w4 = {pack2_bf16<kRTNE>(pv[8 * kk + 0], pv[8 * kk + 1]),
                              pack2_bf16<kRTNE>(pv[8 * kk + 2], pv[8 * kk + 3]),
                              pack2_bf16<kRTNE>(pv[8 * kk + 4], pv[8 * kk + 5]),
                              pack2_bf16<kRTNE>(pv[8 * kk + 6], pv[8 * kk + 7])};
            *reinterpret_cast<u32x4*>(pw + 1024 * kk) = w4;
          }
          pv_left(7);
        }

        // ---- tile barrier: P^T(t) published, tile t+1 landed everywhere, slot of t-1 free ----
        if (t + 2 < ntiles) {
          asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        } else {
          asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        if (t + 3 < ntiles) pend = issue_tile(t + 3, tab_next, true);
      };
      // Tile 0 has no PV before it; every later body carries the previous
      // tile's PV (one code path in the loop, so the accumulators stay put).
      finish(0, body(0, 0, std::false_type{}), ntiles > 3 ? tab_at(3) : 0, std::false_type{});
      for (int t = 1; t < ntiles; ++t) {
        const int tab_next = (t + 3 < ntiles) ? tab_at(t + 3) : 0;
        const int pd = pend;
        pend = false;
        if constexpr (kMaxOnly) {
          finish(t, body(t, pd, std::false_type{}), tab_next, std::false_type{});
        } else {
          finish(t, body(t, pd, std::true_type{}), tab_next, std::true_type{});
        }
      }
      if constexpr (!kMaxOnly) pv_last(ntiles - 1);
    }
  };

  // Each wave posts its rows' (m, l) and its fallback flag, then one barrier.
  auto post_ml = [&]() {
    const float L = xor32_sum(row_l);  // lanes n and n+32 hold the same row
    if (g == 0) {
      mlb[2 * (32 * wave + n)] = row_m;
      mlb[2 * (32 * wave + n) + 1] = L;
    }
    const bool any = __builtin_amdgcn_ballot_w64(grew) != 0;
    if (lane == 0) misc[8 + wave] = any;
    lds_reads_done_barrier_vm0();
  };
  sweep(std::false_type{});
  post_ml();
  // Fallback (only when some row's scores rise more than 2^64 above its first
  // tile): redo the part with the exact row max (max-only sweep, then
  // accumulate). CTA-uniform: the flags are read after a barrier.
  if ((misc[8] | misc[9] | misc[10] | misc[11]) != 0) {
    asm volatile("s_barrier" ::: "memory");  // every wave has read the flags
    row_m = -__builtin_inff();
    sweep(std::true_type{});
    row_m = __builtin_ceilf(row_m * c);
    row_l = 0.f;
    grew = false;
    zero_o();
    sweep(std::false_type{});
    post_ml();
  }

  // ---- epilogue: this wave's 4 d-tiles of the 128 rows -------------------------------
  // Branch-free stores through buffer resources that span exactly the valid
  // query rows of this request: lanes of rows >= qrows fall outside the range
  // and the hardware drops their stores. Lane (n, g), register 4*i4 + e of
  // d-tile dt holds dim 32dt + 8*i4 + 4g + e of row tile rt's row n.
  mfma_result_fence();
  const bool split = un.nparts > 1;
  const size_t rec0 = (size_t)un.rec0 + part;
  constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer access, gfx9 family
  const int row0 = rb * kWRows + n;       // this lane's row in row tile 0
  if (split) {
    // Unnormalised fp32 O of this part, record rec0 in fragment order: the
    // 16 bytes of (wave, row tile RT = 4 rb + rt < rec_rows / 32, d-tile j,
    // i4, lane) at 16 * ((((wave * nrt + RT) * 4 + j) * 4 + i4) * 64 + lane),
    // so every store instruction writes 1 KB contiguous (row-major stores from
    // this register layout write 16 B per 2 KB row: ~3x slower at 256 KB per
    // CTA).
    const int nrt = p.rec_rows / 32;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(ws_rec_o(p, rec0), (short)0, p.rec_rows * kLat * 4, kRsrcWord3);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      if (4 * rb + rt < nrt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            // Whole-vector bit cast: a bit cast of a single vector element
            // reinterprets element 0 with this compiler.
            const f32x4 f = {oacc[4 * j + rt][4 * i4], oacc[4 * j + rt][4 * i4 + 1], oacc[4 * j + rt][4 * i4 + 2],
                             oacc[4 * j + rt][4 * i4 + 3]};
            const u32x4 v = __builtin_bit_cast(u32x4, f);
            const int off = ((((wave * nrt + 4 * rb + rt) * 4 + j) * 4 + i4) * 64 + lane) * 16;
            __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, 0, 0);
          }
        }
      }
    }
  } else {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        p.o_lat + (long long)qb * p.qrows * kLat, (short)0, p.qrows * kLat * 2, kRsrcWord3);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const float L = mlb[2 * (32 * rt + n) + 1];
      const float inv = (L == 0.f) ? 0.f : p.kv_scale * __builtin_amdgcn_rcpf(L);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          u32x2 o;
          o[0] = pack2_bf16_canon<kRTNE>(oacc[4 * j + rt][4 * i4] * inv, oacc[4 * j + rt][4 * i4 + 1] * inv);
          o[1] = pack2_bf16_canon<kRTNE>(oacc[4 * j + rt][4 * i4 + 2] * inv, oacc[4 * j + rt][4 * i4 + 3] * inv);
          const int off = ((row0 + 32 * rt) * kLat + 32 * (4 * wave + j) + 8 * i4 + 4 * g) * 2;
          __builtin_amdgcn_raw_buffer_store_b64(o, rs, off, 0, 0);
        }
      }
    }
  }
  if (split && row_ok && g == 0) {
    float* pml = ws_ml(p) + (rec0 * p.qrows + qrow) * 2;
    pml[0] = row_m;
    pml[1] = mlb[2 * (32 * wave + n) + 1];
  }
  if (p.parts > 1 && part == 0 && rb == 0 && tid == 0) {
    // Per-request (parts, first record) table for the merge kernel.
    int* tbl = ws_tbl(p);
    tbl[2 * b] = un.nparts;
    tbl[2 * b + 1] = un.rec0;
  }
}

int launch_wide_kernel(const Params& p, long long grid, hipStream_t st) {
  if (p.paged)
    hipLaunchKernelGGL(mla_wide_kernel<true>, dim3((unsigned)grid), dim3(kWThreads), 0, st, p);
  else
    hipLaunchKernelGGL(mla_wide_kernel<false>, dim3((unsigned)grid), dim3(kWThreads), 0, st, p);
  return 0;
}

}  // namespace mla
}  // namespace mm
