// Absorbed-MLA decode for MI355X (gfx950): bf16 queries against an fp8 (OCP
// e4m3fn) latent KV cache, 576-wide fused rows ([0:512] latent = K and V,
// [512:576] rope = K only) at one per-tensor kv_scale.
//
//   score[r, j] = (q_lat[r] . c[j, 0:512] + q_pe[r] . c[j, 512:576]) * scale * kv_scale
//   o_lat[r]    = sum_j softmax_j(score[r, :]) * c[j, 0:512] * kv_scale
//
// Replaces the reference's gfx942 single-q and multi-q kernels (moonmath
// reference csrc/mla_decode_a16w8.hip:183-754, csrc/mla_decode_a16w8_multiq.hip
// :282-856) with one gfx950 kernel:
//
//  * A query row r is (draft position t, head h) = (r / H, r % H); draft
//    position t attends tokens [0, S - (q_len - 1 - t)) (end-aligned causal
//    window, reference mla_decode_a16w8.hip:213-217).
//  * One CTA = 32 query rows of one request b and one KV part (one 32-wide
//    v_mfma_f32_32x32x16_bf16 tile of rows). Its 4 waves (one per SIMD) walk
//    interleaved 32-token tiles of the part: wave w takes tiles w, w+4, ...
//    Every wave gathers its own tiles HBM -> LDS with 16-byte DMA into a private
//    2-slot ring (the next tile is in flight while the current one is
//    processed), so the main loop has no CTA barrier.
//  * Operands come straight from the fp8 tile: the K fragment of a 16-dim
//    k-step pair is one ds_read_b128 (16 fp8 of one token), the V^T fragment is
//    one ds_read_b64_tr_b8 (8 tokens of one latent dim); both are widened with
//    v_cvt_scalef32_pk_bf16_fp8 at scale 1, which is exact.
//  * S^T = K Q^T accumulates in VGPRs (two chains); softmax in base 2 with
//    each row's max m on the integer grid, m = ceil(max s * c) of the row's
//    first non-empty tile of the wave, p = exp2(s * c - m) (<= 2^64 for later
//    tiles, so O is never rescaled in the loop); P rounded to bf16 RTNE;
//    O^T = V^T P^T accumulates in AGPRs (16 d-tiles x 16 fp32 per lane).
//    Every combination of partial results uses exact power-of-two weights.
//  * The 4 waves' (O, m, l) are merged through LDS, each wave finalising 4 of
//    the 16 d-tiles. Split-KV parts > 1 write unnormalised fp32 (O, m, l)
//    records that mla_merge_kernel combines with power-of-two weights.
//  * Work split (plan_unit_paged, shared with the other two kernels): the
//    caller's parts budget and one round of CTAs over the CUs bound the number
//    of units (request parts); the device picks the smallest chunk C whose
//    units fit, from the batch's lengths read on the device, and cuts each
//    request into ceil(L / C) equal parts. Units run in request order when they
//    fit one round, otherwise longest first; they are dealt in snake order over
//    the 8 XCDs.
//  * Paged gathers: each wave stages its tiles' slot indices and keeps, per
//    tile, the first slot when the tile's tokens occupy consecutive slots (one
//    SGPR base + per-lane offsets per DMA); any other tile is gathered row by
//    row from per-lane slot lookups.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "mla_common.hpp"

namespace mm {
namespace mla {

constexpr int kRowsPerCta = 32;                // query rows per CTA (one MFMA tile)
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTabPerWave = 512;               // tile-table entries per wave (one segment)

// LDS map (bytes): per-wave 2-slot tile rings, per-wave tile tables (base slot
// of each of the wave's tiles in the current segment), the LDS-resident Q
// dims of the CTA's 32 rows. The merge at the end reuses the tile rings.
constexpr int kRingBytes = 2 * kTileBytes;                  // 36864 per wave
constexpr int kStageBytes = kWaves * kRingBytes;            // 147456
constexpr int kTabOff = kStageBytes;
constexpr int kQpeOff = kTabOff + kWaves * kTabPerWave * 4;  // 155648
constexpr int kLdsBytes = kQpeOff + kRowsPerCta * kQLdsRowBytes;  // 163840
// Staged slot indices: the last 8 KB of each wave's own ring (2048 indices).
constexpr int kIdxStageInRing = kRingBytes - 8192;        // 28672
// Merge area (in the tile rings): [wave][dt][i4][lane] x 16 B of O for 8 d-tiles.
constexpr int kMergeOBytes = 8 * 4 * 64 * 16;              // 32768 per wave and half
static_assert(kWaves * kMergeOBytes <= kStageBytes, "merge area fits the rings");
static_assert(2 * 64 + 1 <= kTabPerWave, "(m, l) and the fallback flag fit a wave's tile table");

// The paged plan's 12 * B bytes of scratch live in one wave's tile ring.
static_assert(12 * kMaxPagedB <= kRingBytes, "plan scratch fits a wave's ring");

template <bool PAGED>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  int* tab = reinterpret_cast<int*>(lds + kTabOff) + (threadIdx.x >> 6) * kTabPerWave;  // this wave's tile table
  char* qpe_lds = lds + kQpeOff;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31;  // MFMA column: query row (S^T, O^T) / token or dim row of A
  const int g = lane >> 5;  // lane half
  char* wring = lds + wave * kRingBytes;

  // ---- work item ----------------------------------------------------------------------
  // Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8) and in
  // blockIdx order within an XCD. Units are dealt to XCDs in snake order (XCD x
  // takes units x, 15-x, 16+x, 31-x, ...) so every XCD gets a similar share
  // (and, when units are ordered longest first, starts with its longest); the
  // ngroups CTAs of a unit run on one XCD (its KV is shared through that L2).
  const int xcd = blockIdx.x % kNumXcds;
  const int k_in_xcd = blockIdx.x / kNumXcds;
  const int uslot = k_in_xcd / p.ngroups;
  const int grp = k_in_xcd % p.ngroups;
  const int u = 16 * (uslot >> 1) + ((uslot & 1) ? 15 - xcd : xcd);
  Unit un;
  if constexpr (PAGED) {
    un = plan_unit_paged(p.seq_lens, p.kv_indptr, p.B, p.parts, p.unit_cap, u, lane, reinterpret_cast<int*>(wring));
  } else {
    un = plan_unit_contig(p.S_fixed, p.B, p.parts, p.unit_cap, u);
  }
  if (u >= un.units) return;  // padding CTA (whole CTA, before any barrier)
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

  // ---- query row of this lane ----------------------------------------------------
  const int qrow = grp * kRowsPerCta + n;  // row within (t, h)
  const bool row_ok = qrow < p.qrows;
  const int qr = row_ok ? qrow : p.qrows - 1;
  const int t_pos = qr / p.H;
  const int lim = S - (p.q_len - 1 - t_pos);  // tokens >= lim are masked for this row
  const long long qoff = (long long)qb * p.qrows + qr;  // row index into [B, q_len, H]

  // Slot indices of this wave's tiles of a segment (32 per tile, two tiles per
  // 4-byte DMA, at most 64 tiles per call) into the last 8 KB of this wave's
  // ring: tile-major, 128 B per tile. Lanes past the segment re-read its last
  // index.
  auto stage_idx = [&](int seg_lo, int seg_hi, int i0, int nb) {
    if constexpr (PAGED) {
      for (int q = 0; q < (nb + 1) / 2; ++q) {
        const int i = i0 + 2 * q + g;
        int tok = seg_lo + kTileTok * (wave + kWaves * i) + n;
        tok = tok < seg_hi ? tok : seg_hi - 1;
        dma4_opaque(p.kv_indices + slot0 + tok, wring + kIdxStageInRing + 256 * q);
      }
    }
  };
  auto seg_end = [&](int seg_lo) {
    const long long e = (long long)seg_lo + kWaves * kTabPerWave * kTileTok;
    return e < kv_hi ? (int)e : kv_hi;
  };
  auto my_tiles = [&](int seg_lo, int seg_hi) {
    const int ntiles = (seg_hi - seg_lo + kTileTok - 1) / kTileTok;
    return (wave < ntiles) ? (ntiles - wave + kWaves - 1) / kWaves : 0;
  };

  // Q fragments (B operand of S^T = K Q^T on v_mfma_f32_32x32x16_bf16; A = K
  // widened exactly from the staged fp8 tile). k-step pair s covers dims
  // 32s + 16g .. +16 of lane half g: the first 8 feed k-step 2s, the next 8
  // k-step 2s+1 (the same dims the K fragment of that lane half holds).
  if (kv_lo < kv_hi) {  // index batch of the first segment, with the Q loads
    const int nm = my_tiles(kv_lo, seg_end(kv_lo));
    stage_idx(kv_lo, seg_end(kv_lo), 0, nm < 64 ? nm : 64);
  }
  bool idx_prestaged = true;
  // The Q loads are issued right after the first tile's gather (first segment
  // of the first sweep), so their latency overlaps the tile's.
  bf16x8 qf[2 * kQRegPairs];
  bool q_ready = false;
  auto load_q = [&]() {
#pragma unroll
    for (int s = 0; s < kQRegPairs; ++s) {
      const uint16_t* src = p.q_lat + qoff * kLat + s * 32 + g * 16;
      qf[2 * s] = *reinterpret_cast<const bf16x8*>(src);
      qf[2 * s + 1] = *reinterpret_cast<const bf16x8*>(src + 8);
    }
    // Q dims [448, 576): 32 rows x 16 chunks of 8 bf16 (chunks 0..7 from q_lat,
    // 8..15 = the rope part from q_pe) into LDS.
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int id = tid + it * kThreads;  // 512 chunks
      const int r = id >> 4, c = id & 15;
      const int rr = grp * kRowsPerCta + r;
      const long long ro = (long long)qb * p.qrows + (rr < p.qrows ? rr : p.qrows - 1);
      const uint16_t* src = (c < 8) ? p.q_lat + ro * kLat + kQLdsDim0 + c * 8 : p.q_pe + ro * kRope + (c - 8) * 8;
      *reinterpret_cast<bf16x8*>(qpe_lds + r * kQLdsRowBytes + 16 * (c ^ (r & 15))) =
          *reinterpret_cast<const bf16x8*>(src);
    }
    // Retire every load here, visibly to the compiler (vmcnt 0, expcnt/lgkmcnt
    // untouched; this also lands the first tile): the tile DMAs are invisible
    // to its wait-count model, so a wait left to the loop would become a
    // per-tile vmcnt countdown that also waits for the prefetched tile.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // qpe_lds published
    q_ready = true;
  };

  // ---- per-lane constant offsets inside a staged tile -------------------------------
  // K read of pair s: token n, piece 2s+g -> n*576 + 16*((2s+g) ^ swz(n)).
  const int koff0 = n * kQK + 16 * (g ^ swz(n));
  const int koff1 = n * kQK + 16 * ((2 + g) ^ swz(n));
  // V^T transpose read (16-lane group G = 2g + mh, member j): member j supplies
  // 8 bytes of token T = 8(e/4) + 4g + e%4 (e = j/2, +16 per k-step kk), dims
  // 32dt + 16mh + 8(j&1) .. +8; swz(T) = 2(e/4) + g for every kk.
  const int vj = lane & 15, vmh = (lane >> 4) & 1, ve = vj >> 1;
  const int vT = 8 * (ve >> 2) + 4 * g + (ve & 3);
  const int vsw = 2 * (ve >> 2) + g;
  const int voff0 = vT * kQK + 16 * (vmh ^ vsw) + 8 * (vj & 1);
  const int voff1 = vT * kQK + 16 * ((2 + vmh) ^ vsw) + 8 * (vj & 1);
  // DMA: instruction k of a tile moves LDS pieces 64k .. 64k+63; with 36 pieces
  // per row, 9 instructions cover exactly 16 token rows, so the lane pattern of
  // k and k+9 is the same 16 rows later. dma_off[k9] = tg*576 + 16*c for the
  // piece slot this lane fills (tg = token within the 16-row group).
  // Offsets are < 2^14: two per VGPR (dma_pk[k9 / 2], low half for even k9).
  uint32_t dma_pk[5];
#pragma unroll
  for (int k9 = 0; k9 < 9; ++k9) {
    const int pc = 64 * k9 + lane;
    const int tg = pc / 36, cs = pc % 36;
    const uint32_t off = tg * kQK + 16 * (cs ^ swz(tg));
    dma_pk[k9 / 2] = (k9 & 1) ? (dma_pk[k9 / 2] | (off << 16)) : off;
  }
  auto dma_off = [&](int k9) -> int { return (int)((dma_pk[k9 / 2] >> (16 * (k9 & 1))) & 0xFFFFu); };
  auto dma_offv = [&](int k9) { return u16_field(dma_pk[k9 / 2], k9 & 1); };

  f32x16 oacc[kDTiles];
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt) oacc[dt] = f32x16{};
  float row_m = -__builtin_inff(), row_l = 0.f;
  bool grew = false;  // a later tile of this row exceeded row_m by more than kGrowLimit
  const float c = p.score_c;

  // One pass over the part's tiles. Accumulate mode: softmax + PV with this
  // row's max fixed at its first non-empty tile. Max-only mode: QK and the row's
  // largest masked score only (row_m then holds the raw score max).
  auto sweep = [&](auto max_only_tag) {
  constexpr bool kMaxOnly = decltype(max_only_tag)::value;
  // Segments of up to kTabPerWave tiles per wave (one for any part up to 64K tokens).
  for (int seg_lo = kv_lo; seg_lo < kv_hi; seg_lo += kWaves * kTabPerWave * kTileTok) {
    const int seg_hi = seg_end(seg_lo);
    const int ntiles = (seg_hi - seg_lo + kTileTok - 1) / kTileTok;
    const int nmine = my_tiles(seg_lo, seg_hi);  // tiles wave, wave+4, ...
    if constexpr (PAGED) {
      // Tile table of this wave's tiles: the slot indices of each tile (32 per
      // tile, two tiles per 4-byte DMA) are staged in this wave's ring, then
      // tab[i] = slot of the tile's first token if its valid tokens occupy
      // consecutive slots (the gather is one base + lane offsets), else -1.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring is free (previous segment drained)
      for (int i0 = 0; i0 < nmine; i0 += 64) {
        const int nb = (nmine - i0 < 64) ? nmine - i0 : 64;
        if (!(idx_prestaged && seg_lo == kv_lo && i0 == 0)) stage_idx(seg_lo, seg_hi, i0, nb);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll 4
        for (int q = 0; q < (nb + 1) / 2; ++q) {
          const int i = i0 + 2 * q + g;
          const int v = *reinterpret_cast<const int*>(wring + kIdxStageInRing + 256 * q + 4 * lane);
          const int f0 = __builtin_amdgcn_readlane(v, 0), f1 = __builtin_amdgcn_readlane(v, 32);
          const int first = g ? f1 : f0;
          const int tok = seg_lo + kTileTok * (wave + kWaves * i) + n;
          const unsigned long long bal = __builtin_amdgcn_ballot_w64(tok >= seg_hi || v == first + n);
          const bool contiguous = ((bal >> (32 * g)) & 0xffffffffull) == 0xffffffffull;
          if (n == 0 && i < nmine) tab[i] = contiguous ? first : -1;
        }
      }
    }
    idx_prestaged = false;  // a later sweep re-stages its indices
    const int eff = lim < seg_hi ? lim : seg_hi;  // this row's token limit in the segment

    // Gather of tile j (tokens seg_lo + 32j ..), j = wave + 4i. Fast path: the
    // tile's rows are consecutive slots (always for the contiguous layout, and
    // for paged tiles inside one page): DMA k reads base + (k/9)*16 rows +
    // dma_off[k%9], with rows past the valid ones clamped to the last valid row
    // in a partial tile. Slow path: every lane looks its row up.
    auto tile_base = [&](int j, const uint8_t*& base) -> bool {
      const int tok0 = seg_lo + j * kTileTok;
      if constexpr (PAGED) {
        const int s0 = __builtin_amdgcn_readfirstlane(tab[j / kWaves]);
        base = p.kv + (long long)s0 * kQK;
        return s0 >= 0;
      } else {
        base = p.kv + ((long long)b * p.S_fixed + tok0) * kQK;
        return true;
      }
    };
    auto issue_partial = [&](int j, const uint8_t* base, const char* dst) {
      const int nvalid = seg_hi - (seg_lo + j * kTileTok);
#pragma unroll 1
      for (int k = 0; k < kDmaPerTile; ++k) {
        const int o = dma_off(k % 9);
        const int tg = (o * 7282) >> 22;  // o / 576 for o < 9216
        int t = (k / 9) * 16 + tg;
        t = t < nvalid ? t : nvalid - 1;
        dma16_opaque(base + t * kQK + (o - tg * kQK), dst + 1024 * k);
      }
    };
    auto issue_slow = [&](int j, const char* dst) {
      const int tok0 = seg_lo + j * kTileTok;
      int tk = tok0 + n;
      tk = tk < seg_hi ? tk : seg_hi - 1;
      const int myrow = p.kv_indices[slot0 + tk];  // lane n: slot of token tok0 + n
#pragma unroll 1
      for (int k = 0; k < kDmaPerTile; ++k) {
        const int o = dma_off(k % 9);
        const int tg = (o * 7282) >> 22;
        const int row = __shfl(myrow, (k / 9) * 16 + tg);
        dma16_opaque(p.kv + (long long)row * kQK + (o - tg * kQK), dst + 1024 * k);
      }
    };
    auto issue_tile = [&](int j, const char* dst) {
      const uint8_t* base;
      if (!tile_base(j, base)) {
        issue_slow(j, dst);
      } else if (seg_lo + (j + 1) * kTileTok > seg_hi) {
        issue_partial(j, base, dst);
      } else {
#pragma unroll
        for (int k = 0; k < kDmaPerTile; ++k) dma16_sbase(base + (k / 9) * 16 * kQK, dma_offv(k % 9), dst + 1024 * k);
      }
    };

    int slot = 0;
    if (wave < ntiles) issue_tile(wave, wring);
    if (!q_ready) load_q();  // CTA-uniform: the first segment of the first sweep
    for (int j = wave; j < ntiles; j += kWaves) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this tile has landed
      const char* st = wring + slot * kTileBytes;
      const char* nst = wring + (slot ^ 1) * kTileBytes;
      const int tok0 = seg_lo + j * kTileTok;
      // Next tile of this wave: a full fast-path gather is spread over the 18
      // QK steps below (one DMA each); any other gather is issued here.
      const uint8_t* nbase = nullptr;
      bool ndma = false;
      if (j + kWaves < ntiles) {
        const bool full = seg_lo + (j + kWaves + 1) * kTileTok <= seg_hi;
        ndma = full && tile_base(j + kWaves, nbase);
        if (!ndma) issue_tile(j + kWaves, nst);
      }
      ndma = __builtin_amdgcn_readfirstlane((int)ndma) != 0;

      // ---- S^T = K Q^T: 18 k-step pairs, two accumulator chains ------------------------
      // K pieces are read kKAhead pairs ahead of their conversion; each step
      // also issues one DMA of the next tile. One straight-line body per DMA
      // mode, so no branch splits the steps; sched_fence() keeps each step's
      // [DMA, read ahead, convert, 2 MFMA] order.
      constexpr int kKAhead = 4;
      auto kaddr = [&](int s) { return st + ((s & 1) ? koff1 : koff0) + 64 * (s >> 1); };
      auto qk = [&](auto with_dma) {
        u32x4 kraw[kKAhead];
#pragma unroll
        for (int s = 0; s < kKAhead; ++s) kraw[s] = *reinterpret_cast<const u32x4*>(kaddr(qk_pair_at(s)));
        bf16x8 qpa, qpb;  // LDS-resident Q of the next pair, read one step ahead
        f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
        for (int s = 0; s < kKPairs; ++s) {
          if constexpr (decltype(with_dma)::value)
            dma16_sbase(nbase + (s / 9) * 16 * kQK, dma_offv(s % 9), nst + 1024 * s);
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
            const char* qrow_p = qpe_lds + n * kQLdsRowBytes;
            const int c0 = 4 * (pn - kQRegPairs) + 2 * g;  // chunk of dims 32 pn + 16g
            qpa = *reinterpret_cast<const bf16x8*>(qrow_p + 16 * (c0 ^ (n & 15)));
            qpb = *reinterpret_cast<const bf16x8*>(qrow_p + 16 * ((c0 + 1) ^ (n & 15)));
          }
          const bf16x8 ka = fp8x8_bf16(raw[0], raw[1]);
          const bf16x8 kb = fp8x8_bf16(raw[2], raw[3]);
          s0 = mfma32(ka, qa, s0);
          s1 = mfma32(kb, qb2, s1);
          sched_fence();
        }
        return s0 + s1;
      };
      const f32x16 sacc = ndma ? qk(std::true_type{}) : qk(std::false_type{});
      // V^T transpose reads for the first PV steps go out before the softmax.
      constexpr int kVAhead = 6;
      auto vaddr = [&](int i) {
        const int kk = i / kDTiles, dt = i % kDTiles;
        return st + ((dt & 1) ? voff1 : voff0) + 64 * (dt >> 1) + kk * 16 * kQK;
      };
      i32x2 vraw[kVAhead];
#pragma unroll
      for (int i = 0; i < kVAhead; ++i) vraw[i] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MM_LDS i32x2*)vaddr(i));

      // Lane (n, g), register i: token tok0 + 8(i/4) + 4g + i%4 of query row n.
      float sv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) sv[i] = sacc[i];
      const int rel = eff - tok0 - 4 * g;  // register i is valid iff 8(i/4) + i%4 < rel
      if (__builtin_amdgcn_ballot_w64(rel < 32)) {  // the window or the range ends in this tile
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] = ((8 * (i >> 2) + (i & 3)) < rel) ? sv[i] : -__builtin_inff();
      }

      // ---- online softmax: running max on the integer grid, fixed per row --------------
      float mx[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) mx[i] = fmaxf(sv[i], sv[i + 8]);
#pragma unroll
      for (int i = 0; i < 4; ++i) mx[i] = fmaxf(mx[i], mx[i + 4]);
      float bm = fmaxf(fmaxf(mx[0], mx[2]), fmaxf(mx[1], mx[3]));
      bm = xor32_max(bm);
      if constexpr (kMaxOnly) {
        row_m = fmaxf(row_m, bm);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // drain the V^T reads
        slot ^= 1;
        continue;
      }
      const float mc = __builtin_ceilf(bm * c);
      if (row_m == -__builtin_inff()) {
        row_m = mc;  // first non-empty tile of the row (O and l are still 0)
      } else {
        grew = grew || (mc > row_m + kGrowLimit);
      }
      const float neg_m = (row_m == -__builtin_inff()) ? 0.f : -row_m;
      // P of k-step 0 (registers 0..7) now; k-step 1 is finished inside the
      // first PV steps, under their MFMAs.
      float pv[16];
      float lsum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], c, neg_m));
        lsum += pv[i];
      }
      bf16x8 pf[2];
      {
        u32x4 pw = {pack2_bf16<kRTNE>(pv[0], pv[1]), pack2_bf16<kRTNE>(pv[2], pv[3]), pack2_bf16<kRTNE>(pv[4], pv[5]),
                    pack2_bf16<kRTNE>(pv[6], pv[7])};
        pf[0] = __builtin_bit_cast(bf16x8, pw);
      }
      sched_fence();

      // ---- O^T += V^T P^T: 16 d-tiles x 2 token k-steps ---------------------------------
#pragma unroll
      for (int i = 0; i < 2 * kDTiles; ++i) {
        const int kk = i / kDTiles, dt = i % kDTiles;
        const i32x2 r = vraw[i % kVAhead];
        if (i + kVAhead < 2 * kDTiles)
          vraw[i % kVAhead] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MM_LDS i32x2*)vaddr(i + kVAhead));
        if (i < 8) {
          pv[8 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[8 + i], c, neg_m));
          lsum += pv[8 + i];
        }
        if (i == 8) {
          u32x4 pw = {pack2_bf16<kRTNE>(pv[8], pv[9]), pack2_bf16<kRTNE>(pv[10], pv[11]),
                      pack2_bf16<kRTNE>(pv[12], pv[13]), pack2_bf16<kRTNE>(pv[14], pv[15])};
          pf[1] = __builtin_bit_cast(bf16x8, pw);
          row_l += lsum;
        }
        pv_mfma(oacc[dt], fp8x8_bf16((uint32_t)r[0], (uint32_t)r[1]), pf[kk]);
        sched_fence();
      }
      slot ^= 1;
    }
  }
  };

  // Each wave posts its (m, l) per lane and its fallback flag into its own
  // tile-table area (no other wave touches it), then one barrier.
  auto post_ml = [&]() {
    mfma_result_fence();
    float* mine = reinterpret_cast<float*>(tab);
    mine[2 * lane] = row_m;
    mine[2 * lane + 1] = row_l;
    if (lane == 0) reinterpret_cast<int*>(tab)[128] = __builtin_amdgcn_ballot_w64(grew) != 0;
    lds_reads_done_barrier_vm0();
  };
  auto ml_of = [&](int v, int i) {
    return reinterpret_cast<const float*>(lds + kTabOff)[v * kTabPerWave + 2 * lane + i];
  };
  auto retry_of = [&]() {
    const int* base = reinterpret_cast<const int*>(lds + kTabOff);
    return (base[128] | base[kTabPerWave + 128] | base[2 * kTabPerWave + 128] | base[3 * kTabPerWave + 128]) != 0;
  };
  sweep(std::false_type{});
  post_ml();
  // Fallback (never taken unless some row's scores rise more than 2^64 above
  // its first tile): every wave redoes its tiles with the exact row max. The
  // decision is CTA-uniform because the sweeps hold CTA barriers.
  if (retry_of()) {
    asm volatile("s_barrier" ::: "memory");  // every wave has read the flags
    row_m = -__builtin_inff();
    sweep(std::true_type{});
    row_m = __builtin_ceilf(row_m * c);
    row_l = 0.f;
    grew = false;
    mfma_result_fence();
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt) oacc[dt] = f32x16{};
    sweep(std::false_type{});
    post_ml();
  }

  // ---- merge the 4 waves' (O, m, l) through LDS ---------------------------------------
  // Rows of lanes n and n+32 are the same query row: m agrees, l is summed at the end.
  // Lane weights of the 4 waves, exact powers of two.
  float mw[kWaves], lw[kWaves];
  float M = -__builtin_inff();
#pragma unroll
  for (int v = 0; v < kWaves; ++v) {
    mw[v] = ml_of(v, 0);
    lw[v] = ml_of(v, 1);
    M = fmaxf(M, mw[v]);
  }
  float wt[kWaves];
  float L = 0.f;
#pragma unroll
  for (int v = 0; v < kWaves; ++v) {
    const float diff = mw[v] - M;  // integer-valued or -inf, <= 0
    wt[v] = (mw[v] == -__builtin_inff()) ? 0.f : ((diff >= -126.f) ? __builtin_ldexpf(1.0f, (int)diff) : 0.f);
    L = __builtin_fmaf(wt[v], lw[v], L);
  }
  L = xor32_sum(L);  // whole-row sum (lanes n and n+32)
  const bool split = un.nparts > 1;
  const float inv = (L == 0.f) ? 0.f : p.kv_scale * __builtin_amdgcn_rcpf(L);
  // The query row again, from the lane id (cheaper than keeping it live
  // through the tile loop).
  const int qrow_e = grp * kRowsPerCta + (int)(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) & 31);
  const bool row_ok_e = qrow_e < p.qrows;
  const size_t rec = ((size_t)un.rec0 + part) * p.qrows + qrow_e;  // row-major records (rec_rows == qrows)
  uint16_t* orow = p.o_lat + ((long long)qb * p.qrows + qrow_e) * kLat;
  float* prow = p.ws + rec * kLat;

#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 1) lds_reads_done_barrier();  // the first half's readers are done
    // Publish this wave's 8 d-tiles of half h: [wave][dt8][i4][lane] x 16 B.
#pragma unroll
    for (int d8 = 0; d8 < 8; ++d8) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const f32x4 v = {oacc[8 * h + d8][4 * i4], oacc[8 * h + d8][4 * i4 + 1], oacc[8 * h + d8][4 * i4 + 2],
                         oacc[8 * h + d8][4 * i4 + 3]};
        *reinterpret_cast<f32x4*>(lds + wave * kMergeOBytes + ((d8 * 4 + i4) * 64 + lane) * 16) = v;
      }
    }
    lds_reads_done_barrier();
    // This wave finalises d-tiles 8h + 2*wave and 8h + 2*wave + 1.
#pragma unroll
    for (int dd = 0; dd < 2; ++dd) {
      const int d8 = 2 * wave + dd;
      const int dt = 8 * h + d8;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int v = 0; v < kWaves; ++v) {
          const f32x4 o = *reinterpret_cast<const f32x4*>(lds + v * kMergeOBytes + ((d8 * 4 + i4) * 64 + lane) * 16);
          acc[0] = __builtin_fmaf(wt[v], o[0], acc[0]);
          acc[1] = __builtin_fmaf(wt[v], o[1], acc[1]);
          acc[2] = __builtin_fmaf(wt[v], o[2], acc[2]);
          acc[3] = __builtin_fmaf(wt[v], o[3], acc[3]);
        }
        // Lane (n, g), register 4*i4 + e of d-tile dt: dim 32dt + 8*i4 + 4g + e.
        const int d = 32 * dt + 8 * i4 + 4 * g;
        if (row_ok_e) {
          if (split) {
            *reinterpret_cast<f32x4*>(prow + d) = acc;
          } else {
            u32x2 o;
            o[0] = pack2_bf16_canon<kRTNE>(acc[0] * inv, acc[1] * inv);
            o[1] = pack2_bf16_canon<kRTNE>(acc[2] * inv, acc[3] * inv);
            *reinterpret_cast<u32x2*>(orow + d) = o;
          }
        }
      }
    }
  }
  if (split && row_ok_e && g == 0 && wave == 0) {
    float* pml = ws_ml(p) + rec * 2;
    pml[0] = M;
    pml[1] = L;
  }
  if (p.parts > 1 && part == 0 && grp == 0 && tid == 0) {
    // Per-request (parts, first record) table for the merge kernel.
    int* tbl = ws_tbl(p);
    tbl[2 * b] = un.nparts;
    tbl[2 * b + 1] = un.rec0;
  }
}

// Merge of NU 4-dim slices of one query row over its request's parts:
// M = max_p m_p, w_p = 2^(m_p - M), out = sum w_p O_p * kv_scale / sum w_p l_p,
// parts in order. o_at(j, u): part j's 16-byte O slice u; ml_at(j): part j's
// (m, l) pair (shared by the slices: one row). The (m, l) pairs and O slices
// of up to kBatch parts are loaded together, so a request of up to kBatch
// parts costs one round of memory latency.
template <int NU, class OAt, class MlAt>
__device__ __forceinline__ void merge_slices(int nparts, float kv_scale, OAt o_at, MlAt ml_at, u32x2 (&out)[NU]) {
  constexpr int kBatch = 8;
  float M = -__builtin_inff();
  f32x4 acc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  float mb[kBatch], lb[kBatch];
  f32x4 ob[kBatch][NU];
  // Parts past the request's last are not loaded (uniform across the CTA: a
  // CTA's cells belong to one request).
  auto load_batch = [&](int j0) {
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (j0 + k < nparts) {
        const float2 m_l = *reinterpret_cast<const float2*>(ml_at(j0 + k));
        mb[k] = m_l.x;
        lb[k] = m_l.y;
#pragma unroll
        for (int u = 0; u < NU; ++u) ob[k][u] = *reinterpret_cast<const f32x4*>(o_at(j0 + k, u));
      } else {
        mb[k] = -__builtin_inff();
        lb[k] = 0.f;
#pragma unroll
        for (int u = 0; u < NU; ++u) ob[k][u] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  auto accumulate = [&](int j0) {
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (j0 + k < nparts) {
        const float diff = mb[k] - M;  // integer-valued or -inf, <= 0
        const float wt =
            (mb[k] == -__builtin_inff()) ? 0.f : ((diff >= -126.f) ? __builtin_ldexpf(1.0f, (int)diff) : 0.f);
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          acc[u][0] = __builtin_fmaf(wt, ob[k][u][0], acc[u][0]);
          acc[u][1] = __builtin_fmaf(wt, ob[k][u][1], acc[u][1]);
          acc[u][2] = __builtin_fmaf(wt, ob[k][u][2], acc[u][2]);
          acc[u][3] = __builtin_fmaf(wt, ob[k][u][3], acc[u][3]);
        }
        L = __builtin_fmaf(wt, lb[k], L);
      }
    }
  };
  if (nparts <= kBatch) {
    load_batch(0);
#pragma unroll
    for (int k = 0; k < kBatch; ++k) M = fmaxf(M, mb[k]);  // repeats of the last part change nothing
    accumulate(0);
  } else {
    for (int j0 = 0; j0 < nparts; j0 += kBatch) {
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int j = j0 + k < nparts ? j0 + k : nparts - 1;
        M = fmaxf(M, ml_at(j)[0]);
      }
    }
    for (int j0 = 0; j0 < nparts; j0 += kBatch) {
      load_batch(j0);
      accumulate(j0);
    }
  }
  const float inv = (L == 0.f) ? 0.f : kv_scale * __builtin_amdgcn_rcpf(L);
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    out[u][0] = pack2_bf16_canon<kRTNE>(acc[u][0] * inv, acc[u][1] * inv);
    out[u][1] = pack2_bf16_canon<kRTNE>(acc[u][2] * inv, acc[u][3] * inv);
  }
}

template <class OAt, class MlAt>
__device__ __forceinline__ u32x2 merge_slice(int nparts, float kv_scale, OAt o_at, MlAt ml_at) {
  u32x2 o[1];
  merge_slices<1>(nparts, kv_scale, [&](int j, int) { return o_at(j); }, ml_at, o);
  return o[0];
}

__device__ __forceinline__ int merge_out_row(const Params& p, int b) {
  int qb = b;
  if (p.rows) {
    qb = p.rows[b];
    qb = qb < 0 ? 0 : (qb >= p.B ? p.B - 1 : qb);
  }
  return qb;
}

// Merge of row-major records: one thread = 4 output dims of one (b, query row).
__global__ __launch_bounds__(256) void mla_merge_kernel(Params p) {
  const long long cell = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long per_b = (long long)p.qrows * (kLat / 4);
  if (cell >= per_b * p.B) return;
  const int b = (int)(cell / per_b);
  const int rem = (int)(cell % per_b);
  const int qrow = rem / (kLat / 4);
  const int d = (rem % (kLat / 4)) * 4;
  const int qb = merge_out_row(p, b);
  const float* ml = ws_ml(p);
  const int* tbl = ws_tbl(p);
  const int nparts = tbl[2 * b];
  const int rec0 = tbl[2 * b + 1];
  if (nparts <= 1) return;  // the decode kernel wrote this request's output
  const u32x2 o = merge_slice(
      nparts, p.kv_scale, [&](int j) { return ws_rec_o(p, (size_t)rec0 + j) + (size_t)qrow * kLat + d; },
      [&](int j) { return ml + (((size_t)rec0 + j) * p.qrows + qrow) * 2; });
  // Non-temporal: written once, read by no later kernel of the call (H=16:
  // 45.8 -> 44.4 us per call; the same in the decode kernels measured neutral
  // or slower).
  __builtin_nontemporal_store(o, reinterpret_cast<u32x2*>(p.o_lat + ((long long)qb * p.qrows + qrow) * kLat + d));
}

// Merge of the 128-row kernel's fragment-order records (see its epilogue):
// CTA (b, wave slice w, row tile rt) reads the 16 KB of its 32 rows x 128 dims
// from each part, 16 contiguous bytes per thread, and writes the rows' 256-byte
// output spans through LDS.
constexpr int kMergeFragThreads = 1024;
// One CTA = one request's 32-row tile of the 128-row kernel's records, output
// dims 256 wp .. 256 wp + 255 (record fragments of waves 2 wp and 2 wp + 1):
// each thread merges the same 16-byte unit of both waves' fragments, so the
// grid (B x 2 x row tiles) is one round of resident CTAs with two slices'
// loads in flight per thread.
__global__ __launch_bounds__(kMergeFragThreads) void mla_merge_frag_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[32][256];
  const int nrt = p.rec_rows / 32;
  const int b = blockIdx.x / (2 * nrt);
  const int kk = blockIdx.x % (2 * nrt);  // wp * nrt + rt
  const int wp = kk / nrt, rt = kk % nrt;
  const int tid = threadIdx.x;
  const int lane = tid & 63, i4 = (tid >> 6) & 3, j = tid >> 8;
  const int n = lane & 31, g = lane >> 5;
  const int* tbl = ws_tbl(p);
  const int nparts = tbl[2 * b];
  const int rec0 = tbl[2 * b + 1];
  if (nparts <= 1) return;  // uniform: the decode kernel wrote this request's output
  const int row = 32 * rt + n;
  const int mrow = row < p.qrows ? row : p.qrows - 1;  // padding rows read a valid (m, l)
  // 16-byte unit of wave w's fragment k = w * nrt + rt in the record.
  const size_t f0 = ((size_t)((2 * wp * nrt + rt) * 4 + j) * 4 + i4) * 64 + lane;
  const size_t f1 = f0 + (size_t)nrt * 4 * 4 * 64;  // wave 2 wp + 1
  const float* ml = ws_ml(p);
  u32x2 o[2];
  merge_slices<2>(
      nparts, p.kv_scale,
      [&](int jj, int u) { return ws_rec_o(p, (size_t)rec0 + jj) + (u ? f1 : f0) * 4; },
      [&](int jj) { return ml + (((size_t)rec0 + jj) * p.qrows + mrow) * 2; }, o);
  *reinterpret_cast<u32x2*>(&tile[n][32 * j + 8 * i4 + 4 * g]) = o[0];
  *reinterpret_cast<u32x2*>(&tile[n][128 + 32 * j + 8 * i4 + 4 * g]) = o[1];
  __syncthreads();
  // 32 rows x 512 B: thread t stores 16 B of row t / 32.
  const int r = tid >> 5, c = tid & 31;
  const int orow = 32 * rt + r;
  if (orow < p.qrows) {
    const int qb = merge_out_row(p, b);
    *reinterpret_cast<u32x4*>(p.o_lat + ((long long)qb * p.qrows + orow) * kLat + 256 * wp + 8 * c) =
        *reinterpret_cast<const u32x4*>(&tile[r][8 * c]);
  }
}

// ---------------------------------------------------------------------------
// 64-token block tables -> the flat per-token slots the decode reads. Request
// b's slots go at stride max_blocks * 64: idx[b * stride + t] = page(b, t / 64)
// * 64 + t % 64 for t < len_b, with page ids clamped to the pool and
// len_b = seq_lens[b] clamped to [0, max_blocks * 64], so no table content
// makes the decode read outside the pool. Index workspace (int32):
// [B * stride slots][B lengths][B + 1 offsets]. One thread per token slot of
// the table (4 pages per 256-thread CTA).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void expand_block_table_kernel(const int* __restrict__ seq_lens,
                                                                 const int* __restrict__ table, int max_blocks,
                                                                 int num_blocks, int B, int* __restrict__ ws) {
  const long long page = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (page >= (long long)B * max_blocks) return;
  const int b = (int)(page / max_blocks), j = (int)(page % max_blocks);
  const long long stride = (long long)max_blocks * 64;
  int len = seq_lens[b];
  len = len < 0 ? 0 : (len > stride ? (int)stride : len);
  const int t = j * 64 + lane;
  if (t < len) {
    int blk = table[page];
    blk = blk < 0 ? 0 : (blk >= num_blocks ? num_blocks - 1 : blk);
    ws[b * stride + t] = blk * 64 + lane;
  }
  if (j == 0 && lane == 0) {
    ws[B * stride + b] = len;
    ws[B * stride + B + b] = (int)(b * stride);
    if (b == B - 1) ws[B * stride + 2 * B] = (int)(B * stride);
  }
}

// Test hook: decode fp8 bytes with the same hardware convert the kernel uses.
__global__ void fp8_to_bf16_kernel(const uint8_t* in, uint16_t* out, int n) {
  const int i = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  uint32_t v = 0;
  for (int k = 0; k < 4; ++k) v |= (uint32_t)(i + k < n ? in[i + k] : 0) << (8 * k);
  const uint32_t lo = fp8x2_bf16<false>(v);
  const uint32_t hi = fp8x2_bf16<true>(v);
  const uint16_t r[4] = {(uint16_t)(lo & 0xFFFF), (uint16_t)(lo >> 16), (uint16_t)(hi & 0xFFFF), (uint16_t)(hi >> 16)};
  for (int k = 0; k < 4; ++k)
    if (i + k < n) out[i + k] = r[k];
}

}  // namespace mla
}  // namespace mm

// ===========================================================================
// Host side: planners + C ABI
// ===========================================================================
namespace {
using namespace mm::mla;

constexpr int kQRowsPerCta = kRowsPerCta;  // 32
constexpr int kNumCUs = 256;
constexpr int kMaxParts = 64;

// Requests of 96..128 query rows (H * q_len) run mla_wide_kernel (one 128-row
// block per CTA); others the 32-row kernel. Measured at B=64, ctx U[1024,8192]
// (steady clocks): H=128 q_len 1: 108 us wide (4 parts) vs 131 us 32-row
// unsplit, 120-124 us 32-row with 2 parts (two rounds of CTAs, in request or
// longest-first order) and 149-153 us with 4 parts; H=128 q_len 2 (two row
// blocks, one round of 256 CTAs with 2 parts, fragment-order records): 187 us
// wide vs 180-182 us 32-row -- with several row blocks the split records
// (rows x parts x 2 KB) outweigh the shared tile loads.
constexpr int kWideMinRows = 96;
constexpr int kWideRowsPerCta = 128;
// Requests of at most 16 query rows run mla_coop_kernel (the 4 waves share each
// tile: no cross-wave merge of the output).
constexpr int kCoopMaxRows = 16;
bool use_wide(int H, int q_len) { return H * q_len >= kWideMinRows && H * q_len <= kWideRowsPerCta; }
bool use_coop(int H, int q_len) { return H * q_len <= kCoopMaxRows; }
int ngroups_for(int H, int q_len) {
  if (use_coop(H, q_len)) return 1;
  const int rows = use_wide(H, q_len) ? kWideRowsPerCta : kQRowsPerCta;
  return (H * q_len + rows - 1) / rows;
}

// O rows of one split record: the 128-row kernel writes whole 32-row tiles in
// its fragment order; the others write qrows row-major rows.
int rec_rows_for(int H, int q_len) {
  const int qrows = H * q_len;
  return use_wide(H, q_len) ? 32 * ((qrows + 31) / 32) : qrows;
}

// Split workspace bytes: O records, (m, l) pairs, the per-request table.
size_t split_ws_bytes(int B, int H, int parts, int q_len) {
  return (size_t)B * parts * ((size_t)rec_rows_for(H, q_len) * kLat + (size_t)H * q_len * 2) * sizeof(float) +
         (size_t)B * 8;
}

// Largest parts the fixed record workspace allows for (B, H, q_len).
int max_parts_for(int B, int H, int q_len) {
  const long long per_part = (long long)B * rec_rows_for(H, q_len);
  long long m = per_part > 0 ? (long long)kMaxRecords / per_part : 1;
  if (m > kMaxParts) m = kMaxParts;
  return m < 1 ? 1 : (int)m;
}

// Units one round of CTAs over the CUs holds (one CTA per CU fits in LDS for
// every kernel here; per-CTA set-up dominates short CTAs, so a second round
// costs more than longer parts). 32-row kernel: its ngroups CTAs per unit
// share the CUs.
int unit_cap_for(int H, int q_len) {
  if (use_coop(H, q_len) || use_wide(H, q_len)) return kNumCUs;
  const int c = kNumCUs / ngroups_for(H, q_len);
  return c < 1 ? 1 : c;
}

// Split planner: enough parts that the kernel's plan can fill the unit cap
// (it then cuts the batch into at most min(B * parts, cap) units), within the
// record workspace. Measured on the 128-row kernel (B=64, H=128, q_len 2):
// 209 us with 4 parts and 448 CTAs, 264 us with 2 parts and 192 CTAs.
int plan_parts(int B, int H, int max_seq_len, int q_len) {
  if (B < 1) B = 1;
  if (q_len < 1) q_len = 1;
  const int units = unit_cap_for(H, q_len);
  int p = (units + B - 1) / B;
  const int by_len = 1 + max_seq_len / 512;  // chunks are at least 512 tokens
  if (p > by_len) p = by_len;
  const int cap = max_parts_for(B, H, q_len);
  if (p > cap) p = cap;
  return p < 1 ? 1 : p;
}

int clamp_parts(int parts, int B, int H, int q_len, bool have_ws) {
  int p = parts < 1 ? 1 : parts;
  const int cap = max_parts_for(B, H, q_len);
  if (p > cap) p = cap;
  if (!have_ws) p = 1;
  return p;
}

// Argument codes shared by every decode launcher (0 = arguments usable).
int check_launch_args(const void* q_lat, const void* q_pe, const void* kv, const void* o_lat, const void* seq_lens,
                      const void* kv_indices, const void* kv_indptr, int B, int H, int S_fixed, int q_len,
                      int lat_dim, int rope_dim, bool paged) {
  if (lat_dim != kLat || rope_dim != kRope) return -2;
  if (H < 1 || H > kMaxHeads) return -3;
  if (q_len < 1 || q_len > kMaxQLen || B < 1) return -4;
  if (paged && B > kMaxPagedB) return -4;
  if (!q_lat || !q_pe || !kv || !o_lat) return -6;
  if (paged && (!seq_lens || !kv_indices || !kv_indptr)) return -6;
  if (!paged && S_fixed < 1) return -7;
  return 0;
}

int launch(const void* q_lat, const void* q_pe, const void* kv, void* o_lat, const void* seq_lens,
           const void* rows, const void* kv_indices, const void* kv_indptr, int B, int H, int S_fixed, int parts,
           int q_len, int lat_dim, int rope_dim, float scale, float kv_scale, void* workspace, void* stream,
           bool paged) {
  const int arg_rc = check_launch_args(q_lat, q_pe, kv, o_lat, seq_lens, kv_indices, kv_indptr, B, H, S_fixed, q_len,
                                       lat_dim, rope_dim, paged);
  if (arg_rc != 0) return arg_rc;
  Params p{};
  p.q_lat = static_cast<const uint16_t*>(q_lat);
  p.q_pe = static_cast<const uint16_t*>(q_pe);
  p.kv = static_cast<const uint8_t*>(kv);
  p.o_lat = static_cast<uint16_t*>(o_lat);
  p.ws = static_cast<float*>(workspace);
  p.seq_lens = static_cast<const int*>(seq_lens);
  p.rows = static_cast<const int*>(rows);
  p.kv_indices = static_cast<const int*>(kv_indices);
  p.kv_indptr = static_cast<const int*>(kv_indptr);
  p.B = B;
  p.H = H;
  p.q_len = q_len;
  p.S_fixed = S_fixed;
  p.parts = clamp_parts(parts, B, H, q_len, workspace != nullptr);
  p.ngroups = ngroups_for(H, q_len);
  p.unit_cap = unit_cap_for(H, q_len);
  p.paged = paged ? 1 : 0;
  p.qrows = H * q_len;
  p.rec_rows = rec_rows_for(H, q_len);
  p.rec_frag = use_wide(H, q_len) ? 1 : 0;
  p.score_c = (float)((double)scale * (double)kv_scale * 1.4426950408889634);
  p.kv_scale = kv_scale;
  // Unit slots per XCD for the snake deal of units 0..U-1, U <= B * parts (the
  // kernel's split plan never exceeds that bound; CTAs past the real count exit).
  const long long umax = (long long)B * p.parts;
  const long long slots_per_xcd = 2 * ((umax - 1) / 16) + (((umax - 1) % 16) >= 8 ? 2 : 1);
  const long long grid = (long long)mm::kNumXcds * slots_per_xcd * p.ngroups;
  if (grid > 0x7FFFFFFFLL) return -8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (use_coop(H, q_len))
    launch_coop_kernel(p, grid, st);
  else if (use_wide(H, q_len))
    launch_wide_kernel(p, grid, st);
  else if (paged)
    hipLaunchKernelGGL(mla_decode_kernel<true>, dim3((unsigned)grid), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(mla_decode_kernel<false>, dim3((unsigned)grid), dim3(kThreads), 0, st, p);
  if (p.parts > 1 && p.rec_frag) {
    const long long ctas = (long long)B * 2 * (p.rec_rows / 32);
    hipLaunchKernelGGL(mla_merge_frag_kernel, dim3((unsigned)ctas), dim3(kMergeFragThreads), 0, st, p);
  } else if (p.parts > 1) {
    const long long cells = (long long)B * p.qrows * (kLat / 4);
    hipLaunchKernelGGL(mla_merge_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, st, p);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

// ---------------------------------------------------------------------------
// Allocation-free launches: the split records and merge table of one launch
// live in a file-scope device array (64.3 MiB, zero-filled at load, held on
// every GPU the library runs on until the process ends). Its device address
// is looked up once per device with hipGetSymbolAddress and kept; host code
// never hands the array's name itself to a kernel (on the host that name is a
// stand-in, not a device address). The decode writes every record and table
// entry the merge reads, so nothing needs clearing between calls; calls that
// overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
constexpr size_t kScratchRecords = 32768;  // B * parts * rec_rows_for(H, q_len) at most
constexpr size_t kScratchBytes = kScratchRecords * (kLat + 2) * sizeof(float) + (size_t)kMaxPagedB * 8;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device (0 or a HIP error code).
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return -10;
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return -10;
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return 0;
}

}  // namespace

extern "C" {

// Records (O [512] + (m, l) per query row and part) plus an 8-byte
// (parts, first record) entry per request.
size_t mla_decode_a16w8_workspace_bytes(void) { return kMaxRecords * (kLat + 2) * sizeof(float) + kMaxRecords * 8; }

size_t mla_decode_a16w8_multiq_workspace_for(int B, int H, int parts, int q_len) {
  if (B < 1 || H < 1 || q_len < 1) return 0;
  return split_ws_bytes(B, H, clamp_parts(parts, B, H, q_len, true), q_len);
}

int launch_mla_decode_a16w8(const void* q_lat, const void* q_pe, const void* c_kv, const void* k_pe, void* o_lat,
                            int B, int H, int S, int lat_dim, int rope_dim, float scale, float kv_scale,
                            float scale_p, void* workspace, void* stream) {
  (void)k_pe;
  (void)scale_p;
  const int parts = workspace ? plan_parts(B, H, S, 1) : 1;
  return launch(q_lat, q_pe, c_kv, o_lat, nullptr, nullptr, nullptr, nullptr, B, H, S, parts, 1, lat_dim, rope_dim,
                scale, kv_scale, workspace, stream, false);
}

int launch_mla_decode_a16w8_paged_dev(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                      const void* seq_lens, const void* rows, const void* kv_indices,
                                      const void* kv_indptr, int B, int H, int parts, int lat_dim, int rope_dim,
                                      float scale, float kv_scale, float scale_p, void* workspace, void* stream,
                                      size_t kv_bytes, int q_len) {
  (void)scale_p;
  (void)kv_bytes;
  return launch(q_lat, q_pe, kv_pool, o_lat, seq_lens, rows, kv_indices, kv_indptr, B, H, 0, parts, q_len, lat_dim,
                rope_dim, scale, kv_scale, workspace, stream, true);
}

int launch_mla_decode_a16w8_paged_dev_noalloc(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                              const void* seq_lens, const void* rows, const void* kv_indices,
                                              const void* kv_indptr, int B, int H, int parts, int lat_dim,
                                              int rope_dim, float scale, float kv_scale, float scale_p, void* stream,
                                              size_t kv_bytes, int q_len) {
  (void)scale_p;
  (void)kv_bytes;
  // The workspace launcher's argument codes first, then the scratch limit.
  const int arg_rc = check_launch_args(q_lat, q_pe, kv_pool, o_lat, seq_lens, kv_indices, kv_indptr, B, H, 0, q_len,
                                       lat_dim, rope_dim, true);
  if (arg_rc != 0) return arg_rc;
  const int eff = clamp_parts(parts, B, H, q_len, true);
  void* ws = nullptr;
  if (eff > 1) {
    if ((size_t)B * eff * rec_rows_for(H, q_len) > kScratchRecords) return -9;
    const int rc = scratch_ptr(&ws);
    if (rc != 0) return rc;
  }
  return launch(q_lat, q_pe, kv_pool, o_lat, seq_lens, rows, kv_indices, kv_indptr, B, H, 0, eff, q_len, lat_dim,
                rope_dim, scale, kv_scale, ws, stream, true);
}

size_t mla_decode_a16w8_blocks_index_bytes(int B, int max_blocks) {
  if (B < 1 || max_blocks < 1) return 0;
  return ((size_t)B * max_blocks * 64 + 2 * (size_t)B + 1) * sizeof(int);
}

int launch_mla_decode_a16w8_paged_blocks_dev(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                             const void* seq_lens, const void* rows, const void* block_table,
                                             int max_blocks, int num_blocks, int B, int H, int parts, int q_len,
                                             int lat_dim, int rope_dim, float scale, float kv_scale, float scale_p,
                                             void* workspace, void* index_workspace, void* stream) {
  (void)scale_p;
  if (!seq_lens || !block_table || !index_workspace) return -6;
  if (B < 1 || B > kMaxPagedB) return -4;
  if (max_blocks < 1 || num_blocks < 1) return -11;
  const long long words = (long long)B * max_blocks * 64 + 2LL * B + 1;
  if (words > 0x7FFFFFFFLL || (long long)num_blocks * 64 > 0x7FFFFFFFLL) return -11;
  int* ws = static_cast<int*>(index_workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const long long pages = (long long)B * max_blocks;
  hipLaunchKernelGGL(expand_block_table_kernel, dim3((unsigned)((pages + 3) / 4)), dim3(256), 0, st,
                     static_cast<const int*>(seq_lens), static_cast<const int*>(block_table), max_blocks, num_blocks,
                     B, ws);
  const long long stride_all = (long long)B * max_blocks * 64;
  return launch(q_lat, q_pe, kv_pool, o_lat, ws + stride_all, rows, ws, ws + stride_all + B, B, H, 0, parts, q_len,
                lat_dim, rope_dim, scale, kv_scale, workspace, stream, true);
}

int launch_mla_decode_a16w8_multiq(const void* q_lat, const void* q_pe, const void* kv, void* o_lat, int B, int H,
                                   int S, int q_len, int lat_dim, int rope_dim, float scale, float kv_scale,
                                   void* workspace, void* stream) {
  const int parts = workspace ? plan_parts(B, H, S, q_len) : 1;
  return launch(q_lat, q_pe, kv, o_lat, nullptr, nullptr, nullptr, nullptr, B, H, S, parts, q_len, lat_dim,
                rope_dim, scale, kv_scale, workspace, stream, false);
}

int launch_mla_decode_a16w8_multiq_paged_dev(const void* q_lat, const void* q_pe, const void* kv_pool, void* o_lat,
                                             const void* seq_lens, const void* rows, const void* kv_indices,
                                             const void* kv_indptr, int B, int H, int parts, int q_len,
                                             int lat_dim, int rope_dim, float scale, float kv_scale,
                                             void* workspace, void* stream, size_t kv_bytes) {
  (void)kv_bytes;
  return launch(q_lat, q_pe, kv_pool, o_lat, seq_lens, rows, kv_indices, kv_indptr, B, H, 0, parts, q_len, lat_dim,
                rope_dim, scale, kv_scale, workspace, stream, true);
}

int mla_decode_a16w8_plan_parts(int B, int H, int max_seq_len, int lat_dim) {
  (void)lat_dim;
  return plan_parts(B, H, max_seq_len, 1);
}

int mla_decode_a16w8_plan_parts_q(int B, int max_seq_len, int q_len, int H) {
  if (q_len > kMaxQLen) return -4;
  return plan_parts(B, H, max_seq_len, q_len < 1 ? 1 : q_len);
}

int mla_decode_a16w8_plan_parts_capped(int B, int H, int max_seq_len, int lat_dim) {
  (void)lat_dim;
  return plan_parts(B, H, max_seq_len, 1);
}

int mla_decode_a16w8_multiq_plan_parts_q(int B, int max_seq_len, int q_len, int H) {
  if (q_len > kMaxQLen) return -4;
  return plan_parts(B, H, max_seq_len, q_len < 1 ? 1 : q_len);
}

int mla_decode_a16w8_max_ctas(void) { return (int)(kMaxRecords / kQRowsPerCta); }

int moonmath_mla_effective_parts(int B, int H, int parts, int q_len, int have_workspace) {
  if (B < 1 || H < 1 || q_len < 1) return 1;
  return clamp_parts(parts, B, H, q_len, have_workspace != 0);
}

int moonmath_fp8e4m3_to_bf16(const void* in, void* out, int n, void* stream) {
  if (!in || !out || n < 0) return -6;
  if (n == 0) return 0;
  const int threads = 256;
  const int blocks = ((n + 3) / 4 + threads - 1) / threads;
  hipLaunchKernelGGL(fp8_to_bf16_kernel, dim3(blocks), dim3(threads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(in), static_cast<uint16_t*>(out), n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // extern "C"
