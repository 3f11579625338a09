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

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "mm_common.hpp"

namespace mm {
namespace mla {

constexpr int kLat = 512;
constexpr int kRope = 64;
constexpr int kQK = kLat + kRope;              // 576 bytes per fp8 row
constexpr int kTileTok = 32;                   // tokens per tile
constexpr int kTileBytes = kTileTok * kQK;     // 18432 fp8 bytes per tile
constexpr int kDmaPerTile = kTileBytes / 1024; // 18 wave-DMA instructions (64 x 16 B)
constexpr int kRowsPerCta = 32;                // query rows per CTA (one MFMA tile)
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kKPairs = kQK / 32;              // 18 pairs of 16-dim k-steps (16 latent + 2 rope)
constexpr int kDTiles = kLat / 32;             // 16 output d-tiles of 32
constexpr int kMaxQLen = 8;
constexpr int kMaxHeads = 128;
constexpr int kIdxCap = 2048;                  // slot indices resident in LDS per sub-range
// A row's running max is fixed at its first non-empty tile; later tiles may
// exceed it by up to 2^64 (p <= 2^64, no fp32 overflow of O or l). Beyond that
// the CTA falls back to an exact-max second pass.
constexpr float kGrowLimit = 64.f;

// LDS map (bytes): per-wave 2-slot tile rings, the slot indices of the current
// sub-range, the rope part of Q. The merge at the end reuses the tile rings.
constexpr int kRingBytes = 2 * kTileBytes;                  // 36864 per wave
constexpr int kStageBytes = kWaves * kRingBytes;            // 147456
constexpr int kIdxOff = kStageBytes;
constexpr int kQpeOff = kIdxOff + kIdxCap * 4;              // 155648
constexpr int kLdsBytes = kQpeOff + kRowsPerCta * kRope * 2;  // 159744
// Merge area: [wave][dt][i4][lane] x 16 B of O for 8 d-tiles, then (m, l).
constexpr int kMergeOBytes = 8 * 4 * 64 * 16;              // 32768 per wave and half
constexpr int kMergeMlOff = kWaves * kMergeOBytes;          // 131072
static_assert(kMergeMlOff + kWaves * 64 * 8 <= kStageBytes, "merge area fits the rings");

// Split partial records: one per (b, part, query row): O [512] fp32, then all
// (m, l) pairs after the last O record. kMaxRecords caps the workspace.
constexpr size_t kMaxRecords = 65536;

struct Params {
  const uint16_t* q_lat;  // [B, q_len, H, 512] bf16 (q_len 1: [B, H, 512])
  const uint16_t* q_pe;   // [B, q_len, H, 64]
  const uint8_t* kv;      // paged: [slots, 576] fp8; contiguous: [B, S, 576]
  uint16_t* o_lat;        // like q_lat
  float* ws;              // split partials (parts > 1)
  const int* seq_lens;    // [B] (paged)
  const int* rows;        // [B] q/out row per request, or null
  const int* kv_indices;  // flat per-token slots (paged)
  const int* kv_indptr;   // [B+1] (paged)
  int B, H, q_len, S_fixed, parts, ngroups, paged;
  int qrows;              // H * q_len
  float score_c;          // scale * kv_scale * log2(e), fp32
  float kv_scale;
};

typedef int i32x2 __attribute__((ext_vector_type(2)));

// Two fp8 of a dword (lo or hi half) -> two bf16, exact (scale 1).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_bf16(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}
__device__ __forceinline__ bf16x8 fp8x8_bf16(uint32_t lo, uint32_t hi) {
  u32x4 o = {fp8x2_bf16<false>(lo), fp8x2_bf16<true>(lo), fp8x2_bf16<false>(hi), fp8x2_bf16<true>(hi)};
  return __builtin_bit_cast(bf16x8, o);
}

// O^T += V^T P^T into an AGPR accumulator. The s_nop covers the VALU-write ->
// MFMA-read distance for operands converted just before (the compiler cannot
// see through the asm); consecutive calls always target different
// accumulators, and every VALU read of an accumulator is preceded by
// mfma_result_fence().
__device__ __forceinline__ void pv_mfma(f32x16& acc, bf16x8 a, bf16x8 b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// 16-byte global -> LDS DMA issued through asm. The kernel counts these loads
// itself (explicit s_waitcnt vmcnt); hiding them from the compiler keeps it
// from adding a conservative vmcnt(0) before every LDS transpose read (it
// cannot prove those reads do not alias an in-flight DMA).
__device__ __forceinline__ void dma16_opaque(const void* gsrc, const char* lds_dst) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)lds_dst;
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gsrc), "{m0}"(m0v) : "memory");
}

// Request holding length rank `rank` (0 = longest) among B requests, in an
// approximate longest-first order: 16 linear length buckets, longest bucket
// first, request index order inside a bucket. Wave-uniform; every wave of a
// CTA computes it independently from the same seq_lens.
__device__ __forceinline__ int request_of_rank(const int* seq_lens, int B, int rank, int lane) {
  int maxl = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int l = (c0 + lane < B) ? seq_lens[c0 + lane] : 0;
    int m = l;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max(m, __shfl_xor(m, off));
    maxl = max(maxl, m);
  }
  maxl = __builtin_amdgcn_readfirstlane(maxl);
  auto bucket_of = [&](int l) {  // 0 = longest lengths
    const long long q = (long long)l * 16 / ((long long)maxl + 1);
    return 15 - (int)q;
  };
  // Bucket sizes over all requests.
  int start[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) start[k] = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const bool valid = c0 + lane < B;
    const int bk = valid ? bucket_of(seq_lens[c0 + lane]) : -1;
#pragma unroll
    for (int k = 0; k < 16; ++k) start[k] += __builtin_popcountll(__builtin_amdgcn_ballot_w64(bk == k));
  }
  int acc = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int c = start[k];
    start[k] = acc;
    acc += c;
  }
  // Position of every request; the one at `rank` wins.
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const bool valid = c0 + lane < B;
    const int bk = valid ? bucket_of(seq_lens[c0 + lane]) : -1;
    int pos = -1;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const unsigned long long m = __builtin_amdgcn_ballot_w64(bk == k);
      if (bk == k) pos = start[k] + __builtin_popcountll(m & lt);
      start[k] += __builtin_popcountll(m);
    }
    const unsigned long long hit = __builtin_amdgcn_ballot_w64(valid && pos == rank);
    if (hit) return c0 + (int)__builtin_ctzll(hit);
  }
  return 0;  // unreachable for rank < B
}

// Staging layout of one tile: token t's 576-byte row at t*576, its 16-byte
// piece c stored at piece slot c ^ swz(t) (a permutation inside each aligned
// group of 4 pieces) so the 32 lanes of a K read and the 8-token groups of a
// V^T transpose read hit distinct LDS banks.
__device__ __forceinline__ int swz(int t) { return (t >> 2) & 3; }

template <bool PAGED>
__global__ __launch_bounds__(kThreads, 1) void mla_decode_kernel(Params p) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  int* idx_lds = reinterpret_cast<int*>(lds + kIdxOff);
  char* qpe_lds = lds + kQpeOff;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31;  // MFMA column: query row (S^T, O^T) / token or dim row of A
  const int g = lane >> 5;  // lane half
  char* wring = lds + wave * kRingBytes;

  // ---- work item ----------------------------------------------------------------------
  // Workgroups are dispatched round-robin over the 8 XCDs (blockIdx % 8) and in
  // blockIdx order within an XCD. Request slots are dealt to XCDs in snake order
  // of decreasing length (XCD x takes length ranks x, 15-x, 16+x, 31-x, ...), so
  // every XCD gets a similar share, the E = parts * ngroups CTAs of a request
  // run on one XCD (its KV is shared through that L2) and each XCD starts its
  // longest requests first.
  const int E = p.parts * p.ngroups;
  const int xcd = blockIdx.x % kNumXcds;
  const int k_in_xcd = blockIdx.x / kNumXcds;
  const int tslot = k_in_xcd / E, e = k_in_xcd % E;
  const int rank = 16 * (tslot >> 1) + ((tslot & 1) ? 15 - xcd : xcd);
  if (rank >= p.B) return;  // padding CTA (whole CTA, before any barrier)
  const int part = e / p.ngroups;
  const int grp = e % p.ngroups;
  const int b = PAGED ? request_of_rank(p.seq_lens, p.B, rank, lane) : rank;
  int qb = b;
  if (p.rows) {
    qb = p.rows[b];
    qb = qb < 0 ? 0 : (qb >= p.B ? p.B - 1 : qb);
  }
  const int S = PAGED ? p.seq_lens[b] : p.S_fixed;
  const int slot0 = PAGED ? p.kv_indptr[b] : 0;
  // Proportional split: each part covers ceil(S / parts) tokens rounded to tiles.
  const int part_tok = ((S + p.parts * kTileTok - 1) / (p.parts * kTileTok)) * kTileTok;
  const int kv_lo = part * part_tok;
  const int kv_hi = (kv_lo + part_tok < S) ? kv_lo + part_tok : S;

  // ---- query row of this lane ----------------------------------------------------
  const int qrow = grp * kRowsPerCta + n;  // row within (t, h)
  const bool row_ok = qrow < p.qrows;
  const int qr = row_ok ? qrow : p.qrows - 1;
  const int t_pos = qr / p.H;
  const int lim = S - (p.q_len - 1 - t_pos);  // tokens >= lim are masked for this row
  const long long qoff = (long long)qb * p.qrows + qr;  // row index into [B, q_len, H]

  // Q fragments (B operand of S^T = K Q^T). k-step pair s covers dims
  // 32s + 16g .. +16 of lane half g: the first 8 feed k-step 2s, the next 8 k-step
  // 2s+1 (the same dims the K fragment of that lane half holds).
  bf16x8 qf[2 * (kKPairs - 2)];
#pragma unroll
  for (int s = 0; s < kKPairs - 2; ++s) {
    const uint16_t* src = p.q_lat + qoff * kLat + s * 32 + g * 16;
    qf[2 * s] = *reinterpret_cast<const bf16x8*>(src);
    qf[2 * s + 1] = *reinterpret_cast<const bf16x8*>(src + 8);
  }
  // Rope part of Q: 32 rows x 64 bf16 in LDS (row n at n * 128 B).
  if (tid < kRowsPerCta * 8) {
    const int r = tid >> 3, c = tid & 7;
    const int rr = grp * kRowsPerCta + r;
    const long long ro = (long long)qb * p.qrows + (rr < p.qrows ? rr : p.qrows - 1);
    *reinterpret_cast<bf16x8*>(qpe_lds + r * 128 + c * 16) =
        *reinterpret_cast<const bf16x8*>(p.q_pe + ro * kRope + c * 8);
  }

  // Retire the Q loads here, visibly to the compiler (vmcnt 0, expcnt/lgkmcnt
  // untouched): the tile DMAs are invisible to its wait-count model, so a Q
  // wait left to the loop would become a per-tile vmcnt countdown that also
  // waits for the prefetched tile.
  __builtin_amdgcn_s_waitcnt(0x0F70);

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
  int dma_off[9];
#pragma unroll
  for (int k9 = 0; k9 < 9; ++k9) {
    const int pc = 64 * k9 + lane;
    const int tg = pc / 36, cs = pc % 36;
    dma_off[k9] = tg * kQK + 16 * (cs ^ swz(tg));
  }

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
  for (int sub_lo = kv_lo; sub_lo < kv_hi; sub_lo += kIdxCap) {
    const int sub_hi = (sub_lo + kIdxCap < kv_hi) ? sub_lo + kIdxCap : kv_hi;
    const int ntiles = (sub_hi - sub_lo + kTileTok - 1) / kTileTok;
    if constexpr (PAGED) {
      lds_reads_done_barrier_vm0();  // every wave is done with the previous indices
      for (int i = tid; i < sub_hi - sub_lo; i += kThreads) idx_lds[i] = p.kv_indices[slot0 + sub_lo + i];
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
      if (sub_lo == kv_lo) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");  // qpe_lds
    }
    const int eff = lim < sub_hi ? lim : sub_hi;  // this row's token limit in the sub-range

    // Gather plan of tile j (tokens sub_lo + 32j ..). Fast path: the 32 rows are
    // consecutive slots (always for the contiguous layout, and for paged tiles
    // inside one page): DMA k reads base + (k/9)*16 rows + dma_off[k%9]. Slow
    // path: every lane looks its row up, with tokens past sub_hi clamped to the
    // last valid one (their scores are masked).
    auto tile_fast = [&](int j, const uint8_t*& base) -> bool {
      const int tok0 = sub_lo + j * kTileTok;
      bool fast = tok0 + kTileTok <= sub_hi;
      long long row0 = (long long)b * p.S_fixed + tok0;
      if constexpr (PAGED) {
        if (fast) {
          const int i0 = __builtin_amdgcn_readfirstlane(idx_lds[tok0 - sub_lo]);
          const int mine = idx_lds[tok0 - sub_lo + n];
          fast = __builtin_amdgcn_ballot_w64(mine == i0 + n) == ~0ull;
          row0 = i0;
        }
      }
      base = p.kv + row0 * kQK;
      return fast;
    };
    auto issue_slow = [&](int j, const char* dst) {
      const int tok0 = sub_lo + j * kTileTok;
#pragma unroll 1
      for (int k = 0; k < kDmaPerTile; ++k) {
        const int k9 = k % 9;
        const int pc = 64 * k9 + lane;
        const int tg = pc / 36, cs = pc - 36 * (pc / 36);
        int tok = tok0 + (k / 9) * 16 + tg;
        tok = tok < sub_hi ? tok : sub_hi - 1;
        long long row;
        if constexpr (PAGED) {
          row = idx_lds[tok - sub_lo];
        } else {
          row = (long long)b * p.S_fixed + tok;
        }
        dma16_opaque(p.kv + row * kQK + 16 * (cs ^ swz(tg)), dst + 1024 * k);
      }
    };
    auto issue_tile = [&](int j, const char* dst) {
      const uint8_t* base;
      if (tile_fast(j, base)) {
#pragma unroll
        for (int k = 0; k < kDmaPerTile; ++k) dma16_opaque(base + (k / 9) * 16 * kQK + dma_off[k % 9], dst + 1024 * k);
      } else {
        issue_slow(j, dst);
      }
    };

    int slot = 0;
    if (wave < ntiles) issue_tile(wave, wring);
    for (int j = wave; j < ntiles; j += kWaves) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this tile has landed
      const char* st = wring + slot * kTileBytes;
      const char* nst = wring + (slot ^ 1) * kTileBytes;
      const int tok0 = sub_lo + j * kTileTok;
      // Next tile of this wave: a fast-path gather is spread over the 18 QK
      // steps below (one DMA each); a slow-path gather is issued here.
      const uint8_t* nbase = nullptr;
      bool ndma = false;
      if (j + kWaves < ntiles) {
        ndma = tile_fast(j + kWaves, nbase);
        if (!ndma) issue_slow(j + kWaves, nst);
      }

      // ---- S^T = K Q^T: 18 k-step pairs, two accumulator chains ------------------------
      // K pieces are read kKAhead pairs ahead of their conversion; sched_fence()
      // keeps each step's [DMA, read ahead, convert, 2 MFMA] order.
      constexpr int kKAhead = 4;
      auto kaddr = [&](int s) { return st + ((s & 1) ? koff1 : koff0) + 64 * (s >> 1); };
      u32x4 kraw[kKAhead];
#pragma unroll
      for (int s = 0; s < kKAhead; ++s) kraw[s] = *reinterpret_cast<const u32x4*>(kaddr(s));
      bf16x8 qpe[4];
      f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
      for (int s = 0; s < kKPairs; ++s) {
        if (ndma) dma16_opaque(nbase + (s / 9) * 16 * kQK + dma_off[s % 9], nst + 1024 * s);
        const u32x4 raw = kraw[s % kKAhead];
        if (s + kKAhead < kKPairs) kraw[s % kKAhead] = *reinterpret_cast<const u32x4*>(kaddr(s + kKAhead));
        if (s == kKPairs - 2 - kKAhead) {  // rope part of Q for the last two pairs
          const char* qp = qpe_lds + n * 128 + g * 32;
          qpe[0] = *reinterpret_cast<const bf16x8*>(qp);
          qpe[1] = *reinterpret_cast<const bf16x8*>(qp + 16);
          qpe[2] = *reinterpret_cast<const bf16x8*>(qp + 64);
          qpe[3] = *reinterpret_cast<const bf16x8*>(qp + 80);
        }
        const bf16x8 ka = fp8x8_bf16(raw[0], raw[1]);
        const bf16x8 kb = fp8x8_bf16(raw[2], raw[3]);
        const bf16x8 qa = (s < kKPairs - 2) ? qf[2 * s] : qpe[2 * (s - (kKPairs - 2))];
        const bf16x8 qb2 = (s < kKPairs - 2) ? qf[2 * s + 1] : qpe[2 * (s - (kKPairs - 2)) + 1];
        s0 = mfma32(ka, qa, s0);
        s1 = mfma32(kb, qb2, s1);
        sched_fence();
      }
      // V^T transpose reads for the first PV steps go out before the softmax.
      constexpr int kVAhead = 8;
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
      for (int i = 0; i < 16; ++i) sv[i] = s0[i] + s1[i];
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

  sweep(std::false_type{});
  // Fallback (never taken unless some row's scores rise more than 2^64 above
  // its first tile): every wave redoes its tiles with the exact row max. The
  // decision is CTA-uniform because the sweeps hold CTA barriers.
  {
    int* flags = reinterpret_cast<int*>(lds + kMergeMlOff);
    lds_reads_done_barrier_vm0();
    if (lane == 0) flags[wave] = __builtin_amdgcn_ballot_w64(grew) != 0;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const bool retry = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
    if (retry) {
      row_m = -__builtin_inff();
      sweep(std::true_type{});
      row_m = __builtin_ceilf(row_m * c);
      row_l = 0.f;
      mfma_result_fence();
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) oacc[dt] = f32x16{};
      sweep(std::false_type{});
    }
  }

  // ---- merge the 4 waves' (O, m, l) through LDS ---------------------------------------
  // Rows of lanes n and n+32 are the same query row: m agrees, l is summed at the end.
  mfma_result_fence();
  lds_reads_done_barrier_vm0();  // every wave is done with its ring
  float* mlarea = reinterpret_cast<float*>(lds + kMergeMlOff);
  mlarea[(wave * 64 + lane) * 2] = row_m;
  mlarea[(wave * 64 + lane) * 2 + 1] = row_l;
  // Lane weights of the 4 waves, exact powers of two.
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  float mw[kWaves], lw[kWaves];
  float M = -__builtin_inff();
#pragma unroll
  for (int v = 0; v < kWaves; ++v) {
    mw[v] = mlarea[(v * 64 + lane) * 2];
    lw[v] = mlarea[(v * 64 + lane) * 2 + 1];
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
  const bool split = p.parts > 1;
  const float inv = (L == 0.f) ? 0.f : p.kv_scale * __builtin_amdgcn_rcpf(L);
  const size_t rec = ((size_t)b * p.parts + part) * p.qrows + qrow;
  uint16_t* orow = p.o_lat + ((long long)qb * p.qrows + qrow) * kLat;
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
        if (row_ok) {
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
  if (split && row_ok && g == 0 && wave == 0) {
    float* pml = p.ws + (size_t)p.B * p.parts * p.qrows * kLat + rec * 2;
    pml[0] = M;
    pml[1] = L;
  }
}

// Merge: one thread = 4 output dims of one (b, query row).
// M = max_p m_p, w_p = 2^(m_p - M), out = sum w_p O_p * kv_scale / sum w_p l_p.
__global__ __launch_bounds__(256) void mla_merge_kernel(Params p) {
  const long long cell = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long per_b = (long long)p.qrows * (kLat / 4);
  if (cell >= per_b * p.B) return;
  const int b = (int)(cell / per_b);
  const int rem = (int)(cell % per_b);
  const int qrow = rem / (kLat / 4);
  const int d = (rem % (kLat / 4)) * 4;
  int qb = b;
  if (p.rows) {
    qb = p.rows[b];
    qb = qb < 0 ? 0 : (qb >= p.B ? p.B - 1 : qb);
  }
  const float* ml = p.ws + (size_t)p.B * p.parts * p.qrows * kLat;
  float M = -__builtin_inff();
  for (int j = 0; j < p.parts; ++j) {
    const size_t rec = ((size_t)b * p.parts + j) * p.qrows + qrow;
    M = fmaxf(M, ml[rec * 2]);
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  for (int j = 0; j < p.parts; ++j) {
    const size_t rec = ((size_t)b * p.parts + j) * p.qrows + qrow;
    const float m_p = ml[rec * 2];
    const float l_p = ml[rec * 2 + 1];
    const float diff = m_p - M;  // integer-valued or -inf, <= 0
    const float wt = (m_p == -__builtin_inff()) ? 0.f : ((diff >= -126.f) ? __builtin_ldexpf(1.0f, (int)diff) : 0.f);
    const f32x4 o = *reinterpret_cast<const f32x4*>(p.ws + rec * kLat + d);
    acc[0] = __builtin_fmaf(wt, o[0], acc[0]);
    acc[1] = __builtin_fmaf(wt, o[1], acc[1]);
    acc[2] = __builtin_fmaf(wt, o[2], acc[2]);
    acc[3] = __builtin_fmaf(wt, o[3], acc[3]);
    L = __builtin_fmaf(wt, l_p, L);
  }
  const float inv = (L == 0.f) ? 0.f : p.kv_scale * __builtin_amdgcn_rcpf(L);
  u32x2 o;
  o[0] = pack2_bf16_canon<kRTNE>(acc[0] * inv, acc[1] * inv);
  o[1] = pack2_bf16_canon<kRTNE>(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<u32x2*>(p.o_lat + ((long long)qb * p.qrows + qrow) * kLat + d) = o;
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
constexpr int kCtasPerCu = 1;
constexpr int kMaxParts = 64;

int ngroups_for(int H, int q_len) { return (H * q_len + kQRowsPerCta - 1) / kQRowsPerCta; }

// Largest parts the fixed record workspace allows for (B, H, q_len).
int max_parts_for(int B, int H, int q_len) {
  const long long per_part = (long long)B * H * q_len;
  long long m = per_part > 0 ? (long long)kMaxRecords / per_part : 1;
  if (m > kMaxParts) m = kMaxParts;
  return m < 1 ? 1 : (int)m;
}

// Split planner: enough CTAs for ~2 rounds over the CUs (ragged lengths balance
// across rounds), at least 4 tiles per wave in a part, within the record workspace.
int plan_parts(int B, int H, int max_seq_len, int q_len) {
  if (B < 1) B = 1;
  if (q_len < 1) q_len = 1;
  const int tiles = (max_seq_len + kTileTok - 1) / kTileTok;
  const int ctas_per_part = B * ngroups_for(H, q_len);
  int p = (2 * kNumCUs * kCtasPerCu + ctas_per_part - 1) / ctas_per_part;
  if (p > tiles / 16) p = tiles / 16;
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

int launch(const void* q_lat, const void* q_pe, const void* kv, void* o_lat, const void* seq_lens,
           const void* rows, const void* kv_indices, const void* kv_indptr, int B, int H, int S_fixed, int parts,
           int q_len, int lat_dim, int rope_dim, float scale, float kv_scale, void* workspace, void* stream,
           bool paged) {
  if (lat_dim != kLat || rope_dim != kRope) return -2;
  if (H < 1 || H > kMaxHeads) return -3;
  if (q_len < 1 || q_len > kMaxQLen || B < 1) return -4;
  if (!q_lat || !q_pe || !kv || !o_lat) return -6;
  if (paged && (!seq_lens || !kv_indices || !kv_indptr)) return -6;
  if (!paged && S_fixed < 1) return -7;
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
  p.paged = paged ? 1 : 0;
  p.qrows = H * q_len;
  p.score_c = (float)((double)scale * (double)kv_scale * 1.4426950408889634);
  p.kv_scale = kv_scale;
  // Request slots per XCD for the snake deal of ranks 0..B-1 (see the kernel).
  const int slots_per_xcd = 2 * ((B - 1) / 16) + (((B - 1) % 16) >= 8 ? 2 : 1);
  const long long grid = (long long)mm::kNumXcds * slots_per_xcd * p.parts * p.ngroups;
  if (grid > 0x7FFFFFFFLL) return -8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (paged)
    hipLaunchKernelGGL(mla_decode_kernel<true>, dim3((unsigned)grid), dim3(kThreads), 0, st, p);
  else
    hipLaunchKernelGGL(mla_decode_kernel<false>, dim3((unsigned)grid), dim3(kThreads), 0, st, p);
  if (p.parts > 1) {
    const long long cells = (long long)B * p.qrows * (kLat / 4);
    hipLaunchKernelGGL(mla_merge_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, st, p);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // namespace

extern "C" {

size_t mla_decode_a16w8_workspace_bytes(void) { return kMaxRecords * (kLat + 2) * sizeof(float); }

size_t mla_decode_a16w8_multiq_workspace_for(int B, int H, int parts, int q_len) {
  if (B < 1 || H < 1 || q_len < 1) return 0;
  const int p = clamp_parts(parts, B, H, q_len, true);
  return (size_t)B * p * H * q_len * (kLat + 2) * sizeof(float);
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
