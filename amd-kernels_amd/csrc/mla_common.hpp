// Shared pieces of the gfx950 absorbed-MLA decode kernels (mla_coop.hip: up
// to 16 query rows per CTA; mla_decode.hip: 32; mla_wide.hip: 128): the fused
// fp8 row format, launch parameters, exact fp8 -> bf16 widening, and the
// device-side split plan the kernels deal their units from.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mm_common.hpp"

namespace mm {
namespace mla {

constexpr int kLat = 512;
constexpr int kRope = 64;
constexpr int kQK = kLat + kRope;              // 576 bytes per fp8 row
constexpr int kTileTok = 32;                   // tokens per tile
constexpr int kTileBytes = kTileTok * kQK;     // 18432 fp8 bytes per tile
constexpr int kDmaPerTile = kTileBytes / 1024; // 18 wave-DMA instructions (64 x 16 B)
constexpr int kKPairs = kQK / 32;              // 18 pairs of 16-dim k-steps (16 latent + 2 rope)
constexpr int kDTiles = kLat / 32;             // 16 output d-tiles of 32
constexpr int kMaxQLen = 8;
constexpr int kMaxHeads = 128;
// A row's running max is fixed at its first non-empty tile; later tiles may
// exceed it by up to 2^64 (p <= 2^64, no fp32 overflow of O or l). Beyond that
// the CTA falls back to an exact-max second pass.
constexpr float kGrowLimit = 64.f;
// Q dims [448, 576) (the last four k-step pairs) stay in LDS, the rest in
// VGPRs: 256 B per query row in LDS, 16-byte chunk c of row r at chunk c ^ (r & 15).
constexpr int kQRegPairs = 14;                 // k-step pairs whose Q lives in VGPRs
constexpr int kQLdsDim0 = kQRegPairs * 32;     // 448
constexpr int kQLdsRowBytes = (kQK - kQLdsDim0) * 2;  // 256
// Order of the k-step pairs in the QK loops: position s handles pair
// qk_pair_at(s). The four LDS-resident pairs run at positions 6..9, not last,
// so their one-step-ahead Q reads overlap the K reads already in flight (and,
// in the 128-row kernel, steps that also carry PV MFMAs): -2% for the 32-row
// kernel at H=128 q_len 2. The scores are fp32 sums in a different order,
// equally close to the exact sum.
__device__ __forceinline__ constexpr int qk_pair_at(int s) { return s < 6 ? s : (s < 10 ? s + 8 : s - 4); }
static_assert(kQRegPairs == 14 && kKPairs == 18, "qk_pair_at permutes 18 pairs with the LDS ones at 6..9");

// Split partial records. Workspace: the O records (one per (b, part): rec_rows
// rows of 512 fp32, row-major, or in the 128-row kernel's fragment order), then
// the (m, l) pair of every (b, part, query row), then an 8-byte (parts, first
// record) entry per request. kMaxRecords caps the O rows of a workspace.
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
  int unit_cap;           // units one round of CTAs over the CUs holds
  int qrows;              // H * q_len
  int rec_rows;           // O rows per split record: qrows, or a multiple of 32 for the fragment order
  int rec_frag;           // 1: O records in the 128-row kernel's fragment order
  float score_c;          // scale * kv_scale * log2(e), fp32
  float kv_scale;
};

// Split workspace regions (see kMaxRecords).
__device__ __forceinline__ float* ws_rec_o(const Params& p, size_t rec) { return p.ws + rec * p.rec_rows * kLat; }
__device__ __forceinline__ float* ws_ml(const Params& p) { return p.ws + (size_t)p.B * p.parts * p.rec_rows * kLat; }
__device__ __forceinline__ int* ws_tbl(const Params& p) {
  return reinterpret_cast<int*>(ws_ml(p) + (size_t)p.B * p.parts * p.qrows * 2);
}

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

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

// Field `k` (16 bits) of a packed pair, extracted where it is used (volatile:
// not hoisted, so the packed pairs are what stays live).
__device__ __forceinline__ uint32_t u16_field(uint32_t w, int k) {
  uint32_t r;
  asm volatile("v_bfe_u32 %0, %1, %2, 16" : "=v"(r) : "v"(w), "i"(16 * k));
  return r;
}

// ---- split plan ------------------------------------------------------------------------
// The caller's `parts` P and the launch's unit cap (the CTAs of one round of
// the grid over the CUs, divided by the CTAs per unit) set a budget of
//   U = max(B, min(B * P, cap))
// units (request parts). Every request is cut into chunks of C tokens, request
// b getting nparts_b = max(1, ceil(L_b / C)) parts of equal size (rounded up to
// 32 tokens; the last part takes the remainder), with C the smallest multiple
// of 32, at least 512, for which sum_b nparts_b <= U -- found by bisection,
// since the count only falls as C grows and C = max_b L_b gives B units. So the
// partial records always fit the B * P * qrows workspace, one round of CTAs
// covers the batch, and the longest part (the CTA that ends last) is as short
// as the budget allows.
constexpr int kMinChunk = 512;
// The paged plan keeps three B-entry tables (12 * B bytes) in LDS scratch.
constexpr int kMaxPagedB = 3072;  // 12 B per request: 36 KB of plan scratch

// ceil(a / d) for 0 <= a, 1 <= d, a + d < 2^32.
__device__ __forceinline__ int ceil_div_u(int a, int d) {
  return (int)(((unsigned)a + (unsigned)d - 1u) / (unsigned)d);
}
__device__ __forceinline__ int nparts_of(int L, int C) { return L <= C ? 1 : ceil_div_u(L, C); }
// Tokens per part of a request of L tokens in np parts: equal shares rounded up
// to whole tiles (the last part takes the remainder).
__device__ __forceinline__ int part_tokens(int L, int np) {
  return (ceil_div_u(L, np) + kTileTok - 1) & ~(kTileTok - 1);
}
__device__ __forceinline__ int unit_budget(int B, int P, int cap) {
  const long long bp = (long long)B * (P < 1 ? 1 : P);
  const long long m = bp < cap ? bp : cap;
  return (int)(m > B ? m : B);
}
// Smallest chunk C (a multiple of 32, >= kMinChunk) with units(C) <= budget,
// for a units(C) that is non-increasing in C with units(max L) = B <= budget.
// Wave-uniform.
template <class UnitsFn>
__device__ int search_chunk(long long sumL, int maxL, int B, int budget, UnitsFn units) {
  int hi = maxL < kMinChunk ? kMinChunk : ((maxL + kTileTok - 1) & ~(kTileTok - 1));
  if (budget <= B) return hi;  // one part per request
  // ceil(L / C) < L / C + 1, so C >= sumL / (budget - B) is feasible too.
  auto ceil_div_ll = [](long long a, int d) -> long long {  // 32-bit division whenever it suffices
    return a < 0x7FFFFFFF ? (long long)ceil_div_u((int)a, d) : (a + d - 1) / d;
  };
  const long long ok = ceil_div_ll(sumL, budget - B);
  if (ok < hi) hi = ok < kMinChunk ? kMinChunk : (int)((ok + kTileTok - 1) & ~(long long)(kTileTok - 1));
  // units(C) >= sumL / C, so C >= sumL / budget.
  const long long need = ceil_div_ll(sumL, budget);
  int lo = need > hi ? hi : (int)need;
  lo = (lo + kTileTok - 1) & ~(kTileTok - 1);
  lo = lo < kMinChunk ? kMinChunk : (lo > hi ? hi : lo);
  while (lo < hi) {
    const int mid = lo + ((hi - lo) / (2 * kTileTok)) * kTileTok;
    if (units(mid) <= budget) {
      hi = mid;
    } else {
      lo = mid + kTileTok;
    }
  }
  return hi;
}

// Wave64 reductions on DPP row shifts / broadcasts (no LDS); wave_incl_scan is
// in mm_common.hpp.
__device__ __forceinline__ int wave_sum_i(int v) { return __builtin_amdgcn_readlane(wave_incl_scan(v), 63); }
__device__ __forceinline__ int wave_max_i(int v) {
  // Invalid DPP sources return `old` = the lane's own value (neutral for max).
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x111, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x112, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x118, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, 63);
}

struct Unit {
  int b;       // request
  int part;    // part within the request
  int nparts;  // parts of the request
  int rec0;    // record part index of the request's part 0 (request-index order)
  int ptok;    // tokens per part of this request
  int units;   // total units (request parts) in the batch
  int len;     // context length of request b
  int slot0;   // first flat slot index of request b (paged: kv_indptr[b])
};

// Unit `u` of the batch. When the units fit one round of CTAs they run in
// request order; otherwise in longest-first order: requests sorted into 16
// linear buckets of their part size (largest first, request index inside a
// bucket), each request's parts consecutive. Wave-uniform, computed by one wave
// in `scratch` (12 * B bytes of LDS that no other wave touches meanwhile). The
// first 64 lengths and kv_indptr entries are loaded in one round of latency, so
// the unit's length and slot offset cost no further round trip for b < 64.
__device__ Unit plan_unit_paged(const int* seq_lens, const int* kv_indptr, int B, int P, int cap, int u, int lane,
                                int* scratch) {
  int* lens = scratch;            // [B] lengths
  int* req_at = scratch + B;      // [B] request at each position
  int* np_at = scratch + 2 * B;   // [B] parts of the request at each position
  const int ip0 = lane < B ? kv_indptr[lane] : 0;
  const int l0 = lane < B ? seq_lens[lane] : 0;  // the first 64 lengths stay in a register
  long long suml = 0;
  int maxl = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int l = c0 == 0 ? l0 : ((c0 + lane < B) ? seq_lens[c0 + lane] : 0);
    if (c0 + lane < B) lens[c0 + lane] = l;
    suml += wave_sum_i(l);  // per-chunk sums stay below 2^31 for lengths < 2^25
    maxl = max(maxl, wave_max_i(l));
  }
  auto len_at = [&](int c0) { return c0 == 0 ? l0 : ((c0 + lane < B) ? lens[c0 + lane] : 0); };
  const int budget = unit_budget(B, P, cap);
  const int C = search_chunk(suml, maxl, B, budget, [&](int c) {
    int n = 0;
    for (int c0 = 0; c0 < B; c0 += 64) n += wave_sum_i(c0 + lane < B ? nparts_of(len_at(c0), c) : 0);
    return n;
  });
  if (budget <= cap) {
    // Every unit gets a CTA of the first round, so their order does not matter:
    // units in request order, which is also the record order (unit u of request
    // b is record rec0(b) + part).
    Unit r{0, 0, 1, 0, kTileTok, 0, 0, 0};
    int run = 0;  // units of the requests before this chunk
    bool found = false;
    for (int c0 = 0; c0 < B; c0 += 64) {
      const bool valid = c0 + lane < B;
      const int l = len_at(c0);
      const int np = valid ? nparts_of(l, C) : 0;
      const int inc = wave_incl_scan(np);
      const int excl = run + inc - np;
      const unsigned long long hit = __builtin_amdgcn_ballot_w64(valid && u >= excl && u < excl + np);
      if (!found && hit) {
        const int hl = (int)__builtin_ctzll(hit);
        r.b = c0 + hl;
        r.rec0 = __builtin_amdgcn_readlane(excl, hl);
        r.part = u - r.rec0;
        r.nparts = __builtin_amdgcn_readlane(np, hl);
        r.len = __builtin_amdgcn_readlane(l, hl);
        found = true;
      }
      run += __builtin_amdgcn_readlane(inc, 63);
    }
    r.units = run;
    r.ptok = part_tokens(r.len, r.nparts);
    r.slot0 = r.b < 64 ? __builtin_amdgcn_readlane(ip0, r.b) : kv_indptr[r.b];
    return r;
  }
  // More requests than the cap (several rounds of CTAs): longest parts first.
  int maxp = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const bool valid = c0 + lane < B;
    const int l = valid ? lens[c0 + lane] : 0;
    const int pt = valid ? part_tokens(l, nparts_of(l, C)) : 0;
    maxp = max(maxp, wave_max_i(pt));
  }
  maxp = __builtin_amdgcn_readfirstlane(maxp);
  auto bucket_of = [&](int pt) {  // 0 = largest parts; pt <= maxp < 2^27
    const unsigned q = (unsigned)pt * 16u / ((unsigned)maxp + 1u);
    return 15 - (int)q;
  };
  int start[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) start[k] = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const bool valid = c0 + lane < B;
    const int l = valid ? lens[c0 + lane] : 0;
    const int bk = valid ? bucket_of(part_tokens(l, nparts_of(l, C))) : -1;
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
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const bool valid = c0 + lane < B;
    const int l = valid ? lens[c0 + lane] : 0;
    const int np = nparts_of(l, C);
    const int bk = valid ? bucket_of(part_tokens(l, np)) : -1;
    int pos = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const unsigned long long m = __builtin_amdgcn_ballot_w64(bk == k);
      if (bk == k) pos = start[k] + __builtin_popcountll(m & lt);
      start[k] += __builtin_popcountll(m);
    }
    if (valid) {
      req_at[pos] = c0 + lane;
      np_at[pos] = np;
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  Unit r{0, 0, 1, 0, kTileTok, 0, 0, 0};
  int run = 0;  // units before this chunk of positions
  bool found = false;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const bool valid = c0 + lane < B;
    const int np = valid ? np_at[c0 + lane] : 0;
    const int inc = wave_incl_scan(np);
    const int excl = run + inc - np;
    const unsigned long long hit = __builtin_amdgcn_ballot_w64(valid && u >= excl && u < excl + np);
    if (!found && hit) {
      const int hl = (int)__builtin_ctzll(hit);
      r.b = __builtin_amdgcn_readlane(req_at[c0 + lane], hl);
      r.part = u - __builtin_amdgcn_readlane(excl, hl);
      r.nparts = __builtin_amdgcn_readlane(np, hl);
      found = true;
    }
    run += __builtin_amdgcn_readlane(inc, 63);
  }
  r.units = run;
  r.len = lens[r.b];
  r.ptok = part_tokens(r.len, r.nparts);
  r.slot0 = r.b < 64 ? __builtin_amdgcn_readlane(ip0, r.b) : kv_indptr[r.b];
  // Record offset: parts of the requests before b, in request-index order.
  int rec0 = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int idx = c0 + lane;
    rec0 += wave_sum_i(idx < B && idx < r.b ? nparts_of(lens[idx], C) : 0);
  }
  r.rec0 = rec0;
  return r;
}

// Unit `u` of a contiguous batch (every request S tokens): the same chunking,
// units in request order.
__device__ __forceinline__ Unit plan_unit_contig(int S, int B, int P, int cap, int u) {
  const int C =
      search_chunk((long long)B * S, S, B, unit_budget(B, P, cap), [&](int c) { return B * nparts_of(S, c); });
  const int np = nparts_of(S, C);
  return Unit{u / np, u % np, np, (u / np) * np, part_tokens(S, np), B * np, S, 0};
}

// 4-byte global -> LDS DMA (lane l's dword lands at lds_dst + 4*l), counted by
// the kernel itself like dma16_opaque.
__device__ __forceinline__ void dma4_opaque(const void* gsrc, const char* lds_dst) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)lds_dst;
  asm volatile("global_load_lds_dword %0, off" ::"v"(gsrc), "{m0}"(m0v) : "memory");
}

// Staging layout of one tile: token t's 576-byte row at t*576, its 16-byte
// piece c stored at piece slot c ^ swz(t) (a permutation inside each aligned
// group of 4 pieces) so the 32 lanes of a K read and the 8-token groups of a
// V^T transpose read hit distinct LDS banks.
__device__ __forceinline__ int swz(int t) { return (t >> 2) & 3; }

// Host launchers of the 128-row kernel (mla_wide.hip) and of the 16-row kernel
// (mla_coop.hip); grid = CTAs.
int launch_wide_kernel(const Params& p, long long grid, hipStream_t st);
int launch_coop_kernel(const Params& p, long long grid, hipStream_t st);

}  // namespace mla
}  // namespace mm
