// Absorbed-MLA decode for MI355X (gfx950): bf16 queries against an fp8 (OCP
// e4m3fn) latent KV cache, 576-wide fused rows ([0:512] latent = K and V,
// [512:576] rope = K only) at one per-tensor kv_scale.
//
//   score[r, j] = (q_lat[r] . c[j, 0:512] + q_pe[r] . c[j, 512:576]) * scale * kv_scale
//   o_lat[r]    = sum_j softmax_j(score[r, :]) * c[j, 0:512] * kv_scale
//
// Replaces the reference's gfx942 single-q and multi-q kernels (moonmath
// reference csrc/mla_decode_a16w8.hip:183-754, csrc/mla_decode_a16w8_multiq.hip
// :282-856) with one gfx950 kernel family:
//
//  * A query row r is (draft position t, head h) = (r / H, r % H); draft
//    position t attends tokens [0, S - (q_len - 1 - t)) (end-aligned causal
//    window, reference mla_decode_a16w8.hip:213-217).
//  * One CTA = kWaves waves = kWaves*16 query rows of one request b and one KV
//    part. The KV stream is walked in 32-token tiles: the fp8 rows are gathered
//    by slot index into an LDS staging buffer with 16-byte DMA (double
//    buffered), then converted ONCE per CTA (v_cvt_scalef32_pk_bf16_fp8, exact)
//    into a bf16 K tile in MFMA fragment order and a transposed bf16 V^T tile,
//    so the conversion is shared by every head of the CTA.
//  * v_mfma_f32_16x16x32_bf16: S^T = K Q^T (each wave owns 16 query columns),
//    online softmax in base 2 with the integer-grid running max (rescales are
//    exact powers of two), P rounded to bf16 RTNE, O^T = V^T P^T with the 512
//    output dims held as 32 independent accumulators per wave.
//  * Split-KV: parts > 1 write unnormalised fp32 (O, m, l) per query row; the
//    merge kernel combines them with exact power-of-two weights.

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mm_common.hpp"

namespace mm {
namespace mla {

constexpr int kLat = 512;
constexpr int kRope = 64;
constexpr int kQK = kLat + kRope;  // 576 bytes per fp8 row
constexpr int kTileTok = 32;       // tokens per tile
constexpr int kKSteps = kQK / 32;  // 18 K-steps of 32 dims (16 latent + 2 rope)
constexpr int kDTiles = kLat / 16; // 32 output d-tiles of 16
constexpr int kRowsPerWave = 16;
constexpr int kMaxQLen = 8;
constexpr int kMaxHeads = 128;

// LDS layout (bytes)
constexpr int kStageBytes = kTileTok * kQK;                  // 18432: fp8 rows, token-major
constexpr int kKTileBytes = 2 * kKSteps * 64 * 16;           // 36864: bf16 K fragments [tt][ks][lane]
constexpr int kVTileBytes = kDTiles * 64 * 16;               // 32768: bf16 V^T fragments [dt][lane]
constexpr int kDmaPieces = kStageBytes / 16;                 // 1152 16-byte pieces per tile
constexpr int kDmaInsts = kDmaPieces / 64;                   // 18 wave-DMA instructions per tile
constexpr int kStages = 3;                                   // fp8 staging ring (DMA 2 tiles ahead)
constexpr int kIdxCap = 4096;                                // slot indices resident in LDS per sub-range
constexpr int kJunkBytes = 1024;                             // sink for padding DMAs

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

template <int WAVES>
__global__ __launch_bounds__(WAVES * 64, 1) void mla_decode_kernel(Params p) {
  constexpr int kThreads = WAVES * 64;
  constexpr int kQRows = WAVES * kRowsPerWave;
  constexpr int kDmaPerWave = (kDmaInsts + WAVES - 1) / WAVES;  // padded to be uniform
  __shared__ __attribute__((aligned(1024)))
      char lds[kStages * kStageBytes + kKTileBytes + kVTileBytes + kIdxCap * 4 + kJunkBytes];
  char* stage = lds;
  char* ktile = lds + kStages * kStageBytes;
  char* vtile = ktile + kKTileBytes;
  int* idx_lds = reinterpret_cast<int*>(vtile + kVTileBytes);
  char* junk = reinterpret_cast<char*>(idx_lds + kIdxCap);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15;  // query column of this lane
  const int g = lane >> 4;  // lane group (0..3)

  // ---- work item: (b, part, group); groups of one (b, part) are adjacent ----
  const int total = p.B * p.parts * p.ngroups;
  const int w = xcd_remap(blockIdx.x, total);
  const int grp = w % p.ngroups;
  const int part = (w / p.ngroups) % p.parts;
  const int b = w / (p.ngroups * p.parts);
  int qb = b;
  if (p.rows) {
    qb = p.rows[b];
    qb = qb < 0 ? 0 : (qb >= p.B ? p.B - 1 : qb);
  }
  const int S = p.paged ? p.seq_lens[b] : p.S_fixed;
  const int slot0 = p.paged ? p.kv_indptr[b] : 0;
  // Proportional split: each part covers ceil(S / parts) tokens rounded to tiles.
  const int part_tok = ((S + p.parts * kTileTok - 1) / (p.parts * kTileTok)) * kTileTok;
  const int kv_lo = part * part_tok;
  const int kv_hi = (kv_lo + part_tok < S) ? kv_lo + part_tok : S;

  // ---- query rows of this lane --------------------------------------------------
  const int qrow = grp * kQRows + wave * kRowsPerWave + n;  // row within (t, h)
  const bool row_ok = qrow < p.qrows;
  const int qr = row_ok ? qrow : p.qrows - 1;
  const int t_pos = qr / p.H;
  const int lim = S - (p.q_len - 1 - t_pos);  // tokens >= lim are masked for this row
  const long long qoff = (long long)qb * p.qrows + qr;   // row index into [B, q_len, H]

  // Q fragments: B operand of S^T = K Q^T, lane (n, g) holds dims 32ks + 8g .. +8.
  bf16x8 qf[kKSteps];
#pragma unroll
  for (int ks = 0; ks < kKSteps; ++ks) {
    const uint16_t* src = (ks < 16) ? p.q_lat + qoff * kLat + ks * 32 + g * 8
                                    : p.q_pe + qoff * kRope + (ks - 16) * 32 + g * 8;
    qf[ks] = *reinterpret_cast<const bf16x8*>(src);
  }

  // ---- DMA of one fp8 tile (32 tokens x 576 B) into a staging slot ---------------
  // Piece P = inst*64 + lane covers token P / 36, bytes (P % 36) * 16 of its row.
  // Every wave issues kDmaPerWave instructions per tile (the padding ones land in
  // the junk area) so vmcnt waits count whole tiles. Tokens past hi are clamped
  // to the last valid one (masked in softmax). Paged rows come from idx_lds,
  // which holds the slots of tokens [sub_lo, sub_lo + kIdxCap).
  auto issue_tile = [&](int tok0, int slot, int sub_lo, int hi) {
    char* st = stage + slot * kStageBytes;
#pragma unroll
    for (int k = 0; k < kDmaPerWave; ++k) {
      const int inst = wave + k * WAVES;
      const int piece = (inst < kDmaInsts ? inst : 0) * 64 + lane;
      const int tok = piece / 36, chunk = piece % 36;
      int j = tok0 + tok;
      j = j < hi ? j : hi - 1;
      const long long row = p.paged ? (long long)idx_lds[j - sub_lo] : (long long)b * p.S_fixed + j;
      char* dst = inst < kDmaInsts ? st + inst * 1024 : junk;
      dma16(p.kv + row * kQK + chunk * 16, (MM_LDS void*)dst);
    }
  };

  // ---- fp8 staging -> bf16 K fragments and bf16 V^T fragments ------------------------
  // K unit (tt, ks, lane=(m, g)): token 16tt + m, dims 32ks + 8g .. +8.
  // V^T unit (dt, lane=(m, g)): dim 16dt + m, tokens tok(g, e) = 16(e/4) + 4g + e%4.
  auto convert_tile = [&](int slot) {
    const char* st = stage + slot * kStageBytes;
    for (int u = tid; u < 2 * kKSteps * 64; u += kThreads) {
      const int ln = u & 63, tk = u >> 6;  // tk = tt * 18 + ks
      const int tt = tk / kKSteps, ks = tk % kKSteps;
      const int tok = tt * 16 + (ln & 15);
      const u32x2 raw = *reinterpret_cast<const u32x2*>(st + tok * kQK + ks * 32 + (ln >> 4) * 8);
      u32x4 o;
      o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.0f, false));
      o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.0f, true));
      o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.0f, false));
      o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.0f, true));
      *reinterpret_cast<u32x4*>(ktile + u * 16) = o;
    }
    // V^T: item = (d-quad dq in 0..127, group gg in 0..3): 8 tokens x 4 dims.
    for (int it = tid; it < 128 * 4; it += kThreads) {
      const int dq = it >> 2, gg = it & 3;
      uint32_t rw[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = 16 * (e >> 2) + 4 * gg + (e & 3);
        rw[e] = *reinterpret_cast<const uint32_t*>(st + tok * kQK + dq * 4);
      }
      // For token pair (2k, 2k+1): bytes [A.d0, B.d0, A.d1, B.d1] and [A.d2, B.d2, A.d3, B.d3].
      uint32_t outw[4][4];  // [dim][pair] bf16x2 (token 2k in lo, 2k+1 in hi)
#pragma unroll
      for (int k2 = 0; k2 < 4; ++k2) {
        const uint32_t a = rw[2 * k2], bb = rw[2 * k2 + 1];
        const uint32_t lo = __builtin_amdgcn_perm(bb, a, 0x05010400u);  // a.b0 b.b0 a.b1 b.b1
        const uint32_t hi = __builtin_amdgcn_perm(bb, a, 0x07030602u);  // a.b2 b.b2 a.b3 b.b3
        outw[0][k2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
        outw[1][k2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
        outw[2][k2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
        outw[3][k2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
      }
#pragma unroll
      for (int dd = 0; dd < 4; ++dd) {
        const int d = dq * 4 + dd;
        const int dt = d >> 4, m = d & 15;
        u32x4 o = {outw[dd][0], outw[dd][1], outw[dd][2], outw[dd][3]};
        *reinterpret_cast<u32x4*>(vtile + (dt * 64 + gg * 16 + m) * 16) = o;
      }
    }
  };

  f32x4 oacc[kDTiles];
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt) oacc[dt] = f32x4{};
  float row_m = kNegFltMax, row_l = 0.f;
  const float c = p.score_c;

  for (int sub_lo = kv_lo; sub_lo < kv_hi; sub_lo += kIdxCap) {
    const int sub_hi = (sub_lo + kIdxCap < kv_hi) ? sub_lo + kIdxCap : kv_hi;
    const int ntiles = (sub_hi - sub_lo + kTileTok - 1) / kTileTok;
    // Every wave is done with the previous sub-range (LDS, DMAs).
    lds_reads_done_barrier_vm0();
    if (p.paged) {
      for (int i = tid; i < sub_hi - sub_lo; i += kThreads) idx_lds[i] = p.kv_indices[slot0 + sub_lo + i];
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    issue_tile(sub_lo, 0, sub_lo, sub_hi);
    issue_tile(sub_lo + (ntiles > 1 ? kTileTok : 0), 1, sub_lo, sub_hi);
    for (int it = 0; it < ntiles; ++it) {
      const int tok0 = sub_lo + it * kTileTok;
      // Tile it has landed (tile it+1 may still be in flight); every wave is done
      // with the bf16 tiles of it-1.
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kDmaPerWave) : "memory");
      // Two tiles ahead into the slot of tile it-1 (past the end: harmless reload).
      const int ahead = it + 2 < ntiles ? it + 2 : ntiles - 1;
      issue_tile(sub_lo + ahead * kTileTok, (it + 2) % kStages, sub_lo, sub_hi);
      convert_tile(it % kStages);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

      // ---- S^T = K Q^T: 2 token tiles x 18 K-steps, 4 accumulator chains ------------
      f32x4 sacc[2][2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) sacc[tt][0] = sacc[tt][1] = f32x4{};
#pragma unroll
      for (int ks = 0; ks < kKSteps; ++ks) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const bf16x8 kf = *reinterpret_cast<const bf16x8*>(ktile + ((tt * kKSteps + ks) * 64 + lane) * 16);
          sacc[tt][ks & 1] = mfma16(kf, qf[ks], sacc[tt][ks & 1]);
        }
      }
      float s[8];  // e = tt*4 + i  <->  token tok0 + 16tt + 4g + i
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tok = tok0 + tt * 16 + 4 * g + i;
          const float v = sacc[tt][0][i] + sacc[tt][1][i];
          s[tt * 4 + i] = (tok < lim && tok < sub_hi) ? v : -__builtin_inff();
        }

      // ---- online softmax (integer-grid running max) --------------------------------
      float bm = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < 8; ++e) bm = fmaxf(bm, s[e]);
      bm = fmaxf(bm, __shfl_xor(bm, 16));
      bm = fmaxf(bm, __shfl_xor(bm, 32));
      const float m_new = fmaxf(row_m, __builtin_ceilf(bm * c));
      const bool grow = m_new > row_m;
      if (__builtin_amdgcn_ballot_w64(grow)) {
        const float diff = row_m - m_new;  // integer-valued, <= 0
        float sc = __builtin_ldexpf(1.0f, (int)fmaxf(diff, -127.f));
        sc = (diff >= -126.f) ? sc : 0.f;
        sc = grow ? sc : 1.f;
        row_l *= sc;
#pragma unroll
        for (int dt = 0; dt < kDTiles; ++dt) oacc[dt] *= sc;
        row_m = m_new;
      }
      const float neg_m = -row_m;
      float pv[8];
      float lsum = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[e], c, neg_m));
        lsum += pv[e];
      }
      row_l += lsum;
      u32x4 pw = {pack2_bf16<kRTNE>(pv[0], pv[1]), pack2_bf16<kRTNE>(pv[2], pv[3]),
                  pack2_bf16<kRTNE>(pv[4], pv[5]), pack2_bf16<kRTNE>(pv[6], pv[7])};
      const bf16x8 pf = __builtin_bit_cast(bf16x8, pw);

      // ---- O^T += V^T P^T: 32 independent d-tile accumulators -------------------------
#pragma unroll
      for (int dt = 0; dt < kDTiles; ++dt) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(vtile + (dt * 64 + lane) * 16);
        oacc[dt] = mfma16(vf, pf, oacc[dt]);
      }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  }

  // ---- epilogue ---------------------------------------------------------------------------
  // Row sums: lanes n, n+16, n+32, n+48 hold partial sums of the same row.
  row_l += __shfl_xor(row_l, 16);
  row_l += __shfl_xor(row_l, 32);
  if (!row_ok) return;
  if (p.parts > 1) {
    const size_t rec = ((size_t)b * p.parts + part) * p.qrows + qrow;
    float* po = p.ws + rec * kLat;
    float* pml = p.ws + (size_t)p.B * p.parts * p.qrows * kLat + rec * 2;
#pragma unroll
    for (int dt = 0; dt < kDTiles; ++dt)
      *reinterpret_cast<f32x4*>(po + dt * 16 + 4 * g) = oacc[dt];
    if (g == 0) {
      pml[0] = row_m;
      pml[1] = row_l;
    }
    return;
  }
  const float inv = (row_l == 0.f) ? 0.f : p.kv_scale * __builtin_amdgcn_rcpf(row_l);
  uint16_t* orow = p.o_lat + ((long long)qb * p.qrows + qrow) * kLat;
#pragma unroll
  for (int dt = 0; dt < kDTiles; ++dt) {
    u32x2 o;
    o[0] = pack2_bf16_canon<kRTNE>(oacc[dt][0] * inv, oacc[dt][1] * inv);
    o[1] = pack2_bf16_canon<kRTNE>(oacc[dt][2] * inv, oacc[dt][3] * inv);
    *reinterpret_cast<u32x2*>(orow + dt * 16 + 4 * g) = o;
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
  float M = kNegFltMax;
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
    float wt = 1.f;
    if (m_p != M) {
      const float diff = m_p - M;
      wt = (diff >= -126.f) ? __builtin_ldexpf(1.0f, (int)fmaxf(diff, -127.f)) : 0.f;
    }
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
  const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, false));
  const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, true));
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

constexpr int kWavesPerCta = 4;
constexpr int kQRowsPerCta = kWavesPerCta * kRowsPerWave;  // 64
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
// across rounds), at least 4 tiles per part, within the record workspace.
int plan_parts(int B, int H, int max_seq_len, int q_len) {
  if (B < 1) B = 1;
  if (q_len < 1) q_len = 1;
  const int tiles = (max_seq_len + kTileTok - 1) / kTileTok;
  const int ctas_per_part = B * ngroups_for(H, q_len);
  int p = (2 * kNumCUs * kCtasPerCu + ctas_per_part - 1) / ctas_per_part;
  if (p > tiles / 4) p = tiles / 4;
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
  const long long grid = (long long)B * p.parts * p.ngroups;
  if (grid > 0x7FFFFFFFLL) return -8;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(mla_decode_kernel<kWavesPerCta>, dim3((unsigned)grid), dim3(kWavesPerCta * 64), 0, st, p);
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
