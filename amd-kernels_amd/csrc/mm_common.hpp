// Shared gfx950 (CDNA4) building blocks for the moonmath kernels: vector types,
// MFMA wrappers, per-mode fp32 -> bf16 rounding, LDS DMA, barriers, XCD remap.
//
// Everything here is written for gfx950 only (wave64, 32x32x16 / 16x16x32 bf16
// MFMA, 16-byte global->LDS DMA, v_permlane32_swap).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

#define MM_LDS __attribute__((address_space(3)))

// Round modes, numbered as in the C ABI (0 = RTNE, 1 = RTNA, 2 = RTZ).
enum RoundMode : int { kRTNE = 0, kRTNA = 1, kRTZ = 2 };

constexpr uint32_t kBf16CanonNaN = 0x7FFFu;
constexpr float kNegFltMax = -3.402823466e+38f;

// ---------------------------------------------------------------------------
// fp32 -> bf16 bit rules (moonmath reference csrc/attention_kernel.hip:110-145):
//   RTNE: u + 0x7FFF + ((u >> 16) & 1), keep the top 16 bits
//   RTNA: u + 0x8000
//   RTZ : u (truncate)
// The "canon" variant maps every NaN to 0x7FFF in all three modes.
// ---------------------------------------------------------------------------
// Pack two fp32 into one dword of two bf16 (lo = a, hi = b).
// RTNE uses the gfx950 hardware convert (v_cvt_pk_bf16_f32), which is IEEE
// round-to-nearest-even and keeps NaN a NaN; RTNA/RTZ use the integer rules.
template <int MODE>
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  if constexpr (MODE == kRTNE) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    bf16x2 v;
    v[0] = (__bf16)a;
    v[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, v);
  } else if constexpr (MODE == kRTNA) {
    const uint32_t ua = __builtin_bit_cast(uint32_t, a) + 0x8000u;
    const uint32_t ub = __builtin_bit_cast(uint32_t, b) + 0x8000u;
    return __builtin_amdgcn_perm(ub, ua, 0x07060302u);
  } else {
    const uint32_t ua = __builtin_bit_cast(uint32_t, a);
    const uint32_t ub = __builtin_bit_cast(uint32_t, b);
    return __builtin_amdgcn_perm(ub, ua, 0x07060302u);
  }
}

// pack2_bf16 with every NaN mapped to 0x7FFF. A NaN input is first replaced
// by the fp32 NaN 0x7FFF0000, which each mode's packing turns into 0x7FFF:
// RTNA's +0x8000 does not carry into bit 16, RTZ truncates, and the RTNE
// convert returns a NaN input's top half unchanged when its quiet bit is set.
// Cost: one class test and one select per value, then the plain pack.
template <int MODE>
__device__ __forceinline__ uint32_t pack2_bf16_canon(float a, float b) {
  const float canon = __builtin_bit_cast(float, kBf16CanonNaN << 16);
  return pack2_bf16<MODE>(__builtin_isnan(a) ? canon : a, __builtin_isnan(b) ? canon : b);
}

// ---------------------------------------------------------------------------
// MFMA
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// Accumulate into an AGPR-resident accumulator. Non-volatile asm, so the
// scheduler may still interleave it with independent work. Hazards the
// compiler cannot see through the asm are covered by the fences below.
__device__ __forceinline__ void mfma32_acc_agpr(bf16x8 a, bf16x8 b, f32x16& acc) {
  asm("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Scheduling fence: nothing moves across it.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }
// Before VALU reads an accumulator written by mfma32_acc_agpr: the 8-pass
// 32x32x16 result needs > 18 wait states before a VALU / accvgpr read.
__device__ __forceinline__ void mfma_result_fence() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
// Before mfma32_acc_agpr reads VGPR/AGPR operands just written by VALU.
__device__ __forceinline__ void mfma_operand_fence() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 4" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Cross-lane: combine lane l with lane l^32 (v_permlane32_swap on gfx950);
// inclusive wave64 prefix sum on DPP row shifts / broadcasts (no LDS).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return v;
}

__device__ __forceinline__ float xor32_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto pr = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)pr[0]), __builtin_bit_cast(float, (uint32_t)pr[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto pr = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  // pr[0] holds the low half in both halves, pr[1] the high half: the sum is
  // formed in the same order (lo + hi) in every lane.
  return __builtin_bit_cast(float, (uint32_t)pr[0]) + __builtin_bit_cast(float, (uint32_t)pr[1]);
}

// ---------------------------------------------------------------------------
// Global -> LDS DMA, 16 bytes per lane: lane l's 16 bytes land at
// lds_dst + 16*l; lds_dst is a generic pointer into __shared__ memory,
// wave-uniform. Issued through asm, for kernels that count their loads
// themselves (explicit s_waitcnt vmcnt): hidden from the compiler's wait-count
// model, an in-flight DMA can neither force a conservative vmcnt(0) before
// LDS reads the compiler cannot prove disjoint from it nor turn the partial
// lgkmcnt waits of in-order LDS reads into lgkmcnt(0) (both measured with
// __builtin_amdgcn_global_load_lds).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void dma16_opaque(const void* gsrc, const char* lds_dst) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)lds_dst;
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(gsrc), "{m0}"(m0v) : "memory");
}
// The same from a wave-uniform base (SGPR pair) plus a 32-bit per-lane offset.
__device__ __forceinline__ void dma16_sbase(const void* sbase, uint32_t voff, const char* lds_dst) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)lds_dst;
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0v) : "memory");
}
// Non-temporal forms (cache-policy bit nt) for data each CTA streams once and
// no other CTA of the launch reads again.
__device__ __forceinline__ void dma16_opaque_nt(const void* gsrc, const char* lds_dst) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)lds_dst;
  asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(gsrc), "{m0}"(m0v) : "memory");
}
__device__ __forceinline__ void dma16_sbase_nt(const void* sbase, uint32_t voff, const char* lds_dst) {
  const uint32_t m0v = (uint32_t)(uintptr_t)(MM_LDS const char*)lds_dst;
  asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "{m0}"(m0v) : "memory");
}
// Barrier without the implicit vmcnt(0) that __syncthreads() carries, so
// prefetch DMA stays in flight across it. VMEM_LEFT = loads allowed to remain
// outstanding (issued after the data the barrier publishes).
template <int VMEM_LEFT>
__device__ __forceinline__ void wait_vmem_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(VMEM_LEFT) : "memory");
}
__device__ __forceinline__ void lds_reads_done_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ void lds_reads_done_barrier_vm0() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---------------------------------------------------------------------------
// XCD-aware work remap. Workgroups are dispatched round-robin over the 8 XCDs
// (blockIdx % 8). Remap so that XCD x runs a contiguous range of logical work
// ids, keeping the q-blocks of one (b, h) head on one XCD and its K/V in that
// XCD's L2.
// ---------------------------------------------------------------------------
constexpr int kNumXcds = 8;
__device__ __forceinline__ int xcd_remap(int idx, int total) {
  const int xcd = idx % kNumXcds;
  const int pos = idx / kNumXcds;
  const int per = total / kNumXcds;
  const int rem = total % kNumXcds;
  return (xcd < rem) ? xcd * (per + 1) + pos : rem * (per + 1) + (xcd - rem) * per + pos;
}

}  // namespace mm
