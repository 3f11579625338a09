// fp8 KV producer for the absorbed-MLA decode (MI355X, gfx950): writes the
// fused 576-byte OCP e4m3fn rows the decode reads ([0:512) latent, [512:576)
// rope) into a paged pool at one per-tensor kv_scale.
//
// The reference keeps no producer of its own: its cache contract is "fused
// fp8 576-wide rows at one per-tensor kv_scale" (moonmath reference
// moonmath_attention/mla.py:17-20, csrc/mla_decode_a16w8_api.cpp:5-8) and its
// tests fill the cache as (x / kv_scale).to(float8) (tests/test_mla_decode.py:
// 34-38). This kernel computes exactly that: q = e4m3fn(fl32(x / kv_scale)),
// round to nearest even, magnitudes above 464 -> NaN (torch's cast), or, with
// `saturate`, clamped to +-448 (NaN stays NaN).
//
// HBM-bound: 1152 bytes read and 576 written per token. One thread per 16
// output bytes (two 16-byte bf16 loads, 8 hardware converts, one 16-byte
// store); the 36 threads of a row write its 576 bytes contiguously.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mm {
namespace kvq {

constexpr int kLat = 512;
constexpr int kRope = 64;
constexpr int kRow = kLat + kRope;    // 576 bytes per fp8 row
constexpr int kChunks = kRow / 16;    // 36 sixteen-byte chunks per row
constexpr int kThreads = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// fp32 -> OCP e4m3fn, two values per instruction: v_cvt_scalef32_pk_fp8_f32
// at scale 1 rounds to nearest even, keeps subnormals, and turns NaN and
// magnitudes above 464 (the midpoint past 448, infinities included) into a
// NaN code (0x7F / 0xFF), which is torch's non-saturating cast (checked
// against a bit-level encoder on every bf16 pattern at several scales).
// Saturating callers clamp |x| > 448 to +-448 first (a NaN fails the compare
// and stays NaN).
typedef short s16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float clamp448(float x) {
  return __builtin_fabsf(x) > 448.f ? __builtin_copysignf(448.f, x) : x;
}

// POW2: kv_scale is a power of two, so x / kv_scale == x * (1 / kv_scale)
// exactly and the correctly rounded division is replaced by one multiply.
template <bool POW2, bool SAT>
__global__ __launch_bounds__(kThreads) void kv_quant_kernel(const uint16_t* __restrict__ c_kv,
                                                            const uint16_t* __restrict__ k_pe,
                                                            uint8_t* __restrict__ pool, const int* __restrict__ slots,
                                                            long long n_tokens, long long num_slots, float kv_scale,
                                                            float inv_scale) {
  const long long item = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (item >= n_tokens * kChunks) return;
  const long long tok = item / kChunks;
  const int chunk = (int)(item - tok * kChunks);
  const uint16_t* src = chunk < kLat / 16 ? c_kv + tok * kLat + chunk * 16 : k_pe + tok * kRope + (chunk - kLat / 16) * 16;
  // Inputs are read once and rows written once: non-temporal accesses. The
  // row loads go out together with the slot load (neither depends on the
  // other), so a thread waits one memory round trip, not two.
  const u32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));      // elements 0..7
  const u32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 8));  // elements 8..15
  const long long slot = slots[tok];
  auto val = [&](uint32_t pair, bool upper) {  // one bf16 of a pair, widened and divided by kv_scale
    const float xv = __builtin_bit_cast(float, upper ? (pair & 0xFFFF0000u) : (pair << 16));
    const float x = POW2 ? xv * inv_scale : xv / kv_scale;
    return SAT ? clamp448(x) : x;
  };
  u32x4 out;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const u32x4& v = w < 2 ? lo : hi;  // output word w = elements 4w .. 4w+3
    const uint32_t p0 = v[(w & 1) * 2], p1 = v[(w & 1) * 2 + 1];
    s16x2 r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(s16x2{0, 0}, val(p0, false), val(p0, true), 1.0f, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, val(p1, false), val(p1, true), 1.0f, true);
    out[w] = __builtin_bit_cast(uint32_t, r);
  }
  // The converted row exists before the slot test (an empty asm use), so the
  // compiler cannot sink the row loads behind the slot's round trip.
  asm volatile("" ::"v"(out));
  if (slot < 0 || slot >= num_slots) return;  // padding token / outside the pool: nothing written
  __builtin_nontemporal_store(out, reinterpret_cast<u32x4*>(pool + slot * kRow + chunk * 16));
}

}  // namespace kvq
}  // namespace mm

extern "C" {

int launch_mla_kv_quantize(const void* c_kv, const void* k_pe, void* kv_pool, const void* slots, long long n_tokens,
                           long long num_slots, float kv_scale, int saturate, void* stream) {
  if (n_tokens < 0 || num_slots < 0) return -4;
  if (n_tokens == 0) return 0;
  if (!c_kv || !k_pe || !kv_pool || !slots) return -6;
  if (!(kv_scale > 0.f) || kv_scale == __builtin_inff()) return -12;
  const long long items = n_tokens * mm::kvq::kChunks;
  const long long grid = (items + mm::kvq::kThreads - 1) / mm::kvq::kThreads;
  if (grid > 0x7FFFFFFFLL) return -8;
  int e2 = 0;
  const bool pow2 = __builtin_frexpf(kv_scale, &e2) == 0.5f && e2 - 1 >= -126 && e2 - 1 <= 126;
  const float inv = pow2 ? __builtin_ldexpf(1.0f, 1 - e2) : 0.f;
  auto* kern = pow2 ? (saturate ? mm::kvq::kv_quant_kernel<true, true> : mm::kvq::kv_quant_kernel<true, false>)
                    : (saturate ? mm::kvq::kv_quant_kernel<false, true> : mm::kvq::kv_quant_kernel<false, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(mm::kvq::kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(c_kv), static_cast<const uint16_t*>(k_pe),
                     static_cast<uint8_t*>(kv_pool), static_cast<const int*>(slots), n_tokens, num_slots, kv_scale,
                     inv);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // extern "C"
