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
// output bytes (two 16-byte bf16 loads, one 16-byte store); the 36 threads of
// a row write its 576 bytes contiguously.
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

// fp32 -> OCP e4m3fn (bias 7, no infinities, 0x7F / 0xFF = NaN, max 448),
// round to nearest even. Overflow (|x| > 464, the midpoint past 448) -> NaN,
// or +-448 when saturating.
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float f, bool saturate) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;                  // NaN
  if (a > 0x43E80000u) return sign | (saturate ? 0x7Eu : 0x7Fu);  // |x| > 464 (incl. inf)
  if (a >= 0x3C800000u) {                                     // |x| >= 2^-6: normal
    // Keep 3 mantissa bits, round to nearest even on the 20 dropped bits; a
    // carry into the exponent is the correctly rounded result.
    const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
    return sign | (r - (120u << 3));                          // rebias 127 -> 7
  }
  // Subnormal (or zero): |x| / 2^-9 rounded to nearest even, 0..8 (8 is the
  // smallest normal, encoded the same way).
  const float m = __builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
  return sign | (uint32_t)m;
}

// POW2: kv_scale is a power of two, so x / kv_scale == x * (1 / kv_scale)
// exactly and the correctly rounded division is replaced by one multiply.
template <bool POW2>
__global__ __launch_bounds__(kThreads) void kv_quant_kernel(const uint16_t* __restrict__ c_kv,
                                                            const uint16_t* __restrict__ k_pe,
                                                            uint8_t* __restrict__ pool, const int* __restrict__ slots,
                                                            long long n_tokens, long long num_slots, float kv_scale,
                                                            float inv_scale, int saturate) {
  const long long item = (long long)blockIdx.x * kThreads + threadIdx.x;
  if (item >= n_tokens * kChunks) return;
  const long long tok = item / kChunks;
  const int chunk = (int)(item - tok * kChunks);
  const long long slot = slots[tok];
  if (slot < 0 || slot >= num_slots) return;  // padding token / outside the pool: nothing written
  const uint16_t* src = chunk < kLat / 16 ? c_kv + tok * kLat + chunk * 16 : k_pe + tok * kRope + (chunk - kLat / 16) * 16;
  const u32x4 lo = *reinterpret_cast<const u32x4*>(src);      // elements 0..7
  const u32x4 hi = *reinterpret_cast<const u32x4*>(src + 8);  // elements 8..15
  const bool sat = saturate != 0;
  u32x4 out;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const u32x4& v = w < 2 ? lo : hi;  // output word w = elements 4w .. 4w+3
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t pair = v[(w & 1) * 2 + (j >> 1)];
      const uint32_t bf = (j & 1) ? (pair >> 16) : (pair & 0xFFFFu);
      const float xv = __builtin_bit_cast(float, bf << 16);
      const float x = POW2 ? xv * inv_scale : xv / kv_scale;
      word |= f32_to_e4m3fn(x, sat) << (8 * j);
    }
    out[w] = word;
  }
  *reinterpret_cast<u32x4*>(pool + slot * kRow + chunk * 16) = out;
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
  auto* kern = pow2 ? mm::kvq::kv_quant_kernel<true> : mm::kvq::kv_quant_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(mm::kvq::kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(c_kv), static_cast<const uint16_t*>(k_pe),
                     static_cast<uint8_t*>(kv_pool), static_cast<const int*>(slots), n_tokens, num_slots, kv_scale,
                     inv, saturate);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // extern "C"
