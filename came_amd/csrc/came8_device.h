// Device-side building blocks of the CAME 8-bit step for gfx950 (CDNA4).
//
// Element types, rounding helpers that reproduce the reference CPU
// arithmetic bit for bit, wavefront (64-lane) reductions with a fixed
// combination order, and the blockwise absmax (de)quantisation formulas of
// the reference (came_pytorch/blockwise_quantization.py:66-82,112-124).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace came8 {

constexpr int kThreads = 256;  // four 64-lane wavefronts per workgroup
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// element types: storage + exact conversions (float <-> storage)
// ---------------------------------------------------------------------------
struct F32 {
  using storage = float;
  static __device__ __forceinline__ float load(storage v) { return v; }
  static __device__ __forceinline__ storage store(float f) { return f; }
};

// bfloat16: the conversion from fp32 rounds to nearest even (gfx950's v_cvt_pk_bf16_f32), the
// rounding c10::BFloat16 applies to every non-NaN value.
struct BF16 {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(storage v) { return __uint_as_float(uint32_t(v) << 16); }
  static __device__ __forceinline__ storage store(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
};

// IEEE half, round-to-nearest-even conversion.
struct F16 {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(storage v) { return float(__builtin_bit_cast(_Float16, v)); }
  static __device__ __forceinline__ storage store(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
};

// Load V consecutive elements (V * sizeof(storage) == 16 bytes when V > 1, 16-byte aligned).
template <typename T, int V>
__device__ __forceinline__ void load_vec(const typename T::storage* __restrict__ p, float (&out)[V]) {
  if constexpr (V == 1) {
    out[0] = T::load(p[0]);
  } else {
    static_assert(V * sizeof(typename T::storage) == 16, "vector chunk must be 16 bytes");
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const typename T::storage* s = reinterpret_cast<const typename T::storage*>(&raw);
#pragma unroll
    for (int v = 0; v < V; ++v) out[v] = T::load(s[v]);
  }
}

// Load / store 8 consecutive elements (16 or 32 bytes, aligned) of any element type.
template <typename T>
__device__ __forceinline__ void load8(const typename T::storage* __restrict__ p, float (&out)[8]) {
  if constexpr (sizeof(typename T::storage) == 4) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const typename T::storage* s = reinterpret_cast<const typename T::storage*>(&raw);
#pragma unroll
    for (int v = 0; v < 8; ++v) out[v] = T::load(s[v]);
  }
}

template <typename T>
__device__ __forceinline__ void store8(typename T::storage* __restrict__ p, const float (&in)[8]) {
  if constexpr (sizeof(typename T::storage) == 4) {
    reinterpret_cast<float4*>(p)[0] = make_float4(in[0], in[1], in[2], in[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(in[4], in[5], in[6], in[7]);
  } else {
    uint4 raw;
    typename T::storage* s = reinterpret_cast<typename T::storage*>(&raw);
#pragma unroll
    for (int v = 0; v < 8; ++v) s[v] = T::store(in[v]);
    *reinterpret_cast<uint4*>(p) = raw;
  }
}

// ---------------------------------------------------------------------------
// reductions with a fixed order (results identical on every run)
// ---------------------------------------------------------------------------
template <typename F>
__device__ __forceinline__ F wave_sum(F v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// max that propagates NaN (torch.amax semantics)
__device__ __forceinline__ float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }

// NaN-propagating max over aligned groups of L lanes (L a power of two <= 64).
template <int L>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) v = nan_max(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ float group_max_rt(float v, int L) {
  for (int o = L / 2; o > 0; o >>= 1) v = nan_max(v, __shfl_xor(v, o, kWave));
  return v;
}

// ---------------------------------------------------------------------------
// blockwise quantisation (reference blockwise_quantization.py:66-82,112-124)
// ---------------------------------------------------------------------------
constexpr float kSignedQ = 127.0f;
constexpr float kUnsignedQ = 255.0f;

// absmax == 0 (or NaN, or negative for unsigned) -> 1.0
__device__ __forceinline__ float fix_absmax(float a) { return (a > 0.0f) ? a : 1.0f; }

// code = clamp(round_half_even((x / absmax) * Q)); division and product rounded separately.
__device__ __forceinline__ int8_t quant_s8(float x, float absmax) {
  float q = rintf((x / absmax) * kSignedQ);
  q = q < -kSignedQ ? -kSignedQ : (q > kSignedQ ? kSignedQ : q);
  return int8_t(int(q));
}
__device__ __forceinline__ uint8_t quant_u8(float x, float absmax) {
  float q = rintf((x / absmax) * kUnsignedQ);
  q = q < 0.0f ? 0.0f : (q > kUnsignedQ ? kUnsignedQ : q);
  return uint8_t(int(q));
}
// dequant: q * (absmax / Q), the scale rounded to fp32 first
__device__ __forceinline__ float deq_s8(int8_t q, float absmax) { return float(q) * (absmax / kSignedQ); }
__device__ __forceinline__ float deq_u8(uint8_t q, float absmax) { return float(q) * (absmax / kUnsignedQ); }

// a / b for b > 0 given y = rcp_for_div(b): q0 = a*y, r = a - q0*b (exact, fused), q1 = q0 + r*y
// (fused) is the correctly rounded quotient when a, b and q1 are normal numbers in [2^-100, 2^100]
// (checked exhaustively over every significand of a for hundreds of divisors, _work-free test in
// tests/test_div_rcp.py); zeros pass through with their sign, every other case takes the IEEE division.
__device__ __forceinline__ float div_rcp(float a, float b, float y) {
  const float q0 = a * y;
  const float r = fmaf(-q0, b, a);
  float q = fmaf(r, y, q0);
  const float aa = fabsf(a), aq = fabsf(q);
  const bool fast = aa >= 0x1p-100f && aa <= 0x1p100f && aq >= 0x1p-100f && aq <= 0x1p100f;
  if (a == 0.0f) {
    q = a;
  } else if (__builtin_expect(!fast, 0)) {
    q = a / b;
  }
  return q;
}

// the reciprocal div_rcp expects; NaN (forcing the IEEE division) for divisors outside [2^-100, 2^100]
__device__ __forceinline__ float rcp_for_div(float b) {
  return (b >= 0x1p-100f && b <= 0x1p100f) ? 1.0f / b : __builtin_nanf("");
}

// quantisation with the block's reciprocal absmax precomputed (same results as quant_s8/quant_u8)
__device__ __forceinline__ int8_t quant_s8_r(float x, float absmax, float rcp) {
  float q = rintf(div_rcp(x, absmax, rcp) * kSignedQ);
  q = q < -kSignedQ ? -kSignedQ : (q > kSignedQ ? kSignedQ : q);
  return int8_t(int(q));
}
__device__ __forceinline__ uint8_t quant_u8_r(float x, float absmax, float rcp) {
  float q = rintf(div_rcp(x, absmax, rcp) * kUnsignedQ);
  q = q < 0.0f ? 0.0f : (q > kUnsignedQ ? kUnsignedQ : q);
  return uint8_t(int(q));
}

// n / d for n < 2^31 with the host-precomputed magic m = floor(2^s / d) + 1, s = 32 + ceil(log2 d)
__device__ __forceinline__ uint32_t udiv_magic(uint32_t n, uint64_t m, uint32_t s) {
  return uint32_t((uint64_t(n) * m) >> s);
}

// 1/sqrt(x) as the reference computes rsqrt on CPU: correctly rounded sqrt, then a correctly rounded divide.
__device__ __forceinline__ float rsqrt_ref(float x) { return 1.0f / sqrtf(x); }

// x.clamp_min(1e-30) with NaN passing through
__device__ __forceinline__ float clamp_min_tiny(float x) { return x < 1e-30f ? 1e-30f : x; }

}  // namespace came8
