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
constexpr int kXcds = 8;  // MI355X: eight XCDs, each with its own L2

// Global-memory view of a pointer taken from a descriptor (loads and stores through it are
// global_* instructions instead of flat_* ones, which also wait on the LDS counter).
#define CAME8_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ CAME8_GLOBAL T* gbl(T* p) {
  return (CAME8_GLOBAL T*)p;
}

// ---------------------------------------------------------------------------
// element types: storage + exact conversions (float <-> storage)
// ---------------------------------------------------------------------------
//
// elem(w, v): element v of consecutive elements packed little-endian in 32-bit words (one
// instruction each: a move, a shift or mask, or a half-precision convert of a word half).
struct F32 {
  using storage = float;
  static __device__ __forceinline__ float load(storage v) { return v; }
  static __device__ __forceinline__ storage store(float f) { return f; }
  static __device__ __forceinline__ float elem(const uint32_t* w, int v) { return __uint_as_float(w[v]); }
};

// bfloat16: the conversion from fp32 rounds to nearest even (gfx950's v_cvt_pk_bf16_f32), the
// rounding c10::BFloat16 applies to every non-NaN value.
struct BF16 {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(storage v) { return __uint_as_float(uint32_t(v) << 16); }
  static __device__ __forceinline__ storage store(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
  static __device__ __forceinline__ float elem(const uint32_t* w, int v) {
    return (v & 1) ? __uint_as_float(w[v >> 1] & 0xffff0000u) : __uint_as_float(w[v >> 1] << 16);
  }
};

// x rounded to fp16 (round to nearest even) and back.  Written with integer operations on x's bits: a
// plain (_Float16) conversion of a product lets the compiler fuse the multiply and the conversion
// into one mixed-precision fma, which rounds the exact product to fp16 once instead of the fp32
// product (two roundings, as the reference computes it); the two differ where the fp32 product
// lands on an fp16 rounding tie.
__device__ __forceinline__ float round_f16(float x) {
  const uint32_t b = __float_as_uint(x);
  if ((b & 0x7f800000u) == 0x7f800000u) return x;  // inf, NaN
  if ((b & 0x7fffffffu) < 0x38800000u)             // |x| < 2^-14: fp16's subnormal grid, 2^-24
    return rintf(x * 0x1p24f) * 0x1p-24f;
  const uint32_t r = (b + 0x0fffu + ((b >> 13) & 1u)) & ~0x1fffu;  // 10 fraction bits, ties to even
  return (r & 0x7fffffffu) > 0x477fe000u ? __uint_as_float((b & 0x80000000u) | 0x7f800000u)  // > 65504
                                         : __uint_as_float(r);
}

// IEEE half, round-to-nearest-even conversion.
struct F16 {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(storage v) { return float(__builtin_bit_cast(_Float16, v)); }
  // round_f16 first: the conversion then sees an fp16 value, never a product it could fuse with
  static __device__ __forceinline__ storage store(float f) { return __builtin_bit_cast(uint16_t, (_Float16)round_f16(f)); }
  static __device__ __forceinline__ float elem(const uint32_t* w, int v) {
    return float(__builtin_bit_cast(_Float16, uint16_t(w[v >> 1] >> (16 * (v & 1)))));
  }
};

// signed byte v of consecutive int8 codes packed in 32-bit words, as a float
__device__ __forceinline__ float code_elem(const uint32_t* w, int v) {
  return float(int32_t(w[v >> 2] << (24 - 8 * (v & 3))) >> 24);
}

// native vector types (HIP's float4 / uint4 classes cannot bind to global-address-space objects)
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// the same with the alignment of their elements only: gfx9 loads vectors from any address (the
// compiler emits one global_load_dwordx4 for these as well)
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4u __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32x2u __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32u __attribute__((aligned(1)));

// Streamed operands (read or written once per pass, each pass's tensors far larger than the caches)
// take the nontemporal hint, `global_load ... nt` / `global_store ... nt` (HBM pure-read rate
// 5.4 -> 6.1 TB/s in a probe), but only where one wavefront instruction covers whole 128-byte lines:
// 16 bytes or less per lane, the lanes contiguous.  Where a lane's 32 bytes come in two 16-byte
// instructions, or a wavefront touches half of a line that another one reads, the hint made the
// kernel slower (fp32 elements 8 to a lane: C5's pass 3 4.53 -> 4.97 ms), and those accesses stay
// plain, as do operands that other workgroups read again (column factors, scales).
#ifndef CAME8_NT_LOADS
#define CAME8_NT_LOADS 1
#endif
#ifndef CAME8_NT_STORES
#define CAME8_NT_STORES 1
#endif
template <typename T>
__device__ __forceinline__ T ld_nt(const CAME8_GLOBAL T* p) {
#if CAME8_NT_LOADS
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}
template <typename T>
__device__ __forceinline__ void st_nt(CAME8_GLOBAL T* p, T v) {
#if CAME8_NT_STORES
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

// 8 consecutive floats from a 4-byte aligned address
__device__ __forceinline__ void load8u_f32(const CAME8_GLOBAL float* __restrict__ p, float (&out)[8]) {
  const f32x4u a = *(const CAME8_GLOBAL f32x4u*)p;
  const f32x4u b = *(const CAME8_GLOBAL f32x4u*)(p + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

// Load / store 8 consecutive elements (16 or 32 bytes, aligned) of any element type (NT: a streamed
// operand; 16-bit elements then load with the nontemporal hint, and 16-bit stores always take it).
template <typename T, bool NT = false>
__device__ __forceinline__ void load8(const CAME8_GLOBAL typename T::storage* __restrict__ p, float (&out)[8]) {
  constexpr bool nt = NT && sizeof(typename T::storage) == 2;  // one 16-byte load per lane
  auto ld = [](const auto* a) __attribute__((always_inline)) { return nt ? ld_nt(a) : *a; };
  if constexpr (sizeof(typename T::storage) == 4) {
    const CAME8_GLOBAL f32x4* q = (const CAME8_GLOBAL f32x4*)p;
    const f32x4 a = ld(q);
    const f32x4 b = ld(q + 1);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  } else {
    const u32x4 raw = ld((const CAME8_GLOBAL u32x4*)p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int v = 0; v < 8; ++v) out[v] = T::elem(w, v);
  }
}

template <typename T>
__device__ __forceinline__ void store8(CAME8_GLOBAL typename T::storage* __restrict__ p, const float (&in)[8]) {
  if constexpr (sizeof(typename T::storage) == 4) {
    CAME8_GLOBAL f32x4* q = (CAME8_GLOBAL f32x4*)p;
    q[0] = f32x4{in[0], in[1], in[2], in[3]};
    q[1] = f32x4{in[4], in[5], in[6], in[7]};
  } else {
    u32x4 raw;
    typename T::storage* s = reinterpret_cast<typename T::storage*>(&raw);
#pragma unroll
    for (int v = 0; v < 8; ++v) s[v] = T::store(in[v]);
    st_nt((CAME8_GLOBAL u32x4*)p, raw);
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

// Cross-lane moves without index arithmetic.  Each pattern is an involution (a lane's partner's
// partner is itself), so a butterfly over them leaves every lane of a group with the same value.
// DPP: quad_perm [1,0,3,2] (lane ^ 1), quad_perm [2,3,0,1] (lane ^ 2), row_half_mirror (within 8
// lanes, i <-> 7 - i), row_mirror (within 16 lanes, i <-> 15 - i); ds_swizzle bit mode: lane ^ 16.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppHalfMirror = 0x141, kDppMirror = 0x140;
__device__ __forceinline__ uint32_t swz_xor16_u32(uint32_t v) {
  return uint32_t(__builtin_amdgcn_ds_swizzle(int(v), 0x401f));
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane) {
  return uint32_t(__builtin_amdgcn_readlane(int(v), lane));
}

// Sum over the 64 lanes in a fixed order (pairs, quads, 8, 16, 32 lanes, then lane 0's half plus
// lane 32's half); every lane returns the same value.
__device__ __forceinline__ float wave_sum(float v) {
  v += __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v)));
  v += __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v)));
  v += __uint_as_float(swz_xor16_u32(__float_as_uint(v)));
  return __uint_as_float(readlane_u32(__float_as_uint(v), 0)) + __uint_as_float(readlane_u32(__float_as_uint(v), 32));
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

// unsigned max over aligned groups of L lanes (L a power of two <= 64); every lane of a group
// returns the group's maximum
template <int L>
__device__ __forceinline__ uint32_t group_max_bits(uint32_t v) {
  if constexpr (L >= 2) v = max(v, dpp_u32<kDppXor1>(v));
  if constexpr (L >= 4) v = max(v, dpp_u32<kDppXor2>(v));
  if constexpr (L >= 8) v = max(v, dpp_u32<kDppHalfMirror>(v));
  if constexpr (L >= 16) v = max(v, dpp_u32<kDppMirror>(v));
  if constexpr (L >= 32) v = max(v, swz_xor16_u32(v));
  if constexpr (L >= 64) v = max(readlane_u32(v, 0), readlane_u32(v, 32));
  return v;
}
__device__ __forceinline__ uint32_t group_max_bits_rt(uint32_t v, int L) {
  switch (L) {
    case 1: return v;
    case 2: return group_max_bits<2>(v);
    case 4: return group_max_bits<4>(v);
    case 8: return group_max_bits<8>(v);
    case 16: return group_max_bits<16>(v);
    case 32: return group_max_bits<32>(v);
    default: return group_max_bits<64>(v);
  }
}

// s_waitcnt vmcnt(0) alone (gfx9 encoding: vmcnt 0, expcnt 7, lgkmcnt 15).  vmcnt counts stores as
// well as loads; while stores are outstanding the compiler cannot tell which load has returned and
// waits for every one at the first use.  Waiting for the stores once, before a prefetching loop
// that issues only loads, lets it wait for exactly one stage inside the loop.
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// a value every lane holds alike, moved to a scalar register (lets branches on it be scalar)
__device__ __forceinline__ float uniform_f32(float v) { return __uint_as_float(readlane_u32(__float_as_uint(v), 0)); }

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

// Division by a block's absmax in quantisation.  With y = RN(1/b), q0 = RN(a*y), r = a - q0*b
// (exact, fused) and q1 = RN(q0 + r*y) (fused) is the correctly rounded a/b whenever a, b and the
// quotient are normal numbers in [2^-100, 2^100] (checked exhaustively over every significand of a
// for hundreds of divisors, tests/test_div_rcp.py).  In quantisation |a| <= b, and only quotients
// |a/b| >= 2^-8 can round to a nonzero code; with b in [2^-40, 2^60] those lie in the exact range,
// and smaller ones give code 0 either way.  Blocks whose absmax is outside that range divide.
__device__ __forceinline__ float div_fast(float a, float b, float y) {
  const float q0 = a * y;
  const float r = fmaf(-q0, b, a);
  return fmaf(r, y, q0);
}

// the reciprocal div_fast expects; NaN for divisors outside [2^-40, 2^60] (callers then divide)
__device__ __forceinline__ float rcp_for_div(float b) {
  return (b >= 0x1p-40f && b <= 0x1p60f) ? 1.0f / b : __builtin_nanf("");
}

// quantisation with rcp = rcp_for_div(absmax) finite (same results as quant_s8 / quant_u8)
__device__ __forceinline__ int8_t quant_s8_fast(float x, float absmax, float rcp) {
  float q = rintf(div_fast(x, absmax, rcp) * kSignedQ);
  q = q < -kSignedQ ? -kSignedQ : (q > kSignedQ ? kSignedQ : q);
  return int8_t(int(q));
}
__device__ __forceinline__ uint8_t quant_u8_fast(float x, float absmax, float rcp) {
  float q = rintf(div_fast(x, absmax, rcp) * kUnsignedQ);
  q = q < 0.0f ? 0.0f : (q > kUnsignedQ ? kUnsignedQ : q);
  return uint8_t(int(q));
}
// Division by the clip divisor (in [1, 2^60], shared by a whole tensor) with y = rcp_for_div(clip):
// the fast path is exact for zero and for every finite numerator with |a| >= 2^-40, whose quotient
// is then a normal number (tests/test_div_rcp.py); it fails only for tiny numerators with subnormal
// quotients and for infinities.  Callers keep a DivGuard per chunk and redo the rare chunks that
// hold other numerators with the IEEE division, element by element, out of the hot path.
__device__ __forceinline__ bool div_exact_needed(float a) {
  const float aa = fabsf(a);
  return !(aa >= 0x1p-40f && aa <= 0x1.fffffep127f) && a != 0.0f;
}

// Range of the nonzero |a| over a chunk, one test per chunk: lo is the least (bits(a) << 1) - 1
// (the sign shifted out; zeros wrap to the largest value and drop out), hi the largest |a|.
struct DivGuard {
  uint32_t lo = 0xffffffffu;
  float hi = 0.0f;
  __device__ __forceinline__ void add(float a) {
    lo = min(lo, (__float_as_uint(a) << 1) - 1u);
    hi = fmaxf(hi, fabsf(a));
  }
  // every numerator is zero or has 2^-40 <= |a| <= FLT_MAX (0x56ffffff = (bits(2^-40) << 1) - 1)
  __device__ __forceinline__ bool fast() const { return lo >= 0x56ffffffu && hi <= 0x1.fffffep127f; }
};

// absmax / 127 for dequantisation: the reciprocal form equals the IEEE quotient for every finite
// absmax (checked over all finite floats); infinities and NaNs divide.
constexpr float kRcpSignedQ = 1.0f / kSignedQ;
__device__ __forceinline__ float scale_s8(float absmax) {
  if (__builtin_expect(!(fabsf(absmax) <= 0x1.fffffep127f), 0)) return absmax / kSignedQ;
  return div_fast(absmax, kSignedQ, kRcpSignedQ);
}

// The 8bit2d layout's quantisation (reference came_kernels.cu:833-847): x times the rounded reciprocal
// of absmax, times Q, each product rounded, then rint and a clamp through fminf / fmaxf.
__device__ __forceinline__ int8_t quant_s8_inv(float x, float inv) {
  const float q = rintf((x * inv) * kSignedQ);
  return int8_t(fminf(kSignedQ, fmaxf(-kSignedQ, q)));
}
// quant_s8_inv of four elements packed into a word (byte v = element v), for a block whose absmax and
// inv = RN(1/absmax) are finite and every |x| <= absmax: then |RN(x*inv)| <= 1 + 2^-23, so
// |(x*inv)*Q| < 127.5 and the clamp never acts, and adding 1.5*2^23 rounds that product to an integer
// k half-to-even (the sum's ulp is 1) leaving k mod 256, the int8 code, in the sum's low byte.
__device__ __forceinline__ uint32_t quant_s8_inv4(const float* x, float inv) {
  constexpr float kRound = 12582912.0f;  // 1.5 * 2^23
  uint32_t b[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) b[v] = __float_as_uint(((x[v] * inv) * kSignedQ) + kRound);
  // byte selectors: 0-3 pick from the second operand, 4-7 from the first, 0x0c gives 0
  const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(b[3], b[2], 0x04000c0cu);
  return lo | hi;
}
__device__ __forceinline__ uint8_t quant_u8_inv(float x, float inv) {
  const float q = rintf((x * inv) * kUnsignedQ);
  return uint8_t(fminf(kUnsignedQ, fmaxf(0.0f, q)));
}

// any rcp (NaN divides)
__device__ __forceinline__ int8_t quant_s8_r(float x, float absmax, float rcp) {
  return rcp == rcp ? quant_s8_fast(x, absmax, rcp) : quant_s8(x, absmax);
}
__device__ __forceinline__ uint8_t quant_u8_r(float x, float absmax, float rcp) {
  return rcp == rcp ? quant_u8_fast(x, absmax, rcp) : quant_u8(x, absmax);
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
