// The clip's update norm in the reference's own summation order, computed in parallel.
//
// The reference clips the update by its RMS, u.norm(2) / sqrt(N) (came_pytorch/CAME8bitFull.py:121-122,
// 1032).  On CPU, torch sums a contiguous fp32 tensor's squares for norm(2) in one thread as eight
// interleaved accumulators, acc[i % 8] = fma(u_i, u_i, acc[i % 8]) over the first N - N % 8 elements,
// then acc[0] + acc[1] + ... + acc[7] left to right, then the remaining elements as separately
// rounded square-and-add, then a correctly rounded sqrt.  Each accumulator is a serial chain of up to
// N / 8 dependent fused multiply-adds (16.4 M for a 32000 x 4096 matrix); its rounding errors are
// part of the result (about 1.5% of the norm at that size), so the exact chain has to be replayed.
//
// Replay without the serial dependence.  While a chain's value s stays inside one binade
// [2^E, 2^(E+1)) (E = -126 also covers the subnormals) it is m * 2^(E-23) with an integer m < 2^24,
// and fma(x, x, s) = (m + n) * 2^(E-23) with n = round(x^2 * 2^(23-E)), provided m + n < 2^24 and
// x^2 * 2^(23-E) is not a half-integer: the exact sum then lies strictly inside the binade, whose
// floats are exactly the multiples of 2^(E-23).  So inside a binade the chain is an integer sum of
// per-element increments that do not depend on s.  Elements whose increment is not determined this
// way are "special": the rounded square x*x is a half-integer after scaling (the true square may be
// a tie, whose rounding depends on m's parity), the scaled square is 2^20 or more, or x*x is
// subnormal, infinite or NaN.  (When the rounded square is not a half-integer, the true square
// rounds the same way: its distance to hi = RN(x*x) is at most half an ulp of hi, less than the
// distance from hi to any half-integer.)
//
//   k_norm_est, k_norm_scan  an estimate of each chain's value along the tensor, from sums the step
//                            has already formed (per row band: rm * sum_j c_j^2 * sum_i g_ij^2 / R_i;
//                            per 1-D tile: the tile's sum of u^2), as an exclusive prefix per tensor.
//   k_norm_seg               one wavefront per segment of kNormSegElems elements (512 per chain):
//                            per chain, the candidate binade Ea of the estimate (and Ea + 1 near a
//                            binade edge), the integer sums of the increments under each, whether
//                            the segment holds special elements, and whether it holds a NaN.
//   k_norm_walk              one workgroup per chain: from s = 0, skips every run of segments whose
//                            record covers the chain's current binade without specials and without
//                            leaving the binade (a block-wide scan of the integer sums), and replays
//                            the segment where that fails element by element with fmaf: the chain's
//                            start, binade crossings, specials, and estimates that missed.
//   k_norm_final             the eight accumulators and the tail in the reference's order, sqrt,
//                            and the clip divisor.
//
// Only the replay uses floating-point addition on the chain; everything else is exact integer
// arithmetic, so the result equals the serial chain bit for bit whatever the estimates were (they
// only decide how many segments are replayed).
#pragma once

#include "came8_kernels.h"

namespace came8 {

constexpr int kNormSegElems = 4096;                    // flat elements per segment (a multiple of 8)
constexpr int kNormChainSeg = kNormSegElems / 8;       // elements per chain per segment
constexpr int kNormChunks = kNormSegElems / (8 * 64);  // 8-element chunks per lane of a segment's wavefront
constexpr int kNormWalkSegs = 16;                      // segments per thread per batch of the walk
constexpr int kNormGroup = 2;                          // chunks per lane loaded together
constexpr float kNormIncrMax = 0x1p20f;                // scaled squares at or above this are special

// binade of a finite s >= 0: E with s in [2^E, 2^(E+1)), or -126 below 2^-125
__device__ __forceinline__ int norm_binade(float s) {
  const int e = int(__float_as_uint(s) >> 23);
  return e == 0 ? -126 : e - 127;
}
// s = m * 2^(E-23) for E = norm_binade(s): the integer m < 2^24, and back
__device__ __forceinline__ uint32_t norm_mant(float s, int E) { return __float_as_uint(s) - (uint32_t(E + 126) << 23); }
__device__ __forceinline__ float norm_value(uint32_t m, int E) { return __uint_as_float((uint32_t(E + 126) << 23) + m); }

// binade of an estimate (any float): -126 for values <= 2^-125 (and NaN), 127 for +inf
__device__ __forceinline__ int norm_est_binade(float v) {
  if (!(v > 0x1p-125f)) return -126;
  if (!(v <= 0x1.fffffep127f)) return 127;
  return norm_binade(v);
}

// The increment of one element whose rounded square is hi under binade E (k = 23 - E) is rint(hi * 2^k),
// exact for the chain whenever that scaled square dh is not a half-integer and below 2^23 (then
// half-integers lie on hi's grid, and a true square that is not one rounds like hi).  The segment
// kernel keeps, per lane and chain, the running sum of rint(dh) and the largest |dh - rint(dh)|; the
// exceptions are then read off per lane once, not tested per element:
//   * a tie (some |dh - rint(dh)| = 0.5): the rounding of that element depends on the chain's parity;
//   * dh >= 2^23: in a normal binade (m >= 2^23) it takes the chain out of the binade by itself, so
//     the segment's sum, at least 2^23, already fails the walk's test m + sum < 2^24;
//   * the subnormal binade (E = -126, k = 149), where hi's own rounding may hide a tie: any nonzero
//     increment there;
//   * NaN or infinite squares: a NaN or infinite sum.
// An exception saturates the segment's sum at kNormFull, which makes the walk replay the segment.
constexpr float kNormSpecial = 0x1p24f;
__device__ __forceinline__ void norm_acc(float hi, int k, float& sum, float& rmax) {
  const float dh = ldexpf(hi, k);
  const float nf = rintf(dh);
  sum += nf;
  rmax = fmaxf(rmax, fabsf(dh - nf));
}
// the lane's sum for one chain as the record's integer, or kNormFull for an exception
__device__ __forceinline__ uint32_t norm_lane_value(float sum, float rmax, int E) {
  const bool bad = !(sum < kNormSpecial) || rmax == 0.5f || (E == -126 && sum != 0.0f);
  return bad ? (1u << 24) : uint32_t(sum);
}

// Record word 0: Ea + 256 (9 bits) | kRecTwo when word 2 holds the sum under Ea + 1.  Words 1 and 2:
// the integer sums of the increments under Ea and Ea + 1, at most 2^24 (2^24: the segment leaves
// the binade or holds a special element).
constexpr uint32_t kRecTwo = 1u << 9;
constexpr uint32_t kNormFull = 1u << 24;

// ---------------------------------------------------------------------------
// estimates
// ---------------------------------------------------------------------------
// Units: row band b of matrix m (unit m * nbands + b; for matrices of the thread-per-matrix passes the
// matrix is its band) or 2048-element tile u of a 1-D tensor.  The estimate of a band is
// rm * sum_j c_j^2 * W_j with W_j = sum over the band's rows of g_ij^2 / R_i (pass 1's column
// partials): the sum of u_ij^2 = (rm / R_i) * c_j^2 * g_ij^2 without the roundings.
__device__ __forceinline__ float norm_unit_rm(const DevTensor& t, int64_t u) {
  return matrix_row_mean(t, t.rsum, u / t.nbands, t.nbands);
}

// WIDE: a workgroup per unit (matrices of at least 256 columns); otherwise a thread per unit.
template <bool WIDE>
__global__ __launch_bounds__(kThreads) void k_norm_est(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                       const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  __shared__ float ssum[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    if constexpr (WIDE) {
      const int64_t u = w - wstart[slot];
      const int64_t m = u / t.nbands;
      const float* __restrict__ W = t.partW + u * t.C;
      const float* __restrict__ cf = t.cfac + m * t.C;
      float s = 0.0f;
      for (int64_t j = tid; j < t.C; j += kThreads) s = fmaf(cf[j] * cf[j], W[j], s);
      s = wave_sum(s);
      if (lane == 0) ssum[wid] = s;
      __syncthreads();
      if (tid == 0) t.nest[u] = norm_unit_rm(t, u) * (((ssum[0] + ssum[1]) + ssum[2]) + ssum[3]);
      __syncthreads();
    } else {
      const int64_t u = (w - wstart[slot]) * kThreads + tid;
      if (u >= t.nunit) continue;
      float e;
      if (t.factored) {
        const int64_t m = u / t.nbands;
        const float* __restrict__ W = t.partW + u * t.C;
        const float* __restrict__ cf = t.cfac + m * t.C;
        float s = 0.0f;
        for (int64_t j = 0; j < t.C; ++j) s = fmaf(cf[j] * cf[j], W[j], s);
        e = norm_unit_rm(t, u) * s;
      } else {
        e = float(t.clip_part[u]);
      }
      t.nest[u] = e;
    }
  }
}

// In-place exclusive prefix of the unit estimates of one tensor per workgroup; nest[nunit] = total.
// Each thread sums a run of consecutive units, the runs' sums are scanned across the workgroup, and
// each thread rewrites its run.
template <int = 0>
__global__ __launch_bounds__(kThreads) void k_norm_scan(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                        int ntens) {
  __shared__ float part[kThreads];
  const int tid = threadIdx.x;
  for (int k = blockIdx.x; k < ntens; k += gridDim.x) {
    const DevTensor& t = T[tids[k]];
    const int64_t n = t.nunit;
    const int64_t per = (n + kThreads - 1) / kThreads;
    const int64_t u0 = min(n, int64_t(tid) * per), u1 = min(n, u0 + per);
    float s = 0.0f;
    for (int64_t u = u0; u < u1; ++u) s += t.nest[u];
    part[tid] = s;
    __syncthreads();
    if (tid == 0) {
      float run = 0.0f;
      for (int i = 0; i < kThreads; ++i) {
        const float v = part[i];
        part[i] = run;
        run += v;
      }
      t.nest[n] = run;
    }
    __syncthreads();
    float run = part[tid];
    for (int64_t u = u0; u < u1; ++u) {
      const float v = t.nest[u];
      t.nest[u] = run;
      run += v;
    }
    __syncthreads();
  }
}

// Estimated sum of u^2 over the flat elements before f (0 <= f <= N), linear inside a unit.
__device__ __forceinline__ float norm_est_at(const DevTensor& t, int64_t f) {
  int64_t u, us, ue;
  if (t.factored) {
    const int64_t row = t.idx32 ? int64_t(udiv_magic(uint32_t(f), t.mC, t.sC)) : f / t.C;
    const int64_t m = t.idx32 ? int64_t(udiv_magic(uint32_t(row), t.mR, t.sR)) : row / t.R;
    if (m >= t.P) return t.nest[t.nunit];
    const int64_t i = row - m * t.R;
    const int64_t b = int64_t(uint32_t(i) / uint32_t(t.rb));  // rows per band <= 256
    u = m * t.nbands + b;
    us = (m * t.R + b * t.rb) * t.C;
    ue = (m * t.R + min((b + 1) * t.rb, t.R)) * t.C;
  } else {
    u = f / kTile;
    if (u >= t.nunit) return t.nest[t.nunit];
    us = u * kTile;
    ue = min(us + kTile, t.N);
  }
  const float p0 = t.nest[u], p1 = t.nest[u + 1];
  return p0 + (p1 - p0) * (float(f - us) / float(ue - us));
}

// ---------------------------------------------------------------------------
// segment records
// ---------------------------------------------------------------------------
// One halving step of norm_lane_sums: lanes with bit O set keep values [H, 2H) and send [0, H) to their
// partner lane ^ O, which keeps [0, H); each adds what it receives (H, O compile-time constants).
template <int H, int O>
__device__ __forceinline__ void norm_halve(uint32_t (&v)[16], int lane) {
  const bool up = (lane & O) != 0;
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const uint32_t mine = up ? v[H + k] : v[k];
    const uint32_t other = up ? v[k] : v[H + k];
    v[k] = mine + uint32_t(__shfl_xor(int(other), O, kWave));
  }
}

// Per-chain sums over the 64 lanes of NV values per lane (NV = 8 or 16).  Halving steps with the
// partners lane ^ 32, ^ 16, ... leave each lane one value, value index (lane >> (6 - log2 NV)), summed
// over the lanes that share those bits; butterfly sums over the remaining low lane bits complete it.
// On return v[0] of lane l holds the total of value l >> 3 (NV = 8) or l >> 2 (NV = 16).
template <int NV>
__device__ __forceinline__ void norm_lane_sums(uint32_t (&v)[16], int lane) {
  if constexpr (NV == 16) {
    norm_halve<8, 32>(v, lane);
    norm_halve<4, 16>(v, lane);
    norm_halve<2, 8>(v, lane);
    norm_halve<1, 4>(v, lane);
  } else {
    norm_halve<4, 32>(v, lane);
    norm_halve<2, 16>(v, lane);
    norm_halve<1, 8>(v, lane);
    v[0] += uint32_t(__shfl_xor(int(v[0]), 4, kWave));
  }
  v[0] += uint32_t(__shfl_xor(int(v[0]), 2, kWave));
  v[0] += uint32_t(__shfl_xor(int(v[0]), 1, kWave));
}

// u at flat index e (u_at), with 32-bit index arithmetic where the flat indices fit.
template <typename TG>
__device__ __forceinline__ float norm_x_at(const DevTensor& t, int64_t e, const Hp& hp) {
  if (t.factored && t.idx32) {
    const uint32_t row = udiv_magic(uint32_t(e), t.mC, t.sC);
    const uint32_t j = uint32_t(e) - row * uint32_t(t.C);
    const uint32_t m = udiv_magic(row, t.mR, t.sR);
    const float gv = TG::load(gbl(static_cast<const typename TG::storage*>(t.g))[e]);
    return (gbl(t.rfac)[row] * gbl(t.cfac)[int64_t(m) * t.C + j]) * gv;
  }
  return u_at<TG>(t, e, hp);
}

// The x = u of the 8 elements at flat index f (a multiple of 8) of a factored tensor whose rows hold
// whole 8-element chunks, 16-byte aligned, with flat indices below 2^31.
template <typename TG>
struct NormChunk {
  float g[8], cf[8], r;
  __device__ __forceinline__ void load(const DevTensor& t, uint32_t f) {
    using GS = typename TG::storage;
    const uint32_t row = udiv_magic(f, t.mC, t.sC);
    const uint32_t j = f - row * uint32_t(t.C);
    const uint32_t m = udiv_magic(row, t.mR, t.sR);
    r = gbl(t.rfac)[row];
    load8<TG>(gbl(static_cast<const GS*>(t.g) + f), g);
    load8<F32>(gbl(t.cfac + int64_t(m) * t.C + j), cf);
  }
};

// The per-lane, per-chain sums of one segment's increments under the candidate binade (ka = 23 - Ea)
// and, with TWO, under Ea + 1, with their largest rounding distances.  FULL: the segment holds all
// kNormSegElems elements.
template <typename TG, bool FAST, bool TWO, bool FULL>
__device__ __forceinline__ void norm_seg_sums(const DevTensor& t, int64_t f0, int64_t f1, int ka, int lane,
                                              const Hp& hp, float (&sa)[8], float (&ra)[8], float (&sb)[8],
                                              float (&rb)[8]) {
  auto account = [&](const float (&x)[8]) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float hi = x[v] * x[v];
      norm_acc(hi, ka, sa[v], ra[v]);
      if constexpr (TWO) norm_acc(hi, ka - 1, sb[v], rb[v]);
    }
  };
  if constexpr (FAST) {
    // in a partial segment, chunks past its end load its last chunk and count for nothing
#pragma unroll 1
    for (int h = 0; h < kNormChunks; h += kNormGroup) {
      NormChunk<TG> ch[kNormGroup];
#pragma unroll
      for (int q = 0; q < kNormGroup; ++q) {
        const int64_t f = f0 + (h + q) * 512 + lane * 8;
        ch[q].load(t, uint32_t(FULL ? f : min(f, f1 - 8)));
      }
#pragma unroll
      for (int q = 0; q < kNormGroup; ++q) {
        const bool in = FULL || f0 + (h + q) * 512 + lane * 8 < f1;
        float x[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) x[v] = in ? (ch[q].r * ch[q].cf[v]) * ch[q].g[v] : 0.0f;
        account(x);
      }
    }
  } else {
    for (int q = 0; q < kNormChunks; ++q) {
      const int64_t f = f0 + q * 512 + lane * 8;
      if (f >= f1) break;
      float x[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) x[v] = norm_x_at<TG>(t, f + v, hp);
      account(x);
    }
  }
}

// Writes the records of one segment from the lanes' per-chain sums.
__device__ __forceinline__ void norm_write_records(const DevTensor& t, int64_t seg, int Ea, bool two, int lane,
                                                   const float (&sa)[8], const float (&ra)[8], const float (&sb)[8],
                                                   const float (&rb)[8]) {
  uint32_t acc[16];
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    acc[v] = norm_lane_value(sa[v], ra[v], Ea);
    acc[8 + v] = two ? norm_lane_value(sb[v], rb[v], Ea + 1) : 0u;
  }
  const int64_t nseg = t.nseg;
  uint32_t* __restrict__ W0 = t.nrec;
  uint32_t* __restrict__ WA = t.nrec + 8 * nseg;
  uint32_t* __restrict__ WB = t.nrec + 16 * nseg;
  if (two) {
    norm_lane_sums<16>(acc, lane);  // lane 4c: chain c under Ea; lane 32 + 4c: under Ea + 1
    const int c = (lane >> 2) & 7;
    if ((lane & 3) == 0) {
      const uint32_t sum = min(acc[0], kNormFull);
      if (lane < 32) {
        W0[c * nseg + seg] = uint32_t(Ea + 256) | kRecTwo;
        WA[c * nseg + seg] = sum;
      } else {
        WB[c * nseg + seg] = sum;
      }
    }
  } else {
    norm_lane_sums<8>(acc, lane);  // lane 8c: chain c under Ea
    const int c = lane >> 3;
    if ((lane & 7) == 0) {
      W0[c * nseg + seg] = uint32_t(Ea + 256);
      WA[c * nseg + seg] = min(acc[0], kNormFull);
      WB[c * nseg + seg] = kNormFull;
    }
  }
}

// Candidate binades of a chain whose estimated value is est: Ea, and whether Ea + 1 is one too.
__device__ __forceinline__ void norm_candidates(float est, int& Ea, bool& two) {
  Ea = norm_est_binade(est * 0.875f);
  two = norm_est_binade(est * 1.015625f) > Ea;
}

constexpr int kNormRunSegs = 64;       // segments per work item of k_norm_seg2d
constexpr int kNormLdsCols = 16384;    // widest rows k_norm_seg2d stages in LDS (64 KB of column factors)

// The per-lane, per-chain sums of one whole segment of a matrix (prefix 1) whose column factors are
// staged in LDS (cl), rows of whole 8-element chunks, 16-byte aligned, 32-bit flat indices.  Every
// gradient chunk and row factor of the segment is loaded first; the column factors come from LDS
// as each chunk is accounted.
template <typename TG, bool TWO>
__device__ __forceinline__ void norm_seg_lds(const DevTensor& t, const float* cl, int64_t f0, int ka, int lane,
                                             float (&sa)[8], float (&ra)[8], float (&sb)[8], float (&rb)[8]) {
  using GS = typename TG::storage;
  constexpr int Q = kNormChunks;
  const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g));
  uint32_t gw[Q][sizeof(GS) * 2];  // 16 or 32 bytes of gradient per chunk
  float r[Q];
  uint32_t col[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const uint32_t f = uint32_t(f0) + uint32_t(q * 512 + lane * 8);
    const uint32_t row = udiv_magic(f, t.mC, t.sC);
    col[q] = f - row * uint32_t(t.C);
    r[q] = gbl(t.rfac)[row];
    if constexpr (sizeof(GS) == 2) {
      const u32x4 v = *(const CAME8_GLOBAL u32x4*)(g + f);
      gw[q][0] = v.x; gw[q][1] = v.y; gw[q][2] = v.z; gw[q][3] = v.w;
    } else {
      const u32x4 a = *(const CAME8_GLOBAL u32x4*)(g + f);
      const u32x4 b = *(const CAME8_GLOBAL u32x4*)(g + f + 4);
      gw[q][0] = a.x; gw[q][1] = a.y; gw[q][2] = a.z; gw[q][3] = a.w;
      gw[q][4] = b.x; gw[q][5] = b.y; gw[q][6] = b.z; gw[q][7] = b.w;
    }
  }
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(cl + col[q]);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(cl + col[q] + 4);
    const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float x = (r[q] * cv[v]) * TG::elem(gw[q], v);
      const float hi = x * x;
      norm_acc(hi, ka, sa[v], ra[v]);
      if constexpr (TWO) norm_acc(hi, ka - 1, sb[v], rb[v]);
    }
  }
}

// Records of the whole segments [0, nseg0) of 2-D factored tensors whose rows hold whole 8-element
// chunks (at most kNormLdsCols), 16-byte aligned, with 32-bit flat indices (the host checks); the last,
// partial segment is k_norm_seg's.  A work item is a run of
// kNormRunSegs segments: the workgroup stages the matrix's column factors in LDS once, and its four
// wavefronts take every fourth segment of the run.
template <typename TG>
__global__ __launch_bounds__(kThreads) void k_norm_seg2d(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  extern __shared__ float cl[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  int32_t staged = -1;
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const int32_t ti = tids[slot];
    const DevTensor& t = T[ti];
    if (ti != staged) {  // uniform over the workgroup
      __syncthreads();
      for (int64_t j = tid * 4; j < t.C; j += kThreads * 4)
        *reinterpret_cast<f32x4*>(cl + j) = *reinterpret_cast<const CAME8_GLOBAL f32x4*>(gbl(t.cfac) + j);
      __syncthreads();
      staged = ti;
    }
    const int64_t run0 = (w - wstart[slot]) * kNormRunSegs;
    const int64_t nrun = min(int64_t(kNormRunSegs), t.nseg0 - run0);
    const int64_t main = t.N - (t.N & 7);
    // the estimate at both ends of the run, linear in between (a chain holds about 1/8 of it)
    const float e0 = uniform_f32(norm_est_at(t, run0 * kNormSegElems)) * 0.125f;
    const float e1 = uniform_f32(norm_est_at(t, min((run0 + nrun) * kNormSegElems, main))) * 0.125f;
#pragma unroll 1
    for (int64_t k = wid; k < nrun; k += 4) {
      const int64_t seg = run0 + k;
      const int64_t f0 = seg * kNormSegElems;
      int Ea;
      bool two;
      norm_candidates(e0 + (e1 - e0) * (float(k) / float(nrun)), Ea, two);
      const int ka = 23 - Ea;
      float sa[8], sb[8], ra[8], rb[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) sa[v] = sb[v] = ra[v] = rb[v] = 0.0f;
      if (two) norm_seg_lds<TG, true>(t, cl, f0, ka, lane, sa, ra, sb, rb);
      else norm_seg_lds<TG, false>(t, cl, f0, ka, lane, sa, ra, sb, rb);
      norm_write_records(t, seg, Ea, two, lane, sa, ra, sb, rb);
    }
  }
}

// Records of the segments [nseg0, nseg).  One wavefront per segment (four per workgroup).  Lane l
// takes the 8-element chunks at
// 512q + 8l (q < kNormChunks) of the segment: element v of a chunk belongs to chain v.  FAST: the
// tensor is factored, its rows hold whole 8-element chunks, the gradient is 16-byte aligned and
// N < 2^31 (the host checks); otherwise every element goes through u_at.
template <typename TG, bool FAST>
__global__ __launch_bounds__(kThreads, 4) void k_norm_seg(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                          const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t seg = t.nseg0 + (w - wstart[slot]) * 4 + wid;
    if (seg >= t.nseg) continue;  // uniform over the wavefront
    const int64_t main = t.N - (t.N & 7);
    const int64_t f0 = seg * kNormSegElems;
    const int64_t f1 = min(f0 + kNormSegElems, main);
    // candidate binades from the estimate at the segment's start (a chain holds about 1/8 of it)
    int Ea;
    bool two;
    norm_candidates(uniform_f32(norm_est_at(t, f0)) * 0.125f, Ea, two);
    const int ka = 23 - Ea;
    float sa[8], sb[8], ra[8], rb[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) sa[v] = sb[v] = ra[v] = rb[v] = 0.0f;
    const bool full = f1 - f0 == kNormSegElems;
    if (two) {
      if (full) norm_seg_sums<TG, FAST, true, true>(t, f0, f1, ka, lane, hp, sa, ra, sb, rb);
      else norm_seg_sums<TG, FAST, true, false>(t, f0, f1, ka, lane, hp, sa, ra, sb, rb);
    } else {
      if (full) norm_seg_sums<TG, FAST, false, true>(t, f0, f1, ka, lane, hp, sa, ra, sb, rb);
      else norm_seg_sums<TG, FAST, false, false>(t, f0, f1, ka, lane, hp, sa, ra, sb, rb);
    }
    norm_write_records(t, seg, Ea, two, lane, sa, ra, sb, rb);
  }
}

// ---------------------------------------------------------------------------
// walk
// ---------------------------------------------------------------------------
// Replays chain c of segment seg from s with fmaf, element by element, as the reference does (one
// wavefront; lane 0 runs the chain).
template <typename TG>
__device__ float norm_replay(const DevTensor& t, int c, int64_t seg, float s, const Hp& hp, float* xs) {
  const int lane = threadIdx.x;
  const int64_t main = t.N - (t.N & 7);
  const int64_t f0 = seg * kNormSegElems;
  const int cnt = int(min(int64_t(kNormChainSeg), (main - f0) / 8));
#pragma unroll
  for (int i = 0; i < kNormChainSeg / kWave; ++i) {
    const int k = i * kWave + lane;
    if (k < cnt) xs[k] = norm_x_at<TG>(t, f0 + 8 * int64_t(k) + c, hp);
  }
  __syncthreads();
  if (lane == 0) {
    int k = 0;
    for (; k + 16 <= cnt; k += 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = xs[k + u];
#pragma unroll
      for (int u = 0; u < 16; ++u) s = fmaf(v[u], v[u], s);
    }
    for (; k < cnt; ++k) s = fmaf(xs[k], xs[k], s);
    xs[kNormChainSeg] = s;
  }
  __syncthreads();
  s = xs[kNormChainSeg];
  __syncthreads();
  return s;
}

constexpr uint32_t kNormSat = 1u << 25;  // saturating integer sums: anything >= 2^24 leaves the binade
__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) { return min(a + b, kNormSat); }

// The increment of a segment's record for a chain in binade E, or kNormSat when the record does not
// cover E.  With s = +inf (E = 128), a segment needs its replay only if it may hold a NaN: an
// exception, which saturates both sums.
__device__ __forceinline__ uint32_t norm_rec_add(uint32_t w0, uint32_t wa, uint32_t wb, int E) {
  const int Ea = int(w0 & 511u) - 256;
  const bool two = (w0 & kRecTwo) != 0;
  const uint32_t fin = E == Ea ? wa : ((two && E == Ea + 1) ? wb : kNormSat);
  const uint32_t inf = (wa >= kNormFull && (!two || wb >= kNormFull)) ? kNormSat : 0u;
  return E == 128 ? inf : fin;
}

constexpr int kNormWalkThreads = kWave;  // one wavefront per chain

// One wavefront per (tensor, chain).  Each batch: every lane sums the records of its run of
// kNormWalkSegs segments under the chain's binade, a scan over the lanes finds the first segment
// whose record does not cover the binade or takes the chain out of it, every segment before it is
// skipped with its integer sum, and that segment is replayed.
template <typename TG>
__global__ __launch_bounds__(kNormWalkThreads) void k_norm_walk(const DevTensor* __restrict__ T,
                                                                const int32_t* __restrict__ tids,
                                                                const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  __shared__ float xs[kNormChainSeg + 1];
  const int lane = threadIdx.x;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int c = int(w - wstart[slot]);
    const int64_t nseg = t.nseg;
    const CAME8_GLOBAL uint32_t* __restrict__ W0 = gbl(t.nrec + c * nseg);
    const CAME8_GLOBAL uint32_t* __restrict__ WA = gbl(t.nrec + (8 + c) * nseg);
    const CAME8_GLOBAL uint32_t* __restrict__ WB = gbl(t.nrec + (16 + c) * nseg);
    float s = 0.0f;
    int64_t seg = 0;
    while (seg < nseg && s == s) {  // a NaN chain stays NaN
      const bool inf = !(s <= 0x1.fffffep127f);
      const int E = inf ? 128 : norm_binade(s);
      const uint32_t m = inf ? 0u : norm_mant(s, E);
      const uint32_t room = kNormFull - m;  // the chain leaves its binade once its increments reach this
      const int64_t base = seg + int64_t(lane) * kNormWalkSegs;
      uint32_t add[kNormWalkSegs], r0[kNormWalkSegs], ra[kNormWalkSegs], rb[kNormWalkSegs];
#pragma unroll
      for (int j = 0; j < kNormWalkSegs; ++j) {  // every load first, then the decoding
        const int64_t k = min(base + j, nseg - 1);
        r0[j] = W0[k];
        ra[j] = WA[k];
        rb[j] = WB[k];
      }
#pragma unroll
      for (int j = 0; j < kNormWalkSegs; ++j) add[j] = norm_rec_add(r0[j], ra[j], rb[j], E);
      // this lane's run: the sum of its records up to the first one that stops the chain
      uint32_t run = 0;
      bool stop = false;
#pragma unroll
      for (int j = 0; j < kNormWalkSegs; ++j) {
        if (base + j < nseg && !stop) {
          if (add[j] >= kNormSat) stop = true;
          else run = sat_add(run, add[j]);
        }
      }
      // inclusive scan of the runs over the lanes (saturating sums, in lane order)
      uint32_t incl = run;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t y = uint32_t(__shfl_up(int(incl), o, kWave));
        if (lane >= o) incl = sat_add(incl, y);
      }
      const uint32_t prev = uint32_t(__shfl_up(int(incl), 1, kWave));
      const uint32_t excl = lane == 0 ? 0u : prev;  // exact while the chain has not left its binade
      const uint32_t tot = uint32_t(__shfl(int(incl), kWave - 1, kWave));
      // the first lane whose run is cut short or takes the chain out of its binade
      const uint64_t bal = __ballot(base < nseg && (stop || sat_add(excl, run) >= room));
      if (bal == 0) {
        if (!inf) s = norm_value(m + tot, E);  // tot < room
        seg = min(nseg, seg + int64_t(kNormWalkThreads) * kNormWalkSegs);
        continue;
      }
      const int first = __builtin_ctzll(bal);
      uint32_t acc = excl;
      int64_t k = base;
#pragma unroll
      for (int j = 0; j < kNormWalkSegs; ++j) {
        if (k == base + j && base + j < nseg && add[j] < kNormSat && acc + add[j] < room) {
          acc += add[j];
          k = base + j + 1;
        }
      }
      const uint32_t mm = m + uint32_t(__shfl(int(acc), first, kWave));
      const int64_t ks = __shfl(k, first, kWave);
      s = norm_replay<TG>(t, c, ks, inf ? s : norm_value(mm, E), hp, xs);
      seg = ks + 1;
    }
    if (lane == 0) t.nchain[c] = s;
    __syncthreads();
  }
}

// The eight accumulators added left to right, the tail elements as rounded square-and-add, sqrt, and
// the clip divisor.  A thread per tensor.
template <typename TG>
__global__ __launch_bounds__(kThreads) void k_norm_final(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         int ntens, Hp hp) {
  const int k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= ntens) return;
  const DevTensor& t = T[tids[k]];
  float b = t.nchain[0];
  for (int j = 1; j < 8; ++j) b = b + t.nchain[j];
  for (int64_t d = t.N - (t.N & 7); d < t.N; ++d) {
    const float u = u_at<TG>(t, d, hp);
    const float uu = u * u;
    b = b + uu;
  }
  const float c = clip_from_norm(sqrtf(b), t.N, hp);
  t.clip[0] = c;
  t.clip[1] = rcp_for_div(c);
}

}  // namespace came8
