// The clip's update norm in the reference's own summation order, computed in parallel.
//
// The reference clips the update by its RMS, u.norm(2) / sqrt(N) (came_pytorch/CAME8bitFull.py:121-122,
// 1032).  On CPU, torch sums a contiguous fp32 tensor's squares for norm(2) in one thread as eight
// interleaved accumulators, acc[i % 8] = fma(u_i, u_i, acc[i % 8]) over the first N - N % 8 elements,
// then acc[0] + acc[1] + ... + acc[7] left to right, then the N % 8 remaining elements: when four or
// more remain, the next four as rounded squares added one at a time, b = (b + RN(u*u)), then the last
// N % 4 as fused multiply-adds, b = fma(u, u, b); then a correctly rounded sqrt.  Each accumulator is a serial chain of up to
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
// a tie, whose rounding depends on m's parity), or x*x is infinite or NaN; an element whose increment
// takes the chain out of the binade ends the run of known increments.  (When the rounded square is
// not a half-integer, the true square rounds the same way: its distance to hi = RN(x*x) is at most
// half an ulp of hi, less than the distance from hi to any half-integer, for every binade above the
// subnormal one, whose half-integers lie on hi's grid.)
//
//   k_norm_est               an estimate of each chain's value along the tensor, from sums the step
//                            has already formed (per row band: rm * sum_j c_j^2 * sum_i g_ij^2 / R_i;
//                            per 1-D tile: the tile's sum of u^2); the records kernels add the units
//                            before a segment themselves (norm_unit_prefix).
//   k_norm_seg               one workgroup per segment of kNormSegElems elements (512 per chain):
//                            per chain, the candidate binade Ea of the estimate (and Ea + 1 near a
//                            binade edge), the integer sums of the increments under each, whether
//                            the segment holds special elements, and whether it holds a NaN; and
//                            the chain's fp32 sum of the segment's rounded squares.
//   k_norm_bsum, k_norm_fix  each chain's own estimate (the prefix of its segment sums), and records
//                            rebuilt under that estimate's binades where the tensor-wide estimate
//                            (an eighth of the prefix) named others.  The chains of heavy-tailed
//                            updates drift far apart; without the rebuild most of their segments
//                            would miss and be replayed.
//   k_norm_walk              one wavefront per chain: applies the first segment from s = 0 element by
//                            element (no record of it is read: a tensor of one segment forms none),
//                            then skips every run of segments whose record covers the chain's current
//                            binade without specials and without leaving the binade (a wavefront scan
//                            of the integer sums), and replays the segment where that fails: binade
//                            crossings, specials, and estimates that missed.  A replay holds the
//                            segment's 512 elements in the wavefront and applies the increments of the
//                            chain's binade with a saturating prefix sum up to the first element that
//                            leaves the binade or is special, that element with fmaf, and so on: one
//                            round per crossing or special element.
//   k_norm_final             the eight accumulators and the tail in the reference's order, sqrt,
//                            and the clip divisor.
//
// Only the replay's fmaf of an element that leaves the binade (or is special) uses floating-point
// addition on the chain; everything else is exact integer arithmetic, so the result equals the
// serial chain bit for bit whatever the estimates were (they only decide how many segments are
// replayed).
//
// The subnormal binade E = -126 (unit 2^-149, which is also the spacing of subnormal squares) has
// one more special element: |x| = 2^-75, whose square 2^-150 is half a unit (a tie) but rounds to 0
// as x * x.  (For |x| = k * 2^-75 with odd k > 1 the square rounds to a nonzero multiple of the
// unit, which is special there already.)
#pragma once

#include "came8_kernels.h"

namespace came8 {

constexpr int kNormSegElems = 4096;                    // flat elements per segment (a multiple of 8)
constexpr int kNormChainSeg = kNormSegElems / 8;       // elements per chain per segment
constexpr int kNormChunks = kNormSegElems / (8 * 64);  // 8-element chunks per lane of a segment's wavefront
// segments per thread per batch of the walk: after each replay the walk scans its lanes' records again,
// so a batch of fewer records per lane makes each scan shorter, at one batch load more per 64 * this
// many segments (with the replays' loads issued together: C1 0.2058 / 0.1997 ms and C2 2.131 / 2.115
// ms with 8 / 4, C4 the same; 16 and 32 slower)
constexpr int kNormWalkSegs = 4;
static_assert(kNormWalkSegs % 4 == 0, "the walk loads each lane's records four at a time");
constexpr int kNormGroup = 2;                          // chunks per lane loaded together
constexpr int64_t kNormMaxUnits = 4096;                // estimate units per tensor of single-band matrices
                                                       // or tiles (more are grouped)

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
// kernel keeps, per lane and chain, the running sum of rint(dh) and either the largest |dh - rint(dh)|
// or (k_norm_seg2d) per chain a wavefront mask of the lanes that met a tie (a compare into a scalar
// register and a scalar or: one VALU instruction per element instead of two); the exceptions are then
// read off per lane once:
//   * a tie (some |dh - rint(dh)| = 0.5): the rounding of that element depends on the chain's parity;
//   * dh >= 2^23: in a normal binade (m >= 2^23) it takes the chain out of the binade by itself, so
//     the segment's sum, at least 2^23, already fails the walk's test m + sum < 2^24;
//   * the subnormal binade (E = -126, k = 149), where hi's own rounding may hide a tie: any nonzero
//     increment there, and any |x| = 2^-75 (NormAcc's TINY form);
//   * NaN or infinite squares: a NaN or infinite sum.
// An exception saturates the segment's sum at kNormFull, which makes the walk replay the segment.
constexpr float kNormSpecial = 0x1p24f;
__device__ __forceinline__ void norm_acc(float hi, int k, float& sum, float& rmax) {
  const float dh = ldexpf(hi, k);
  const float nf = rintf(dh);
  sum += nf;
  rmax = fmaxf(rmax, fabsf(dh - nf));
}
// the same, returning whether the element is a tie
__device__ __forceinline__ bool norm_acc_tie(float hi, int k, float& sum) {
  const float dh = ldexpf(hi, k);
  const float nf = rintf(dh);
  sum += nf;
  return fabsf(dh - nf) == 0.5f;
}
// the lane's sum for one chain as the record's integer, or kNormFull for an exception
__device__ __forceinline__ uint32_t norm_lane_value(float sum, bool tie, int E) {
  const bool bad = !(sum < kNormSpecial) || tie || (E == -126 && sum != 0.0f);
  return bad ? (1u << 24) : uint32_t(sum);
}
__device__ __forceinline__ uint32_t norm_lane_value(float sum, float rmax, int E) {
  return norm_lane_value(sum, rmax == 0.5f, E);
}
// lane `lane`'s bit of a wavefront mask
__device__ __forceinline__ bool norm_bit(uint64_t mask, int lane) { return ((mask >> lane) & 1u) != 0; }

// Record word 0: Ea + 256 (9 bits) | kRecTwo when word 2 holds the sum under Ea + 1.  Words 1 and 2:
// the integer sums of the increments under Ea and Ea + 1, at most 2^24 (2^24: the segment leaves
// the binade or holds a special element).
constexpr uint32_t kRecTwo = 1u << 9;
constexpr uint32_t kNormFull = 1u << 24;

// ---------------------------------------------------------------------------
// estimates
// ---------------------------------------------------------------------------
// Units: row band b of matrix m (unit m * nbands + b; for matrices of the thread-per-matrix passes the
// matrix is its band) or 2048-element tile u of a 1-D tensor.  The sum of u_ij^2 over a band is
// rm * sum_i (1 / R_i) * sum_j c_j^2 * g_ij^2 without the roundings.  A matrix of the thread-per-matrix
// passes has it from W_j = sum_i g_ij^2 / R_i (their column partials): rm * sum_j c_j^2 * W_j.  The band
// passes of the default clip mode keep no W (k_fact_pass1n); their estimate gives every row of the band
// the band's column profile of g^2 (the partials U_j):
//   rm * (sum_i e_i / R_i) * (sum_j c_j^2 U_j) / (sum_j U_j),   e_i = sum_j g_ij^2,
// exact when the rows' profiles agree (Gaussian rows: ~1e-5 relative per band) and a few percent off
// on heavy-tailed rows; k_norm_fix rebuilds the records of a chain that the estimate misleads.
__device__ __forceinline__ float norm_unit_rm(const DevTensor& t, int64_t u) {
  return matrix_row_mean(t, t.rsum, u / t.nbands, t.nbands);
}

// WIDE: a workgroup per unit (matrices of at least 256 columns); otherwise a thread per unit.
template <bool WIDE>
__global__ __launch_bounds__(kThreads) void k_norm_est(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                       const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  __shared__ float ssum[4], usum[4];
  __shared__ double rsm[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    if constexpr (WIDE) {  // band passes (never the thread-per-matrix ones)
      const int64_t u = w - wstart[slot];
      const int64_t m = u / t.nbands;
      const float* __restrict__ Up = t.partU + u * t.C;
      const float* __restrict__ cf = t.cfac + m * t.C;
      // kEstBatch columns per thread loaded before the first is added (an estimate: the order is free)
      constexpr int kEstBatch = 8;
      float acc[kEstBatch] = {}, accu[kEstBatch] = {};
      int64_t j = tid;
      for (; j + (kEstBatch - 1) * kThreads < t.C; j += kEstBatch * kThreads) {
        float c[kEstBatch], uv[kEstBatch];
#pragma unroll
        for (int q = 0; q < kEstBatch; ++q) {
          c[q] = cf[j + q * kThreads];
          uv[q] = Up[j + q * kThreads];
        }
#pragma unroll
        for (int q = 0; q < kEstBatch; ++q) {
          acc[q] = fmaf(c[q] * c[q], uv[q], acc[q]);
          accu[q] += uv[q];
        }
      }
      for (; j < t.C; j += kThreads) {
        acc[0] = fmaf(cf[j] * cf[j], Up[j], acc[0]);
        accu[0] += Up[j];
      }
      // the matrix's mean row state (norm_unit_rm's): the workgroup sums the band sums, thread k over
      // sums k, k + 256, ... (one round of loads, not one thread's chain after the reductions)
      double rp = 0.0;
      for (int64_t k = tid; k < t.nbands; k += kThreads) rp += double(t.rsum[m * t.nbands + k]);
      float s = 0.0f, su = 0.0f;
#pragma unroll
      for (int q = 0; q < kEstBatch; ++q) {
        s += acc[q];
        su += accu[q];
      }
      s = wave_sum(s);
      su = wave_sum(su);
      rp = wave_sum(rp);
      if (lane == 0) {
        ssum[wid] = s;
        usum[wid] = su;
        rsm[wid] = rp;
      }
      __syncthreads();
      if (tid == 0) {
        const float cs = ((ssum[0] + ssum[1]) + ssum[2]) + ssum[3];
        const float us = ((usum[0] + usum[1]) + usum[2]) + usum[3];
        const float rm = row_mean_of_sum(t, ((rsm[0] + rsm[1]) + rsm[2]) + rsm[3]);
        t.nest[u] = us > 0.0f ? rm * t.esum[u] * (cs / us) : 0.0f;
      }
      __syncthreads();
    } else {
      const int64_t u = (w - wstart[slot]) * kThreads + tid;
      if (u >= t.nunit) continue;
      // the unit's ngrp base units: row bands, or (ngrp > 1) whole single-band matrices, or tiles
      const int64_t nbase = t.factored ? t.P * t.nbands : t.nclip;
      const int64_t b0 = u * t.ngrp, b1 = min(nbase, b0 + t.ngrp);
      float e = 0.0f;
      for (int64_t b = b0; b < b1; ++b) {
        if (t.factored && t.R * t.C <= kTinyElems) {  // the thread-per-matrix passes wrote W
          const int64_t m = b / t.nbands;
          const float* __restrict__ W = t.partW + b * t.C;
          const float* __restrict__ cf = t.cfac + m * t.C;
          float s = 0.0f;
          for (int64_t j = 0; j < t.C; ++j) s = fmaf(cf[j] * cf[j], W[j], s);
          e += norm_unit_rm(t, b) * s;
        } else if (t.factored) {  // a band pass of the default mode: the band's profile of g^2
          const int64_t m = b / t.nbands;
          const float* __restrict__ Up = t.partU + b * t.C;
          const float* __restrict__ cf = t.cfac + m * t.C;
          float s = 0.0f, su = 0.0f;
          for (int64_t j = 0; j < t.C; ++j) {
            s = fmaf(cf[j] * cf[j], Up[j], s);
            su += Up[j];
          }
          e += su > 0.0f ? norm_unit_rm(t, b) * t.esum[b] * (s / su) : 0.0f;
        } else {
          e += float(t.clip_part[b]);
        }
      }
      t.nest[u] = e;
    }
  }
}

// The estimated sum of u^2 over the units before unit u (0 <= u <= nunit), from the units' own
// estimates: the wavefront adds them, lane l over units l, l + 64, ..., eight loads in flight.  Every
// lane of the wavefront calls it with the same u and gets the same value.  (The order of the sum is
// free: an estimate decides only which segments are replayed, never the result.)
__device__ __forceinline__ float norm_unit_prefix(const DevTensor& t, int64_t u) {
  const int lane = threadIdx.x & (kWave - 1);
  const CAME8_GLOBAL float* __restrict__ e = gbl(t.nest);
  float s = 0.0f;
  int64_t k = lane;
  for (; k + 7 * kWave < u; k += 8 * kWave) {
    float v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = e[k + q * kWave];
#pragma unroll
    for (int q = 0; q < 8; ++q) s += v[q];
  }
  for (; k < u; k += kWave) s += e[k];
  return wave_sum(s);
}

// Estimated sum of u^2 over the flat elements before f (0 <= f <= N), linear inside a unit.
__device__ __forceinline__ float norm_est_at(const DevTensor& t, int64_t f) {
  int64_t u, us, ue;
  if (t.factored) {
    const int64_t row = t.idx32 ? int64_t(udiv_magic(uint32_t(f), t.mC, t.sC)) : f / t.C;
    const int64_t m = t.idx32 ? int64_t(udiv_magic(uint32_t(row), t.mR, t.sR)) : row / t.R;
    if (m >= t.P) return norm_unit_prefix(t, t.nunit);
    const int64_t i = row - m * t.R;
    if (t.ngrp > 1) {  // groups of ngrp single-band matrices
      u = m / t.ngrp;
      us = u * t.ngrp * t.R * t.C;
      ue = min(t.P, (u + 1) * t.ngrp) * t.R * t.C;
    } else {
      const int64_t b = int64_t(uint32_t(i) / uint32_t(t.rb));  // rows per band <= 256
      u = m * t.nbands + b;
      us = (m * t.R + b * t.rb) * t.C;
      ue = (m * t.R + min((b + 1) * t.rb, t.R)) * t.C;
    }
  } else {
    u = f / (kTile * t.ngrp);
    if (u >= t.nunit) return norm_unit_prefix(t, t.nunit);
    us = u * kTile * t.ngrp;
    ue = min(us + kTile * t.ngrp, t.N);
  }
  return norm_unit_prefix(t, u) + gbl(t.nest)[u] * (float(f - us) / float(ue - us));
}

// ---------------------------------------------------------------------------
// segment records
// ---------------------------------------------------------------------------
// One halving step of norm_group_sums: lanes with bit O set keep values [H, 2H) and send [0, H) to their
// partner lane ^ O, which keeps [0, H); each adds what it receives (H, O compile-time constants).
template <int H, int O, typename T, int L>
__device__ __forceinline__ void norm_halve(T (&v)[L], int lane) {
  const bool up = (lane & O) != 0;
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const T mine = up ? v[H + k] : v[k];
    const T other = up ? v[k] : v[H + k];
    v[k] = mine + __shfl_xor(other, O, kWave);
  }
}

// Per-value sums over groups of G lanes (G a power of two up to 64) of NV values per lane (NV = 8 or
// 16).  Halving steps with the partners lane ^ G/2, ^ G/4, ... leave each lane NV / G values (NV > G)
// or one, summed over the lanes that share the lane bits halved so far; butterfly sums over the
// remaining low lane bits complete it (NV < G).  On return, lane i of a group (i = lane % G) holds
// the totals of values i * NV / G + k in v[k], k < NV / G (NV >= G), or of value i / (G / NV) in v[0]
// (NV < G).
template <int O, int H, typename T, int L>
__device__ __forceinline__ void norm_group_steps(T (&v)[L], int lane) {
  if constexpr (O >= 1) {
    if constexpr (H >= 1) {
      norm_halve<H, O>(v, lane);
    } else {
      v[0] += __shfl_xor(v[0], O, kWave);
    }
    norm_group_steps<O / 2, H / 2>(v, lane);
  }
}
template <int G, int NV, typename T, int L>
__device__ __forceinline__ void norm_group_sums(T (&v)[L], int lane) {
  static_assert(L >= NV && G >= 2 && G <= kWave && (G & (G - 1)) == 0, "bad group");
  norm_group_steps<G / 2, NV / 2>(v, lane);
}
// The same over the whole wavefront: v[0] of lane l holds the total of value l >> 3 (NV = 8) or l >> 2
// (NV = 16).
template <int NV, typename T, int L>
__device__ __forceinline__ void norm_lane_sums(T (&v)[L], int lane) {
  norm_group_sums<kWave, NV>(v, lane);
}

// u_at of the 8 elements e[v] (in bounds) of any tensor, every operand loaded before the first is
// used: the tensor's kind is tested once for the 8, so that no branch between the elements makes the
// wavefront wait out each element's loads in turn.
template <typename TG>
__device__ __forceinline__ void norm_x_any8(const DevTensor& t, const int64_t (&e)[8], const Hp& hp, float (&x)[8]) {
  using GS = typename TG::storage;
  const CAME8_GLOBAL GS* __restrict__ gp = gbl(static_cast<const GS*>(t.g));
  float gv[8], a[8], b[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) gv[v] = TG::load(gp[e[v]]);
  if (t.factored) {
    const CAME8_GLOBAL float* __restrict__ rf = gbl(t.rfac);
    const CAME8_GLOBAL float* __restrict__ cf = gbl(t.cfac);
    if (t.idx32) {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const uint32_t row = udiv_magic(uint32_t(e[v]), t.mC, t.sC);
        const uint32_t j = uint32_t(e[v]) - row * uint32_t(t.C);
        const uint32_t m = udiv_magic(row, t.mR, t.sR);
        a[v] = rf[row];
        b[v] = cf[int64_t(m) * t.C + j];
      }
    } else {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int64_t row = e[v] / t.C;
        const int64_t j = e[v] - row * t.C;
        a[v] = rf[row];
        b[v] = cf[(row / t.R) * t.C + j];
      }
    }
#pragma unroll
    for (int v = 0; v < 8; ++v) x[v] = (a[v] * b[v]) * gv[v];
  } else {
    if (t.fp32st) {
#pragma unroll
      for (int v = 0; v < 8; ++v) a[v] = gbl(st_sq_row(t))[e[v]];
    } else {
#pragma unroll
      for (int v = 0; v < 8; ++v) a[v] = deq_u8(gbl(t.rq)[e[v]], gbl(t.ra)[blk_of(e[v], hp)]);
    }
#pragma unroll
    for (int v = 0; v < 8; ++v) x[v] = rsqrt_ref(vec_v_from(gv[v], a[v], hp)) * gv[v];
  }
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

// The same for a factored tensor of at least 8 columns whose rows do not hold whole chunks: the chunk
// may end in the next row (and the next matrix); its gradient is still 16-byte aligned.
template <typename TG>
__device__ __forceinline__ void norm_chunk_rows(const DevTensor& t, uint32_t f, float (&x)[8]) {
  using GS = typename TG::storage;
  const uint32_t C = uint32_t(t.C);
  const uint32_t row = udiv_magic(f, t.mC, t.sC);
  const uint32_t j = f - row * C;
  const uint32_t m0 = udiv_magic(row, t.mR, t.sR);
  float gv[8];
  load8<TG>(gbl(static_cast<const GS*>(t.g) + f), gv);
  const bool cross = j + 8 > C;  // the elements from C - j on are the next row's
  const uint32_t m1 = cross ? udiv_magic(row + 1, t.mR, t.sR) : m0;
  const float r0 = gbl(t.rfac)[row];
  const float r1 = cross ? gbl(t.rfac)[row + 1] : r0;
  const CAME8_GLOBAL float* __restrict__ cf = gbl(t.cfac);
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const bool nx = j + v >= C;
    const uint32_t col = nx ? j + v - C : j + v;
    const float c = cf[int64_t(nx ? m1 : m0) * C + col];
    x[v] = ((nx ? r1 : r0) * c) * gv[v];
  }
}

// How a norm kernel loads the x of a tensor's 8-element chunks: kNormVec for factored tensors whose rows
// hold whole chunks, kNormRows for other factored tensors of at least 8 columns (both: gradient 16-byte
// aligned, N < 2^31; the host checks), kNormAny (u_at of each element) for the rest.
constexpr int kNormAny = 0, kNormRows = 1, kNormVec = 2;

// Per-lane, per-chain accumulators of one segment: the integer sums of the increments under the
// candidate binades Ea (sa) and Ea + 1 (sb), their largest rounding distances (ra, rb), and the fp32
// sum of the rounded squares (hs).
struct NormAcc {
  float sa[8], ra[8], sb[8], rb[8], hs[8];
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int v = 0; v < 8; ++v) sa[v] = ra[v] = sb[v] = rb[v] = hs[v] = 0.0f;
  }
  // element x of chain v under ka = 23 - Ea (TWO: and ka - 1).  TINY: Ea = -126, where |x| = 2^-75
  // is a tie that x * x hides.
  template <bool TWO, bool TINY>
  __device__ __forceinline__ void add(int v, float x, int ka) {
    const float hi = x * x;
    hs[v] += hi;
    norm_acc(hi, ka, sa[v], ra[v]);
    if constexpr (TWO) norm_acc(hi, ka - 1, sb[v], rb[v]);
    if constexpr (TINY) ra[v] = fabsf(x) == 0x1p-75f ? 0.5f : ra[v];
  }
  // both binades, with the TINY rule when tiny (the rebuild of k_norm_fix, a binade per chain)
  __device__ __forceinline__ void add_both(int v, float x, int ka, bool tiny) {
    const float hi = x * x;
    norm_acc(hi, ka, sa[v], ra[v]);
    norm_acc(hi, ka - 1, sb[v], rb[v]);
    ra[v] = tiny && fabsf(x) == 0x1p-75f ? 0.5f : ra[v];
  }
  __device__ __forceinline__ bool tie_a(int v, int) const { return ra[v] == 0.5f; }
  __device__ __forceinline__ bool tie_b(int v, int) const { return rb[v] == 0.5f; }
};

// NormAcc of k_norm_seg2d: the ties as per-chain wavefront masks of the lanes that met one (ta, tb;
// scalar registers), which takes one VALU instruction per element and binade fewer than the largest
// rounding distance.  (The other record kernels, whose loops are not unrolled, keep NormAcc: their
// sixteen masks there spill scalar registers.)  Every lane of the wavefront takes part in add.
struct NormAccM {
  float sa[8], sb[8], hs[8];
  uint64_t ta[8], tb[8];
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      sa[v] = sb[v] = hs[v] = 0.0f;
      ta[v] = tb[v] = 0;
    }
  }
  template <bool TWO, bool TINY>
  __device__ __forceinline__ void add(int v, float x, int ka) {
    const float hi = x * x;
    hs[v] += hi;
    ta[v] |= __ballot(norm_acc_tie(hi, ka, sa[v]));
    if constexpr (TWO) tb[v] |= __ballot(norm_acc_tie(hi, ka - 1, sb[v]));
    if constexpr (TINY) ta[v] |= __ballot(fabsf(x) == 0x1p-75f);
  }
  // An empty asm that reads and writes the sums: in a fully unrolled segment the code generator would
  // otherwise defer the roundings to the segment's end (their results are read only there) and hold
  // every square until then.
  template <bool TWO>
  __device__ __forceinline__ void pin() {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      asm volatile("" : "+v"(sa[v]), "+v"(hs[v]), "+s"(ta[v]));
      if constexpr (TWO) asm volatile("" : "+v"(sb[v]), "+s"(tb[v]));
    }
  }
  __device__ __forceinline__ bool tie_a(int v, int lane) const { return norm_bit(ta[v], lane); }
  __device__ __forceinline__ bool tie_b(int v, int lane) const { return norm_bit(tb[v], lane); }
};

// The x of the 8 elements at flat index f (a multiple of 8): element v belongs to chain v.  Elements
// at or past f1 (a multiple of 8) are 0.
template <typename TG, int FORM>
__device__ __forceinline__ void norm_chunk_x(const DevTensor& t, int64_t f, int64_t f1, const Hp& hp,
                                             float (&x)[8]) {
  const bool in = f < f1;
  if constexpr (FORM == kNormVec) {
    NormChunk<TG> ch;
    ch.load(t, uint32_t(in ? f : f1 - 8));
#pragma unroll
    for (int v = 0; v < 8; ++v) x[v] = in ? (ch.r * ch.cf[v]) * ch.g[v] : 0.0f;
  } else if constexpr (FORM == kNormRows) {
    norm_chunk_rows<TG>(t, uint32_t(in ? f : f1 - 8), x);
#pragma unroll
    for (int v = 0; v < 8; ++v) x[v] = in ? x[v] : 0.0f;
  } else {  // a chunk past f1 reads the last chunk before it (f1 >= 8)
    int64_t e[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) e[v] = (in ? f : f1 - 8) + v;
    norm_x_any8<TG>(t, e, hp, x);
#pragma unroll
    for (int v = 0; v < 8; ++v) x[v] = in ? x[v] : 0.0f;
  }
}

// The per-lane, per-chain sums of one segment's increments under the candidate binade (ka = 23 - Ea)
// and, with TWO, under Ea + 1, with their largest rounding distances and the sums of the squares.
// FULL: the segment holds all kNormSegElems elements.
template <typename TG, int FORM, bool TWO, bool TINY, bool FULL>
__device__ __forceinline__ void norm_seg_sums(const DevTensor& t, int64_t f0, int64_t f1, int ka, int lane,
                                              const Hp& hp, NormAcc& a, int h0 = 0, int h1 = kNormChunks) {
  auto account = [&](const float (&x)[8]) {
#pragma unroll
    for (int v = 0; v < 8; ++v) a.add<TWO, TINY>(v, x[v], ka);
  };
  if constexpr (FORM == kNormRows) {
#pragma unroll 1
    for (int h = h0; h < h1; h += kNormGroup) {
      float x[kNormGroup][8];
#pragma unroll
      for (int q = 0; q < kNormGroup; ++q)
        norm_chunk_x<TG, kNormRows>(t, f0 + (h + q) * 512 + lane * 8, FULL ? f0 + kNormSegElems : f1, hp, x[q]);
#pragma unroll
      for (int q = 0; q < kNormGroup; ++q) account(x[q]);
    }
  } else if constexpr (FORM == kNormVec) {
    // in a partial segment, chunks past its end load its last chunk and count for nothing
#pragma unroll 1
    for (int h = h0; h < h1; h += kNormGroup) {
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
  } else {  // chunks past the segment's end count for nothing
#pragma unroll 1
    for (int h = h0; h < h1; h += kNormGroup) {
      float x[kNormGroup][8];
#pragma unroll
      for (int q = 0; q < kNormGroup; ++q)
        norm_chunk_x<TG, kNormAny>(t, f0 + (h + q) * 512 + lane * 8, FULL ? f0 + kNormSegElems : f1, hp, x[q]);
#pragma unroll
      for (int q = 0; q < kNormGroup; ++q) account(x[q]);
    }
  }
}

// Writes the records of one segment from the per-lane, per-chain sums of the workgroup's wavefronts
// (each took a part of the segment's chunks), and the chains' sums of squares.  Each wavefront sums its
// lanes' integer records (a lane's sum is an exact integer below 2^24, or 2^24 when it holds a tie or
// leaves the binade) and caps the total at 2^24; wavefront 0 adds the four totals in order, caps again
// and writes the records.  xacc and xhs are LDS of the workgroup; every thread of it calls this.
__device__ __forceinline__ void norm_write_records(const DevTensor& t, int64_t seg, int Ea, bool two, int lane,
                                                   int wid, const NormAcc& a, uint32_t (*xacc)[16], float (*xhs)[8]) {
  uint32_t acc[16];
  float hs[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    acc[v] = norm_lane_value(a.sa[v], a.tie_a(v, lane), Ea);
    acc[8 + v] = two ? norm_lane_value(a.sb[v], a.tie_b(v, lane), Ea + 1) : 0u;
    hs[v] = a.hs[v];
  }
  norm_lane_sums<8>(hs, lane);    // lane 8c: chain c
  norm_lane_sums<16>(acc, lane);  // lane 4c: chain c under Ea; lane 32 + 4c: under Ea + 1
  if ((lane & 7) == 0) xhs[wid][lane >> 3] = hs[0];
  if ((lane & 3) == 0) xacc[wid][lane >> 2] = min(acc[0], kNormFull);
  __syncthreads();
  if (wid == 0) {
    const int64_t nseg = t.nseg;
    const int c = lane & 7;
    if (lane < 16) {
      uint32_t sum = 0;
#pragma unroll
      for (int k = 0; k < kThreads / kWave; ++k) sum += xacc[k][lane];
      sum = min(sum, kNormFull);
      if (lane < 8) {
        t.nrec[c * nseg + seg] = uint32_t(Ea + 256) | (two ? kRecTwo : 0u);
        t.nrec[(8 + c) * nseg + seg] = sum;
      } else {
        t.nrec[(16 + c) * nseg + seg] = two ? sum : kNormFull;
      }
    }
    if (lane < 8) {
      float h = xhs[0][lane];
#pragma unroll
      for (int k = 1; k < kThreads / kWave; ++k) h += xhs[k][lane];
      t.nsum[lane * nseg + seg] = h;
    }
  }
  __syncthreads();  // xacc and xhs are written again by the next segment
}

// Candidate binades of a chain whose estimated value is est: Ea, and whether Ea + 1 is one too.
__device__ __forceinline__ void norm_candidates(float est, int& Ea, bool& two) {
  Ea = norm_est_binade(est * 0.875f);
  two = norm_est_binade(est * 1.015625f) > Ea;
}

constexpr int kNormRunSegs = 64;       // segments per work item of k_norm_seg2d (at most; 16 for small tensors)
constexpr int kNormLdsCols = 16384;    // column factors k_norm_seg2d stages in LDS (64 KB; rows of whole chunks
                                       // up to this wide, other rows 8 less)
constexpr int kNormSegLanes = 16;      // lanes per segment in k_norm_seg2d (narrowest rows: 8 * this)
constexpr int kNormSegAhead = 8;       // chunks per lane in flight there

// The per-lane, per-chain sums of one whole segment per group of G lanes (lane i = lane % G of the
// group takes the 8-element chunks at f0 + 8 * G * q + 8 * i) of a matrix (prefix 1) whose column
// factors are staged in LDS (cl), rows at least 8 * G wide, gradient 16-byte aligned, 32-bit flat
// indices.  A chunk's row and column follow from the previous chunk's by one wrap, as the rows are at
// least 8 * G wide.  ROWS: rows that are not whole chunks; a chunk may end in the next row, whose
// column factors continue in cl past C (the staging repeats the first 8 there) and whose row factor
// the elements from C - col on take (a select per element: a branch around it would double the
// unrolled loop, which then no longer unrolls).  The schedule is fixed by hand, a step per chunk: the column factors
// of the next chunk are read from LDS, this chunk is accounted, and the gradient and row factor of
// the chunk kNormSegAhead on are loaded into the registers this one frees.  Scheduling barriers keep
// the compiler from hoisting the loads further, and NormAcc::pin keeps each chunk's roundings in its
// step (either would cost registers, not time).
template <typename TG, int G, bool TWO, bool TINY, bool ROWS>
__device__ __forceinline__ void norm_seg_lds(const DevTensor& t, const float* cl, uint32_t f0, int ka, int li,
                                             NormAccM& a) {
  using GS = typename TG::storage;
  constexpr int Q = kNormSegElems / (8 * G), D = kNormSegAhead, NW = int(sizeof(GS)) * 2;
  static_assert(Q >= D, "segment chunks");
  const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g));
  const CAME8_GLOBAL float* __restrict__ rf = gbl(t.rfac);
  const uint32_t C = uint32_t(t.C), rlast = uint32_t(t.R) - 1u;
  uint32_t f = f0 + uint32_t(li * 8);
  uint32_t row = udiv_magic(f, t.mC, t.sC);
  uint32_t col = f - row * C;
  uint32_t gw[D][NW];  // 16 or 32 bytes of gradient per chunk
  float r[D], r1[ROWS ? D : 1];
  uint32_t cc[D];
  auto issue = [&](int s) __attribute__((always_inline)) {
    cc[s] = col;
    r[s] = rf[row];
    if constexpr (ROWS) r1[s] = rf[min(row + 1u, rlast)];  // the next row's, for a chunk that ends there
    if constexpr (sizeof(GS) == 2) {
      const u32x4 v = ld_nt((const CAME8_GLOBAL u32x4*)(g + f));
      gw[s][0] = v.x; gw[s][1] = v.y; gw[s][2] = v.z; gw[s][3] = v.w;
    } else {
      const u32x4 b0 = *(const CAME8_GLOBAL u32x4*)(g + f);  // two per lane: no hint
      const u32x4 b1 = *(const CAME8_GLOBAL u32x4*)(g + f + 4);
      gw[s][0] = b0.x; gw[s][1] = b0.y; gw[s][2] = b0.z; gw[s][3] = b0.w;
      gw[s][4] = b1.x; gw[s][5] = b1.y; gw[s][6] = b1.z; gw[s][7] = b1.w;
    }
    f += 8 * G;
    col += 8 * G;
    const bool wrap = col >= C;
    col = wrap ? col - C : col;
    row += wrap ? 1u : 0u;
  };
  // the column factors of a chunk at column col (ROWS: 4-byte aligned, read in pairs)
  auto read_c = [&](uint32_t col, float (&cv)[8]) __attribute__((always_inline)) {
    if constexpr (ROWS) {
#pragma unroll
      for (int v = 0; v < 8; ++v) cv[v] = cl[col + v];
    } else {
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(cl + col);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(cl + col + 4);
      cv[0] = c0.x; cv[1] = c0.y; cv[2] = c0.z; cv[3] = c0.w;
      cv[4] = c1.x; cv[5] = c1.y; cv[6] = c1.z; cv[7] = c1.w;
    }
  };
#pragma unroll
  for (int q = 0; q < D; ++q) issue(q);
  float cn[8];
  read_c(cc[0], cn);
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    __builtin_amdgcn_sched_barrier(0);
    const int s = q % D;
    float cv[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) cv[v] = cn[v];
    if (q + 1 < Q) read_c(cc[(q + 1) % D], cn);
    if constexpr (ROWS) {
      const uint32_t b = C - cc[s];  // the chunk's elements in its first row
#pragma unroll
      for (int v = 0; v < 8; ++v)
        a.add<TWO, TINY>(v, ((uint32_t(v) < b ? r[s] : r1[s]) * cv[v]) * TG::elem(gw[s], v), ka);
      a.template pin<TWO>();
    } else {
#pragma unroll
      for (int v = 0; v < 8; ++v) a.add<TWO, TINY>(v, (r[s] * cv[v]) * TG::elem(gw[s], v), ka);
      a.template pin<TWO>();
    }
    if (q + D < Q) issue(s);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Writes the records of the segment of each active group of G lanes (li = lane % G) from the lanes'
// per-chain sums, and the chains' sums of squares.  Ea: the group's binade; two: sums under Ea + 1
// were formed (uniform over the wavefront).
template <int G>
__device__ __forceinline__ void norm_write_records_g(const DevTensor& t, int64_t seg, int Ea, bool two, bool act,
                                                     int lane, const NormAccM& a) {
  const int li = lane & (G - 1);
  uint32_t acc[16];
  float hs[8];
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    acc[v] = norm_lane_value(a.sa[v], a.tie_a(v, lane), Ea);
    acc[8 + v] = two ? norm_lane_value(a.sb[v], a.tie_b(v, lane), Ea + 1) : 0u;
    hs[v] = a.hs[v];
  }
  const int64_t nseg = t.nseg;
  uint32_t* __restrict__ W0 = t.nrec;
  uint32_t* __restrict__ WA = t.nrec + 8 * nseg;
  uint32_t* __restrict__ WB = t.nrec + 16 * nseg;
  // value index i / (G / NV) (NV < G) or i * NV / G + k (NV >= G) after norm_group_sums
  norm_group_sums<G, 8>(hs, lane);
  constexpr int H8 = G > 8 ? G / 8 : 1, K8 = G < 8 ? 8 / G : 1;
#pragma unroll
  for (int k = 0; k < K8; ++k) {
    const int c = G >= 8 ? li / H8 : li * K8 + k;
    if (act && li % H8 == 0) t.nsum[c * nseg + seg] = hs[k];
  }
  if (two) {
    norm_group_sums<G, 16>(acc, lane);
    constexpr int H16 = G > 16 ? G / 16 : 1, K16 = G < 16 ? 16 / G : 1;
#pragma unroll
    for (int k = 0; k < K16; ++k) {
      const int i = G >= 16 ? li / H16 : li * K16 + k;  // i < 8: chain i under Ea; else chain i - 8 under Ea + 1
      if (act && li % H16 == 0) {
        const uint32_t sum = min(acc[k], kNormFull);
        if (i < 8) {
          W0[i * nseg + seg] = uint32_t(Ea + 256) | kRecTwo;
          WA[i * nseg + seg] = sum;
        } else {
          WB[(i - 8) * nseg + seg] = sum;
        }
      }
    }
  } else {
    norm_group_sums<G, 8>(acc, lane);
#pragma unroll
    for (int k = 0; k < K8; ++k) {
      const int c = G >= 8 ? li / H8 : li * K8 + k;
      if (act && li % H8 == 0) {
        W0[c * nseg + seg] = uint32_t(Ea + 256);
        WA[c * nseg + seg] = min(acc[k], kNormFull);
        WB[c * nseg + seg] = kNormFull;
      }
    }
  }
}

// The segments of one wavefront in a run of k_norm_seg2d: segments k0 + sub for k0 = wid * SPW,
// wid * SPW + 4 * SPW, ... below nrun, sub = lane / G.  TWO and TINY hold for all of them.
template <typename TG, int G, bool TWO, bool TINY, bool ROWS>
__device__ __forceinline__ void norm_seg2d_wave(const DevTensor& t, const float* cl, int64_t run0, int64_t nrun,
                                                float e0, float e1, int wid, int lane) {
  constexpr int SPW = kWave / G;
  const int li = lane & (G - 1), sub = lane / G;
#pragma unroll 1
  for (int64_t k0 = int64_t(wid) * SPW; k0 < nrun; k0 += (kThreads / kWave) * SPW) {
    // a group past the run's end takes its last segment again and writes nothing
    const bool act = k0 + sub < nrun;
    const int64_t k = act ? k0 + sub : nrun - 1;
    const int64_t seg = run0 + k;
    int Ea;
    bool two;
    norm_candidates(e0 + (e1 - e0) * (float(k) / float(nrun)), Ea, two);
    NormAccM a;
    a.clear();
    wait_vm_all();  // the previous records' stores: the chunk loads' waits then count only loads
    norm_seg_lds<TG, G, TWO, TINY, ROWS>(t, cl, uint32_t(seg * kNormSegElems), 23 - Ea, li, a);
    norm_write_records_g<G>(t, seg, Ea, TWO, act, lane, a);
  }
}

// Records of the whole segments [0, nseg0) of 2-D factored tensors whose rows are at least
// 8 * kNormSegLanes and at most kNormLdsCols wide, gradient 16-byte aligned, with 32-bit flat indices
// (the host checks); FORM kNormVec when the rows hold whole 8-element chunks, else kNormRows.  The last,
// partial segment is k_norm_seg's.  A work item is a run of nrun (16 to kNormRunSegs)
// segments: the workgroup stages the matrix's column factors in LDS once, and each wavefront takes
// kWave / kNormSegLanes consecutive segments at a time, a group of kNormSegLanes lanes per segment.
// A wavefront forms the sums under Ea + 1 for all its segments of the run when one of them needs them
// (a record with both sums is never wrong), and the subnormal rule when one of them is in that binade;
// the choice is made once per run, so that no code is shared between the forms' segment loops (the
// compiler would hoist a shared start, and the registers it holds, above the branch).
template <typename TG, int FORM>
__global__ __launch_bounds__(kThreads) void k_norm_seg2d(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  static_assert(FORM == kNormVec || FORM == kNormRows, "k_norm_seg2d forms");
  constexpr bool ROWS = FORM == kNormRows;
  constexpr int G = kNormSegLanes, SPW = kWave / G;  // lanes per segment, segments per wavefront
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
      if constexpr (ROWS) {  // C + 8 factors: the row's, then its first 8 again (for chunks that wrap)
        for (int64_t j = tid; j < t.C + 8; j += kThreads) cl[j] = gbl(t.cfac)[j < t.C ? j : j - t.C];
      } else {
        for (int64_t j = tid * 4; j < t.C; j += kThreads * 4)
          *reinterpret_cast<f32x4*>(cl + j) = *reinterpret_cast<const CAME8_GLOBAL f32x4*>(gbl(t.cfac) + j);
      }
      __syncthreads();
      staged = ti;
    }
    const int64_t run0 = (w - wstart[slot]) * t.nrun;
    const int64_t nrun = min(t.nrun, t.nseg0 - run0);
    const int64_t main = t.N - (t.N & 7);
    // the estimate at both ends of the run, linear in between (a chain holds about 1/8 of it)
    const float e0 = uniform_f32(norm_est_at(t, run0 * kNormSegElems)) * 0.125f;
    const float e1 = uniform_f32(norm_est_at(t, min((run0 + nrun) * kNormSegElems, main))) * 0.125f;
    bool any_two = false, any_tiny = false;
    for (int64_t k0 = int64_t(wid) * SPW; k0 < nrun; k0 += (kThreads / kWave) * SPW) {
      const int64_t k = min(k0 + lane / G, nrun - 1);
      int Ea;
      bool two;
      norm_candidates(e0 + (e1 - e0) * (float(k) / float(nrun)), Ea, two);
      any_two |= two;
      any_tiny |= Ea == -126;
    }
    if (__any(any_tiny)) norm_seg2d_wave<TG, G, true, true, ROWS>(t, cl, run0, nrun, e0, e1, wid, lane);
    else if (__any(any_two)) norm_seg2d_wave<TG, G, true, false, ROWS>(t, cl, run0, nrun, e0, e1, wid, lane);
    else norm_seg2d_wave<TG, G, false, false, ROWS>(t, cl, run0, nrun, e0, e1, wid, lane);
  }
}

// Records of the segments [nseg0, nseg).  One workgroup per segment: lane l of wavefront w takes the
// 8-element chunks at 512q + 8l of the segment for q in [w, w + 1) * kNormGroup (element v of a chunk
// belongs to chain v), and norm_write_records adds the wavefronts' sums.  FORM: how the chunks are
// loaded (norm_chunk_x).
template <typename TG, int FORM>
__global__ __launch_bounds__(kThreads, 4) void k_norm_seg(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                          const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  static_assert(kNormChunks == (kThreads / kWave) * kNormGroup, "a wavefront per kNormGroup chunk steps");
  __shared__ uint32_t xacc[kThreads / kWave][16];
  __shared__ float xhs[kThreads / kWave][8];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    // one segment per work item; wavefront wid takes its chunk steps [wid, wid + 1) * kNormGroup
    const int64_t seg = t.nseg0 + (w - wstart[slot]);
    const int h0 = wid * kNormGroup, h1 = h0 + kNormGroup;
    const int64_t main = t.N - (t.N & 7);
    const int64_t f0 = seg * kNormSegElems;
    const int64_t f1 = min(f0 + kNormSegElems, main);
    // candidate binades from the estimate at the segment's start (a chain holds about 1/8 of it)
    int Ea;
    bool two;
    norm_candidates(uniform_f32(norm_est_at(t, f0)) * 0.125f, Ea, two);
    const int ka = 23 - Ea;
    NormAcc a;
    a.clear();
    const bool full = f1 - f0 == kNormSegElems;
    if (Ea == -126) {
      norm_seg_sums<TG, FORM, true, true, false>(t, f0, f1, ka, lane, hp, a, h0, h1);
    } else if (two) {
      if (full) norm_seg_sums<TG, FORM, true, false, true>(t, f0, f1, ka, lane, hp, a, h0, h1);
      else norm_seg_sums<TG, FORM, true, false, false>(t, f0, f1, ka, lane, hp, a, h0, h1);
    } else {
      if (full) norm_seg_sums<TG, FORM, false, false, true>(t, f0, f1, ka, lane, hp, a, h0, h1);
      else norm_seg_sums<TG, FORM, false, false, false>(t, f0, f1, ka, lane, hp, a, h0, h1);
    }
    norm_write_records(t, seg, Ea, two, lane, wid, a, xacc, xhs);
  }
}

// The x of the 8 elements of the chunk at flat index f (a multiple of 8, in a whole segment) of a tensor
// that k_norm_seg2d takes, with the column factors staged in LDS (cl) as it stages them.  ROWS: the
// chunk may end in the next row (kNormRows).
template <typename TG, bool ROWS>
__device__ __forceinline__ void norm_chunk_lds(const DevTensor& t, const float* cl, uint32_t f, float (&x)[8]) {
  using GS = typename TG::storage;
  const uint32_t C = uint32_t(t.C);
  const uint32_t row = udiv_magic(f, t.mC, t.sC);
  const uint32_t col = f - row * C;
  float gv[8];
  load8<TG>(gbl(static_cast<const GS*>(t.g) + f), gv);
  const float r0 = gbl(t.rfac)[row];
  if constexpr (ROWS) {
    const float r1 = gbl(t.rfac)[min(row + 1u, uint32_t(t.R) - 1u)];
    const uint32_t b = C - col;  // the chunk's elements in its first row
#pragma unroll
    for (int v = 0; v < 8; ++v) x[v] = ((uint32_t(v) < b ? r0 : r1) * cl[col + v]) * gv[v];
  } else {
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(cl + col);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(cl + col + 4);
    const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int v = 0; v < 8; ++v) x[v] = (r0 * cv[v]) * gv[v];
  }
}

// Stages the column factors of a tensor that k_norm_seg2d takes in LDS (cl) as k_norm_seg2d does: ROWS,
// C + 8 factors (the row's, then its first 8 again).  Every thread of the workgroup calls it.
template <bool ROWS>
__device__ __forceinline__ void norm_stage_cols(const DevTensor& t, float* cl) {
  const int tid = threadIdx.x;
  if constexpr (ROWS) {
    for (int64_t j = tid; j < t.C + 8; j += kThreads) cl[j] = gbl(t.cfac)[j < t.C ? j : j - t.C];
  } else {
    for (int64_t j = tid * 4; j < t.C; j += kThreads * 4)
      *reinterpret_cast<f32x4*>(cl + j) = *reinterpret_cast<const CAME8_GLOBAL f32x4*>(gbl(t.cfac) + j);
  }
}

// ---------------------------------------------------------------------------
// each chain's own estimate, and records rebuilt under it
// ---------------------------------------------------------------------------
constexpr int kNormFixSegs = kThreads;  // segments per block of the chains' estimates and per work item of k_norm_fix
constexpr int64_t kNormFixDirect = 4;   // tensors of at most this many blocks: k_norm_fix adds the segments' sums itself

// Each chain's sum of squares over a block of kNormFixSegs segments (nbsum[c][block]), for the prefix
// k_norm_fix forms.  One work item per block; thread i takes segment i of the block.
template <int = 0>
__global__ __launch_bounds__(kThreads) void k_norm_bsum(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                        const int64_t* __restrict__ wstart, int ntens) {
  __shared__ float part[kThreads / kWave][8];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t nseg = t.nseg;
    const int64_t blk = w - wstart[slot];
    const int64_t seg = blk * kNormFixSegs + tid;
    float v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) v[c] = seg < nseg ? t.nsum[c * nseg + seg] : 0.0f;
    norm_lane_sums<8>(v, lane);  // lane 8c: chain c over the wavefront
    if ((lane & 7) == 0) part[wid][lane >> 3] = v[0];
    __syncthreads();
    if (tid < 8) t.nbsum[tid * t.nblk + blk] = (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]);
    __syncthreads();
  }
}

// The chains' estimates at the segments of one work item of k_norm_fix, into est[c][thread]: the sums of
// the blocks before it (k_norm_bsum) plus an exclusive scan of the item's own segment sums.
__device__ __forceinline__ void norm_item_estimates(const DevTensor& t, int64_t blk, const float (&v)[8],
                                                    float (&est)[8][kNormFixSegs], float (&part)[kThreads / kWave][8],
                                                    float (&base)[8]) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // the blocks before this one: thread i adds chain i % 8's blocks i / 8, i / 8 + 32, ... in that order,
  // four loads in flight at a time.  A tensor of at most kNormFixDirect blocks has no block sums
  // (k_norm_bsum skips it): its threads add the segments' sums themselves.
  {
    float acc = 0.0f;
    const int c = tid & 7;
    constexpr int kStep = kThreads / 8;
    const bool direct = t.nblk <= kNormFixDirect;  // uniform
    const float* __restrict__ nb = direct ? t.nsum + c * t.nseg : t.nbsum + c * t.nblk;
    const int64_t nend = direct ? blk * kNormFixSegs : blk;
    int64_t b = tid >> 3;
    for (; b + 3 * kStep < nend; b += 4 * kStep) {
      float y[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) y[u] = nb[b + u * kStep];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc += y[u];
    }
    for (; b < nend; b += kStep) acc += nb[b];
    est[c][tid >> 3] = acc;  // scratch: 32 partials per chain
  }
  __syncthreads();
  if (tid < 8) {
    float acc = 0.0f;
    for (int k = 0; k < kThreads / 8; ++k) acc += est[tid][k];
    base[tid] = acc;
  }
  __syncthreads();
  // this item's segments (v: this thread's segment's sums of squares, 0 past the tensor's segments):
  // an exclusive scan over the threads, per chain
  float incl[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) incl[c] = v[c];
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float y = __shfl_up(incl[c], o, kWave);
      incl[c] += lane >= o ? y : 0.0f;
    }
  }
  if (lane == kWave - 1) {
#pragma unroll
    for (int c = 0; c < 8; ++c) part[wid][c] = incl[c];
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    float off = base[c];
    for (int k = 0; k < kThreads / kWave; ++k) off += k < wid ? part[k][c] : 0.0f;
    est[c][tid] = off + (incl[c] - v[c]);
  }
  __syncthreads();
}


// Writes the records of the chains in mask from a rebuild under a binade pair per chain (Ea[c], Ea[c] + 1).
__device__ __forceinline__ void norm_write_records_pc(const DevTensor& t, int64_t seg, const int (&Ea)[8],
                                                      uint32_t mask, int lane, const NormAcc& a) {
  uint32_t acc[16];
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    acc[v] = norm_lane_value(a.sa[v], a.tie_a(v, lane), Ea[v]);
    acc[8 + v] = norm_lane_value(a.sb[v], a.tie_b(v, lane), Ea[v] + 1);
  }
  norm_lane_sums<16>(acc, lane);  // lane 4c: chain c under Ea[c]; lane 32 + 4c: under Ea[c] + 1
  const int c = (lane >> 2) & 7;
  int Ec = Ea[0];
#pragma unroll
  for (int v = 1; v < 8; ++v) Ec = c == v ? Ea[v] : Ec;
  if ((lane & 3) == 0 && ((mask >> c) & 1u)) {
    const int64_t nseg = t.nseg;
    const uint32_t sum = min(acc[0], kNormFull);
    if (lane < 32) {
      t.nrec[c * nseg + seg] = uint32_t(Ec + 256) | kRecTwo;
      t.nrec[(8 + c) * nseg + seg] = sum;
    } else {
      t.nrec[(16 + c) * nseg + seg] = sum;
    }
  }
}

// Records rebuilt under each chain's own estimate.  A work item is kNormFixSegs consecutive segments
// of one tensor, one per thread: the chains' estimates at each segment (norm_item_estimates, taken as
// within [-2%, +0.5%] of the chain) are checked against the segment's eight records, and the segments
// where a record's binades do not cover a chain's are listed in LDS and shared out to the wavefronts,
// which rebuild them a segment at a time under each chain's own candidates Ea and Ea + 1 (both sums
// always).  FORM as for k_norm_seg.  The whole segments of a tensor that k_norm_seg2d takes (nseg0 > 0)
// read their column factors from LDS, staged once per tensor as k_norm_seg2d stages them.
template <typename TG, int FORM>
__global__ __launch_bounds__(kThreads) void k_norm_fix(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                       const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  extern __shared__ float cl[];            // column factors (launches with tensors that k_norm_seg2d takes)
  __shared__ uint32_t list[kNormFixSegs];  // (thread << 8) | mask of the chains to rebuild
  __shared__ int nlist;
  __shared__ float est_l[8][kNormFixSegs];
  __shared__ float part[kThreads / kWave][8];
  __shared__ float base_l[8];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  int32_t staged = -1;
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const int32_t ti = tids[slot];
    const DevTensor& t = T[ti];
    const int64_t nseg = t.nseg;
    const int64_t blk = w - wstart[slot];
    const int64_t base = blk * kNormFixSegs;
    const int64_t seg = base + tid;
    if (tid == 0) nlist = 0;
    // this thread's segment's sums of squares and record words, loaded before the estimates' sums
    float v[8];
    uint32_t w0s[8];
    {
      const int64_t sc = seg < nseg ? seg : nseg - 1;  // nseg >= 1 for a tensor in the list
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        v[c] = t.nsum[c * nseg + sc];
        w0s[c] = t.nrec[c * nseg + sc];
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) v[c] = seg < nseg ? v[c] : 0.0f;
    }
    norm_item_estimates(t, blk, v, est_l, part, base_l);  // synchronises the workgroup
    uint32_t need = 0;
    if (seg < nseg) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float est = est_l[c][tid];
        const uint32_t w0 = w0s[c];
        const int Ea = int(w0 & 511u) - 256;
        const bool two = (w0 & kRecTwo) != 0;
        const int lo = norm_est_binade(est * 0.98f), hi = norm_est_binade(est * 1.005f);
        const bool ok = (lo == Ea || (two && lo == Ea + 1)) && (hi == Ea || (two && hi == Ea + 1));
        need |= ok ? 0u : (1u << c);
      }
    }
    if (need != 0) list[atomicAdd(&nlist, 1)] = (uint32_t(tid) << 8) | need;
    __syncthreads();
    const int n = nlist;
    const int64_t main = t.N - (t.N & 7);
    constexpr bool kLds = FORM != kNormAny;
    if (kLds && n > 0 && t.nseg0 > 0 && ti != staged) {  // uniform over the workgroup
      norm_stage_cols<FORM == kNormRows>(t, cl);
      __syncthreads();
      staged = ti;
    }
    for (int k = wid; k < n; k += kThreads / kWave) {  // uniform over the wavefront
      const uint32_t e = list[k];
      const int64_t sf = base + (e >> 8);
      int Ea[8], ka[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        bool two;
        norm_candidates(est_l[c][e >> 8], Ea[c], two);
        ka[c] = 23 - Ea[c];
      }
      NormAcc a;
      a.clear();
      const int64_t f0 = sf * kNormSegElems, f1 = min(f0 + kNormSegElems, main);
      if (kLds && sf < t.nseg0) {  // uniform over the wavefront
#pragma unroll 1
        for (int h = 0; h < kNormChunks; h += kNormGroup) {
          float x[kNormGroup][8];
#pragma unroll
          for (int q = 0; q < kNormGroup; ++q)
            norm_chunk_lds<TG, FORM == kNormRows>(t, cl, uint32_t(f0 + (h + q) * 512 + lane * 8), x[q]);
#pragma unroll
          for (int q = 0; q < kNormGroup; ++q)
#pragma unroll
            for (int v = 0; v < 8; ++v) a.add_both(v, x[q][v], ka[v], Ea[v] == -126);
        }
      } else {
#pragma unroll 1
        for (int h = 0; h < kNormChunks; h += kNormGroup) {
          float x[kNormGroup][8];
#pragma unroll
          for (int q = 0; q < kNormGroup; ++q) norm_chunk_x<TG, FORM>(t, f0 + (h + q) * 512 + lane * 8, f1, hp, x[q]);
#pragma unroll
          for (int q = 0; q < kNormGroup; ++q)
#pragma unroll
            for (int v = 0; v < 8; ++v) a.add_both(v, x[q][v], ka[v], Ea[v] == -126);
        }
      }
      norm_write_records_pc(t, sf, Ea, e & 255u, lane, a);
    }
    __syncthreads();  // the list is reused by the next item
  }
}

// ---------------------------------------------------------------------------
// walk
// ---------------------------------------------------------------------------
constexpr uint32_t kNormSat = 1u << 25;  // saturating integer sums: anything >= 2^24 leaves the binade
__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b) { return min(a + b, kNormSat); }

// Cross-lane steps of the walk, all 64 lanes active.  DPP: row_shr:n (0x110 + n; lanes shifted in from
// before their row's start read 0), row_bcast:15 (0x142) and row_bcast:31 (0x143) with row masks
// (rows outside them add 0), wave_shr:1 (0x138).
template <int CTRL, int ROWS, bool BOUND>
__device__ __forceinline__ uint32_t norm_dpp(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, ROWS, 0xf, BOUND));
}
// inclusive scan of saturating sums over the wavefront, in lane order
__device__ __forceinline__ uint32_t norm_wave_scan(uint32_t v) {
  v = sat_add(v, norm_dpp<0x111, 0xf, true>(v));
  v = sat_add(v, norm_dpp<0x112, 0xf, true>(v));
  v = sat_add(v, norm_dpp<0x114, 0xf, true>(v));
  v = sat_add(v, norm_dpp<0x118, 0xf, true>(v));  // each row of 16 scanned
  v = sat_add(v, norm_dpp<0x142, 0xa, false>(v));  // rows 1 and 3 add the totals of rows 0 and 2
  v = sat_add(v, norm_dpp<0x143, 0xc, false>(v));  // rows 2 and 3 add the total of rows 0 and 1
  return v;
}
// the inclusive value of the previous lane (0 for lane 0)
__device__ __forceinline__ uint32_t norm_wave_prev(uint32_t incl) { return norm_dpp<0x138, 0xf, true>(incl); }
// lane `src`'s value (src uniform)
__device__ __forceinline__ uint32_t norm_lane(uint32_t v, int src) { return uint32_t(__builtin_amdgcn_readlane(int(v), src)); }
__device__ __forceinline__ float norm_lane(float v, int src) { return __uint_as_float(norm_lane(__float_as_uint(v), src)); }

// Replays chain c over segment seg from s, equal to the reference's serial fmaf loop bit for bit (one
// wavefront).  Lane l holds the chain's elements 8l .. 8l + 7 of the segment.  A round takes every
// remaining element's increment under s's binade, a saturating prefix sum of them in element order,
// and the first element that is special or whose prefix takes the chain out of the binade; the
// elements before it are one integer add, that element is one fmaf, and the next round starts after
// it.  A finite chain only grows, so the rounds are the segment's binade crossings and special
// elements, plus one.  An infinite chain changes only at a NaN element; a NaN chain not at all.
template <typename TG>
__device__ float norm_replay(const DevTensor& t, int c, int64_t seg, float s, const Hp& hp) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t main = t.N - (t.N & 7);
  const int64_t f0 = seg * kNormSegElems;
  const int cnt = int(min(int64_t(kNormChainSeg), (main - f0) / 8));  // at least 1
  float x[8], h[8];
  {
    // an element past the segment's end reads the segment's first element of the chain and counts
    // for nothing
    int64_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = f0 + 8 * int64_t(lane * 8 + j < cnt ? lane * 8 + j : 0) + c;
    norm_x_any8<TG>(t, e, hp, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = lane * 8 + j < cnt ? x[j] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = x[j] * x[j];
  if (s == 0.0f) {
    // A chain's first segment crosses a binade every few elements, and its early increments keep many
    // fractional bits, so ties are common too: instead of a round per crossing or tie, its elements are
    // applied one by one (the reference's own loop), each broadcast from its lane.  Elements past the
    // segment's end are 0, and fmaf(0, 0, s) is s, so the loop needs no branch.
#pragma unroll
    for (int k = 0; k < kNormChainSeg; ++k) {
      const float xk = norm_lane(x[k & 7], k >> 3);
      s = fmaf(xk, xk, s);
    }
    return s;
  }
  int pos = 0;  // the elements before pos are applied
  while (pos < cnt) {  // uniform
    if (!(s <= 0x1.fffffep127f)) {
      if (s != s) break;
      uint32_t nanm = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int k = lane * 8 + j;
        nanm |= (k >= pos && k < cnt && x[j] != x[j]) ? (1u << j) : 0u;
      }
      const uint64_t bal = __ballot(nanm != 0);
      if (bal != 0) {
        const int fl = __builtin_ctzll(bal);
        const int jj = int(norm_lane(uint32_t(__builtin_ctz(nanm | 0x100u)), fl));
        float xe = x[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) xe = jj == j ? x[j] : xe;
        xe = norm_lane(xe, fl);
        s = fmaf(xe, xe, s);
      }
      break;
    }
    const int E = norm_binade(s);
    const uint32_t m = norm_mant(s, E);
    const uint32_t room = kNormFull - m;  // an increment prefix that reaches this leaves the binade
    const int kk = 23 - E;
    uint32_t incl[8], spm = 0, run = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = lane * 8 + j;
      const bool live = k >= pos && k < cnt;
      const float dh = ldexpf(h[j], kk);
      const float nf = rintf(dh);
      const bool special = fabsf(dh - nf) == 0.5f || (E == -126 && (nf != 0.0f || fabsf(x[j]) == 0x1p-75f));
      const uint32_t n = nf < 0x1p25f ? uint32_t(nf) : kNormSat;  // NaN and inf squares saturate
      run = sat_add(run, live ? n : 0u);
      incl[j] = run;
      spm |= (live && special) ? (1u << j) : 0u;
    }
    const uint32_t winc = norm_wave_scan(run);  // inclusive scan of the lanes' runs
    const uint32_t excl = norm_wave_prev(winc);
    uint32_t evm = spm;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = lane * 8 + j;
      evm |= (k >= pos && k < cnt && sat_add(excl, incl[j]) >= room) ? (1u << j) : 0u;
    }
    const uint64_t bal = __ballot(evm != 0);
    if (bal == 0) {
      s = norm_value(m + norm_lane(winc, kWave - 1), E);  // below room
      break;
    }
    const int fl = __builtin_ctzll(bal);
    const int j0 = __builtin_ctz(evm | 0x100u);  // this lane's first event (8: none)
    uint32_t before = excl;                      // the increments before that event, on lane fl
    float xe = x[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) {
      before = j0 == j ? excl + incl[j - 1] : before;
      xe = j0 == j ? x[j] : xe;
    }
    const int jj = int(norm_lane(uint32_t(j0), fl));
    before = norm_lane(before, fl);
    xe = norm_lane(xe, fl);
    s = fmaf(xe, xe, norm_value(m + before, E));
    pos = fl * 8 + jj + 1;
  }
  return s;
}

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

// One wavefront per (tensor, chain).  A batch loads the records of kWave * kNormWalkSegs segments, a
// run of kNormWalkSegs per lane.  Then, from the chain's position: every lane sums its records under
// the chain's binade, a scan over the lanes finds the first segment whose record does not cover the
// binade or takes the chain out of it, every segment before it is skipped with its integer sum, that
// segment is replayed, and the scan resumes after it with the records already loaded.
template <typename TG>
__global__ __launch_bounds__(kNormWalkThreads) void k_norm_walk(const DevTensor* __restrict__ T,
                                                                const int32_t* __restrict__ tids,
                                                                const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  const int lane = threadIdx.x;
  const int64_t total = wstart[ntens];
  // Workgroup w runs on XCD w % 8 (the dispatcher deals a launch's workgroups to the eight XCDs in
  // turn).  The items, eight per tensor (its chains), go to the XCDs in eight contiguous ranges, so
  // that a tensor's chains share one XCD's L2: they mostly replay the same segments at about the same
  // time, and each replay reads the cache lines that hold all eight chains' elements.
  const int64_t per = total % kXcds == 0 ? total / kXcds : 0;
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int64_t item = per > 0 ? (w % kXcds) * per + w / kXcds : w;
    const int slot = find_slot(wstart, ntens, item);
    const DevTensor& t = T[tids[slot]];
    const int c = int(item - wstart[slot]);
    const int64_t nseg = t.nseg;
    const CAME8_GLOBAL uint32_t* __restrict__ W0 = gbl(t.nrec + c * nseg);
    const CAME8_GLOBAL uint32_t* __restrict__ WA = gbl(t.nrec + (8 + c) * nseg);
    const CAME8_GLOBAL uint32_t* __restrict__ WB = gbl(t.nrec + (16 + c) * nseg);
    // the first segment is replayed from zero without reading its record (a tensor of one segment forms
    // none)
    float s = nseg > 0 ? norm_replay<TG>(t, c, 0, 0.0f, hp) : 0.0f;
    int64_t seg = 1;
    while (seg < nseg && s == s) {  // a NaN chain stays NaN
      // the batch starts at a multiple of kNormWalkSegs; its segments before seg count for nothing
      const int64_t bstart = seg & ~int64_t(kNormWalkSegs - 1);
      const int64_t base = bstart + int64_t(lane) * kNormWalkSegs;
      const int64_t bend = min(nseg, bstart + int64_t(kWave) * kNormWalkSegs);
      uint32_t r0[kNormWalkSegs], ra[kNormWalkSegs], rb[kNormWalkSegs];
      if (base + kNormWalkSegs <= nseg) {  // consecutive records of each array: 4-dword loads
#pragma unroll
        for (int q = 0; q < kNormWalkSegs / 4; ++q) {
          const u32x4u a0 = *reinterpret_cast<const CAME8_GLOBAL u32x4u*>(W0 + base + 4 * q);
          const u32x4u aa = *reinterpret_cast<const CAME8_GLOBAL u32x4u*>(WA + base + 4 * q);
          const u32x4u ab = *reinterpret_cast<const CAME8_GLOBAL u32x4u*>(WB + base + 4 * q);
          r0[4 * q] = a0.x; r0[4 * q + 1] = a0.y; r0[4 * q + 2] = a0.z; r0[4 * q + 3] = a0.w;
          ra[4 * q] = aa.x; ra[4 * q + 1] = aa.y; ra[4 * q + 2] = aa.z; ra[4 * q + 3] = aa.w;
          rb[4 * q] = ab.x; rb[4 * q + 1] = ab.y; rb[4 * q + 2] = ab.z; rb[4 * q + 3] = ab.w;
        }
      } else {  // the array's end: clamped loads (the records past it count for nothing)
#pragma unroll
        for (int j = 0; j < kNormWalkSegs; ++j) {
          const int64_t k = min(base + j, nseg - 1);
          r0[j] = W0[k];
          ra[j] = WA[k];
          rb[j] = WB[k];
        }
      }
      while (seg < bend && s == s) {  // the segments [seg, bend) of this batch
        const bool inf = !(s <= 0x1.fffffep127f);
        const int E = inf ? 128 : norm_binade(s);
        const uint32_t m = inf ? 0u : norm_mant(s, E);
        const uint32_t room = kNormFull - m;  // the chain leaves its binade once its increments reach this
        // this lane's run: the sum of its records from seg on, up to the first one that stops the chain
        uint32_t add[kNormWalkSegs], run = 0;
        bool stop = false;
#pragma unroll
        for (int j = 0; j < kNormWalkSegs; ++j) {
          add[j] = norm_rec_add(r0[j], ra[j], rb[j], E);
          if (base + j >= seg && base + j < bend && !stop) {
            if (add[j] >= kNormSat) stop = true;
            else run = sat_add(run, add[j]);
          }
        }
        // inclusive scan of the runs over the lanes (saturating sums, in lane order)
        const uint32_t incl = norm_wave_scan(run);
        const uint32_t excl = norm_wave_prev(incl);  // exact while the chain has not left its binade
        const uint32_t tot = norm_lane(incl, kWave - 1);
        // the first lane whose run is cut short or takes the chain out of its binade
        const uint64_t bal = __ballot(stop || sat_add(excl, run) >= room);
        if (bal == 0) {
          if (!inf) s = norm_value(m + tot, E);  // tot < room
          seg = bend;
          break;
        }
        const int first = __builtin_ctzll(bal);
        uint32_t acc = excl;
        int64_t k = max(base, seg);
#pragma unroll
        for (int j = 0; j < kNormWalkSegs; ++j) {
          if (k == base + j && k < bend && add[j] < kNormSat && acc + add[j] < room) {
            acc += add[j];
            k = base + j + 1;
          }
        }
        const uint32_t mm = m + norm_lane(acc, first);
        const int64_t ks = int64_t(norm_lane(uint32_t(k), first)) | (int64_t(norm_lane(uint32_t(uint64_t(k) >> 32), first)) << 32);
        s = norm_replay<TG>(t, c, ks, inf ? s : norm_value(mm, E), hp);
        seg = ks + 1;
      }
    }
    if (lane == 0) t.nchain[c] = s;
  }
}

// The eight accumulators added left to right, then the N % 8 tail elements in torch's order (a block
// of four rounded squares added one at a time when four or more remain, then the rest as fused
// multiply-adds), sqrt, and the clip divisor.  A thread per tensor.
template <typename TG>
__global__ __launch_bounds__(kThreads) void k_norm_final(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         int ntens, Hp hp) {
  const int k = blockIdx.x * kThreads + threadIdx.x;
  if (k >= ntens) return;
  const DevTensor& t = T[tids[k]];
  float b = t.nchain[0];
  for (int j = 1; j < 8; ++j) b = b + t.nchain[j];
  int64_t d = t.N - (t.N & 7);
  if (t.N - d >= 4) {
    for (const int64_t e = d + 4; d < e; ++d) {
      const float u = u_at<TG>(t, d, hp);
      const float uu = u * u;  // rounded on its own (the build does not contract)
      b = b + uu;
    }
  }
  for (; d < t.N; ++d) {
    const float u = u_at<TG>(t, d, hp);
    b = fmaf(u, u, b);
  }
  const float c = clip_from_norm(sqrtf(b), t.N, hp);
  t.clip[0] = c;
  t.clip[1] = rcp_for_div(c);
}

}  // namespace came8
