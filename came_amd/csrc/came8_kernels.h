// Kernels of the CAME 8-bit step (gfx950).  Included once, by came8.hip.
//
// One optimizer step over a list of tensors runs as a short chain of
// multi-tensor launches on one stream (every launch covers all tensors of its
// kind):
//
//   P1  band pass over G of every factored tensor: row sums of g^2+eps0 (whole
//       rows per workgroup, so the new row state R_i is known locally), column
//       partial sums of g^2+eps0 and of g^2/R_i per row band.
//   A   1-D tensors: sum of u^2 per 2048-element tile.
//   F1a per matrix: mean of the new row state (rm).
//   F1b row-state blocks: r_i = rsqrt(R_i/rm), uint8 requantisation of R;
//       column-state blocks: C_j = EMA(mean_i), clamp 1e-30, c_j = rsqrt(C_j),
//       uint8 requantisation, and the clip numerator  rm * c_j^2 * sum_i g^2/R_i.
//   CLIP per tensor: update-RMS clip divisor.
//   P2  band pass over G and the int8 momentum: u, m_new, residual
//       (u-m)^2+eps1; row sums -> residual row state, column partials.
//   F2a/F2b residual factors rr_i, cr_j and their uint8 requantisation.
//   P3  flat pass over whole quantisation blocks: u, m_new, step, weight decay,
//       parameter write, int8 requantisation of m.
//   B   1-D tensors: v, u/clip, m, parameter write, int8 + uint8 requantisation.
//
// The arithmetic of every element follows the reference's CPU path
// (came_pytorch/CAME8bitFull.py:1006-1075) operation for operation, with the
// same roundings (fused multiply-add where torch's CPU kernels fuse, IEEE
// division and square root, round-half-even).  Reductions use fixed
// combination orders, so results are identical from run to run.
#pragma once

#include <type_traits>

#include "came8_device.h"

namespace came8 {

// Per-tensor descriptor in device memory (built by the host plan).
struct alignas(128) DevTensor {  // each descriptor on whole cache lines
  void* p;
  const void* g;
  int8_t* mq;     // exp_avg codes [N]
  float* ma;      // exp_avg absmax [nbm]
  uint8_t* rq;    // factored: [2][P*R]; 1-D: exp_avg_sq codes [N]
  float* ra;      // factored: [2][nbr]; 1-D: [nbm]
  uint8_t* cq;    // [2][P*C]
  float* ca;      // [2][nbc]
  int64_t P, R, C, N;
  int64_t nbr, nbc, nbm;  // absmax blocks of one row state, one col state, exp_avg
  int64_t nbands;         // row bands per matrix
  int64_t rb;             // rows per band
  // scratch (workspace)
  float* Rn;      // new row state (fp32)           [P*R]
  float* rfac;    // rsqrt(R/rm)                     [P*R]
  float* RRn;     // new residual row state          [P*R]
  float* rrfac;   //                                 [P*R]
  float* Cn;      // new column state (clamped)      [P*C]
  float* cfac;    //                                 [P*C]
  float* CRn;     //                                 [P*C]
  float* crfac;   //                                 [P*C]
  float* partU;   // column partials of g^2+eps0     [P*nbands*C]
  float* partW;   // column partials of g^2/R_i      [P*nbands*C]
  float* partRes; // column partials of residual     [P*nbands*C]
  float* rsum;    // row states summed per band      [P*nbands]  (mean row state: their sum / R)
  float* rrsum;   // residual row states per band    [P*nbands]
  double* clip_part;  // clip numerator partials     [nclip]
  float* clip;        // clip divisor and rcp_for_div of it [2]
  int64_t nclip;
  // reference-order norm (the clip's update norm replayed as the reference's eight fp32 chains)
  int64_t nseg;       // chain segments of kNormSegElems flat elements over the first N - N % 8
  int64_t nseg0;      // leading whole segments of the LDS-staged kernel (0: every segment is the other's)
  int64_t nrun;       // segments per work item of the LDS-staged kernel
  int64_t nunit;      // estimate units: row bands of every matrix (factored), 2048-element tiles (1-D),
  int64_t ngrp;       //   or groups of ngrp single-band matrices / tiles (ngrp > 1 bounds nunit)
  float* nest;        // estimated sum of u^2 per unit, then its exclusive prefix [nunit + 1]
  uint32_t* nrec;     // per chain and segment: binade/flags, two integer sums [3][8][nseg]
  float* nsum;        // per chain and segment: fp32 sum of the rounded squares      [8][nseg]
  float* nbsum;       // their sums per block of 256 segments                        [8][nblk]
  int64_t nblk;
  float* nchain;      // the eight chain accumulators                           [8]
  uint64_t mC, mR;    // magic multipliers for n / C and n / R (n < 2^31)
  uint32_t sC, sR;    // and their shifts
  int32_t idx32;      // N < 2^31: flat indices fit the magic division
  int32_t rowal;      // the quantisation block size divides C (every row starts a block)
  int32_t p3_rb;      // band form of P3: rows per work item,
  int32_t p3_nseg;    // column segments per row,
  int64_t p3_nbands;  // row bands per matrix (0: the tensor uses the tile form)
  int32_t c8;         // C % 8 == 0: 8 consecutive elements never cross a row
  int32_t vec_ok;     // p, g, codes 16-byte aligned (flat passes may use vector access)
  int32_t factored;
  int32_t fp32st;     // fp32 states (CAMECUDA layout): mq -> float m, rq/ra -> float second-moment /
                      // residual rows (rq -> float v for 1-D), cq/ca -> float columns; ma unused
  // 8bit2d layout (reference CAME8bit2D): ma holds one absmax per 16x16 tile of m; rq/ra, cq/ca are
  // the second-moment row / column states and rrq/rra, rcq/rca the residual ones; t2col receives
  // each tile's residual sums per column [tr][C], t2row (scalar momentum pass only) per row [R][tc];
  // rrsum then holds one sum of residual row states per tile row
  int32_t mode2d;
  int32_t tr, tc;     // tile rows, tile columns
  uint8_t* rrq;
  float* rra;
  uint8_t* rcq;
  float* rca;
  float* t2row;
  float* t2col;
  int32_t v2d, v2dp;  // vector forms of the momentum pass / parameter write apply
  int32_t fp16u;      // this unfactored tensor takes the fp16-rounded update (CAME8_TENSOR_FP16_UPDATE)
  // CAME8_STATE_Q8_MATRIX with P > 1: quantisation blocks restart at every matrix (the reference's CUDA
  // N-D layout); blocks per matrix of the momentum (R*C elements), of a row state (R) and of a column
  // state (C).  nbm, nbr, nbc are then P times these.
  int32_t pm;
  int64_t pmb_m, pmb_r, pmb_c;
  // default clip mode: per row band the sum of e_i / R_i (e_i the row's sum of g^2), which the
  // clip-norm estimates weigh with the band's column partials of g^2 [P*nbands]
  float* esum;
};

// fp32-state views of the state pointers
__device__ __forceinline__ float* st_m(const DevTensor& t) { return reinterpret_cast<float*>(t.mq); }
__device__ __forceinline__ float* st_sq_row(const DevTensor& t) { return reinterpret_cast<float*>(t.rq); }
__device__ __forceinline__ float* st_sq_col(const DevTensor& t) { return reinterpret_cast<float*>(t.cq); }

// Hyper-parameters as the fp32 constants the reference's CPU ops use.
struct Hp {
  float b1, a1, b2, a2, b3, a3;  // beta, (1 - beta) computed in double then rounded
  float eps0, eps1;
  float awd;       // -wd*lr rounded to fp32 (fp32 params)
  float awd_bf16;  // the same rounded to bf16 (torch's reduced-precision add_ alpha)
  float awd_f16;
  float alr;       // -lr
  float thr;       // clip_threshold
  int32_t wd;      // weight_decay != 0
  int32_t B;       // quantisation block size
  int32_t log2B;   // log2(B) if B is a power of two, else -1
  uint32_t sB;     // magic division by B (indices < 2^31, which the host guarantees for
  uint64_t mB;     // block sizes that are not powers of two)
  float a1f, a2f, a3f;  // 8bit2d: 1 - beta computed in float
  float wdfac;          // 8bit2d: multiplicative weight decay 1 - lr * wd, computed in float
  const void* zeros;    // kZeroBytes of zeros in the workspace (reads that must count for nothing)
  int32_t fp16u;        // 1-D tensors: the momentum takes the update rounded to fp16 (CAME8_FLAG_FP16_UPDATE)
  int32_t noW;          // default clip mode: the band passes wrote no column sums of g^2/R_i (partW)
};
constexpr int kZeroBytes = 32768;  // >= TPB*V*K elements of any band-pass shape

__device__ __forceinline__ int64_t blk_of(int64_t e, const Hp& hp) {
  return hp.log2B >= 0 ? (e >> hp.log2B) : int64_t(udiv_magic(uint32_t(e), hp.mB, hp.sB));
}
// the same without a branch: (e * mB) >> sB is e >> log2(B) for a power of two (mB = 1) and the
// magic division otherwise (e < 2^31 then, so the product stays below 2^64)
__device__ __forceinline__ int64_t blk_of_nb(int64_t e, const Hp& hp) {
  return int64_t((uint64_t(e) * hp.mB) >> hp.sB);
}

// Block of row state `row` (0 <= row < P*R), of column state i (0 <= i < P*C) and of momentum element e:
// flat blocks, or per-matrix blocks (t.pm) that restart at every matrix's first row / column / element.
// Per-matrix tensors hold fewer than 2^31 elements (the host checks), so the matrix of an index comes from
// the 32-bit magic divisions by R and C.
__device__ __forceinline__ int64_t rblk(const DevTensor& t, int64_t row, const Hp& hp) {
  if (!t.pm) return blk_of(row, hp);
  const int64_t b = udiv_magic(uint32_t(row), t.mR, t.sR);
  return b * t.pmb_r + blk_of(row - b * t.R, hp);
}
__device__ __forceinline__ int64_t cblk(const DevTensor& t, int64_t i, const Hp& hp) {
  if (!t.pm) return blk_of(i, hp);
  const int64_t b = udiv_magic(uint32_t(i), t.mC, t.sC);
  return b * t.pmb_c + blk_of(i - b * t.C, hp);
}
// matrix of momentum element e (per-matrix tensors): floor(floor(e / C) / R)
__device__ __forceinline__ int64_t pm_matrix(const DevTensor& t, int64_t e) {
  return udiv_magic(udiv_magic(uint32_t(e), t.mC, t.sC), t.mR, t.sR);
}
__device__ __forceinline__ int64_t mblk(const DevTensor& t, int64_t e, const Hp& hp) {
  if (!t.pm) return blk_of(e, hp);
  const int64_t b = pm_matrix(t, e);
  return b * t.pmb_m + blk_of(e - b * (t.R * t.C), hp);
}
// wstart has n+1 entries, wstart[0] = 0; returns k with wstart[k] <= w < wstart[k+1]
__device__ __forceinline__ int find_slot(const int64_t* __restrict__ wstart, int n, int64_t w) {
  int lo = 0, hi = n;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (wstart[mid] <= w) lo = mid; else hi = mid;
  }
  return lo;
}

template <typename TP>
__device__ __forceinline__ float wd_alpha(const Hp& hp);
template <> __device__ __forceinline__ float wd_alpha<F32>(const Hp& hp) { return hp.awd; }
template <> __device__ __forceinline__ float wd_alpha<BF16>(const Hp& hp) { return hp.awd_bf16; }
template <> __device__ __forceinline__ float wd_alpha<F16>(const Hp& hp) { return hp.awd_f16; }

// p <- p + (-wd*lr)*p (if wd != 0), rounded to the param type; then p + (-lr)*step, rounded again
// (reference CAME8bitFull.py:1053-1056).
template <typename TP>
__device__ __forceinline__ float param_update(float p, float step, const Hp& hp) {
  if (hp.wd) p = TP::load(TP::store(fmaf(p, wd_alpha<TP>(hp), p)));
  return fmaf(step, hp.alr, p);
}

constexpr int kTile = 2048;  // elements per workgroup tile in the flat passes (8 per thread)
constexpr int kMaxBandRows = 256;

// ===========================================================================
// P1 / P2: band passes over whole rows
// ===========================================================================
// A workgroup of TPB threads owns a band of consecutive rows of one matrix.
// Thread t owns column chunks t, t+TPB, ..., t+TPB*(K-1) of V elements each
// (V = 16 bytes of the gradient type when rows are 16-byte aligned, else 1).
// When C <= TPB*V*K a row is read once: it stays in registers, in its storage
// type, between the row reduction and the column accumulation, and the next
// stage of rows is already loading while the current one is reduced (two
// register buffers).  Wider rows are handled in column segments after a first
// sweep that forms the row sums.

// V consecutive gradient elements, kept as raw 32-bit words until used (V = 1, or 16 bytes; U: the
// 16 bytes need only the element's alignment).
template <typename TG, int V, bool U = false>
struct Chunk {
  static constexpr int NWD = V == 1 ? 1 : 4;
  uint32_t w[NWD];
  __device__ __forceinline__ void load(const CAME8_GLOBAL typename TG::storage* __restrict__ p) {
    if constexpr (V == 1) {
      if constexpr (sizeof(typename TG::storage) == 4) w[0] = __float_as_uint(p[0]);
      else w[0] = uint32_t(p[0]);
    } else {
      static_assert(V * sizeof(typename TG::storage) == 16, "vector chunk must be 16 bytes");
      using VT = typename std::conditional<U, u32x4u, u32x4>::type;
      const VT r = ld_nt((const CAME8_GLOBAL VT*)p);
      w[0] = r.x; w[1] = r.y; w[2] = r.z; w[3] = r.w;
    }
  }
  // elements v < skip read as zero: word i keeps the halves (or the word) at or past `skip`
  __device__ __forceinline__ void mask(const uint32_t (&m)[NWD]) {
#pragma unroll
    for (int i = 0; i < NWD; ++i) w[i] &= m[i];
  }
  __device__ __forceinline__ float operator[](int v) const { return TG::elem(w, v); }
};

// V consecutive int8 codes (V-byte aligned for V = 4, 8, unless U), as raw words.
template <int V, bool U = false>
struct CodeChunk {
  static constexpr int NWD = (V + 3) / 4;
  uint32_t w[NWD];
  __device__ __forceinline__ void load(const CAME8_GLOBAL int8_t* __restrict__ p) {
    if constexpr (V == 8) {
      using VT = typename std::conditional<U, u32x2u, u32x2>::type;
      const VT r = ld_nt((const CAME8_GLOBAL VT*)p);
      w[0] = r.x; w[1] = r.y;
    } else if constexpr (V == 4) {
      using WT = typename std::conditional<U, u32u, uint32_t>::type;
      w[0] = ld_nt((const CAME8_GLOBAL WT*)p);
    } else {
#pragma unroll
      for (int i = 0; i < NWD; ++i) w[i] = 0;
#pragma unroll
      for (int v = 0; v < V; ++v) w[v >> 2] |= uint32_t(uint8_t(p[v])) << (8 * (v & 3));
    }
  }
  __device__ __forceinline__ float operator[](int v) const { return code_elem(w, v); }
  // dequantised old momentum: code * (absmax / 127), the scale rounded first
  __device__ __forceinline__ float mold(int v, float scale) const { return code_elem(w, v) * scale; }
};

// V consecutive fp32 momentum values (fp32-state layout), V-element aligned for V = 4, 8 unless U
template <int V, bool U = false>
struct M32Chunk {
  float m[V];
  __device__ __forceinline__ void load(const CAME8_GLOBAL float* __restrict__ p) {
    if constexpr (V % 4 == 0) {
      using VT = typename std::conditional<U, f32x4u, f32x4>::type;
#pragma unroll
      for (int i = 0; i < V / 4; ++i) {
        const CAME8_GLOBAL VT* q = (const CAME8_GLOBAL VT*)p + i;
        const VT r = V == 4 ? ld_nt(q) : *q;  // the hint only for one 16-byte load per lane
        m[4 * i] = r.x; m[4 * i + 1] = r.y; m[4 * i + 2] = r.z; m[4 * i + 3] = r.w;
      }
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) m[v] = p[v];
    }
  }
  __device__ __forceinline__ float mold(int v, float) const { return m[v]; }
};

// V int8 codes as floats (V consecutive, V-byte aligned)
template <int V>
__device__ __forceinline__ void load_codes(const CAME8_GLOBAL int8_t* __restrict__ q, float (&out)[V]) {
  CodeChunk<V> c;
  c.load(q);
#pragma unroll
  for (int v = 0; v < V; ++v) out[v] = c[v];
}

// Rows whose length is not a multiple of V (UA variants of the band passes): every chunk is read with
// unaligned vector loads, and the row's last, partial chunk instead reads the row's last V elements;
// its first `skip` elements belong to the chunk before it and are masked out.  Word masks for
// element size es bytes: element v of word i is kept when v >= skip.
__device__ __forceinline__ uint32_t keep_mask(int i, int skip, int es) {
  const int lo = i * (4 / es);             // first element of word i
  const int n = skip - lo;                 // elements of word i to drop
  if (n <= 0) return 0xffffffffu;
  if (n >= 4 / es) return 0u;
  return 0xffffffffu << (8 * es * n);      // little-endian: the low elements go first
}

// Rows per register stage: about 64 bytes of gradient per thread, 1..16 rows.
template <typename TG, int V, int K>
struct Stage {
  static constexpr int bytes = int(sizeof(typename TG::storage)) * V * K;
  static constexpr int S = (64 / bytes) < 1 ? 1 : ((64 / bytes) > 16 ? 16 : (64 / bytes));
};

// Row and column accumulators of the band passes: fp64.  A row or column of heavy-tailed gradients
// can hold one element that outweighs the rest by ten orders of magnitude; fp32 partial sums then
// keep only what the dominant term's last few ulps allow, in an order-dependent way, while fp64
// sums are exact for every practical purpose (fp64 fused multiply-adds issue at the fp32 rate on
// CDNA4).  A band's column partials are rounded to fp32 once when stored.
template <int V, int K>
using ColAcc = double;

// Sum S per-thread row partials over the workgroup (NW wavefronts) in a fixed order;
// red is a [2][16][NW] LDS buffer whose half alternates between calls.
template <int S, int NW>
__device__ __forceinline__ void block_row_sums(const double (&ps)[S], double (*red)[16][NW], int par, double (&tot)[S]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const double w = wave_sum(ps[s]);
    if (lane == 0) red[par][s][wid] = w;
  }
  __syncthreads();
#pragma unroll
  for (int s = 0; s < S; ++s) {
    double t = red[par][s][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[par][s][w];
    tot[s] = t;
  }
}

// Work item -> (tensor, matrix, band) of a band launch.
struct BandItem {
  const DevTensor* t;
  int64_t b, band, r0, r1;
};
__device__ __forceinline__ BandItem band_item(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                              const int64_t* __restrict__ wstart, int ntens, int64_t w) {
  const int slot = find_slot(wstart, ntens, w);
  const DevTensor& t = T[tids[slot]];
  const int64_t local = w - wstart[slot];
  BandItem it;
  it.t = &t;
  it.b = local / t.nbands;
  it.band = local - it.b * t.nbands;
  it.r0 = it.band * t.rb;
  it.r1 = (it.r0 + t.rb < t.R) ? (it.r0 + t.rb) : t.R;
  return it;
}

// a + x*y in the accumulator's type (one fused multiply-add)
template <typename Acc>
__device__ __forceinline__ Acc acc_fma(Acc a, float x, float y) {
  if constexpr (std::is_same<Acc, double>::value) return fma(double(x), double(y), a);
  else return fmaf(x, y, a);
}
// a + x*x*w, the product formed in the accumulator's type
template <typename Acc>
__device__ __forceinline__ Acc acc_fma_w(Acc a, float x, float w) {
  if constexpr (std::is_same<Acc, double>::value) return fma(double(x) * double(w), double(x), a);
  else return fmaf(x * w, x, a);
}

// ---------------- P1 ----------------
// Row sums of g^2 (whole rows per workgroup, so the new row state R_i is known locally) and, per
// band, the column partial sums of g^2 + eps0 and of g^2/R_i.  These sums feed the factors, which
// are held to a relative tolerance rather than a bit pattern: each element costs one fused
// multiply-add per sum, and eps0 is added once per summed element count instead of per element.
template <typename TG, int V, int K, int TPB, bool UA = false>
__global__ __launch_bounds__(TPB) void k_fact_pass1(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                    const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using GS = typename TG::storage;
  using Acc = ColAcc<V, K>;
  constexpr int NW = TPB / kWave;
  // one-chunk vector rows take one-row stages: 76 VGPRs instead of 124 (six workgroups per CU
  // instead of four) outweigh the extra row-sum exchange per row (C3 pass 1: 0.76 -> 0.70 ms)
  constexpr int S = (V > 1 && K == 1) ? 1 : Stage<TG, V, K>::S;
  constexpr int64_t segw = int64_t(TPB) * V * K;
  __shared__ double red[2][16][NW];
  __shared__ float rowR[kMaxBandRows];
  __shared__ float rowold[kMaxBandRows];  // the band's old row states
  const int tid = threadIdx.x;
  int par = 0;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const BandItem it = band_item(T, tids, wstart, ntens, w);
    const DevTensor& t = *it.t;
    const int64_t R = t.R, C = t.C, b = it.b, r0 = it.r0, r1 = it.r1;
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g) + (b * R) * C);
    const CAME8_GLOBAL uint8_t* __restrict__ rq = gbl(t.rq);
    const CAME8_GLOBAL float* __restrict__ ra = gbl(t.ra);
    // the row state block of band row rr is rbb + blk_of(roff + r0 + rr): flat blocks over the tensor's
    // rows, or per-matrix blocks from the band's matrix b's first row (uniform per band)
    const int64_t rbb = t.pm ? b * t.pmb_r : 0, roff = t.pm ? 0 : b * R;
    CAME8_GLOBAL float* __restrict__ Rn = gbl(t.Rn);
    const float fC = float(C);
    const int64_t nseg = (C + segw - 1) / segw;
    CAME8_GLOBAL float* __restrict__ pU = gbl(t.partU + (b * t.nbands + it.band) * C);
    CAME8_GLOBAL float* __restrict__ pW = gbl(t.partW + (b * t.nbands + it.band) * C);
    double bandR = 0.0;  // sum of this band's new row states, in row order (every thread alike)
    const float band_eps = float(r1 - r0) * hp.eps0;  // eps0 of each element of a column partial
    // The old row states go through LDS: a per-row global load inside the stage loop would wait for
    // the next stage's loads as well.  The caller issues the band's first loads before this, so that
    // their latencies overlap.
    auto stage_rows = [&]() __attribute__((always_inline)) {
      for (int64_t rr = tid; rr < r1 - r0; rr += TPB) {
        const int64_t row = b * R + r0 + rr;
        rowold[rr] = t.fp32st ? gbl(st_sq_row(t))[row] : deq_u8(rq[row], ra[rbb + blk_of(roff + r0 + rr, hp)]);
      }
      wait_vm_all();  // on every path: the stage loop's waits then count only its own loads
      __syncthreads();
    };
    // new row state from the row's sum of g^2 (eps0 added once per element count)
    // (the mean through 1/C: within 1 ulp of tot / C, and equal to it for power-of-two C)
    const float invC = 1.0f / fC;
    auto row_state = [&](int64_t row, double sum_g2) {
      const float tot = float(sum_g2 + double(C) * double(hp.eps0));
      const float Rold = rowold[row - b * R - r0];
      const float mean = tot * invC;
      return t.mode2d ? (Rold * hp.b2) + (hp.a2f * mean) : fmaf(mean, hp.a2, Rold * hp.b2);
    };

    if (nseg == 1) {
      // The stage loop issues only loads (the new row states stay in LDS until after it) and issues
      // them unconditionally, so that the compiler waits for exactly one stage while the next is in
      // flight: a chunk past the row end (cok false) loads the row's first chunk and is skipped, a
      // row past the band end loads the band's last row and is ignored.
      // column sums of g^2 in fp64 (the column second moment is held to 1e-6); of g^2/R_i in fp32 (it
      // only enters the clip, and an outlier's g^2/R_i outweighs the rest of its column by about C/R,
      // not by orders of magnitude, since the outlier's row sum R_i holds it too)
      Acc colU[K][V];
      float colW[K][V];
#pragma unroll
      for (int k = 0; k < K; ++k)
#pragma unroll
        for (int v = 0; v < V; ++v) {
          colU[k][v] = Acc(0);
          colW[k][v] = 0.0f;
        }
      using CK = Chunk<TG, V, UA>;
      CK A[S][K], Bf[S][K];
      int32_t coff[K], cskip[K];
      bool cok[K];
      uint32_t gmask[UA ? K : 1][CK::NWD];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int32_t c = (tid + k * TPB) * V;
        cok[k] = c < C;  // without UA, C % V == 0: a chunk that starts inside the row ends inside it
        coff[k] = cok[k] ? c : 0;
        cskip[k] = 0;
        if constexpr (UA) {  // the row's partial last chunk reads the row's last V elements
          if (cok[k] && c + V > C) {
            coff[k] = int32_t(C) - V;
            cskip[k] = c - coff[k];
          }
#pragma unroll
          for (int i = 0; i < CK::NWD; ++i) gmask[k][i] = keep_mask(i, cskip[k], int(sizeof(GS)));
        }
      }
      // rows past the band end read the workspace's zero block (at least TPB*V*K elements long)
      const CAME8_GLOBAL GS* __restrict__ zrow = gbl(static_cast<const GS*>(hp.zeros));
      auto load_stage = [&](CK (&buf)[S][K], int64_t r) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const CAME8_GLOBAL GS* __restrict__ grow = (r + s < r1) ? g + (r + s) * C : zrow;
#pragma unroll
          for (int k = 0; k < K; ++k) buf[s][k].load(grow + coff[k]);
        }
      };
      auto process = [&](CK (&buf)[S][K], int64_t r) __attribute__((always_inline)) {
        // row partials and the column sums of g^2 (neither needs the row sums), then the row sums
        // over the workgroup, then the column sums of g^2/R_i.  A row past the band end holds zeros
        // and adds nothing anywhere; so do the masked leading elements of a partial last chunk.
        if constexpr (UA) {
#pragma unroll
          for (int s = 0; s < S; ++s)
#pragma unroll
            for (int k = 0; k < K; ++k) buf[s][k].mask(gmask[k]);
        }
        double ps[S];
#pragma unroll
        for (int s = 0; s < S; ++s) {
          ps[s] = 0.0;
#pragma unroll
          for (int k = 0; k < K; ++k) {
            if (cok[k]) {
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const double x = double(buf[s][k][v]);
                ps[s] = fma(x, x, ps[s]);
                colU[k][v] = fma(x, x, colU[k][v]);
              }
            }
          }
        }
        double tot[S];
        block_row_sums<S, NW>(ps, red, par, tot);
        par ^= 1;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const bool rok = r + s < r1;
          float invR = 0.0f;
          if (rok) {
            const float Rnew = row_state(b * R + r + s, tot[s]);
            if (tid == 0) rowR[r + s - r0] = Rnew;
            bandR += Rnew;
            // 1/R_i only weighs the clip's column sums: the hardware reciprocal (within 1 ulp) will do
            invR = __builtin_amdgcn_rcpf(Rnew);
          }
#pragma unroll
          for (int k = 0; k < K; ++k) {
            if (cok[k]) {
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const float x = buf[s][k][v];
                colW[k][v] = fmaf(x * invR, x, colW[k][v]);
              }
            }
          }
        }
      };
      // the row staging waits for every load issued so far, which also retires the previous band's
      // stores
      load_stage(A, r0);
      stage_rows();
      for (int64_t r = r0; r < r1; r += 2 * S) {
        load_stage(Bf, r + S);
        process(A, r);
        load_stage(A, r + 2 * S);
        process(Bf, r + S);
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if (cok[k]) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            if (UA && v < cskip[k]) continue;
            pU[coff[k] + v] = float(colU[k][v]) + band_eps;
            pW[coff[k] + v] = colW[k][v];
          }
        }
      }
      __syncthreads();
      for (int64_t rr = tid; rr < r1 - r0; rr += TPB) Rn[b * R + r0 + rr] = rowR[rr];
    } else if constexpr (!UA) {  // (the host gives UA variants single-sweep rows only)
      // Rows wider than one sweep of the workgroup: the row sums first, row by row, then the column
      // partials segment by segment (the band is read twice).  A row's K chunks of a segment are
      // loaded together, before any is used: a chunk past the row end loads the row's first chunk
      // and is skipped; in phase B two rows' loads are in flight.
      stage_rows();
      using CK = Chunk<TG, V>;
      auto seg_col = [&](int64_t seg, int k) { return seg * segw + (int64_t(tid) + int64_t(k) * TPB) * V; };
      // phase A: row sums over all segments
      for (int64_t r = r0; r < r1; ++r) {
        double ps[1] = {0.0};
        for (int64_t seg = 0; seg < nseg; ++seg) {
          CK x[K];
#pragma unroll
          for (int k = 0; k < K; ++k) {
            const int64_t c0 = seg_col(seg, k);
            x[k].load(g + r * C + (c0 < C ? c0 : 0));
          }
#pragma unroll
          for (int k = 0; k < K; ++k) {
            if (seg_col(seg, k) < C) {
#pragma unroll
              for (int v = 0; v < V; ++v) ps[0] = acc_fma(ps[0], x[k][v], x[k][v]);
            }
          }
        }
        double tot[1];
        block_row_sums<1, NW>(ps, red, par, tot);
        par ^= 1;
        const int64_t row = b * R + r;
        const float Rnew = row_state(row, tot[0]);
        bandR += Rnew;
        if (tid == 0) {
          Rn[row] = Rnew;
          rowR[r - r0] = Rnew;
        }
      }
      __syncthreads();
      // phase B: column partials segment by segment
      for (int64_t seg = 0; seg < nseg; ++seg) {
        Acc colU[K][V], colW[K][V];
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
          for (int v = 0; v < V; ++v) colU[k][v] = colW[k][v] = Acc(0);
        for (int64_t r = r0; r < r1; r += 2) {
          const bool two = r + 1 < r1;
          CK x0[K], x1[K];
#pragma unroll
          for (int k = 0; k < K; ++k) {
            const int64_t c0 = seg_col(seg, k);
            const int64_t cc = c0 < C ? c0 : 0;
            x0[k].load(g + r * C + cc);
            x1[k].load(g + (two ? r + 1 : r) * C + cc);
          }
          const float invR0 = 1.0f / rowR[r - r0];
          const float invR1 = two ? 1.0f / rowR[r + 1 - r0] : 0.0f;
#pragma unroll
          for (int k = 0; k < K; ++k) {
            if (seg_col(seg, k) < C) {
#pragma unroll
              for (int v = 0; v < V; ++v) {
                colU[k][v] = acc_fma(colU[k][v], x0[k][v], x0[k][v]);
                colW[k][v] = acc_fma_w(colW[k][v], x0[k][v], invR0);
              }
              if (two) {
#pragma unroll
                for (int v = 0; v < V; ++v) {
                  colU[k][v] = acc_fma(colU[k][v], x1[k][v], x1[k][v]);
                  colW[k][v] = acc_fma_w(colW[k][v], x1[k][v], invR1);
                }
              }
            }
          }
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const int64_t c0 = seg_col(seg, k);
          if (c0 < C) {
#pragma unroll
            for (int v = 0; v < V; ++v) {
              pU[c0 + v] = float(colU[k][v]) + band_eps;
              pW[c0 + v] = float(colW[k][v]);
            }
          }
        }
      }
      __syncthreads();  // rowR is reused by the next work item
    }
    if (tid == 0) t.rsum[b * t.nbands + it.band] = float(bandR);
    __syncthreads();  // rowold is rewritten by the next work item
  }
}

// ---------------- P1, default clip mode ----------------
// Pass 1 without the column sums of g^2/R_i.  Only the exactly rounded clip and the clip-norm
// estimates use them; in the default mode the estimates take instead each band's sum of e_i/R_i
// (e_i the row's sum of g^2; esum) with the band's column profile of g^2 (the partials of U), and the
// exact clip is not formed.  No column sum then needs a row's R_i, so:
//   * the stage loop has no barrier: each wave's share of a row sum goes to LDS (rows past the band
//     end to a dummy row), and the band's rows are combined once, after its last stage;
//   * rows wider than one sweep of the workgroup are taken in column segments (MS), each over all of
//     the band's rows, the per-wave row sums adding up over the segments; every element is read once.
// The row sums, new row states and column partials are those of k_fact_pass1 (the same fp64 sums;
// a row's waves combined in the same order for single-sweep rows).
template <typename TG, int V, int K, int TPB, bool UA = false, bool MS = false>
__global__ __launch_bounds__(TPB) void k_fact_pass1n(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                     const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using GS = typename TG::storage;
  using Acc = ColAcc<V, K>;
  using CK = Chunk<TG, V, UA>;
  constexpr int NW = TPB / kWave;
  // aligned 128-thread workgroups of fp32 gradients (narrow rows) take twice the rows per stage: more
  // bytes in flight per wave (as pass 2's)
  constexpr int S = ((V > 1 && K == 1) ? 2 : Stage<TG, V, K>::S) * ((TPB == 128 && sizeof(GS) == 4 && !UA) ? 2 : 1);
  constexpr int64_t segw = int64_t(TPB) * V * K;
  __shared__ double rowpart[2][kMaxBandRows + 1][NW];  // per-wave row sums of a band (+1: a dummy row)
  __shared__ float rowval[kMaxBandRows];  // the band's new row states
  __shared__ float rowe[kMaxBandRows];    // e_i / R_i
  __shared__ float rowold[kMaxBandRows];  // the band's old row states
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  int bpar = 0;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const BandItem it = band_item(T, tids, wstart, ntens, w);
    const DevTensor& t = *it.t;
    const int64_t R = t.R, C = t.C, b = it.b, r0 = it.r0, r1 = it.r1;
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g) + (b * R) * C);
    const CAME8_GLOBAL uint8_t* __restrict__ rq = gbl(t.rq);
    const CAME8_GLOBAL float* __restrict__ ra = gbl(t.ra);
    const int64_t rbb = t.pm ? b * t.pmb_r : 0, roff = t.pm ? 0 : b * R;  // row state blocks, as in k_fact_pass1
    CAME8_GLOBAL float* __restrict__ Rn = gbl(t.Rn);
    const int64_t nseg = (C + segw - 1) / segw;
    CAME8_GLOBAL float* __restrict__ pU = gbl(t.partU + (b * t.nbands + it.band) * C);
    const float band_eps = float(r1 - r0) * hp.eps0;  // eps0 of each element of a column partial
    const float invC = 1.0f / float(C);
    // The old row states go through LDS (a per-row global load at the band's end would wait for the
    // stage loop's loads as well); MS clears the per-wave row sums, which add up over the segments.
    auto stage_rows = [&]() __attribute__((always_inline)) {
      for (int64_t rr = tid; rr < r1 - r0; rr += TPB) {
        const int64_t row = b * R + r0 + rr;
        rowold[rr] = t.fp32st ? gbl(st_sq_row(t))[row] : deq_u8(rq[row], ra[rbb + blk_of(roff + r0 + rr, hp)]);
      }
      if constexpr (MS) {
        for (int64_t i = tid; i < (r1 - r0) * NW; i += TPB) rowpart[bpar][i / NW][i % NW] = 0.0;
        if (tid < NW) rowpart[bpar][kMaxBandRows][tid] = 0.0;
      }
      wait_vm_all();  // on every path: the stage loop's waits then count only its own loads
      __syncthreads();
    };
    int32_t coff[K], cskip[K];
    bool cok[K];
    uint32_t gmask[UA ? K : 1][CK::NWD];
    Acc colU[K][V];
    auto setup_segment = [&](int64_t cbase) __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int32_t c = int32_t(cbase) + (tid + k * TPB) * V;
        cok[k] = c < C;  // without UA, C % V == 0: a chunk that starts inside the row ends inside it
        coff[k] = cok[k] ? c : 0;
        cskip[k] = 0;
        if constexpr (UA) {  // the row's partial last chunk reads the row's last V elements
          if (cok[k] && c + V > C) {
            coff[k] = int32_t(C) - V;
            cskip[k] = c - coff[k];
          }
#pragma unroll
          for (int i = 0; i < CK::NWD; ++i) gmask[k][i] = keep_mask(i, cskip[k], int(sizeof(GS)));
        }
#pragma unroll
        for (int v = 0; v < V; ++v) colU[k][v] = Acc(0);
      }
    };
    // The stage loop issues loads only, unconditionally: a chunk past the row end (cok false) loads the
    // row's first chunk and is skipped, and a row past the band end loads the band's last row and adds
    // nothing (its row sum goes to the dummy row).
    auto load_stage = [&](CK (&buf)[S][K], int64_t r) __attribute__((always_inline)) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const CAME8_GLOBAL GS* __restrict__ grow = g + ((r + s < r1) ? (r + s) : (r1 - 1)) * C;
#pragma unroll
        for (int k = 0; k < K; ++k) buf[s][k].load(grow + coff[k]);
      }
    };
    auto process = [&](CK (&buf)[S][K], int64_t r) __attribute__((always_inline)) {
      if constexpr (UA) {  // the masked leading elements of a partial last chunk read as zero
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int k = 0; k < K; ++k) buf[s][k].mask(gmask[k]);
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const bool rok = r + s < r1;  // uniform
        double ps = 0.0;
        if (rok) {
#pragma unroll
          for (int k = 0; k < K; ++k) {
            if (cok[k]) {
#pragma unroll
              for (int v = 0; v < V; ++v) {
                const double x = double(buf[s][k][v]);
                ps = fma(x, x, ps);
                colU[k][v] = fma(x, x, colU[k][v]);
              }
            }
          }
        }
        const double wsum = wave_sum(ps);
        const int64_t slot = rok ? (r + s - r0) : int64_t(kMaxBandRows);
        if (lane == 0) {
          if constexpr (MS) rowpart[bpar][slot][wid] += wsum;
          else rowpart[bpar][slot][wid] = wsum;
        }
      }
    };
    auto segment = [&](int64_t cbase) __attribute__((always_inline)) {
      setup_segment(cbase);
      CK A[S][K], Bf[S][K];
      load_stage(A, r0);
      for (int64_t r = r0; r < r1; r += 2 * S) {
        load_stage(Bf, r + S);
        process(A, r);
        load_stage(A, r + 2 * S);
        process(Bf, r + S);
      }
#pragma unroll
      for (int k = 0; k < K; ++k) {
        if (cok[k]) {
#pragma unroll
          for (int v = 0; v < V; ++v)
            if (!UA || v >= cskip[k]) pU[coff[k] + v] = float(colU[k][v]) + band_eps;
        }
      }
    };
    stage_rows();
    if constexpr (MS) {
      for (int64_t seg = 0; seg < nseg; ++seg) {
        segment(seg * segw);
        if (seg + 1 < nseg) wait_vm_all();  // the partials' stores: the next stage loop waits for loads only
      }
    } else {
      segment(0);  // (the host gives the other variants single-sweep rows only)
    }
    __syncthreads();
    // row totals over the waves in a fixed order, the new row states, and e_i / R_i; the first wave
    // adds up the band's (lane l over rows l, l+64, ..., then the lanes in the wave sum's order)
    for (int64_t rr = tid; rr < r1 - r0; rr += TPB) {
      double tot = rowpart[bpar][rr][0];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) tot += rowpart[bpar][rr][w2];
      const float Rold = rowold[rr];
      const float mean = float(tot + double(C) * double(hp.eps0)) * invC;
      const float Rnew = t.mode2d ? (Rold * hp.b2) + (hp.a2f * mean) : fmaf(mean, hp.a2, Rold * hp.b2);
      Rn[b * R + r0 + rr] = Rnew;
      rowval[rr] = Rnew;
      rowe[rr] = Rnew > 0.0f ? float(tot) / Rnew : 0.0f;
    }
    __syncthreads();
    if (wid == 0) {
      double sr = 0.0, se = 0.0;
      for (int64_t rr = lane; rr < r1 - r0; rr += kWave) {
        sr += rowval[rr];
        se += rowe[rr];
      }
      sr = wave_sum(sr);
      se = wave_sum(se);
      if (lane == 0) {
        t.rsum[b * t.nbands + it.band] = float(sr);
        t.esum[b * t.nbands + it.band] = float(se);
      }
    }
    bpar ^= 1;  // the next band writes the other half (after this band's barriers above)
    __syncthreads();  // rowold is rewritten by the next work item
  }
}

// ---------------- P1 / P2 for tiny matrices ----------------
// Tensors whose matrices hold at most kTinyElems elements (conv kernels such as 320x320x3x3 are
// 102400 matrices of 3x3; 1280x640x1x1 is 819200 matrices of one element) take one thread per
// matrix instead of a workgroup per band: the matrix is its own band (nbands = 1), and the thread
// writes what the band passes write -- new row states, the band's row-state sum, the column partial
// sums -- with the same per-element arithmetic, its sums in fp64 in index order.
constexpr int kTinyElems = 64;

template <typename TG>
__global__ __launch_bounds__(kThreads) void k_tiny_pass1(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using GS = typename TG::storage;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t b = (w - wstart[slot]) * kThreads + threadIdx.x;  // the matrix
    if (b >= t.P) continue;
    const int64_t R = t.R, C = t.C;
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g) + b * R * C);
    CAME8_GLOBAL float* __restrict__ Rn = gbl(t.Rn + b * R);
    const float invC = 1.0f / float(C);
    double bandR = 0.0;
    for (int64_t i = 0; i < R; ++i) {
      double s = 0.0;
      for (int64_t j = 0; j < C; ++j) {
        const double x = double(TG::load(g[i * C + j]));
        s = fma(x, x, s);
      }
      const int64_t row = b * R + i;
      const float Rold = t.fp32st ? st_sq_row(t)[row] : deq_u8(t.rq[row], t.ra[rblk(t, row, hp)]);
      const float mean = float(s + double(C) * double(hp.eps0)) * invC;
      const float Rnew = fmaf(mean, hp.a2, Rold * hp.b2);
      Rn[i] = Rnew;
      bandR += Rnew;
    }
    const float band_eps = float(R) * hp.eps0;
    for (int64_t j = 0; j < C; ++j) {
      double u = 0.0;
      float wsum = 0.0f;
      for (int64_t i = 0; i < R; ++i) {
        const float x = TG::load(g[i * C + j]);
        u = fma(double(x), double(x), u);
        wsum = fmaf(x * __builtin_amdgcn_rcpf(Rn[i]), x, wsum);
      }
      gbl(t.partU)[b * C + j] = float(u) + band_eps;
      gbl(t.partW)[b * C + j] = wsum;
    }
    gbl(t.rsum)[b] = float(bandR);
  }
}

template <typename TG>
__global__ __launch_bounds__(kThreads) void k_tiny_pass2(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using GS = typename TG::storage;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t b = (w - wstart[slot]) * kThreads + threadIdx.x;
    if (b >= t.P) continue;
    const int64_t R = t.R, C = t.C, e0 = b * R * C;
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g) + e0);
    const CAME8_GLOBAL float* __restrict__ rf = gbl(t.rfac + b * R);
    const CAME8_GLOBAL float* __restrict__ cf = gbl(t.cfac + b * C);
    const float clip = t.clip[0];
    const float crcp = 1.0f / clip;  // as the band pass: the divisor is >= 1
    const int64_t PR = t.P * R;
    // d = u - m of element (i, j), as the band pass forms it
    auto d_at = [&](int64_t i, int64_t j) {
      const int64_t e = e0 + i * C + j;
      const float mo = t.fp32st ? st_m(t)[e]
                                : float(t.mq[e]) * div_fast(t.ma[t.pm ? mblk(t, e, hp) : blk_of_nb(e, hp)], kSignedQ, kRcpSignedQ);
      const float u = div_fast((rf[i] * cf[j]) * TG::load(g[i * C + j]), clip, crcp);
      const float m = fmaf(u, hp.a1, mo * hp.b1);
      return u - m;
    };
    double bandRR = 0.0;
    for (int64_t i = 0; i < R; ++i) {
      double s = 0.0;
      for (int64_t j = 0; j < C; ++j) {
        const float d = d_at(i, j);
        s = fma(double(d), double(d), s);
      }
      const int64_t row = b * R + i;
      const float tot = float(s + double(C) * double(hp.eps1));
      const float RRold = t.fp32st ? t.ra[row] : deq_u8(t.rq[PR + row], t.ra[t.nbr + rblk(t, row, hp)]);
      const float RRnew = fmaf(tot / float(C), hp.a3, RRold * hp.b3);
      gbl(t.RRn)[row] = RRnew;
      bandRR += RRnew;
    }
    const float band_eps = float(R) * hp.eps1;
    for (int64_t j = 0; j < C; ++j) {
      double s = 0.0;
      for (int64_t i = 0; i < R; ++i) {
        const float d = d_at(i, j);
        s = fma(double(d), double(d), s);
      }
      gbl(t.partRes)[b * C + j] = float(s) + band_eps;
    }
    gbl(t.rrsum)[b] = float(bandRR);
  }
}

// ---------------- P2 ----------------
// Residual row and column sums of a band.  Per element the reference forms u = (r_i*c_j)*g / clip,
// m = fma(u, 1-b1, m_old*b1) and res = (u - m)^2 + eps1 (CAME8bitFull.py:1032-1036) and keeps only
// the means of res along rows and columns; the momentum itself is formed again, and kept, in pass 3.
// This pass forms u and m with the reference's own operations and roundings (the division by the
// clip divisor through its reciprocal, exact for the numerators that matter; m_old = code*(absmax/127)),
// so d = u - m is the reference's; it then sums d*d with fused multiply-adds and adds eps1 once per
// summed element count.  The sums differ from the reference's only in the order of addition and the
// rounding of d*d: a few 1e-8 relative even where one element dominates a short column.
// The 16-bit-gradient UA variants of 256 threads are held to two resident workgroups per CU: left
// free, the compiler spills a few registers to AGPRs and the total leaves room for one only.
// MS: rows wider than one sweep, taken in column segments (a variant of its own: the segment loop
// costs registers that the single-sweep variants, at the edge of two resident workgroups, lack).
template <typename TG, int V, int K, int TPB, bool F32ST, bool UA = false, bool MS = false>
__global__ __launch_bounds__(TPB, (UA && sizeof(typename TG::storage) == 2 && TPB == 256) ? 2 : 1) void k_fact_pass2(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                    const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using GS = typename TG::storage;
  using Acc = ColAcc<V, K>;
  constexpr int NW = TPB / kWave;
  // one-chunk vector rows take two-row stages instead of four: 157 VGPRs instead of 227 (three
  // workgroups per CU instead of two); the stage loop has no barrier (C3 pass 2: 1.00 -> 0.89 ms)
  // Aligned 128-thread workgroups of fp32 gradients take twice the rows per stage, as pass 1's do (C2's
  // 1024-wide rows: the step 2.053 -> 2.029 ms).  Not the others: for 16-bit gradients it took C3's
  // 2048-wide rows from 4.35 to 4.66 ms, and C5's unaligned fp32 rows slowed down too (their registers
  // then leave fewer waves per SIMD).
  constexpr int S = ((V > 1 && K == 1) ? 2 : Stage<TG, V, K>::S) * ((TPB == 128 && sizeof(GS) == 4 && !UA) ? 2 : 1);
  constexpr int64_t segw = int64_t(TPB) * V * K;
  __shared__ double rowpart[2][kMaxBandRows + 1][NW];  // per-wave row sums of a band (+1: a dummy row)
  __shared__ float rowval[kMaxBandRows];           // the band's new residual row states
  __shared__ float rowsc[kMaxBandRows];            // the band's row factors r_i
  __shared__ float rowold[kMaxBandRows];           // the band's old residual row states
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  int bpar = 0;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const BandItem it = band_item(T, tids, wstart, ntens, w);
    const DevTensor& t = *it.t;
    const int64_t R = t.R, C = t.C, b = it.b, r0 = it.r0, r1 = it.r1;
    const int64_t ebase = (b * R) * C;
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g) + ebase);
    const CAME8_GLOBAL int8_t* __restrict__ mq = gbl(t.mq + ebase);
    const CAME8_GLOBAL float* __restrict__ m32 = gbl(static_cast<const float*>(st_m(t)) + ebase);
    const CAME8_GLOBAL float* __restrict__ ma = gbl(t.ma);
    const CAME8_GLOBAL float* __restrict__ cf = gbl(t.cfac + b * C);
    const CAME8_GLOBAL float* __restrict__ rfac = gbl(t.rfac);
    const CAME8_GLOBAL uint8_t* __restrict__ rq = gbl(t.rq);
    const CAME8_GLOBAL float* __restrict__ ra = gbl(t.ra);
    const int64_t rbb = t.pm ? b * t.pmb_r : 0, roff = t.pm ? 0 : b * R;  // row state blocks, as in pass 1
    CAME8_GLOBAL float* __restrict__ RRn = gbl(t.RRn);
    const float clip = uniform_f32(t.clip[0]);
    const float crcp = 1.0f / clip;  // the clip divisor is >= 1, so division through it is exact or 1 ulp off
    const float fC = float(C);
    const float band_eps = float(r1 - r0) * hp.eps1;  // eps1 of each element of a column partial
    const int64_t nseg = (C + segw - 1) / segw;
    CAME8_GLOBAL float* __restrict__ pR = gbl(t.partRes + (b * t.nbands + it.band) * C);
    const int64_t PR = t.P * R;
    constexpr bool f32st = F32ST;  // fp32 states (CAMECUDA layout); the host keys the launch by it

    // d = u - m of one element (x the gradient, mo the dequantised old momentum)
    auto d_of = [&](float ri, float cj, float x, float mo) __attribute__((always_inline)) {
      const float u = div_fast((ri * cj) * x, clip, crcp);
      const float m = fmaf(u, hp.a1, mo * hp.b1);
      return u - m;
    };
    // new residual row state of band row rr from its sum of d^2
    auto row_state = [&](int64_t rr, double sum_e2) {
      const float tot = float(sum_e2 + double(C) * double(hp.eps1));
      const float RRnew = fmaf(tot / fC, hp.a3, rowold[rr] * hp.b3);
      RRn[b * R + r0 + rr] = RRnew;
      return RRnew;
    };
    // The band's row scalars (r_i, old residual states) go through LDS: a per-row global load inside
    // the stage loop, or at the band's end, would wait for the next stage's loads as well.  The
    // caller issues the band's first loads before this, so that their latencies overlap.
    auto stage_rows = [&]() __attribute__((always_inline)) {
      for (int64_t rr = tid; rr < r1 - r0; rr += TPB) {
        const int64_t row = b * R + r0 + rr;
        rowsc[rr] = rfac[row];
        rowold[rr] = f32st ? gbl(t.ra)[row] : deq_u8(rq[PR + row], ra[t.nbr + rbb + blk_of(roff + r0 + rr, hp)]);
      }
      if constexpr (MS) {  // the per-wave row sums add up over the column segments (the dummy row too)
        for (int64_t i = tid; i < (r1 - r0) * NW; i += TPB) rowpart[bpar][i / NW][i % NW] = 0.0;
        if (tid < NW) rowpart[bpar][kMaxBandRows][tid] = 0.0;
      }
      wait_vm_all();  // on every path: the stage loop's waits then count only its own loads
      __syncthreads();
    };
    if (MS || nseg == 1) {  // (the host gives the other variants single-sweep rows only)
      // The band's columns in segments of one sweep of the workgroup (MS; otherwise the sweep covers a
      // row), each over all of the band's rows: the column sums of a segment are complete when its
      // rows are, and the per-wave row sums add up over the segments in LDS.  Every element is read
      // once.
      // The stage loop is branch-free, so that the compiler can wait for exactly one stage's loads
      // while the next stage's are in flight: a chunk past the row end (cok false) loads the row's
      // first chunk instead, and a row past the band end loads the band's last row; both contribute
      // zero (their r_i, c_j and momentum scale are zero) and their sums are never stored.
      float cj[K][V];
      int32_t coff[K], cskip[K];
      bool cok[K];
      uint32_t cmask[UA ? K : 1][CodeChunk<V>::NWD];
      Acc colR[K][V];
      int32_t cbk[K];
      int64_t seg = 0;  // the column segment
      auto setup_segment = [&](int64_t cbase) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
          const int32_t c = int32_t(cbase) + (tid + k * TPB) * V;
          cok[k] = c < C;  // without UA, C % V == 0: a chunk that starts inside the row ends inside it
          coff[k] = cok[k] ? c : 0;
          cskip[k] = 0;
          if constexpr (UA) {  // the row's partial last chunk reads the row's last V elements
            if (cok[k] && c + V > C) {
              coff[k] = int32_t(C) - V;
              cskip[k] = c - coff[k];
            }
#pragma unroll
            for (int i = 0; i < CodeChunk<V>::NWD; ++i) cmask[k][i] = keep_mask(i, cskip[k], 1);
          }
          // a masked leading element has c_j = 0 (so u = 0) and a zeroed code (so m = 0)
#pragma unroll
          for (int v = 0; v < V; ++v) cj[k][v] = (cok[k] && v >= cskip[k]) ? cf[coff[k] + v] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
          for (int v = 0; v < V; ++v) colR[k][v] = Acc(0);
        // When B divides C a row starts a block: the block of chunk k is the row's first block plus
        // the chunk's (per-thread) block offset cbk[k].
#pragma unroll
        for (int k = 0; k < K; ++k) cbk[k] = t.rowal ? int32_t(blk_of(coff[k], hp)) : 0;
      };
      // AL: rows start quantisation blocks; ST: fp32 states
      auto run = [&](auto AL, auto ST) __attribute__((always_inline)) {
        constexpr bool kF32 = decltype(ST)::value;
        constexpr bool kAligned = decltype(AL)::value && !kF32;
        using MB = typename std::conditional<kF32, M32Chunk<V, UA>, CodeChunk<V, UA>>::type;
        // a stage: S rows of gradient chunks, momentum chunks and (8-bit states) the chunks' block
        // absmax, all issued together so that waiting for one stage never waits for the next.
        // UA: a chunk may straddle two quantisation blocks; it holds both scales and the number of
        // its elements in the first block.
        struct StageBuf {
          Chunk<TG, V, UA> g[S][K];
          MB q[S][K];
          float a[S][K];
          float a2[UA ? S : 1][UA ? K : 1];
          int32_t split[UA ? S : 1][UA ? K : 1];
        };
        StageBuf A, Bs;
        auto load_stage = [&](StageBuf& sb, int64_t r) __attribute__((always_inline)) {
#pragma unroll
          for (int s = 0; s < S; ++s) {
            const int64_t rs = (r + s < r1) ? (r + s) : (r1 - 1);
            const int64_t erow = ebase + rs * C;
            const CAME8_GLOBAL float* __restrict__ marow = kAligned ? ma + blk_of_nb(erow, hp) : ma;
#pragma unroll
            for (int k = 0; k < K; ++k) {
              sb.g[s][k].load(g + rs * C + coff[k]);
              if constexpr (kF32) {
                sb.q[s][k].load(m32 + rs * C + coff[k]);
              } else if constexpr (UA) {
                sb.q[s][k].load(mq + rs * C + coff[k]);
                // per-matrix blocks (t.pm; the host sends such tensors to this variant or to V = 1): block
                // numbers from the band's matrix's first element, after that matrix's first block
                const int64_t e0 = (t.pm ? rs * C : erow) + coff[k];
                const CAME8_GLOBAL float* __restrict__ mab = t.pm ? ma + b * t.pmb_m : ma;
                const int64_t b0 = blk_of_nb(e0, hp), b1 = blk_of_nb(e0 + V - 1, hp);
                sb.a[s][k] = mab[b0];
                sb.a2[s][k] = mab[b1];
                sb.split[s][k] = int32_t((b0 + 1) * int64_t(hp.B) - e0);
              } else {
                sb.q[s][k].load(mq + rs * C + coff[k]);
                if constexpr (V == 1) {  // one element: its own block, per matrix when t.pm
                  sb.a[s][k] = t.pm ? ma[b * t.pmb_m + blk_of_nb(rs * C + coff[k], hp)] : ma[blk_of_nb(erow + coff[k], hp)];
                } else {  // flat momentum blocks (the host routes per-matrix ones elsewhere)
                  sb.a[s][k] = kAligned ? marow[cbk[k]] : ma[blk_of_nb(erow + coff[k], hp)];
                }
              }
            }
          }
        };
        auto process = [&](StageBuf& sb, int64_t r) __attribute__((always_inline)) {
          auto& gb = sb.g;
          auto& qb = sb.q;
          auto& ab = sb.a;
          double ps[S];
#pragma unroll
          for (int s = 0; s < S; ++s) {
            ps[s] = 0.0f;
            const bool rok = r + s < r1;
            const float ri_l = rowsc[(rok ? (r + s) : (r1 - 1)) - r0];
            const float ri = rok ? ri_l : 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
              const bool ok = rok && cok[k];
              // momentum scale absmax/127 (fp32 states: 1), zero for a chunk that counts for nothing
              float sc, sc2 = 0.0f;
              if constexpr (kF32) sc = ok ? 1.0f : 0.0f;
              else sc = ok ? div_fast(ab[s][k], kSignedQ, kRcpSignedQ) : 0.0f;
              if constexpr (UA && !kF32) {
                sc2 = ok ? div_fast(sb.a2[s][k], kSignedQ, kRcpSignedQ) : 0.0f;
                qb[s][k].w[0] &= cmask[k][0];
                if constexpr (CodeChunk<V>::NWD > 1) qb[s][k].w[1] &= cmask[k][1];
              }
#pragma unroll
              for (int v = 0; v < V; ++v) {
                float mo;
                if constexpr (kF32) mo = (UA && v < cskip[k]) ? 0.0f : qb[s][k].m[v] * sc;
                else if constexpr (UA) mo = qb[s][k][v] * (v < sb.split[s][k] ? sc : sc2);
                else mo = qb[s][k][v] * sc;
                const float d = d_of(ri, cj[k][v], gb[s][k][v], mo);
                ps[s] = acc_fma(ps[s], d, d);
                colR[k][v] = acc_fma(colR[k][v], d, d);
              }
            }
          }
          // each wave's share of the row sums (rows past the band end go to the dummy row); the
          // band's rows are combined after its last stage
#pragma unroll
          for (int s = 0; s < S; ++s) {
            const double wsum = wave_sum(ps[s]);
            const int64_t slot = (r + s < r1) ? (r + s - r0) : int64_t(kMaxBandRows);
            if (lane == 0) {  // MS: the segments add up (stage_rows clears the sums)
              if constexpr (MS) rowpart[bpar][slot][wid] += wsum;
              else rowpart[bpar][slot][wid] = wsum;
            }
          }
        };
        // two register stages in flight; the prefetches are unconditional (rows past the band end
        // reload its last row, from cache, and count for nothing).  The row staging (before the
        // first segment) and the wait after each segment's column partials retire every store
        // issued so far.  (Issuing the first stage before the staging keeps that stage's registers
        // live across the staging and the barrier, which costs this kernel more than the
        // overlapped latency gains.)
        if (seg == 0) stage_rows();
        load_stage(A, r0);
        for (int64_t r = r0; r < r1; r += 2 * S) {
          load_stage(Bs, r + S);
          process(A, r);
          load_stage(A, r + 2 * S);
          process(Bs, r + S);
        }
      };
      auto segment = [&]() __attribute__((always_inline)) {
        if constexpr (F32ST) run(std::false_type{}, std::true_type{});
        else if constexpr (UA) run(std::false_type{}, std::false_type{});
        else if (t.rowal) run(std::true_type{}, std::false_type{});
        else run(std::false_type{}, std::false_type{});
#pragma unroll
        for (int k = 0; k < K; ++k) {
          if (cok[k]) {
#pragma unroll
            for (int v = 0; v < V; ++v)
              if (!UA || v >= cskip[k]) pR[coff[k] + v] = float(colR[k][v]) + band_eps;
          }
        }
      };
      if constexpr (MS) {
        for (seg = 0; seg < nseg; ++seg) {
          setup_segment(seg * segw);
          segment();
          if (seg + 1 < nseg) wait_vm_all();  // the partials' stores: the next stage loop waits for loads only
        }
      } else {
        setup_segment(0);
        segment();
      }
      __syncthreads();
      // row totals over the waves in a fixed order; the new residual row states go through LDS so
      // that the first wave can add them up: lane l over rows l, l+64, ..., then the lanes in the
      // fixed order of the wave sum
      for (int rr = tid; rr < r1 - r0; rr += TPB) {
        double tot = rowpart[bpar][rr][0];
#pragma unroll
        for (int w2 = 1; w2 < NW; ++w2) tot += rowpart[bpar][rr][w2];
        rowval[rr] = row_state(rr, tot);
      }
      __syncthreads();
      if (wid == 0) {
        double sum = 0.0;
        for (int64_t rr = lane; rr < r1 - r0; rr += kWave) sum += rowval[rr];
        sum = wave_sum(sum);
        if (lane == 0) t.rrsum[b * t.nbands + it.band] = float(sum);
      }
      bpar ^= 1;  // the next band writes the other half (after this band's barriers above)
    }
    __syncthreads();  // rowsc is rewritten by the next work item
  }
}

// ===========================================================================
// F1b / F2b: factors and uint8 requantisation of the row / column states
// ===========================================================================
// Work item = one quantisation block of the row state (first nbr items of a
// tensor) or of the column state (next nbc items).

// Loads per batch of the strided sums below: a batch is issued before its first add, so a column
// sum over n partials waits for n / kSumBatch memory round trips instead of n.
constexpr int kSumBatch = 16;

// sum of n floats at stride s in fp64, in index order
__device__ __forceinline__ double ordered_sum_f64(const float* __restrict__ p, int64_t n, int64_t s) {
  double acc = 0.0;
  int64_t k = 0;
  for (; k + kSumBatch <= n; k += kSumBatch) {
    float v[kSumBatch];
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) v[u] = p[(k + u) * s];
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) acc += double(v[u]);
  }
  for (; k < n; ++k) acc += double(p[k * s]);
  return acc;
}

// sum of n floats at stride s in fp32, in index order from 0.0f (a running sum, as a sequential loop)
__device__ __forceinline__ float ordered_sum_f32(const float* __restrict__ p, int64_t n, int64_t s) {
  float acc = 0.0f;
  int64_t k = 0;
  for (; k + kSumBatch <= n; k += kSumBatch) {
    float v[kSumBatch];
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) v[u] = p[(k + u) * s];
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) acc += v[u];
  }
  for (; k < n; ++k) acc += p[k * s];
  return acc;
}

// A matrix's mean row state from the sum of its row states.
__device__ __forceinline__ float row_mean_of_sum(const DevTensor& t, double s) {
  const float m = float(s) / float(t.R);
  if (t.mode2d) return m > 0.0f ? m : 1.0f;  // 8bit2d: a mean that is not positive counts as 1
  return clamp_min_tiny(m);
}
// Mean row state of matrix b, max(mean, 1e-30): the per-band sums the band pass wrote (each an fp64
// sum rounded once), added in band order in fp64 (the reference: R.mean(dim=-1,
// keepdim=True).clamp_min(1e-30), CAME8bitFull.py:1021,1044).
__device__ __forceinline__ float matrix_row_mean(const DevTensor& t, const float* __restrict__ bandsum, int64_t b,
                                                 int64_t nb) {
  return row_mean_of_sum(t, ordered_sum_f64(bandsum + b * nb, nb, 1));
}

// Sums over the nbands band partials of one column (stride C) of one or two partial arrays: four
// interleaved fp64 accumulators (band k into accumulator k % 4), combined as (a0 + a1) + (a2 + a3).
template <int NA>
__device__ __forceinline__ void band_column_sums(const float* __restrict__ p0, const float* __restrict__ p1,
                                                 int64_t nbands, int64_t C, double* out) {
  double a[NA][4] = {};
  int64_t k = 0;
  for (; k + kSumBatch <= nbands; k += kSumBatch) {
    float v[NA][kSumBatch];
#pragma unroll
    for (int u = 0; u < kSumBatch; ++u) {
      v[0][u] = p0[(k + u) * C];
      if constexpr (NA > 1) v[NA - 1][u] = p1[(k + u) * C];
    }
#pragma unroll
    for (int x = 0; x < NA; ++x)
#pragma unroll
      for (int u = 0; u < kSumBatch; ++u) a[x][u & 3] += double(v[x][u]);
  }
  for (; k < nbands; ++k) {
    a[0][0] += double(p0[k * C]);
    if constexpr (NA > 1) a[NA - 1][0] += double(p1[k * C]);
  }
#pragma unroll
  for (int x = 0; x < NA; ++x) out[x] = (a[x][0] + a[x][1]) + (a[x][2] + a[x][3]);
}
template <bool RES>
__global__ __launch_bounds__(kThreads) void k_factor_blocks(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                            const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  __shared__ float smax[4];
  __shared__ double ssum[4], msum[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t local = w - wstart[slot];
    const bool is_row = local < t.nbr;
    const int64_t blk = is_row ? local : local - t.nbr;
    int64_t i0, i1;
    if (t.pm) {  // blocks restart at every matrix: block blk is block jb of matrix mb's R (or C) states
      const int64_t per = is_row ? t.pmb_r : t.pmb_c, n = is_row ? t.R : t.C;
      const int64_t mb = blk / per, jb = blk - mb * per;
      i0 = mb * n + jb * hp.B;
      i1 = (jb * hp.B + hp.B < n) ? (i0 + hp.B) : (mb * n + n);
    } else {
      const int64_t len = is_row ? t.P * t.R : t.P * t.C;
      i0 = blk * hp.B;
      i1 = (i0 + hp.B < len) ? (i0 + hp.B) : len;
    }
    const bool partial = (i1 - i0) < hp.B;  // zero padding joins the max
    float vmax = partial ? 0.0f : -__builtin_inff();
    double csum = 0.0;
    const float beta = RES ? hp.b3 : hp.b2;
    const float alpha = RES ? hp.a3 : hp.a2;
    const float alpha_f = RES ? hp.a3f : hp.a2f;
    if (is_row) {
      const float* __restrict__ Rsrc = RES ? t.RRn : t.Rn;
      float* __restrict__ fac = RES ? t.rrfac : t.rfac;
      const float* __restrict__ bsum = RES ? t.rrsum : t.rsum;
      // the 8bit2d momentum pass sums its residual row states per tile row
      const int64_t nsum = (RES && t.mode2d) ? int64_t(t.tr) : t.nbands;
      int64_t mb = i0 / t.R;  // matrix of the block's first row; blocks may span matrices
      const float vfirst = i0 + tid < i1 ? Rsrc[i0 + tid] : 0.0f;  // loaded before the mean's sums
      float mean;
      if ((i1 - 1) / t.R == mb) {
        // the block's rows are one matrix's (uniform): the workgroup sums the matrix's band sums together,
        // thread k over sums k, k + 256, ..., then in a fixed order (one round of loads instead of one
        // thread's chain over all of them)
        double ms = 0.0;
        for (int64_t k = tid; k < nsum; k += kThreads) ms += double(bsum[mb * nsum + k]);
        ms = wave_sum(ms);
        if (lane == 0) msum[wid] = ms;
        __syncthreads();  // (msum is written again only after the block maximum's barrier below)
        mean = row_mean_of_sum(t, ((msum[0] + msum[1]) + msum[2]) + msum[3]);
      } else {
        mean = matrix_row_mean(t, bsum, mb, nsum);
      }
      for (int64_t i = i0 + tid; i < i1; i += kThreads) {
        const int64_t bi = i / t.R;
        if (bi != mb) {
          mb = bi;
          mean = matrix_row_mean(t, bsum, mb, nsum);
        }
        const float v = i == i0 + tid ? vfirst : Rsrc[i];
        fac[i] = rsqrt_ref(v / mean);
        vmax = nan_max(vmax, v);
        if (t.fp32st) (RES ? t.ra : st_sq_row(t))[i] = v;  // the fp32 row state itself
      }
    } else {
      const int64_t off = RES ? t.P * t.C : 0;
      const int64_t aoff = RES ? t.nbc : 0;
      const float* __restrict__ part = RES ? t.partRes : t.partU;
      float* __restrict__ Cdst = RES ? t.CRn : t.Cn;
      float* __restrict__ fac = RES ? t.crfac : t.cfac;
      const float fR = float(t.R);
      int64_t cmb = -1;  // matrix whose mean row state crm holds
      float crm = 0.0f;
      for (int64_t i = i0 + tid; i < i1; i += kThreads) {
        const int64_t b = i / t.C;
        const int64_t j = i - b * t.C;
        float* __restrict__ cst = RES ? t.ca : st_sq_col(t);  // fp32 column state
        float Cold, Cv;
        double W = 0.0;  // column sum of the clip weights (!RES)
        if (t.mode2d) {
          // 8bit2d: residual column sums come from the tile partials (tiles in order); no clamp
          float s2 = 0.0f;
          if (RES) {
            s2 = ordered_sum_f32(t.t2col + i, t.tr, t.C);
          } else {
            double sw[2];
            band_column_sums<2>(part + (b * t.nbands) * t.C + j, t.partW + (b * t.nbands) * t.C + j, t.nbands, t.C, sw);
            s2 = float(sw[0]);
            W = sw[1];
          }
          Cold = RES ? deq_u8(t.rcq[i], t.rca[blk_of(i, hp)]) : deq_u8(t.cq[i], t.ca[blk_of(i, hp)]);
          Cv = (Cold * beta) + (alpha_f * (s2 / fR));
        } else {
          const float* __restrict__ pp = part + (b * t.nbands) * t.C + j;
          // the old state's loads go out before the partial sums' (their latencies overlap)
          Cold = t.fp32st ? cst[i] : deq_u8(t.cq[off + i], t.ca[aoff + cblk(t, i, hp)]);
          double sw[2] = {0.0, 0.0};  // column sums of the partials, and for !RES of the clip weights
          // (in the default clip mode the band passes wrote no partW: the clip partial is not used)
          if (RES || hp.noW) band_column_sums<1>(pp, nullptr, t.nbands, t.C, sw);
          else band_column_sums<2>(pp, t.partW + (b * t.nbands) * t.C + j, t.nbands, t.C, sw);
          const double s = sw[0];
          W = sw[1];
          Cv = clamp_min_tiny(fmaf(float(s) / fR, alpha, Cold * beta));
        }
        const float c = rsqrt_ref(Cv);
        Cdst[i] = Cv;
        fac[i] = c;
        if (t.fp32st) cst[i] = Cv;
        vmax = nan_max(vmax, Cv);
        if (!RES && (t.mode2d || !hp.noW)) {  // the clip partial (k_clip: exact mode, and 8bit2d tensors always)
          if (b != cmb) {
            cmb = b;
            crm = matrix_row_mean(t, t.rsum, b, t.nbands);
          }
          csum += double(crm) * double(c) * double(c) * W;
        }
      }
    }
    // block max and clip partial (fixed order)
    vmax = group_max<64>(vmax);
    if (!RES) csum = wave_sum(csum);
    if (lane == 0) {
      smax[wid] = vmax;
      ssum[wid] = csum;
    }
    __syncthreads();
    const float amax = fix_absmax(nan_max(nan_max(smax[0], smax[1]), nan_max(smax[2], smax[3])));
    if (tid == 0) {
      if (!RES && !is_row) t.clip_part[blk] = ((ssum[0] + ssum[1]) + ssum[2]) + ssum[3];
      if (t.mode2d) {
        if (is_row) (RES ? t.rra : t.ra)[blk] = amax;
        else (RES ? t.rca : t.ca)[blk] = amax;
      } else if (!t.fp32st) {
        if (is_row) t.ra[(RES ? t.nbr : 0) + blk] = amax;
        else t.ca[(RES ? t.nbc : 0) + blk] = amax;
      }
    }
    const float arcp = rcp_for_div(amax);
    if (t.fp32st) {
      // fp32 states were written above; no codes
    } else if (t.mode2d) {
      const float inv = 1.0f / amax;
      const float* __restrict__ src = is_row ? (RES ? t.RRn : t.Rn) : (RES ? t.CRn : t.Cn);
      uint8_t* __restrict__ q = is_row ? (RES ? t.rrq : t.rq) : (RES ? t.rcq : t.cq);
      for (int64_t i = i0 + tid; i < i1; i += kThreads) q[i] = quant_u8_inv(src[i], inv);
    } else if (is_row) {
      const float* __restrict__ Rsrc = RES ? t.RRn : t.Rn;
      uint8_t* __restrict__ q = t.rq + (RES ? t.P * t.R : 0);
      for (int64_t i = i0 + tid; i < i1; i += kThreads) q[i] = quant_u8_r(Rsrc[i], amax, arcp);
    } else {
      const float* __restrict__ Csrc = RES ? t.CRn : t.Cn;
      uint8_t* __restrict__ q = t.cq + (RES ? t.P * t.C : 0);
      for (int64_t i = i0 + tid; i < i1; i += kThreads) q[i] = quant_u8_r(Csrc[i], amax, arcp);
    }
    __syncthreads();  // smax / ssum reused by the next item
  }
}

// ===========================================================================
// 1-D tensors, pass A: sum of u^2 per tile, u = rsqrt(clamp(v)) * g
// ===========================================================================
// the new second moment of a 1-D element from its gradient and its old (dequantised) second moment
__device__ __forceinline__ float vec_v_from(float gv, float vold, const Hp& hp) {
  return clamp_min_tiny(fmaf(gv * gv + hp.eps0, hp.a2, vold * hp.b2));
}
template <typename TG>
__device__ __forceinline__ float vec_v_new(const DevTensor& t, int64_t e, float gv, const Hp& hp) {
  const float vold = t.fp32st ? st_sq_row(t)[e] : deq_u8(t.rq[e], t.ra[blk_of(e, hp)]);
  return vec_v_from(gv, vold, hp);
}
// The clamped indices of a thread's 8 elements e0 .. e0 + 7 of a 1-D tensor (an element at or past N
// reads element N - 1 and counts for nothing), and their gradients and old second moments, every
// load issued before the first is used: a branch per element would wait out each element's loads in
// turn.
template <typename TG>
__device__ __forceinline__ void vec_load8(const DevTensor& t, int64_t e0, const Hp& hp, int64_t (&ec)[8],
                                          float (&gv)[8], float (&vo)[8]) {
  using GS = typename TG::storage;
  const GS* __restrict__ g = static_cast<const GS*>(t.g);
#pragma unroll
  for (int v = 0; v < 8; ++v) ec[v] = min(e0 + v, t.N - 1);
#pragma unroll
  for (int v = 0; v < 8; ++v) gv[v] = TG::load(g[ec[v]]);
  if (t.fp32st) {
#pragma unroll
    for (int v = 0; v < 8; ++v) vo[v] = st_sq_row(t)[ec[v]];
  } else {
#pragma unroll
    for (int v = 0; v < 8; ++v) vo[v] = deq_u8(t.rq[ec[v]], t.ra[blk_of(ec[v], hp)]);
  }
}

template <typename TG>
__global__ __launch_bounds__(kThreads) void k_vec_passA(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                        const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  __shared__ double ssum[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t tile = w - wstart[slot];
    const int64_t e0 = tile * kTile + int64_t(tid) * 8;
    int64_t ec[8];
    float gv[8], vo[8];
    vec_load8<TG>(t, e0, hp, ec, gv, vo);
    double s = 0.0;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      if (e0 + v < t.N) {
        const float u = rsqrt_ref(vec_v_from(gv[v], vo[v], hp)) * gv[v];
        s += double(u) * double(u);
      }
    }
    s = wave_sum(s);
    if (lane == 0) ssum[wid] = s;
    __syncthreads();
    if (tid == 0) t.clip_part[tile] = ((ssum[0] + ssum[1]) + ssum[2]) + ssum[3];
    __syncthreads();
  }
}

// ===========================================================================
// CLIP: per-tensor divisor  max(||u|| / sqrt(N) / clip_threshold, 1)
// ===========================================================================
__device__ __forceinline__ float clip_from_norm(float norm, int64_t N, const Hp& hp) {
  const float rms = norm / float(sqrt(double(N)));
  const float q = rms / hp.thr;
  return q < 1.0f ? 1.0f : q;
}

// only2d: leave every tensor but those of the 8bit2d layout alone (the others take the norm in the
// reference's order, came8_norm.h)
template <int = 0>  // a template only so that every translation unit may include this header
__global__ __launch_bounds__(kThreads) void k_clip(const DevTensor* __restrict__ T, int ntens, int only2d, Hp hp) {
  __shared__ double ssum[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  for (int k = blockIdx.x; k < ntens; k += gridDim.x) {
    const DevTensor& t = T[k];
    if (only2d && !t.mode2d) continue;  // uniform over the workgroup
    double s = 0.0;
    for (int64_t i = tid; i < t.nclip; i += kThreads) s += t.clip_part[i];
    s = wave_sum(s);
    if (lane == 0) ssum[wid] = s;
    __syncthreads();
    if (tid == 0) {
      const double tot = ((ssum[0] + ssum[1]) + ssum[2]) + ssum[3];
      float c;
      if (t.mode2d) {  // 8bit2d: sqrtf(sum / n) in float (came_kernels.cu:2619-2620)
        const float q = sqrtf(float(tot) / float(t.N)) / hp.thr;
        c = q < 1.0f ? 1.0f : q;
      } else {
        c = clip_from_norm(float(sqrt(tot)), t.N, hp);
      }
      t.clip[0] = c;
      t.clip[1] = rcp_for_div(c);
    }
    __syncthreads();
  }
}

// Unclipped update u at flat index e, computed exactly as the reference does.
template <typename TG>
__device__ __forceinline__ float u_at(const DevTensor& t, int64_t e, const Hp& hp) {
  const float gv = TG::load(static_cast<const typename TG::storage*>(t.g)[e]);
  if (t.factored) {
    const int64_t row = e / t.C;
    const int64_t j = e - row * t.C;
    const int64_t b = row / t.R;
    return (t.rfac[row] * t.cfac[b * t.C + j]) * gv;
  }
  return rsqrt_ref(vec_v_new<TG>(t, e, gv, hp)) * gv;
}

// ===========================================================================
// P3: flat pass over whole quantisation blocks (factored tensors)
// ===========================================================================
// 2048-element tiles, 8 consecutive elements per thread, L = B/8 lanes per
// quantisation block (B a power of two in [8, 2048]).
//
// A tile that lies inside its tensor, of a tensor whose rows hold whole 8-element groups and whose
// buffers are 16-byte aligned, takes the fast path: one branch per tile on a workgroup-uniform
// condition, vector loads and stores, the reciprocal divisions, and the rare elements outside their
// exact range handled by selects.  Other tiles (tensor tails, ragged shapes) take the general
// per-element path.  Both give the same values.

// Maximum of per-thread values over the L lanes of each quantisation block (L = B/8 <= 256); every
// thread of the workgroup must call it (L > 64 synchronises through LDS).
__device__ __forceinline__ uint32_t block_max_bits(uint32_t v, int L, uint32_t (*wmax)[4], int& par) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (L <= 64) return group_max_bits_rt(v, L);
  v = group_max_bits<64>(v);
  if (lane == 0) wmax[par][wid] = v;
  __syncthreads();
  const int wpb = L >> 6;  // waves per block
  const int w0 = (wid / wpb) * wpb;
  v = wmax[par][w0];
  for (int k = 1; k < wpb; ++k) v = max(v, wmax[par][w0 + k]);
  par ^= 1;
  return v;
}

// |m| as an ordered bit pattern (a NaN orders above every number, so a maximum propagates it as
// torch.amax does)
__device__ __forceinline__ uint32_t abs_bits(float m) { return __float_as_uint(m) & 0x7fffffffu; }

// 8 codes packed little-endian into two words
__device__ __forceinline__ u32x2 pack_codes(const int32_t (&c)[8]) {
  u32x2 r;
  r.x = __builtin_amdgcn_perm(uint32_t(c[1]), uint32_t(c[0]), 0x0c0c0400u) |
        __builtin_amdgcn_perm(uint32_t(c[3]), uint32_t(c[2]), 0x04000c0cu);
  r.y = __builtin_amdgcn_perm(uint32_t(c[5]), uint32_t(c[4]), 0x0c0c0400u) |
        __builtin_amdgcn_perm(uint32_t(c[7]), uint32_t(c[6]), 0x04000c0cu);
  return r;
}

// m_new and the updated parameters of 8 elements that share a row and a quantisation block
// (reference CAME8bitFull.py:1032-1036 and 1047-1056): the reciprocal divisions, and the rare
// operands outside their exact range through selects.
// With F32ST (fp32 states) q holds the old momentum values and amax_old is not used; otherwise q
// holds the int8 codes of a block whose absmax is amax_old.
template <typename TP, bool F32ST>
__device__ __forceinline__ void p3_math8(const float (&gv)[8], const float (&q)[8], float (&pv)[8], float (&m)[8],
                                         float amax_old, float ri, float rri, const float (&cj)[8],
                                         const float (&crj)[8], float clip, float crcp, bool clip_fast, const Hp& hp) {
  float a[8];
  DivGuard gd;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    a[v] = (ri * cj[v]) * gv[v];
    gd.add(a[v]);
  }
  if (__builtin_expect(clip_fast && gd.fast() && (F32ST || fabsf(amax_old) <= 0x1.fffffep127f), 1)) {
    const float scale = F32ST ? 0.0f : div_fast(amax_old, kSignedQ, kRcpSignedQ);
#pragma unroll
    for (int v = 0; v < 8; ++v)
      m[v] = fmaf(div_fast(a[v], clip, crcp), hp.a1, (F32ST ? q[v] : q[v] * scale) * hp.b1);
  } else {
    const float scale = F32ST ? 0.0f : amax_old / kSignedQ;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float u = (clip_fast && !div_exact_needed(a[v])) ? div_fast(a[v], clip, crcp) : a[v] / clip;
      m[v] = fmaf(u, hp.a1, (F32ST ? q[v] : q[v] * scale) * hp.b1);
    }
  }
#pragma unroll
  for (int v = 0; v < 8; ++v) pv[v] = param_update<TP>(pv[v], (rri * crj[v]) * m[v], hp);
}

// p3_math8 for 8 elements that may lie on two rows: a row factor per element
template <typename TP, bool F32ST>
__device__ __forceinline__ void p3_math8r(const float (&gv)[8], const float (&q)[8], float (&pv)[8], float (&m)[8],
                                          float amax_old, const float (&ri)[8], const float (&rri)[8],
                                          const float (&cj)[8], const float (&crj)[8], float clip, float crcp,
                                          bool clip_fast, const Hp& hp) {
  float a[8];
  DivGuard gd;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    a[v] = (ri[v] * cj[v]) * gv[v];
    gd.add(a[v]);
  }
  if (__builtin_expect(clip_fast && gd.fast() && (F32ST || fabsf(amax_old) <= 0x1.fffffep127f), 1)) {
    const float scale = F32ST ? 0.0f : div_fast(amax_old, kSignedQ, kRcpSignedQ);
#pragma unroll
    for (int v = 0; v < 8; ++v)
      m[v] = fmaf(div_fast(a[v], clip, crcp), hp.a1, (F32ST ? q[v] : q[v] * scale) * hp.b1);
  } else {
    const float scale = F32ST ? 0.0f : amax_old / kSignedQ;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float u = (clip_fast && !div_exact_needed(a[v])) ? div_fast(a[v], clip, crcp) : a[v] / clip;
      m[v] = fmaf(u, hp.a1, (F32ST ? q[v] : q[v] * scale) * hp.b1);
    }
  }
#pragma unroll
  for (int v = 0; v < 8; ++v) pv[v] = param_update<TP>(pv[v], (rri[v] * crj[v]) * m[v], hp);
}

// int8 codes of 8 values of a block whose absmax is amax (abits: the block maximum of |m| as bits)
__device__ __forceinline__ u32x2 p3_quant8(const float (&m)[8], float amax, uint32_t abits) {
  const float arcp = rcp_for_div(amax);
  int32_t c[8];
  if (__builtin_expect(arcp == arcp && abits <= 0x7f800000u, 1)) {
    // |m| <= amax, so |m / amax| <= 1 and the code needs no clamp
#pragma unroll
    for (int v = 0; v < 8; ++v) c[v] = int32_t(rintf(div_fast(m[v], amax, arcp) * kSignedQ));
  } else {
#pragma unroll
    for (int v = 0; v < 8; ++v) c[v] = quant_s8(m[v], amax);
  }
  return pack_codes(c);
}

template <typename TP, typename TG, bool F32ST>
__global__ __launch_bounds__(kThreads) void k_fact_pass3(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using PS = typename TP::storage;
  using GS = typename TG::storage;
  __shared__ uint32_t wmax[2][4];
  const int tid = threadIdx.x;
  const int L = hp.B >> 3;  // lanes per block
  int par = 0;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t base = (w - wstart[slot]) * kTile;
    const int64_t e0 = base + int64_t(tid) * 8;
    const int64_t N = t.N, C = t.C, R = t.R;
    CAME8_GLOBAL PS* __restrict__ p = gbl(static_cast<PS*>(t.p));
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g));
    CAME8_GLOBAL int8_t* __restrict__ mq = gbl(t.mq);
    CAME8_GLOBAL float* __restrict__ ma = gbl(t.ma);
    const CAME8_GLOBAL float* __restrict__ rfac = gbl(t.rfac);
    const CAME8_GLOBAL float* __restrict__ rrfac = gbl(t.rrfac);
    const CAME8_GLOBAL float* __restrict__ cfac = gbl(t.cfac);
    const CAME8_GLOBAL float* __restrict__ crfac = gbl(t.crfac);
    const float clip = uniform_f32(t.clip[0]), crcp = uniform_f32(t.clip[1]);
    const bool clip_fast = crcp == crcp;
    const int64_t blk = blk_of(e0, hp);  // 8 elements share a block (B >= 8)
    int64_t row, bb;
    if (t.idx32) {
      const uint32_t r32 = udiv_magic(uint32_t(e0), t.mC, t.sC);
      row = r32;
      bb = udiv_magic(r32, t.mR, t.sR);
    } else {
      row = e0 / C;
      bb = row / R;
    }
    int64_t j = e0 - row * C;

    if (t.vec_ok && (t.c8 || C >= 8) && base + kTile <= N) {
      // ---- fast tile: vector access to 8 elements of one quantisation block ----
      float gv[8], pv[8], q[8], m[8];
      load8<TG, true>(g + e0, gv);
      load8<TP, true>(p + e0, pv);
      if constexpr (F32ST) load8<F32, true>(gbl(st_m(t)) + e0, q);
      else load_codes<8>(mq + e0, q);
      const float amax_old = F32ST ? 0.0f : ma[blk];
      if (t.c8) {
        // the 8 elements share a row; their column factors are contiguous and aligned
        float cj[8], crj[8];
        const float ri = rfac[row], rri = rrfac[row];
        load8<F32>(cfac + bb * C + j, cj);
        load8<F32>(crfac + bb * C + j, crj);
        p3_math8<TP, F32ST>(gv, q, pv, m, amax_old, ri, rri, cj, crj, clip, crcp, clip_fast, hp);
      } else if (!__any(j + 8 > C)) {
        // rows of C >= 8 elements that are not a whole number of 8-element groups, where no chunk of
        // the wavefront reaches the next row (most of them): one row's factors, unaligned loads
        float cj[8], crj[8];
        const float ri = rfac[row], rri = rrfac[row];
        load8u_f32(cfac + bb * C + j, cj);
        load8u_f32(crfac + bb * C + j, crj);
        p3_math8<TP, F32ST>(gv, q, pv, m, amax_old, ri, rri, cj, crj, clip, crcp, clip_fast, hp);
      } else {
        // the same rows where some chunk of the wavefront ends in the next row: the 8 elements
        // lie on at most two rows.  Element v is column j + v of `row`, or, past the row's end,
        // column j + v - C of row + 1 (which may begin the next matrix).  The factors come as two
        // unaligned 8-column loads, C apart, and a select per element; the lanes a select drops
        // read workspace memory next to the factor arrays (each array is padded to 256 bytes and
        // the column state arrays precede the column factors), never outside the workspace.
        const int64_t bb1 = (row + 1 - bb * R == R) ? bb + 1 : bb;
        const float r0 = rfac[row], rr0 = rrfac[row], r1 = rfac[row + 1], rr1 = rrfac[row + 1];
        float c0[8], cr0[8], c1[8], cr1[8], ri[8], rri[8], cj[8], crj[8];
        load8u_f32(cfac + bb * C + j, c0);
        load8u_f32(crfac + bb * C + j, cr0);
        load8u_f32(cfac + bb1 * C + j - C, c1);
        load8u_f32(crfac + bb1 * C + j - C, cr1);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const bool wrap = j + v >= C;
          ri[v] = wrap ? r1 : r0;
          rri[v] = wrap ? rr1 : rr0;
          cj[v] = wrap ? c1[v] : c0[v];
          crj[v] = wrap ? cr1[v] : cr0[v];
        }
        p3_math8r<TP, F32ST>(gv, q, pv, m, amax_old, ri, rri, cj, crj, clip, crcp, clip_fast, hp);
      }
      store8<TP>(p + e0, pv);
      if constexpr (F32ST) {
        store8<F32>(gbl(st_m(t)) + e0, m);
        continue;
      }

      uint32_t abits = 0;
#pragma unroll
      for (int v = 0; v < 8; ++v) abits = max(abits, abs_bits(m[v]));
      abits = block_max_bits(abits, L, wmax, par);
      const float amax = fix_absmax(__uint_as_float(abits));
      if ((e0 & (hp.B - 1)) == 0) ma[blk] = amax;
      st_nt((CAME8_GLOBAL u32x2*)(mq + e0), p3_quant8(m, amax, abits));
    } else {
      // ---- general tile: element by element ----
      float m[8], pv[8];
      if (e0 < N) {
        const float scale = F32ST ? 0.0f : ma[blk] / kSignedQ;
        int64_t i = row - bb * R;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          if (e0 + v < N) {
            pv[v] = TP::load(p[e0 + v]);
            const float ri = rfac[row], rri = rrfac[row];
            const float cj = cfac[bb * C + j], crj = crfac[bb * C + j];
            const float u = ((ri * cj) * TG::load(g[e0 + v])) / clip;
            const float mold = F32ST ? st_m(t)[e0 + v] : float(mq[e0 + v]) * scale;
            m[v] = fmaf(u, hp.a1, mold * hp.b1);
            pv[v] = param_update<TP>(pv[v], (rri * crj) * m[v], hp);
          } else {
            m[v] = 0.0f;
            pv[v] = 0.0f;
          }
          if (++j == C) {
            j = 0;
            ++row;
            if (++i == R) {
              i = 0;
              ++bb;
            }
          }
        }
      } else {
#pragma unroll
        for (int v = 0; v < 8; ++v) m[v] = pv[v] = 0.0f;
      }
      if constexpr (F32ST) {
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          if (e0 + v < N) {
            st_m(t)[e0 + v] = m[v];
            p[e0 + v] = TP::store(pv[v]);
          }
        }
        continue;
      }
      uint32_t abits = 0;
#pragma unroll
      for (int v = 0; v < 8; ++v) abits = max(abits, abs_bits(m[v]));
      abits = block_max_bits(abits, L, wmax, par);
      const float amax = fix_absmax(__uint_as_float(abits));
      if (e0 < N) {
        if ((e0 & (hp.B - 1)) == 0) ma[blk] = amax;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          if (e0 + v < N) {
            mq[e0 + v] = quant_s8(m[v], amax);
            p[e0 + v] = TP::store(pv[v]);
          }
        }
      }
    }
  }
}

// ===========================================================================
// P3, band form: rows stream through a workgroup that keeps its columns' factors in registers
// ===========================================================================
// For tensors whose rows start quantisation blocks (B divides C; B a power of two in [8, 2048]) and
// whose buffers are 16-byte aligned.  A work item is (matrix, band of p3_rb rows, column segment
// of whole blocks, at most 2048 columns); thread t owns 8 consecutive columns of the segment, loads
// their c and cr factors once, and walks the band's rows with the next row's loads in flight.
// The arithmetic is p3_math8 / p3_quant8, as in the tile kernel.

// 8 consecutive elements of type T kept as raw 32-bit words until used
template <typename T>
struct Raw8 {
  static constexpr int NWD = int(sizeof(typename T::storage)) * 2;
  uint32_t w[NWD];
  // NT: the nontemporal hint, for a 16-byte load per lane whose wavefront covers whole lines
  template <bool NT = (NWD == 4)>
  __device__ __forceinline__ void load(const CAME8_GLOBAL typename T::storage* __restrict__ p) {
    const CAME8_GLOBAL u32x4* q = (const CAME8_GLOBAL u32x4*)p;
#pragma unroll
    for (int i = 0; i < NWD / 4; ++i) {
      const u32x4 r = NT ? ld_nt(q + i) : q[i];
      w[4 * i] = r.x; w[4 * i + 1] = r.y; w[4 * i + 2] = r.z; w[4 * i + 3] = r.w;
    }
  }
  __device__ __forceinline__ float operator[](int v) const { return T::elem(w, v); }
};

template <typename TP, typename TG, bool F32ST>
__global__ __launch_bounds__(kThreads) void k_fact_pass3b(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                          const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using PS = typename TP::storage;
  using GS = typename TG::storage;
  __shared__ uint32_t wmax[2][4];
  const int tid = threadIdx.x;
  const int L = hp.B >> 3;  // lanes per block
  int par = 0;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t R = t.R, C = t.C;
    const int64_t nseg = t.p3_nseg;
    const int64_t local = w - wstart[slot];
    const int64_t per_mat = t.p3_nbands * nseg;
    const int64_t b = local / per_mat;
    const int64_t rem = local - b * per_mat;
    const int64_t band = rem / nseg, seg = rem - band * nseg;
    const int64_t r0 = band * t.p3_rb;
    const int64_t r1 = (r0 + t.p3_rb < R) ? (r0 + t.p3_rb) : R;
    const int64_t bpr = C >> hp.log2B;  // blocks per row
    const int64_t blk0 = seg * bpr / nseg, blk1 = (seg + 1) * bpr / nseg;
    const bool active = tid < (blk1 - blk0) * L;
    const int64_t col = (blk0 << hp.log2B) + int64_t(tid) * 8;
    const int64_t cblk = blk0 + (tid >> (hp.log2B - 3));  // this thread's block within a row

    CAME8_GLOBAL PS* __restrict__ p = gbl(static_cast<PS*>(t.p));
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g));
    CAME8_GLOBAL int8_t* __restrict__ mq = gbl(t.mq);
    CAME8_GLOBAL float* __restrict__ ma = gbl(t.ma);
    const CAME8_GLOBAL float* __restrict__ rfac = gbl(t.rfac);
    const CAME8_GLOBAL float* __restrict__ rrfac = gbl(t.rrfac);
    const float clip = uniform_f32(t.clip[0]), crcp = uniform_f32(t.clip[1]);
    const bool clip_fast = crcp == crcp;

    float cj[8], crj[8];
    if (active) {
      load8<F32>(gbl(t.cfac) + b * C + col, cj);
      load8<F32>(gbl(t.crfac) + b * C + col, crj);
    }
    using MB = typename std::conditional<F32ST, M32Chunk<8>, CodeChunk<8>>::type;
    Raw8<TG> gA, gB;
    Raw8<TP> pA, pB;
    MB qA, qB;
    float aA = 0.0f, aB = 0.0f;
    auto load_row = [&](int64_t r, Raw8<TG>& gr, Raw8<TP>& pr, MB& qr, float& am) {
      const int64_t e = (b * R + r) * C + col;
      gr.load(g + e);
      pr.load(p + e);
      if constexpr (F32ST) {
        qr.load(gbl(st_m(t)) + e);
      } else {
        qr.load(mq + e);
        am = ma[(b * R + r) * bpr + cblk];
      }
    };
    auto do_row = [&](int64_t r, const Raw8<TG>& gr, const Raw8<TP>& pr, const MB& qr, float am) {
      const int64_t row = b * R + r;
      const float ri = uniform_f32(rfac[row]), rri = uniform_f32(rrfac[row]);
      float m[8], pv[8];
      uint32_t abits = 0;
      if (active) {
        float gv[8], q[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          gv[v] = gr[v];
          q[v] = qr.mold(v, 1.0f);  // the code itself, or the fp32 momentum
          pv[v] = pr[v];
        }
        p3_math8<TP, F32ST>(gv, q, pv, m, am, ri, rri, cj, crj, clip, crcp, clip_fast, hp);
        if constexpr (F32ST) {
          const int64_t e = row * C + col;
          store8<TP>(p + e, pv);
          store8<F32>(gbl(st_m(t)) + e, m);
          return;
        }
#pragma unroll
        for (int v = 0; v < 8; ++v) abits = max(abits, abs_bits(m[v]));
      }
      if constexpr (F32ST) return;
      abits = block_max_bits(abits, L, wmax, par);
      if (active) {
        const int64_t e = row * C + col;
        store8<TP>(p + e, pv);
        const float amax = fix_absmax(__uint_as_float(abits));
        if ((tid & (L - 1)) == 0) ma[row * bpr + cblk] = amax;
        st_nt((CAME8_GLOBAL u32x2*)(mq + e), p3_quant8(m, amax, abits));
      }
    };
    if (active) load_row(r0, gA, pA, qA, aA);
    for (int64_t r = r0; r < r1; r += 2) {
      if (active && r + 1 < r1) load_row(r + 1, gB, pB, qB, aB);
      do_row(r, gA, pA, qA, aA);
      if (r + 1 < r1) {
        if (active && r + 2 < r1) load_row(r + 2, gA, pA, qA, aA);
        do_row(r + 1, gB, pB, qB, aB);
      }
    }
  }
}

// ===========================================================================
// 1-D tensors, pass B: v, u/clip, m, parameter write, requantisation
// ===========================================================================
template <typename TP, typename TG>
__global__ __launch_bounds__(kThreads) void k_vec_passB(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                        const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using PS = typename TP::storage;
  __shared__ float wmax[2][2][4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int L = hp.B >> 3;
  int par = 0;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t tile = w - wstart[slot];
    const int64_t e0 = tile * kTile + int64_t(tid) * 8;
    const int64_t N = t.N;
    PS* __restrict__ p = static_cast<PS*>(t.p);
    const float clip = t.clip[0];
    float m[8], vv[8], pv[8];
    {
      int64_t ec[8];
      float gv[8], vo[8], mo[8], po[8];
      vec_load8<TG>(t, e0, hp, ec, gv, vo);
#pragma unroll
      for (int v = 0; v < 8; ++v) po[v] = TP::load(p[ec[v]]);
      if (t.fp32st) {
#pragma unroll
        for (int v = 0; v < 8; ++v) mo[v] = st_m(t)[ec[v]];
      } else {
#pragma unroll
        for (int v = 0; v < 8; ++v) mo[v] = deq_s8(t.mq[ec[v]], t.ma[blk_of(ec[v], hp)]);
      }
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        if (e0 + v < N) {
          vv[v] = vec_v_from(gv[v], vo[v], hp);
          float uu = rsqrt_ref(vv[v]) * gv[v];
          if ((hp.fp16u || t.fp16u) && !t.fp32st) uu = round_f16(uu);
          const float u = uu / clip;
          m[v] = fmaf(u, hp.a1, mo[v] * hp.b1);
          pv[v] = param_update<TP>(po[v], m[v], hp);
        } else {
          m[v] = 0.0f;
          vv[v] = 0.0f;
        }
      }
    }
    if (t.fp32st) {  // fp32 states: store the values (uniform per work item)
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int64_t e = e0 + v;
        if (e < N) {
          st_m(t)[e] = m[v];
          st_sq_row(t)[e] = vv[v];
          p[e] = TP::store(pv[v]);
        }
      }
      continue;
    }
    float am = 0.0f, av = 0.0f;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      am = nan_max(am, fabsf(m[v]));
      av = nan_max(av, vv[v]);
    }
    if (L <= 64) {
      am = group_max_rt(am, L);
      av = group_max_rt(av, L);
    } else {
      am = group_max<64>(am);
      av = group_max<64>(av);
      if (lane == 0) {
        wmax[par][0][wid] = am;
        wmax[par][1][wid] = av;
      }
      __syncthreads();
      const int wpb = L >> 6;
      const int w0 = (wid / wpb) * wpb;
      am = wmax[par][0][w0];
      av = wmax[par][1][w0];
      for (int k = 1; k < wpb; ++k) {
        am = nan_max(am, wmax[par][0][w0 + k]);
        av = nan_max(av, wmax[par][1][w0 + k]);
      }
      par ^= 1;
    }
    am = fix_absmax(am);
    av = fix_absmax(av);
    const float amr = rcp_for_div(am), avr = rcp_for_div(av);
    if (e0 < N && ((e0 & (hp.B - 1)) == 0)) {
      t.ma[blk_of(e0, hp)] = am;
      t.ra[blk_of(e0, hp)] = av;
    }
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int64_t e = e0 + v;
      if (e < N) {
        t.mq[e] = quant_s8_r(m[v], am, amr);
        t.rq[e] = quant_u8_r(vv[v], av, avr);
        p[e] = TP::store(pv[v]);
      }
    }
  }
}

// ===========================================================================
// Generic block-size fallback for P3 / B: one workgroup per quantisation
// block, any block size.  Values are recomputed in a second sweep after the
// block absmax is known.
// ===========================================================================
template <typename TG>
__device__ __forceinline__ float m_new_fact(const DevTensor& t, int64_t e, float clip, const Hp& hp) {
  float uu = u_at<TG>(t, e, hp);
  if ((hp.fp16u || t.fp16u) && !t.factored) uu = round_f16(uu);
  const float u = uu / clip;
  return fmaf(u, hp.a1, deq_s8(t.mq[e], t.ma[mblk(t, e, hp)]) * hp.b1);
}

template <typename TP, typename TG>
__global__ __launch_bounds__(kThreads) void k_generic_update(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                             const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using PS = typename TP::storage;
  __shared__ float wm[2][4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t blk = w - wstart[slot];
    int64_t i0, i1;
    if (t.pm) {  // block jb of matrix mb
      const int64_t rc = t.R * t.C, mb = blk / t.pmb_m, jb = blk - mb * t.pmb_m;
      i0 = mb * rc + jb * hp.B;
      i1 = (jb * hp.B + hp.B < rc) ? (i0 + hp.B) : (mb * rc + rc);
    } else {
      i0 = blk * hp.B;
      i1 = (i0 + hp.B < t.N) ? (i0 + hp.B) : t.N;
    }
    const float clip = t.clip[0];
    const typename TG::storage* __restrict__ g = static_cast<const typename TG::storage*>(t.g);
    PS* __restrict__ p = static_cast<PS*>(t.p);
    // sweep 1: block absmax of the new momentum (and of the new 1-D second moment)
    float am = 0.0f, av = 0.0f;
    for (int64_t e = i0 + tid; e < i1; e += kThreads) {
      am = nan_max(am, fabsf(m_new_fact<TG>(t, e, clip, hp)));
      if (!t.factored) av = nan_max(av, vec_v_new<TG>(t, e, TG::load(g[e]), hp));
    }
    am = group_max<64>(am);
    av = group_max<64>(av);
    if (lane == 0) {
      wm[0][wid] = am;
      wm[1][wid] = av;
    }
    __syncthreads();
    am = fix_absmax(nan_max(nan_max(wm[0][0], wm[0][1]), nan_max(wm[0][2], wm[0][3])));
    av = fix_absmax(nan_max(nan_max(wm[1][0], wm[1][1]), nan_max(wm[1][2], wm[1][3])));
    // sweep 2: each element is recomputed from its old codes and rewritten by the same
    // thread; the old block scales are overwritten only after the barrier below
    for (int64_t e = i0 + tid; e < i1; e += kThreads) {
      const float m = m_new_fact<TG>(t, e, clip, hp);
      float step;
      if (t.factored) {
        const int64_t row = e / t.C;
        const int64_t j = e - row * t.C;
        const int64_t b = row / t.R;
        step = (t.rrfac[row] * t.crfac[b * t.C + j]) * m;
      } else {
        step = m;
        t.rq[e] = quant_u8(vec_v_new<TG>(t, e, TG::load(g[e]), hp), av);
      }
      p[e] = TP::store(param_update<TP>(TP::load(p[e]), step, hp));
      t.mq[e] = quant_s8(m, am);
    }
    __syncthreads();
    if (tid == 0) {
      t.ma[blk] = am;
      if (!t.factored) t.ra[blk] = av;
    }
    __syncthreads();
  }
}

// ===========================================================================
// 8bit2d layout: momentum quantised in 16x16 tiles (reference CAME8bit2D; arithmetic order of
// came_kernels.cu:2584-2684, 2685-2780, 3333-3367)
// ===========================================================================
constexpr int kTile2 = 16;
constexpr int kParam2Groups = 4;                    // 8-element groups per thread of the vector parameter write
constexpr int kParam2Items = kParam2Groups * kTile;  // elements per work item of the vector parameter write
constexpr int kParam2BandRows = 32;  // rows per work item of the band form of the parameter write

// one element of the momentum pass from its clipped update u = (g*r)*c / clip:
// m = m_old*b1 + u*(1-b1); res = (u - m)^2 + eps1
__device__ __forceinline__ void m2d_from_u(float u, float mold, const Hp& hp, float& m, float& res) {
  const float mn = (mold * hp.b1) + (u * hp.a1f);
  const float d = u - mn;
  m = mn;
  res = (d * d) + hp.eps1;
}
__device__ __forceinline__ void m2d_elem(float gv, float ri, float cj, float clip, float mold, const Hp& hp, float& m,
                                         float& res) {
  const float u = ((gv * ri) * cj) / clip;
  const float mn = (mold * hp.b1) + (u * hp.a1f);
  const float d = u - mn;
  m = mn;
  res = (d * d) + hp.eps1;
}

// residual row state of one row from its sum over the tiles: RR_old*b3 + (1-b3)*(sum/C)
__device__ __forceinline__ float rr2d_new(const DevTensor& t, int64_t row, float sum, const Hp& hp) {
  const float old = deq_u8(gbl(t.rrq)[row], gbl(t.rra)[blk_of(row, hp)]);
  return (old * hp.b3) + (hp.a3f * (sum / float(t.C)));
}

// Momentum pass, vector form (C a multiple of 16; gradient and codes 16-byte aligned).  Work item =
// (tensor, tile row ty): rows [16*ty, +16) across all columns, 16 tiles at a time.  Lane l of wave w
// holds row l%16 of tile 4*w + l/16 of the chunk: 16 consecutive elements, loaded as vectors.  Per
// tile: the absmax of the new momentum (a max over the tile's 16 lanes, 0 -> 1) and its int8
// codes; each tile row's residual sum (in-lane, columns in order) and each tile column's (rows in
// order, through LDS, written to t2col[ty*C + col]).  The rows' tile sums are added in tile order
// chunk by chunk; at the end of the item come the residual row states and their sum over the
// item's rows (rrsum[ty]).  An inactive lane (a row or tile past the edge) carries zeros.
template <typename TG>
__global__ __launch_bounds__(kThreads) void k_2d_rows(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                      const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using GS = typename TG::storage;
  __shared__ float xres[4][kWave][kTile2 + 1];  // per wave: 4 tiles x 16 rows x 16 residuals (+1: banks)
  __shared__ __align__(16) float rpart[kTile2][kTile2];  // [row][tile of the chunk]: each tile row's residual sum
  __shared__ float racc[kTile2];                // running row sums, tiles in order
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int i = lane & (kTile2 - 1), s = lane >> 4;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t R = t.R, C = t.C, tc = t.tc;
    const int64_t ty = w - wstart[slot];
    const int64_t r0 = ty * kTile2;
    const int nrows = int((R - r0) < kTile2 ? (R - r0) : kTile2);
    const bool rvalid = i < nrows;
    const int64_t row = r0 + (rvalid ? i : 0);
    const CAME8_GLOBAL GS* __restrict__ grow = gbl(static_cast<const GS*>(t.g) + row * C);
    CAME8_GLOBAL int8_t* __restrict__ qrow = gbl(t.mq + row * C);
    const CAME8_GLOBAL float* __restrict__ cf = gbl(static_cast<const float*>(t.cfac));
    CAME8_GLOBAL float* __restrict__ ma = gbl(t.ma + ty * tc);
    // global (not generic) stores: a generic store also counts in the LDS counter, and the wait for
    // the LDS writes before each barrier would then wait for the store to reach memory
    CAME8_GLOBAL float* __restrict__ t2col = gbl(t.t2col + ty * C);
    const float clip = uniform_f32(t.clip[0]), crcp = uniform_f32(t.clip[1]);
    const bool clip_fast = crcp == crcp;  // the reciprocal division serves this divisor
    const float ri = gbl(t.rfac)[row];
    if (tid < kTile2) racc[tid] = 0.0f;
    for (int64_t tx0 = 0; tx0 < tc; tx0 += kTile2) {
      const int64_t tx = tx0 + wid * 4 + s;
      const bool tvalid = tx < tc;
      const bool act = tvalid && rvalid;
      const int64_t c0 = tx * kTile2;
      // m is set and read only on active lanes, and only active lanes write their residuals to LDS:
      // the reads below stop at the block's rows and tiles, so an inactive lane's slots are never read
      float m[kTile2];
      // the tile's largest |m| as bits, from the largest signed and unsigned raw bits: a max over
      // the nonnegative elements and one over the negative elements' magnitudes (or both over the
      // nonnegative ones)
      int32_t smax = 0;
      uint32_t umax = 0;
      if (act) {
        Raw8<TG> ga, gb;
        // plain loads and stores: a lane's 32 bytes of gradient come in two instructions, and a
        // wavefront's codes are 64 bytes of each of 16 rows
        ga.template load<false>(grow + c0);
        gb.template load<false>(grow + c0 + 8);
        const u32x4 q = *(const CAME8_GLOBAL u32x4*)(qrow + c0);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        const float am_old = ma[tx];
        // u = (g*r)*c / clip: the reciprocal division where it gives the quotient exactly (every
        // numerator of the chunk zero or in its range), else the IEEE division element by element
        float u[kTile2];
        DivGuard gd;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const f32x4 c4 = *(const CAME8_GLOBAL f32x4*)(cf + c0 + 4 * k);
          const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int j = 4 * k + v;
            u[j] = ((j < 8 ? ga[j] : gb[j - 8]) * ri) * cv[v];
            gd.add(u[j]);
          }
        }
        if (__builtin_expect(clip_fast && gd.fast(), 1)) {
#pragma unroll
          for (int j = 0; j < kTile2; ++j) u[j] = div_fast(u[j], clip, crcp);
        } else {
#pragma unroll
          for (int j = 0; j < kTile2; ++j)
            u[j] = (clip_fast && !div_exact_needed(u[j])) ? div_fast(u[j], clip, crcp) : u[j] / clip;
        }
        // the guard `am_old > 0 ? code*scale : 0` folded into the scale: code*0 is a zero too (its sign
        // can differ, which changes no code, sum or parameter)
        // (after the loads: scale_s8's rare branch would make the column-factor loads wait for am_old)
        const float sc_old = am_old > 0.0f ? scale_s8(am_old) : 0.0f;
        float rsum = 0.0f;
#pragma unroll
        for (int j = 0; j < kTile2; ++j) {
          const float mold = code_elem(qw, j) * sc_old;
          float res;
          m2d_from_u(u[j], mold, hp, m[j], res);
          smax = max(smax, int32_t(__float_as_uint(m[j])));
          umax = max(umax, __float_as_uint(m[j]));
          rsum += res;
          xres[wid][lane][j] = res;
        }
        rpart[i][wid * 4 + s] = rsum;
      }
      // the tile's 16 rows are 16 consecutive lanes
      const uint32_t abits = group_max_bits<kTile2>(max(uint32_t(smax), umax & 0x7fffffffu));
      if (act) {
        const float amax = fix_absmax(__uint_as_float(abits));
        const float inv = 1.0f / amax;
        uint32_t ow[4];
        if (__builtin_expect(abits <= 0x7f7fffffu && inv <= 0x1.fffffep127f, 1)) {
          // no infinity or NaN in the tile and a finite reciprocal
#pragma unroll
          for (int k = 0; k < 4; ++k) ow[k] = quant_s8_inv4(m + 4 * k, inv);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            uint32_t wv = 0;
#pragma unroll
            for (int v = 0; v < 4; ++v) wv |= uint32_t(uint8_t(quant_s8_inv(m[4 * k + v], inv))) << (8 * v);
            ow[k] = wv;
          }
        }
        *(CAME8_GLOBAL u32x4*)(qrow + c0) = u32x4{ow[0], ow[1], ow[2], ow[3]};
        if (i == 0) ma[tx] = amax;
      }
      __syncthreads();
      if (tvalid) {  // lane (s, i): column i of its tile, the block's rows in order
        float cs = 0.0f;
        if (nrows == kTile2) {
#pragma unroll
          for (int k = 0; k < kTile2; ++k) cs += xres[wid][s * kTile2 + k][i];
        } else {
          for (int k = 0; k < nrows; ++k) cs += xres[wid][s * kTile2 + k][i];
        }
        t2col[c0 + i] = cs;
      }
      if (tid < nrows) {  // row tid's tile sums of the chunk, tiles in order
        float a = racc[tid];
        const int64_t nt = (tc - tx0) < kTile2 ? (tc - tx0) : kTile2;
        if (nt == kTile2) {
          const f32x4* rp = reinterpret_cast<const f32x4*>(&rpart[tid][0]);
#pragma unroll
          for (int k = 0; k < kTile2 / 4; ++k) {
            const f32x4 v = rp[k];
            a = (((a + v.x) + v.y) + v.z) + v.w;
          }
        } else {
          for (int64_t k = 0; k < nt; ++k) a += rpart[tid][k];
        }
        racc[tid] = a;
      }
      __syncthreads();
    }
    if (tid < nrows) {
      const float v = rr2d_new(t, r0 + tid, racc[tid], hp);
      gbl(t.RRn)[r0 + tid] = v;
      racc[tid] = v;
    }
    __syncthreads();
    if (tid == 0) {
      double sum = 0.0;
      for (int k = 0; k < nrows; ++k) sum += racc[k];
      gbl(t.rrsum)[ty] = float(sum);
    }
    __syncthreads();  // racc / LDS reused by the next item
  }
}

// Momentum pass, scalar form (any C and alignment).  Work item = (tensor, tile row ty, group of 256
// columns); wave w owns columns [256*cg + 64*w, +64) of the tile row's 16 rows, one column per lane,
// so a tile is 16 lanes of one wave.  The same per-element arithmetic and tile codes as the vector
// form; each tile's residual sums per column go to t2col[ty*C + col] and per row to
// t2row[row*tc + tx], which k_2d_res_rows then adds in tile order.
template <typename TG>
__global__ __launch_bounds__(kThreads) void k_2d_tiles(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                       const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using GS = typename TG::storage;
  __shared__ float lres[4][kTile2][kWave + 1];  // +1: rows of a tile fall in different banks
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t R = t.R, C = t.C;
    const int64_t ncg = (C + 255) / 256;
    const int64_t local = w - wstart[slot];
    const int64_t ty = local / ncg, cg = local - ty * ncg;
    const int64_t r0 = ty * kTile2;
    const int nrows = int((R - r0) < kTile2 ? (R - r0) : kTile2);
    const int64_t col = cg * 256 + int64_t(wid) * kWave + lane;
    const bool cvalid = col < C;
    const int64_t tile = ty * t.tc + (col >> 4);
    const CAME8_GLOBAL GS* __restrict__ g = gbl(static_cast<const GS*>(t.g));
    CAME8_GLOBAL int8_t* __restrict__ mq = gbl(t.mq);
    const float clip = uniform_f32(t.clip[0]);
    const float cj = cvalid ? t.cfac[col] : 0.0f;
    const float am_old = cvalid ? t.ma[tile] : 0.0f;
    const float sc_old = am_old / kSignedQ;
    float m[kTile2], res[kTile2];
    uint32_t abits = 0;
#pragma unroll
    for (int i = 0; i < kTile2; ++i) {
      m[i] = 0.0f;
      res[i] = 0.0f;
      if (i < nrows && cvalid) {
        const int64_t e = (r0 + i) * C + col;
        const float mold = am_old > 0.0f ? float(mq[e]) * sc_old : 0.0f;
        m2d_elem(TG::load(g[e]), t.rfac[r0 + i], cj, clip, mold, hp, m[i], res[i]);
      }
      abits = max(abits, abs_bits(m[i]));
    }
    abits = group_max_bits<kTile2>(abits);
    const float amax = fix_absmax(__uint_as_float(abits));
    const float inv = 1.0f / amax;
    if (cvalid) {
      if ((lane & (kTile2 - 1)) == 0) t.ma[tile] = amax;
      float csum = 0.0f;
#pragma unroll
      for (int i = 0; i < kTile2; ++i) {
        if (i < nrows) mq[(r0 + i) * C + col] = quant_s8_inv(m[i], inv);
        csum += res[i];
      }
      t.t2col[ty * C + col] = csum;
    }
    // per-row sums of each tile: the 16 columns in order, through LDS
#pragma unroll
    for (int i = 0; i < kTile2; ++i) lres[wid][i][lane] = res[i];
    __syncthreads();
    {
      const int i = lane & (kTile2 - 1), k = lane >> 4;
      const int64_t c0 = cg * 256 + int64_t(wid) * kWave + k * kTile2;
      float rsum = 0.0f;
#pragma unroll
      for (int j = 0; j < kTile2; ++j) rsum += lres[wid][i][k * kTile2 + j];
      if (i < nrows && c0 < C) t.t2row[(r0 + i) * t.tc + (c0 >> 4)] = rsum;
    }
    __syncthreads();  // lres is reused by the next work item
  }
}

// Residual row states after the scalar momentum pass.  Work item = (tensor, tile row ty): each of its
// rows' sum over the tiles in order, the new state, and the states' sum over the rows (rrsum[ty]).
template <int = 0>  // a template only so that every translation unit may include this header
__global__ __launch_bounds__(kThreads) void k_2d_res_rows(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                          const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  __shared__ float rowval[kTile2];
  const int tid = threadIdx.x;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t ty = w - wstart[slot];
    const int64_t r0 = ty * kTile2;
    const int nrows = int((t.R - r0) < kTile2 ? (t.R - r0) : kTile2);
    if (tid < nrows) {
      const int64_t row = r0 + tid;
      float s = 0.0f;
      for (int64_t tx = 0; tx < t.tc; ++tx) s += t.t2row[row * t.tc + tx];
      const float v = rr2d_new(t, row, s, hp);
      t.RRn[row] = v;
      rowval[tid] = v;
    }
    __syncthreads();
    if (tid == 0) {
      double s = 0.0;
      for (int k = 0; k < nrows; ++k) s += rowval[k];
      t.rrsum[ty] = float(s);
    }
    __syncthreads();
  }
}

// parameter write of one element: p <- round(p * (1 - lr*wd)) when wd != 0 (the reference does this
// in its momentum pass; nothing reads p in between), then p <- round(p - lr*((m_q*rr)*cr)), one
// fused multiply-add, m_q = code * (tile absmax / 127)
template <typename TP>
__device__ __forceinline__ float p2d_new(float pv, float code, float sc, float rr, float cr, const Hp& hp) {
  if (hp.wd) pv = TP::load(TP::store(pv * hp.wdfac));
  const float step = ((code * sc) * rr) * cr;
  return fmaf(step, hp.alr, pv);
}

// Parameter write, vector form (C a multiple of 16; parameter and codes 16-byte aligned).  A thread
// takes kParam2Groups groups of 8 consecutive elements (half a tile row each), kTile elements apart,
// and issues the loads of all its groups before the first arithmetic, so that one memory round
// trip serves kParam2Items elements per workgroup.  A group past the end loads the tensor's last
// group instead and stores nothing.
template <typename TP>
__global__ __launch_bounds__(kThreads) void k_2d_param_v(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using PS = typename TP::storage;
  constexpr int G = kParam2Groups;
  const int tid = threadIdx.x;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t base = (w - wstart[slot]) * kParam2Items + int64_t(tid) * 8;
    CAME8_GLOBAL PS* __restrict__ p = gbl(static_cast<PS*>(t.p));
    const CAME8_GLOBAL int8_t* __restrict__ mq = gbl(t.mq);
    const CAME8_GLOBAL float* __restrict__ ma = gbl(t.ma);
    const CAME8_GLOBAL float* __restrict__ rrfac = gbl(t.rrfac);
    const CAME8_GLOBAL float* __restrict__ crfac = gbl(static_cast<const float*>(t.crfac));
    Raw8<TP> praw[G];
    u32x2 q[G];
    float am[G], rr[G], cr[G][8];
    bool ok[G];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int64_t e = base + int64_t(gi) * kTile;
      ok[gi] = e < t.N;
      const int64_t el = ok[gi] ? e : t.N - 8;
      const int64_t row = t.idx32 ? int64_t(udiv_magic(uint32_t(el), t.mC, t.sC)) : el / t.C;
      const int64_t c0 = el - row * t.C;
      praw[gi].load(p + el);
      q[gi] = ld_nt((const CAME8_GLOBAL u32x2*)(mq + el));
      am[gi] = ma[(row >> 4) * t.tc + (c0 >> 4)];
      rr[gi] = rrfac[row];
      load8<F32>(crfac + c0, cr[gi]);
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      if (!ok[gi]) continue;
      const int64_t e = base + int64_t(gi) * kTile;
      const uint32_t qw[2] = {q[gi].x, q[gi].y};
      const float sc = am[gi] / kSignedQ;
      float pv[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) pv[v] = p2d_new<TP>(praw[gi][v], code_elem(qw, v), sc, rr[gi], cr[gi][v], hp);
      store8<TP>(p + e, pv);
    }
  }
}

// Parameter write, band form (C a multiple of 16; parameter and codes 16-byte aligned).  A work item
// is (kParam2BandRows rows, a segment of at most kTile columns); thread t owns 8 columns (half a
// tile row), loads their residual column factors once and streams the rows with the next row's
// loads in flight.  The same arithmetic as k_2d_param_v.
template <typename TP>
__global__ __launch_bounds__(kThreads) void k_2d_param_b(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                         const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using PS = typename TP::storage;
  const int tid = threadIdx.x;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t R = t.R, C = t.C, tc = t.tc;
    const int64_t nseg = (C + kTile - 1) / kTile;
    const int64_t local = w - wstart[slot];
    const int64_t band = local / nseg, seg = local - band * nseg;
    const int64_t r0 = band * kParam2BandRows;
    const int64_t r1 = (r0 + kParam2BandRows < R) ? (r0 + kParam2BandRows) : R;
    const int64_t col = seg * kTile + int64_t(tid) * 8;
    if (col >= C) continue;  // no barrier below: idle lanes may leave the item
    CAME8_GLOBAL PS* __restrict__ p = gbl(static_cast<PS*>(t.p));
    const CAME8_GLOBAL int8_t* __restrict__ mq = gbl(t.mq);
    const CAME8_GLOBAL float* __restrict__ ma = gbl(t.ma) + (col >> 4);
    const CAME8_GLOBAL float* __restrict__ rrfac = gbl(t.rrfac);
    float cr[8];
    load8<F32>(gbl(static_cast<const float*>(t.crfac)) + col, cr);
    Raw8<TP> pA, pB;
    u32x2 qA, qB;
    float aA = 0.0f, aB = 0.0f, rA = 0.0f, rB = 0.0f;
    auto load_row = [&](int64_t r, Raw8<TP>& pr, u32x2& q, float& am, float& rr) {
      const int64_t e = r * C + col;
      pr.load(p + e);
      q = ld_nt((const CAME8_GLOBAL u32x2*)(mq + e));
      am = ma[(r >> 4) * tc];
      rr = rrfac[r];
    };
    auto do_row = [&](int64_t r, const Raw8<TP>& pr, const u32x2& q, float am, float rr) {
      const uint32_t qw[2] = {q.x, q.y};
      const float sc = am / kSignedQ;
      float pv[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) pv[v] = p2d_new<TP>(pr[v], code_elem(qw, v), sc, rr, cr[v], hp);
      store8<TP>(p + r * C + col, pv);
    };
    load_row(r0, pA, qA, aA, rA);
    for (int64_t r = r0; r < r1; r += 2) {
      if (r + 1 < r1) load_row(r + 1, pB, qB, aB, rB);
      do_row(r, pA, qA, aA, rA);
      if (r + 1 < r1) {
        if (r + 2 < r1) load_row(r + 2, pA, qA, aA, rA);
        do_row(r + 1, pB, qB, aB, rB);
      }
    }
  }
}

// Parameter write, scalar form (any C and alignment): 8 consecutive elements per thread, 2048 per item.
template <typename TP>
__global__ __launch_bounds__(kThreads) void k_2d_param(const DevTensor* __restrict__ T, const int32_t* __restrict__ tids,
                                                       const int64_t* __restrict__ wstart, int ntens, Hp hp) {
  using PS = typename TP::storage;
  const int tid = threadIdx.x;
  const int64_t total = wstart[ntens];
  for (int64_t w = blockIdx.x; w < total; w += gridDim.x) {
    const int slot = find_slot(wstart, ntens, w);
    const DevTensor& t = T[tids[slot]];
    const int64_t e0 = (w - wstart[slot]) * kTile + int64_t(tid) * 8;
    PS* __restrict__ p = static_cast<PS*>(t.p);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int64_t e = e0 + v;
      if (e < t.N) {
        const int64_t row = t.idx32 ? int64_t(udiv_magic(uint32_t(e), t.mC, t.sC)) : e / t.C;
        const int64_t col = e - row * t.C;
        const float sc = t.ma[(row >> 4) * t.tc + (col >> 4)] / kSignedQ;
        p[e] = TP::store(p2d_new<TP>(TP::load(p[e]), float(t.mq[e]), sc, t.rrfac[row], t.crfac[col], hp));
      }
    }
  }
}

// ===========================================================================
// standalone blockwise quantisation (fp32 -> int8/uint8 + absmax) and dequantisation
// ===========================================================================
template <bool SIGNED>
__global__ __launch_bounds__(kThreads) void k_quantize(const float* __restrict__ x, int64_t n, int32_t B, int64_t nblocks,
                                                       void* __restrict__ q, float* __restrict__ absmax) {
  __shared__ float wm[4];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  for (int64_t blk = blockIdx.x; blk < nblocks; blk += gridDim.x) {
    const int64_t i0 = blk * B;
    const int64_t i1 = (i0 + B < n) ? (i0 + B) : n;
    float a = (SIGNED || (i1 - i0) < B) ? 0.0f : -__builtin_inff();
    for (int64_t i = i0 + tid; i < i1; i += kThreads) a = nan_max(a, SIGNED ? fabsf(x[i]) : x[i]);
    a = group_max<64>(a);
    if (lane == 0) wm[wid] = a;
    __syncthreads();
    a = fix_absmax(nan_max(nan_max(wm[0], wm[1]), nan_max(wm[2], wm[3])));
    for (int64_t i = i0 + tid; i < i1; i += kThreads) {
      if (SIGNED) static_cast<int8_t*>(q)[i] = quant_s8(x[i], a);
      else static_cast<uint8_t*>(q)[i] = quant_u8(x[i], a);
    }
    if (tid == 0) absmax[blk] = a;
    __syncthreads();
  }
}

template <bool SIGNED>
__global__ __launch_bounds__(kThreads) void k_dequantize(const void* __restrict__ q, const float* __restrict__ absmax, int64_t n,
                                                         int32_t B, float* __restrict__ out) {
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < n; i += int64_t(gridDim.x) * kThreads) {
    const float a = absmax[i / B];
    out[i] = SIGNED ? deq_s8(static_cast<const int8_t*>(q)[i], a) : deq_u8(static_cast<const uint8_t*>(q)[i], a);
  }
}

}  // namespace came8
