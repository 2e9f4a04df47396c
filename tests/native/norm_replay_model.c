/*
 * CPU model of the library's replay of an fp32 fused-multiply-add chain s = fma(x, x, s), the
 * accumulation order of torch's CPU norm(2) (came_amd/csrc/came8_norm.h), written to check its
 * exactness argument against the serial chain on adversarial inputs.  Test infrastructure only.
 *
 * Segment records follow the kernel's rules: a segment holds 512 chain elements; lane l (64 lanes)
 * accounts elements 64q + l (q < 8) in an fp32 running sum of rint(x*x * 2^(23-E)) and the largest
 * |dh - rint(dh)|; a lane's value saturates at 2^24 for a tie (0.5), a sum of 2^24 or more (or NaN), or
 * a nonzero sum in the subnormal binade; the segment's value is the lanes' integer sum, at most 2^24.
 * The walk skips a segment whose record covers the chain's binade when m + value < 2^24 and replays
 * the others element by element.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int binade(float s) {
  uint32_t b;
  memcpy(&b, &s, 4);
  int e = (int)(b >> 23);
  return e == 0 ? -126 : e - 127;
}
static int est_binade(double v) {
  if (!(v > 0x1p-125)) return -126;
  if (!(v <= 0x1.fffffep127)) return 127;
  return binade((float)v);
}
static uint32_t seg_value(const float* x, int64_t k0, int64_t cnt, int E) {
  uint64_t tot = 0;
  for (int lane = 0; lane < 64; ++lane) {
    float sum = 0.0f, rmax = 0.0f;
    for (int q = 0; q < 8; ++q) {
      int64_t k = 64 * q + lane;
      if (k >= cnt) continue;
      float v = x[k0 + k];
      float hi = v * v;
      float dh = ldexpf(hi, 23 - E);
      float nf = rintf(dh);
      sum += nf;
      rmax = fmaxf(rmax, fabsf(dh - nf));
    }
    int bad = !(sum < 0x1p24f) || rmax == 0.5f || (E == -126 && sum != 0.0f);
    tot += bad ? (1u << 24) : (uint32_t)sum;
  }
  return tot > (1u << 24) ? (1u << 24) : (uint32_t)tot;
}

float chain_serial(const float* x, int64_t n) {
  float s = 0.0f;
  for (int64_t k = 0; k < n; ++k) s = fmaf(x[k], x[k], s);
  return s;
}

/* est[g]: estimated chain value at the start of segment g; returns the chain, *replays the count */
float chain_replay(const float* x, int64_t n, const double* est, int64_t* replays) {
  const int L = 512;
  int64_t nseg = (n + L - 1) / L;
  int* Ea = malloc(sizeof(int) * (nseg ? nseg : 1));
  int* two = malloc(sizeof(int) * (nseg ? nseg : 1));
  uint32_t* wa = malloc(sizeof(uint32_t) * (nseg ? nseg : 1));
  uint32_t* wb = malloc(sizeof(uint32_t) * (nseg ? nseg : 1));
  for (int64_t g = 0; g < nseg; ++g) {
    int64_t k0 = g * L, cnt = n - k0 < L ? n - k0 : L;
    Ea[g] = est_binade(est[g] * 0.875);
    two[g] = est_binade(est[g] * 1.015625) > Ea[g];
    wa[g] = seg_value(x, k0, cnt, Ea[g]);
    wb[g] = two[g] ? seg_value(x, k0, cnt, Ea[g] + 1) : (1u << 24);
  }
  float s = 0.0f;
  *replays = 0;
  for (int64_t g = 0; g < nseg && s == s; ++g) {
    int64_t k0 = g * L, cnt = n - k0 < L ? n - k0 : L;
    int ok = 0;
    if (s <= 0x1.fffffep127f) {
      int E = binade(s);
      uint32_t b;
      memcpy(&b, &s, 4);
      uint32_t m = b - ((uint32_t)(E + 126) << 23);
      uint32_t add = E == Ea[g] ? wa[g] : ((two[g] && E == Ea[g] + 1) ? wb[g] : (1u << 25));
      if ((uint64_t)m + add < (1u << 24)) {
        uint32_t r = ((uint32_t)(E + 126) << 23) + m + add;
        memcpy(&s, &r, 4);
        ok = 1;
      }
    } else if (wa[g] < (1u << 24) || (two[g] && wb[g] < (1u << 24))) {
      ok = 1; /* s = +inf and no element of the segment can be NaN */
    }
    if (!ok) {
      ++*replays;
      for (int64_t k = 0; k < cnt; ++k) s = fmaf(x[k0 + k], x[k0 + k], s);
    }
  }
  free(Ea);
  free(two);
  free(wa);
  free(wb);
  return s;
}
