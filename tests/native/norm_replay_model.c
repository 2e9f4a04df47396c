/*
 * CPU model of the library's replay of an fp32 fused-multiply-add chain s = fma(x, x, s), the
 * accumulation order of torch's CPU norm(2) (came_amd/csrc/came8_norm.h), written to check its
 * exactness argument against the serial chain on adversarial inputs.  Test infrastructure only.
 *
 * Segment records follow the kernel's rules: a segment holds 512 chain elements; lane l (64 lanes)
 * accounts elements 64q + l (q < 8) in an fp32 running sum of rint(x*x * 2^(23-E)) and the largest
 * |dh - rint(dh)|; a lane's value saturates at 2^24 for a tie (0.5), a sum of 2^24 or more (or NaN), or
 * a nonzero sum in the subnormal binade; the segment's value is the lanes' integer sum, at most 2^24.
 * In the subnormal binade (E = -126, unit 2^-149) an element |x| = 2^-75 also counts as a tie: its
 * square 2^-150 is half a unit, which x*x rounds to 0.
 * The walk skips a segment whose record covers the chain's binade when m + value < 2^24 and replays
 * the others.  A replay (segment_replay) follows the kernel's wavefront form: lane l holds the chain
 * elements 8l .. 8l + 7 of the segment; each round takes every element's integer increment under the
 * chain's current binade, a saturating prefix over lanes and elements, and the first element where the
 * prefix leaves the binade or the element is special; the elements before it are one integer add, that
 * element is one fmaf, and the next round starts after it.
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
      if (E == -126 && fabsf(v) == 0x1p-75f) rmax = 0.5f; /* x*x = 2^-150 rounds to 0 but is a tie */
    }
    int bad = !(sum < 0x1p24f) || rmax == 0.5f || (E == -126 && sum != 0.0f);
    tot += bad ? (1u << 24) : (uint32_t)sum;
  }
  return tot > (1u << 24) ? (1u << 24) : (uint32_t)tot;
}

#define SAT (1u << 25)
static uint32_t sat_add(uint32_t a, uint32_t b) {
  uint32_t v = a + b;
  return v < SAT ? v : SAT;
}
static float value_of(uint32_t m, int E) {
  uint32_t r = ((uint32_t)(E + 126) << 23) + m;
  float v;
  memcpy(&v, &r, 4);
  return v;
}

/* one segment of cnt <= 512 chain elements x[0 .. cnt) from s; *rounds counts the rounds */
float segment_replay(const float* x, int cnt, float s, int64_t* rounds) {
  int pos = 0;
  while (pos < cnt) {
    ++*rounds;
    if (!(s <= 0x1.fffffep127f)) { /* +inf or NaN: only a NaN element changes an infinite chain */
      if (s != s) break;
      int first = -1;
      for (int k = pos; k < cnt; ++k)
        if (x[k] != x[k]) { first = k; break; }
      if (first >= 0) s = fmaf(x[first], x[first], s);
      break;
    }
    const int E = binade(s);
    uint32_t b;
    memcpy(&b, &s, 4);
    const uint32_t m = b - ((uint32_t)(E + 126) << 23);
    const uint32_t room = (1u << 24) - m;
    uint32_t incl[512], run[64], excl[64];
    int special[512];
    for (int lane = 0; lane < 64; ++lane) {
      uint32_t r = 0;
      for (int j = 0; j < 8; ++j) {
        const int k = lane * 8 + j;
        const int live = k >= pos && k < cnt;
        const float v = k < cnt ? x[k] : 0.0f;
        const float h = v * v;
        const float dh = ldexpf(h, 23 - E);
        const float nf = rintf(dh);
        uint32_t n = nf < 0x1p25f ? (uint32_t)nf : SAT;
        special[k] = live && (fabsf(dh - nf) == 0.5f || (E == -126 && (nf != 0.0f || fabsf(v) == 0x1p-75f)));
        r = sat_add(r, live ? n : 0u);
        incl[k] = r;
      }
      run[lane] = r;
    }
    uint32_t acc = 0;
    for (int lane = 0; lane < 64; ++lane) {
      excl[lane] = acc;
      acc = sat_add(acc, run[lane]);
    }
    int ev = -1;
    for (int k = 0; k < 512 && ev < 0; ++k) {
      const int lane = k / 8;
      const int live = k >= pos && k < cnt;
      if (live && (special[k] || sat_add(excl[lane], incl[k]) >= room)) ev = k;
    }
    if (ev < 0) {
      s = value_of(m + acc, E);
      break;
    }
    const int lane = ev / 8, j = ev % 8;
    const uint32_t before = excl[lane] + (j > 0 ? incl[ev - 1] : 0u);
    s = value_of(m + before, E);
    s = fmaf(x[ev], x[ev], s);
    pos = ev + 1;
  }
  return s;
}

float chain_serial_from(const float* x, int64_t n, float s) {
  for (int64_t k = 0; k < n; ++k) s = fmaf(x[k], x[k], s);
  return s;
}

float chain_serial(const float* x, int64_t n) {
  float s = 0.0f;
  for (int64_t k = 0; k < n; ++k) s = fmaf(x[k], x[k], s);
  return s;
}

/* est[g]: estimated chain value at the start of segment g; returns the chain, *replays the count of
   replayed segments and *rounds the wavefront rounds they took */
float chain_replay_stats(const float* x, int64_t n, const double* est, int64_t* replays, int64_t* rounds) {
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
  *rounds = 0;
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
      s = segment_replay(x + k0, (int)cnt, s, rounds);
    }
  }
  free(Ea);
  free(two);
  free(wa);
  free(wb);
  return s;
}

float chain_replay(const float* x, int64_t n, const double* est, int64_t* replays) {
  int64_t rounds = 0;
  return chain_replay_stats(x, n, est, replays, &rounds);
}
