// libcame8: MI355X (gfx950) CAME 8-bit optimizer step behind a C ABI (include/came8.h).
//
// Host side: validates the tensor list, builds a launch plan (per-tensor
// descriptors with scratch pointers inside the caller's workspace, work lists
// grouped by kernel variant), uploads it into the head of the workspace when
// it changed, and enqueues the multi-tensor launch chain on the caller's
// stream.  No host synchronisation, no allocation, no memset.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <tuple>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/came8.h"
#include "came8_dispatch.h"
#include "came8_kernels.h"
#include "came8_norm.h"

using namespace came8;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x, size_t a = kAlign) { return (x + a - 1) / a * a; }
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// A launch of few bands leaves most CUs idle (one 2048x2048 matrix is 8 bands), and a launch whose
// bands fill the resident workgroups a little more than k times runs a (k+1)-th round almost empty.
// The bands of the tensors one band launch steps together are halved together (down to
// kMinShrunkBandRows rows, at most kMaxShrink times), to the size that minimises a schedule
// estimate of the launch (band_shrinks).
constexpr int64_t kMinShrunkBandRows = 8;
constexpr int kMaxShrink = 6;
constexpr int64_t kMinLaunchBands = 2048;  // without a device to ask: the least work items per launch
// Fixed time of a band (its start, its row sums, its partial stores), about 5 us, in elements the
// whole GPU streams meanwhile: a workgroup among `slots` spends it as kBandFixedElems / slots.
// (2e6 and 3.2e7 pick other shrinks on C2, C3 and C5 and measure within 1% of this value.)
constexpr double kBandFixedElems = 8.4e6;

// Rows per band: about 1M elements per workgroup work item, whole rows, at most 256 rows, divided by
// 2^shrink.  Every band writes one fp32 partial per column and statistic, which the factor kernels
// read back, so the band size sets that traffic (8-12 bytes per column per band).
int64_t band_rows(int64_t R, int64_t C, int shrink = 0) {
  int64_t rb = std::max<int64_t>(1, (int64_t(1) << 20) / std::max<int64_t>(C, 1));
  rb = std::min<int64_t>(rb, kMaxBandRows);
  rb = std::max<int64_t>(std::min<int64_t>(rb, kMinShrunkBandRows), rb >> shrink);
  return std::min<int64_t>(rb, R);
}


float round_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return f;
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

float round_to_f16(float f) { return float(_Float16(f)); }

// Kernel-variant keys.
struct BandKey {
  // st: fp32 states (pass 2), no column sums of g^2/R_i (pass 1: k_fact_pass1n); ua: rows of any
  // length/alignment; ms: rows wider than a sweep in column segments (pass 2, k_fact_pass1n)
  int gdt, V, K, TPB, st = 0, ua = 0, ms = 0;
  bool operator<(const BandKey& o) const {
    return std::tie(gdt, V, K, TPB, st, ua, ms) < std::tie(o.gdt, o.V, o.K, o.TPB, o.st, o.ua, o.ms);
  }
};
struct TypeKey {
  int pdt, gdt, st = 0;  // st: fp32 states
  bool operator<(const TypeKey& o) const { return std::tie(pdt, gdt, st) < std::tie(o.pdt, o.gdt, o.st); }
};

struct WorkList {
  std::vector<int32_t> tids;
  std::vector<int64_t> wstart;  // prefix of work items, size tids+1
  size_t tids_off = 0, wstart_off = 0;  // byte offsets inside the plan blob
  int64_t total() const { return wstart.empty() ? 0 : wstart.back(); }
};

struct Plan {
  std::vector<DevTensor> dev;
  std::map<BandKey, WorkList> band;      // P1 of the exact clip mode (factored tensors of the full8bit / fp32 layouts)
  std::map<BandKey, WorkList> bandN;     // P1 of the default clip mode, the same tensors (k_fact_pass1n; st = 1)
  std::map<BandKey, WorkList> band2dw;   // P1 of the 8bit2d tensors (both modes: their clip takes W)
  std::map<BandKey, WorkList> band2;     // P2 (factored tensors of the full8bit / fp32 layouts)
  std::map<int, WorkList> tiny1;         // P1 of tensors of tiny matrices (per 256 matrices), by grad type
  std::map<int, WorkList> tiny2;         // P2 of tensors of tiny matrices, by grad type
  std::map<TypeKey, WorkList> upd;       // P3, tile form (fast block sizes)
  std::map<TypeKey, WorkList> updb;      // P3, band form
  std::map<TypeKey, WorkList> vecB;      // 1-D pass B (fast block sizes)
  std::map<int, WorkList> vecA;          // 1-D pass A, by grad type
  std::map<int, WorkList> vecAn;         // the same for the default clip mode: tensors of several segments
  std::map<TypeKey, WorkList> generic;   // P3 / B for other block sizes (per quantisation block)
  // the clip's norm in the reference's order (came8_norm.h)
  WorkList nest_w;                       // unit estimates, a workgroup per row band (matrices >= 256 wide)
  WorkList nest_n;                       // unit estimates, a thread per unit (per 256 units)
  std::map<int, WorkList> nseg2d;        // segment records of matrices, runs of nrun segments, by 3 * grad type + form
  std::map<int, WorkList> nseg;          // the other segments' records, by 3 * grad type + chunk form
  WorkList nbsum;                        // the chains' sums per block of segments (one item per block)
  std::map<int, WorkList> nfix;          // records rebuilt under the chains' own estimates, by 3 * grad type + form
  std::map<int, WorkList> nwalk;         // chain walks (8 items per tensor), by grad type
  std::map<int, WorkList> nfinal;        // accumulators + tail + clip (one item per tensor), by grad type
  // The long-chain group (walk_split): factored tensors whose clip-norm chains are much longer than the
  // others'.  In the default norm mode their walk, clip and pass 2 run on the side stream, so that the
  // other tensors' pass 2 does not wait for the longest chain; band2 / tiny2 / nwalk / nfinal then hold
  // the other tensors only.
  bool walk_split = false;
  std::map<BandKey, WorkList> band2L;
  std::map<int, WorkList> tiny2L, nwalkL, nfinalL;
  WorkList factor;                       // F1b / F2b (per state block)
  std::map<int, WorkList> tiles2d_v;     // 8bit2d momentum pass, vector form (per tile row), by grad type
  std::map<int, WorkList> tiles2d;       // 8bit2d momentum pass, scalar form (per 16 rows x 256 columns)
  WorkList res2d;                        // 8bit2d residual row states after the scalar form (per tile row)
  std::map<int, WorkList> param2d_v;     // 8bit2d parameter write, vector form, by param type
  std::map<int, WorkList> param2d_b;     // 8bit2d parameter write, band form (rows >= 1024 wide)
  std::map<int, WorkList> param2d;       // 8bit2d parameter write, scalar form, by param type
  size_t plan_bytes = 0;
  size_t zero_off = 0;  // kZeroBytes of zeros inside the plan blob
  size_t total_bytes = 0;
  std::vector<uint8_t> blob;
};

void add_item(WorkList& wl, int32_t tid, int64_t count) {
  if (wl.wstart.empty()) wl.wstart.push_back(0);
  wl.tids.push_back(tid);
  wl.wstart.push_back(wl.wstart.back() + count);
}

bool fast_block(int B) { return B >= 8 && B <= kTile && (B & (B - 1)) == 0; }

// rows per work item of the band form of P3 (at most).  Measured on C4 / C2 pass 3: 4 rows 10.69 / 0.948 ms,
// 8 rows 10.37 / 0.923, 16 rows 10.48 / 0.948, 32 rows 10.55 (C4), 64 rows 10.90 (C4)
constexpr int kP3BandRows = 8;
constexpr int64_t kP3MinItems = 1024;  // band-form P3 work items wanted per launch (4 per CU)
constexpr int64_t kP3BandMinCols = 1024;  // narrower rows leave too many of a workgroup's lanes idle
// The clip-norm walk takes 12-17 ns per segment of a tensor's chain and runs serially along it; below
// this longest chain, the long-chain group's gain is less than its fork and join cost (20-50 us).
constexpr int64_t kWalkSplitMinSegs = 8192;

int log2_or_minus1(int B) {
  if (B <= 0 || (B & (B - 1)) != 0) return -1;
  int l = 0;
  while ((1 << l) < B) ++l;
  return l;
}

// Kernel shape of the band passes of a factored tensor: V elements per chunk (16 bytes of the
// gradient type when rows are 16-byte aligned and a chunk never straddles a quantisation block,
// else 1), K chunks per thread, TPB threads per workgroup.  `multiseg` when a row is wider than
// one sweep of the workgroup.
struct BandShapeSel {
  int V, K, TPB;
  bool multiseg;
  bool ua;  // vector chunks over rows that are not whole chunks or not aligned (V > 1, one sweep)
};

BandShapeSel band_variant(const came8_tensor& t, int64_t C, int32_t B, int pass, bool pm_m = false) {
  const int vw = t.grad_dtype == CAME8_F32 ? 4 : 8;
  // pm_m (pass 2): per-matrix momentum blocks that are not flat ones take the unaligned variant or V = 1,
  // whose block lookups handle them
  const bool aligned = !pm_m && (C % vw == 0) && (B % vw == 0) && (reinterpret_cast<uintptr_t>(t.grad) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(t.exp_avg_q) % vw == 0);
  BandShapeSel sel{aligned ? vw : 1, 0, 256, false, false};
  // other rows of at least vw elements take vector chunks with unaligned loads (a partial last chunk
  // re-reads the row's last vw elements), when one sweep of the widest shape covers them and a chunk
  // can straddle at most two quantisation blocks
  if (!aligned && C >= vw && B >= vw && C <= int64_t(512) * 4 * vw) {
    sel.V = vw;
    sel.ua = true;
  }
  const int64_t chunks = ceil_div(C, sel.V);
  // Rows of at most 256 vector chunks take 128-thread workgroups, two chunks a thread: a thread's
  // share of each row's sums then covers twice the elements, and a CU holds more workgroups (C2's
  // 1024-wide fp32 rows: pass 2 0.45 -> 0.40 ms).  Wider rows take 256-thread workgroups first: two of
  // them per CU keep one's barriers off the other's loads.  Pass 2 takes rows wider than one sweep in column segments (its MS variants, (3, 256) and, for
  // V = 1, (32, 256)), and for 16-bit gradients already rows wider than (3, 256) covers: it reads
  // each element once either way, and a 512-thread workgroup of its register use (~250) is alone
  // on its CU (C4's 11008-wide rows: 1.13 -> 1.03 ms).  Pass 1, whose column sums of g^2/R_i need
  // the whole row first, and the UA variants take the wider sweeps.
  static const int vec_k[][2] = {{1, 128}, {2, 128}, {2, 256}, {3, 256}, {2, 512}, {3, 512}, {4, 512}};
  static const int one_k[][2] = {{1, 256}, {2, 256}, {4, 256}, {8, 256}, {16, 256}, {32, 256}};
  const int (*cand)[2] = sel.V > 1 ? vec_k : one_k;
  const bool p2seg = pass == 2 && !sel.ua;
  const int nc = sel.V > 1 ? ((p2seg && sel.V == 8) ? 4 : 7) : 6;
  for (int i = 0; i < nc; ++i) {
    if (int64_t(cand[i][0]) * cand[i][1] >= chunks) {
      sel.K = cand[i][0];
      sel.TPB = cand[i][1];
      return sel;
    }
  }
  sel.K = p2seg ? (sel.V > 1 ? 3 : 32) : cand[nc - 1][0];
  sel.TPB = p2seg ? 256 : cand[nc - 1][1];
  sel.multiseg = true;
  return sel;
}

// magic multiplier and shift for n / d with n < 2^31 (floor(2^s / d) + 1, s = 32 + ceil(log2 d))
void magic_div(int64_t d, uint64_t& m, uint32_t& s) {
  uint32_t l = 0;
  while ((int64_t(1) << l) < d) ++l;
  s = 32 + l;
  m = uint64_t(((__uint128_t(1) << s) / uint64_t(d)) + 1);
}

// A factored tensor of the full8bit / fp32 layouts whose matrices are at most kTinyElems elements
// takes the thread-per-matrix passes.
bool tiny_matrix(const came8_tensor& t, bool s2d) {
  return t.factored && !s2d && t.rows >= 1 && t.cols >= 1 && t.rows * t.cols <= kTinyElems;
}

// The clip-norm estimate of a tensor takes a workgroup per row band (matrices at least a workgroup
// wide) rather than a thread per unit.
bool norm_est_wide(const came8_tensor& t, const DevTensor& d) {
  return t.factored && !tiny_matrix(t, false) && d.C >= kThreads;
}

BandFn band_fn(int gdt, bool pass2, int V, int K, int TPB, int st, int ua, int ms);

// The calling thread's current device, or -1 when no device answers (a host without a GPU).
int current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();  // leave no sticky error behind for the caller's next HIP call
    dev = -1;
  }
  return dev;
}

// Workgroups of kernel fn (tpb threads) resident on the current device at once: CUs times the
// workgroups one CU holds (registers, LDS).  0 when no device answers (sizing on a host without a
// GPU).  Cached per kernel and device.
int64_t resident_slots(const void* fn, int tpb) {
  static std::mutex mu;
  static std::map<std::tuple<const void*, int, int>, int64_t> cache;
  if (fn == nullptr) return 0;
  const int dev = current_device();
  std::lock_guard<std::mutex> lk(mu);
  const auto key = std::make_tuple(fn, tpb, dev);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int cus = 0, per_cu = 0;
  int64_t slots = 0;
  if (dev >= 0 && hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, tpb, 0) == hipSuccess)
    slots = int64_t(cus) * std::max(per_cu, 1);
  else
    (void)hipGetLastError();  // leave no sticky error behind for the caller's next HIP call
  cache[key] = slots;
  return slots;
}

// Finish time of work items of the given costs, started in order on `slots` workgroups, each item
// on the workgroup that frees first (how the hardware dispatches a grid of one item per workgroup).
double schedule_makespan(const std::vector<double>& cost, int64_t slots) {
  std::vector<double> heap;  // finish times, a min-heap
  heap.reserve(size_t(std::min<int64_t>(slots, int64_t(cost.size()))));
  double end = 0.0;
  for (const double c : cost) {
    double t0 = 0.0;
    if (int64_t(heap.size()) < slots) {
      heap.push_back(t0 + c);
      std::push_heap(heap.begin(), heap.end(), std::greater<double>());
    } else {
      std::pop_heap(heap.begin(), heap.end(), std::greater<double>());
      t0 = heap.back();
      heap.back() = t0 + c;
      std::push_heap(heap.begin(), heap.end(), std::greater<double>());
    }
    end = std::max(end, t0 + c);
  }
  return end;
}

// The 2^shrink of band_rows for every tensor.  Tensors that share a band-pass kernel variant (one
// launch) share a shrink: the one that minimises the estimated time of the launch's two passes --
// each band costs its elements plus its fixed time, scheduled on the workgroups that pass 1 and pass 2
// keep resident (a workgroup streams 1/slots of the GPU's rate) -- plus the factor kernels' reads of
// the per-band column partials (three fp32 arrays).  Without a device to ask, the least shrink that gives
// the launch kMinLaunchBands work items.
std::vector<int> band_shrinks(const came8_tensor* ts, int32_t n, int32_t B) {
  std::vector<int> out(n, 0);
  std::map<BandKey, std::vector<int>> groups;
  // what the result depends on (the plan is built on every step); slots differ between device kinds
  std::vector<int64_t> sig{B, n, current_device()};
  for (int i = 0; i < n; ++i) {
    const came8_tensor& t = ts[i];
    if (!t.factored || t.rows < 1 || t.cols < 1 || t.prefix < 1) continue;
    if (tiny_matrix(t, t.state_kind == CAME8_STATE_8BIT2D)) continue;
    const BandShapeSel sel = band_variant(t, t.cols, B, 1);
    groups[BandKey{t.grad_dtype, sel.V, sel.K, sel.TPB, 0, sel.ua}].push_back(i);
    sig.insert(sig.end(), {i, t.rows, t.cols, t.prefix, t.grad_dtype, t.state_kind, sel.V, sel.K, sel.TPB, sel.ua});
  }
  static std::mutex memo_mu;
  static std::map<std::vector<int64_t>, std::vector<int>> memo;
  {
    std::lock_guard<std::mutex> lk(memo_mu);
    auto it = memo.find(sig);
    if (it != memo.end()) return it->second;
  }
  for (auto& kv : groups) {
    const BandKey& k = kv.first;
    const came8_tensor& t0 = ts[kv.second.front()];
    const bool s2d = t0.state_kind == CAME8_STATE_8BIT2D;
    const int st = t0.state_kind == CAME8_STATE_FP32 ? 1 : 0;
    const BandShapeSel s2 = band_variant(t0, t0.cols, B, 2);  // alike over the group
    const int64_t slots1 = resident_slots(reinterpret_cast<const void*>(band_fn(k.gdt, false, k.V, k.K, k.TPB, 0, k.ua, 0)), k.TPB);
    const int64_t slots2 = s2d ? 0 : resident_slots(reinterpret_cast<const void*>(band_fn(k.gdt, true, s2.V, s2.K, s2.TPB, st, s2.ua, s2.multiseg)), s2.TPB);
    int best = 0;
    if (slots1 <= 0) {
      for (; best < kMaxShrink; ++best) {
        int64_t bands = 0;
        for (int i : kv.second) bands += ts[i].prefix * ceil_div(ts[i].rows, band_rows(ts[i].rows, ts[i].cols, best));
        if (bands >= kMinLaunchBands) break;
      }
    } else {
      double best_t = 0.0;
      int64_t prev_rb_sum = -1;
      for (int s = 0; s <= kMaxShrink; ++s) {
        std::vector<double> elems;
        double partial = 0.0;
        int64_t rb_sum = 0;
        for (int i : kv.second) {
          const came8_tensor& t = ts[i];
          const int64_t rb = band_rows(t.rows, t.cols, s);
          rb_sum += rb;
          const int64_t nb = ceil_div(t.rows, rb);
          for (int64_t m = 0; m < t.prefix; ++m)
            for (int64_t bnd = 0; bnd < nb; ++bnd)
              elems.push_back(double(std::min(rb, t.rows - bnd * rb)) * double(t.cols));
          partial += 3.0 * double(t.prefix * nb) * double(t.cols);
        }
        if (rb_sum == prev_rb_sum) break;  // every band is at its least height already
        prev_rb_sum = rb_sum;
        // one pass: the busiest workgroup's elements, at 1/slots of the GPU's rate
        auto pass_time = [&](int64_t slots) {
          std::vector<double> cost(elems);
          for (double& c : cost) c += kBandFixedElems / double(slots);
          return schedule_makespan(cost, slots) * double(slots);
        };
        double est = pass_time(slots1) + 2.0 * partial;
        if (slots2 > 0) est += 1.5 * pass_time(slots2);
        if (s == 0 || est < best_t) {
          best_t = est;
          best = s;
        }
      }
    }
    for (int i : kv.second) out[i] = best;
  }
  std::lock_guard<std::mutex> lk(memo_mu);
  if (memo.size() >= 64) memo.clear();
  memo[sig] = out;
  return out;
}

int build_plan(const came8_tensor* ts, int32_t n, int32_t B, char* ws_base, Plan& plan) {
  if (n < 0) return fail(CAME8_EINVAL, "came8: n_tensors must be >= 0");
  if (n > 0 && ts == nullptr) return fail(CAME8_EINVAL, "came8: tensors is NULL");
  if (B <= 0) return fail(CAME8_EINVAL, "came8: block_size must be > 0, got " + std::to_string(B));
  plan.dev.assign(n, DevTensor{});
  // --- scratch layout (after the plan blob; offsets relative to the scratch start) ---
  std::vector<size_t> scr_off(n, 0);
  size_t scr = 0;
  const std::vector<int> shrink = (B > 0 && n > 0) ? band_shrinks(ts, n, B) : std::vector<int>(std::max(n, 0), 0);
  for (int i = 0; i < n; ++i) {
    const came8_tensor& t = ts[i];
    const std::string who = "came8: tensor " + std::to_string(i) + ": ";
    if (t.state_kind != CAME8_STATE_Q8 && t.state_kind != CAME8_STATE_FP32 && t.state_kind != CAME8_STATE_8BIT2D &&
        t.state_kind != CAME8_STATE_Q8_MATRIX)
      return fail(CAME8_EINVAL, who + "unknown state_kind " + std::to_string(t.state_kind));
    if (t.state_kind == CAME8_STATE_Q8_MATRIX && !t.factored)
      return fail(CAME8_EINVAL, who + "per-matrix blocks need a factored tensor");
    if (t.state_kind == CAME8_STATE_Q8_MATRIX && t.prefix > 1 && t.prefix * t.rows * t.cols >= (int64_t(1) << 31))
      return fail(CAME8_EINVAL, who + "per-matrix blocks need fewer than 2^31 elements");
    const bool f32st = t.state_kind == CAME8_STATE_FP32;
    const bool s2d = t.state_kind == CAME8_STATE_8BIT2D;
    if (s2d) {
      if (!t.factored || t.prefix != 1) return fail(CAME8_EINVAL, who + "8bit2d states need a 2-D tensor (factored, prefix 1)");
      if (B != 256) return fail(CAME8_EINVAL, who + "8bit2d states support block_size=256 only, got " + std::to_string(B));
      if (!t.res_row_q || !t.res_row_absmax || !t.res_col_q || !t.res_col_absmax)
        return fail(CAME8_EINVAL, who + "null residual state");
      if ((t.res_row_partial == nullptr) != (t.res_col_partial == nullptr))
        return fail(CAME8_EINVAL, who + "give both tile partial buffers or neither");
    }
    if (!t.param || !t.grad || !t.exp_avg_q || !t.row_q || (!f32st && !t.exp_avg_absmax) ||
        ((!f32st || t.factored) && !t.row_absmax))
      return fail(CAME8_EINVAL, who + "null pointer");
    if (f32st && !fast_block(B))
      return fail(CAME8_EINVAL, who + "fp32 states need a power-of-two block size in [8, 2048]");
    for (int dt : {t.param_dtype, t.grad_dtype})
      if (dt != CAME8_F32 && dt != CAME8_BF16 && dt != CAME8_F16) return fail(CAME8_EINVAL, who + "unsupported dtype");
    if (t.prefix < 1 || t.rows < 1 || t.cols < 1) return fail(CAME8_EINVAL, who + "empty or negative shape");
    if (!t.factored && (t.prefix != 1 || t.rows != 1)) return fail(CAME8_EINVAL, who + "1-D tensors take prefix = rows = 1");
    if ((t.tensor_flags & ~CAME8_TENSOR_FP16_UPDATE) != 0 || t.reserved != 0)
      return fail(CAME8_EINVAL, who + "unknown tensor_flags bits or nonzero reserved field");
    if (t.factored && (!t.col_q || !t.col_absmax)) return fail(CAME8_EINVAL, who + "null column state");
    if ((B & (B - 1)) != 0 && t.prefix * t.rows * t.cols >= (int64_t(1) << 31))
      return fail(CAME8_EINVAL, who + "block sizes that are not powers of two need fewer than 2^31 elements");
    DevTensor& d = plan.dev[i];
    d.p = t.param;
    d.g = t.grad;
    d.mq = t.exp_avg_q;
    d.ma = t.exp_avg_absmax;
    d.rq = t.row_q;
    d.ra = t.row_absmax;
    d.cq = t.col_q;
    d.ca = t.col_absmax;
    d.P = t.prefix;
    d.R = t.rows;
    d.C = t.cols;
    d.N = t.prefix * t.rows * t.cols;
    // per-matrix blocks: only where they differ from flat ones (P > 1); blocks per matrix of the
    // momentum, a row state and a column state
    d.pm = (t.state_kind == CAME8_STATE_Q8_MATRIX && t.prefix > 1) ? 1 : 0;
    d.pmb_m = ceil_div(t.rows * t.cols, int64_t(B));
    d.pmb_r = ceil_div(t.rows, int64_t(B));
    d.pmb_c = ceil_div(t.cols, int64_t(B));
    d.nbm = d.pm ? t.prefix * d.pmb_m : std::max<int64_t>(1, ceil_div(d.N, B));
    d.factored = t.factored ? 1 : 0;
    d.fp32st = f32st ? 1 : 0;
    d.fp16u = (!t.factored && !f32st && !s2d && (t.tensor_flags & CAME8_TENSOR_FP16_UPDATE)) ? 1 : 0;
    d.mode2d = s2d ? 1 : 0;
    bool v2d = false, v2dp = false;  // vector forms of the 8bit2d momentum pass / parameter write
    if (s2d) {
      const uintptr_t a16 = 15;
      const bool c16 = t.cols % 16 == 0, mq16 = (reinterpret_cast<uintptr_t>(t.exp_avg_q) & a16) == 0;
      v2d = c16 && mq16 && (reinterpret_cast<uintptr_t>(t.grad) & a16) == 0;
      v2dp = c16 && mq16 && (reinterpret_cast<uintptr_t>(t.param) & a16) == 0;
      d.tr = int32_t(ceil_div(t.rows, 16));
      d.tc = int32_t(ceil_div(t.cols, 16));
      d.rrq = t.res_row_q;
      d.rra = t.res_row_absmax;
      d.rcq = t.res_col_q;
      d.rca = t.res_col_absmax;
    }
    const uintptr_t pp = reinterpret_cast<uintptr_t>(t.param), gp = reinterpret_cast<uintptr_t>(t.grad),
                    mp = reinterpret_cast<uintptr_t>(t.exp_avg_q);
    d.vec_ok = (pp % 16 == 0 && gp % 16 == 0 && mp % 8 == 0) ? 1 : 0;
    size_t off = 0;
    auto take = [&](size_t bytes) {
      const size_t o = off;
      off += align_up(bytes);
      return o;
    };
    struct Offs {
      size_t Rn, rfac, RRn, rrfac, Cn, cfac, CRn, crfac, pU, pW, pR, rm, rmr, esm, clipp, clip, t2r, t2c, nest, nrec,
          nsum, nbsum, nch;
    } o{};
    d.idx32 = d.N < (int64_t(1) << 31) ? 1 : 0;
    d.rowal = (d.C % B) == 0 ? 1 : 0;
    d.c8 = (d.C % 8 == 0) ? 1 : 0;
    // band form of P3: rows start blocks, vector access, rows wide enough to occupy the lanes
    d.p3_rb = 0;
    d.p3_nseg = 0;
    d.p3_nbands = 0;
    if (t.factored && !s2d && fast_block(B) && d.rowal && d.vec_ok && d.C >= kP3BandMinCols) {
      const int64_t bpr = d.C / B, bmax = kTile / B;  // blocks per row, per segment
      d.p3_nseg = int32_t(ceil_div(bpr, bmax));
      d.p3_rb = kP3BandRows;
      d.p3_nbands = ceil_div(d.R, int64_t(kP3BandRows));
    }
    magic_div(d.C, d.mC, d.sC);
    magic_div(d.R, d.mR, d.sR);
    if (t.factored) {
      d.rb = tiny_matrix(t, s2d) ? d.R : band_rows(d.R, d.C, shrink[i]);
      d.nbands = ceil_div(d.R, d.rb);
      d.nbr = d.pm ? d.P * d.pmb_r : std::max<int64_t>(1, ceil_div(d.P * d.R, B));
      d.nbc = d.pm ? d.P * d.pmb_c : std::max<int64_t>(1, ceil_div(d.P * d.C, B));
      d.nclip = d.nbc;
      const size_t pr = size_t(d.P * d.R) * 4, pc = size_t(d.P * d.C) * 4;
      const size_t part = size_t(d.P * d.nbands * d.C) * 4;
      o.Rn = take(pr); o.rfac = take(pr); o.RRn = take(pr); o.rrfac = take(pr);
      o.Cn = take(pc); o.cfac = take(pc); o.CRn = take(pc); o.crfac = take(pc);
      o.pU = take(part); o.pW = take(part);
      if (s2d) {  // tile residual sums per column [tr][C] and (scalar pass) per row [R][tc], unless the caller's
        if (!t.res_row_partial) {
          if (!v2d) o.t2r = take(size_t(d.R) * size_t(d.tc) * 4);
          o.t2c = take(size_t(d.C) * size_t(d.tr) * 4);
        }
      } else {
        o.pR = take(part);
      }
      o.rm = take(size_t(d.P * d.nbands) * 4);
      o.esm = take(size_t(d.P * d.nbands) * 4);
      o.rmr = take(size_t(d.P * (s2d ? std::max<int64_t>(d.nbands, d.tr) : d.nbands)) * 4);
      o.clipp = take(size_t(d.nclip) * 8);
      o.clip = take(8);
    } else {
      d.rb = 1;
      d.nbands = 1;
      d.nbr = d.nbm;
      d.nbc = 0;
      d.nclip = ceil_div(d.N, kTile);
      o.clipp = take(size_t(d.nclip) * 8);
      o.clip = take(8);
    }
    // reference-order norm: unit estimates, segment records, chain accumulators (not for 8bit2d,
    // whose clip is the reference's float sum)
    d.nseg = 0;
    d.nseg0 = 0;
    d.nrun = kNormRunSegs;
    d.nunit = 0;
    d.ngrp = 1;
    if (!s2d) {
      d.nseg = ceil_div(d.N - (d.N & 7), kNormSegElems);
      const bool lds = t.factored && d.idx32 && reinterpret_cast<uintptr_t>(t.grad) % 16 == 0 && d.P == 1 &&
                       !tiny_matrix(t, false) && d.C >= 8 * kNormSegLanes && d.C + (d.c8 ? 0 : 8) <= kNormLdsCols;
      d.nseg0 = lds ? (d.N - (d.N & 7)) / kNormSegElems : 0;
      // runs of 64 segments (the column factors staged once per 256K elements); a tensor of fewer than
      // 256 such runs takes shorter ones, down to 16, so that it still spreads over the CUs
      d.nrun = d.nseg0 >= 256 * int64_t(kNormRunSegs) ? kNormRunSegs : (d.nseg0 >= 128 * int64_t(kNormRunSegs) ? 32 : 16);
      const int64_t nbase = t.factored ? d.P * d.nbands : d.nclip;
      // the thread-per-unit estimate groups single-band matrices and tiles into at most kNormMaxUnits units
      if (!norm_est_wide(t, d) && (!t.factored || d.nbands == 1)) d.ngrp = ceil_div(nbase, kNormMaxUnits);
      d.nunit = ceil_div(nbase, d.ngrp);
      o.nest = take(size_t(d.nunit + 1) * 4);
      o.nrec = take(size_t(d.nseg) * 3 * 8 * 4);
      o.nsum = take(size_t(d.nseg) * 8 * 4);
      d.nblk = ceil_div(d.nseg, int64_t(kNormFixSegs));
      o.nbsum = take(size_t(d.nblk) * 8 * 4);
      o.nch = take(8 * 4);
    }
    scr_off[i] = scr;
    // store offsets temporarily as integers in the pointer fields (rebased below)
    auto at = [&](size_t x) { return reinterpret_cast<float*>(scr + x); };
    if (t.factored) {
      d.Rn = at(o.Rn); d.rfac = at(o.rfac); d.RRn = at(o.RRn); d.rrfac = at(o.rrfac);
      d.Cn = at(o.Cn); d.cfac = at(o.cfac); d.CRn = at(o.CRn); d.crfac = at(o.crfac);
      d.partU = at(o.pU); d.partW = at(o.pW);
      if (s2d) {
        d.t2row = t.res_row_partial ? t.res_row_partial : (v2d ? nullptr : at(o.t2r));
        d.t2col = t.res_col_partial ? t.res_col_partial : at(o.t2c);
        d.v2d = v2d ? 1 : 0;
        d.v2dp = v2dp ? 1 : 0;
      } else {
        d.partRes = at(o.pR);
      }
      d.rsum = at(o.rm); d.rrsum = at(o.rmr); d.esum = at(o.esm);
    }
    d.clip_part = reinterpret_cast<double*>(scr + o.clipp);
    d.clip = at(o.clip);
    if (!s2d) {
      d.nest = at(o.nest);
      d.nrec = reinterpret_cast<uint32_t*>(scr + o.nrec);
      d.nsum = at(o.nsum);
      d.nbsum = at(o.nbsum);
      d.nchain = at(o.nch);
    }
    scr += off;
  }
  // Few band-form P3 work items (small matrices) would leave most CUs idle: lower every band's
  // height until the launch has kP3MinItems items or the bands are one row high.
  for (int32_t rb = kP3BandRows; rb > 1; rb >>= 1) {
    int64_t items = 0;
    for (const DevTensor& d : plan.dev) items += d.p3_nbands > 0 ? d.P * d.p3_nbands * d.p3_nseg : 0;
    if (items == 0 || items >= kP3MinItems) break;
    for (DevTensor& d : plan.dev)
      if (d.p3_nbands > 0) {
        d.p3_rb = rb >> 1;
        d.p3_nbands = ceil_div(d.R, int64_t(d.p3_rb));
      }
  }

  // --- work lists ---
  const bool fastB = fast_block(B);
  // The long-chain group: factored tensors with more than half the longest chain's segments, when the
  // longest chain is long (kWalkSplitMinSegs) and the group holds at most 60% of the factored elements.
  std::vector<char> longc(size_t(n), 0);
  {
    int64_t maxseg = 0;
    for (int i = 0; i < n; ++i)
      if (!plan.dev[i].mode2d) maxseg = std::max(maxseg, plan.dev[i].nseg);
    double nall = 0.0, nlong = 0.0;
    bool any_short = false;
    for (int i = 0; i < n; ++i) {
      const DevTensor& d = plan.dev[i];
      if (d.mode2d || !ts[i].factored) continue;
      nall += double(d.N);
      if (2 * d.nseg > maxseg) {
        longc[i] = 1;
        nlong += double(d.N);
      } else {
        any_short = true;
      }
    }
    plan.walk_split = maxseg >= kWalkSplitMinSegs && any_short && nlong <= 0.6 * nall;
    if (!plan.walk_split) longc.assign(size_t(n), 0);
  }
  for (int i = 0; i < n; ++i) {
    const came8_tensor& t = ts[i];
    const DevTensor& d = plan.dev[i];
    const TypeKey tk{t.param_dtype, t.grad_dtype, d.fp32st};
    if (d.mode2d) {
      const BandShapeSel sel = band_variant(t, d.C, B, 1);
      add_item(plan.band2dw[BandKey{t.grad_dtype, sel.V, sel.K, sel.TPB, 0, sel.ua}], i, d.nbands);
      add_item(plan.factor, i, d.nbr + d.nbc);
      if (d.v2d) {
        add_item(plan.tiles2d_v[t.grad_dtype], i, d.tr);
      } else {
        add_item(plan.tiles2d[t.grad_dtype], i, int64_t(d.tr) * ceil_div(d.C, 256));
        add_item(plan.res2d, i, d.tr);
      }
      if (d.v2dp && d.C >= kP3BandMinCols)
        add_item(plan.param2d_b[t.param_dtype], i, ceil_div(d.R, int64_t(kParam2BandRows)) * ceil_div(d.C, int64_t(kTile)));
      else if (d.v2dp)
        add_item(plan.param2d_v[t.param_dtype], i, ceil_div(d.N, kParam2Items));
      else add_item(plan.param2d[t.param_dtype], i, ceil_div(d.N, kTile));
      continue;  // the clip of this layout has no parity-mode variant (the reference sums it with float atomics)
    }
    if (t.factored) {
      if (tiny_matrix(t, false)) {
        add_item(plan.tiny1[t.grad_dtype], i, ceil_div(d.P, int64_t(kThreads)));
        add_item((longc[i] ? plan.tiny2L : plan.tiny2)[t.grad_dtype], i, ceil_div(d.P, int64_t(kThreads)));
      } else {
        const bool pm_m = d.pm && (d.R * d.C) % B != 0;
        const BandShapeSel sel1 = band_variant(t, d.C, B, 1), sel2 = band_variant(t, d.C, B, 2, pm_m);
        // the default mode's pass 1 takes pass 2's row shapes (column segments for wide rows)
        const BandShapeSel sel1n = band_variant(t, d.C, B, 2);
        add_item(plan.band[BandKey{t.grad_dtype, sel1.V, sel1.K, sel1.TPB, 0, sel1.ua}], i, d.P * d.nbands);
        add_item(plan.bandN[BandKey{t.grad_dtype, sel1n.V, sel1n.K, sel1n.TPB, 1, sel1n.ua, sel1n.multiseg}], i,
                 d.P * d.nbands);
        add_item((longc[i] ? plan.band2L : plan.band2)[BandKey{t.grad_dtype, sel2.V, sel2.K, sel2.TPB, d.fp32st, sel2.ua,
                                                              sel2.multiseg}], i, d.P * d.nbands);
      }
      add_item(plan.factor, i, d.nbr + d.nbc);
      // per-matrix momentum blocks that end inside a matrix (B does not divide R*C) are not the flat
      // passes' blocks: such tensors take the per-block kernel
      const bool pm_odd = d.pm && (d.R * d.C) % B != 0;
      if (fastB && !pm_odd) {
        if (d.p3_nbands > 0) add_item(plan.updb[tk], i, d.P * d.p3_nbands * d.p3_nseg);
        else add_item(plan.upd[tk], i, ceil_div(d.N, kTile));
      } else if (fastB) {
        add_item(plan.generic[tk], i, d.nbm);
      }
    } else {
      add_item(plan.vecA[t.grad_dtype], i, d.nclip);
      // in the default clip mode pass A's tile sums only feed the norm's estimates
      if (d.nseg > 1) add_item(plan.vecAn[t.grad_dtype], i, d.nclip);
      if (fastB) add_item(plan.vecB[tk], i, ceil_div(d.N, kTile));
    }
    if (!fastB) add_item(plan.generic[tk], i, d.nbm);
    // The walk replays every chain's first segment from zero without reading its record, so a tensor of
    // one segment needs no estimates, records or rebuild.
    if (d.nseg > 1) {
      if (norm_est_wide(t, d)) add_item(plan.nest_w, i, d.nunit);
      else add_item(plan.nest_n, i, ceil_div(d.nunit, int64_t(kThreads)));
      // the vector forms need rows of whole aligned 8-element chunks and 32-bit flat indices; matrices
      // (prefix 1) up to kNormLdsCols wide take runs of segments with their column factors in LDS
      const bool vec = t.factored && d.idx32 && reinterpret_cast<uintptr_t>(t.grad) % 16 == 0;
      const int form = vec && d.c8 ? kNormVec : (vec && d.C >= 8 ? kNormRows : kNormAny);
      if (d.nseg0 > 0)
        add_item(plan.nseg2d[t.grad_dtype * 3 + (d.c8 ? kNormVec : kNormRows)], i, ceil_div(d.nseg0, d.nrun));
      if (d.nseg > d.nseg0) add_item(plan.nseg[t.grad_dtype * 3 + form], i, d.nseg - d.nseg0);
      if (d.nblk > kNormFixDirect) add_item(plan.nbsum, i, d.nblk);
      add_item(plan.nfix[t.grad_dtype * 3 + form], i, ceil_div(d.nseg, int64_t(kNormFixSegs)));
    }
    add_item((longc[i] ? plan.nwalkL : plan.nwalk)[t.grad_dtype], i, 8);
    add_item((longc[i] ? plan.nfinalL : plan.nfinal)[t.grad_dtype], i, 1);
  }

  // --- blob: DevTensor[n] then every work list (tids, wstart) ---
  size_t off = align_up(sizeof(DevTensor) * size_t(n), 16);
  auto place = [&](WorkList& wl) {
    wl.tids_off = off;
    off = align_up(off + wl.tids.size() * 4, 16);
    wl.wstart_off = off;
    off = align_up(off + wl.wstart.size() * 8, 16);
  };
  for (auto& kv : plan.band) place(kv.second);
  for (auto& kv : plan.bandN) place(kv.second);
  for (auto& kv : plan.band2dw) place(kv.second);
  for (auto& kv : plan.band2) place(kv.second);
  for (auto& kv : plan.tiny1) place(kv.second);
  for (auto& kv : plan.tiny2) place(kv.second);
  for (auto& kv : plan.tiles2d_v) place(kv.second);
  for (auto& kv : plan.tiles2d) place(kv.second);
  for (auto& kv : plan.param2d_v) place(kv.second);
  for (auto& kv : plan.param2d_b) place(kv.second);
  for (auto& kv : plan.param2d) place(kv.second);
  place(plan.res2d);
  for (auto& kv : plan.upd) place(kv.second);
  for (auto& kv : plan.updb) place(kv.second);
  for (auto& kv : plan.vecB) place(kv.second);
  for (auto& kv : plan.vecA) place(kv.second);
  for (auto& kv : plan.vecAn) place(kv.second);
  for (auto& kv : plan.generic) place(kv.second);
  place(plan.nest_w);
  place(plan.nest_n);
  for (auto& kv : plan.nseg2d) place(kv.second);
  for (auto& kv : plan.nseg) place(kv.second);
  place(plan.nbsum);
  for (auto& kv : plan.nfix) place(kv.second);
  for (auto& kv : plan.nwalk) place(kv.second);
  for (auto& kv : plan.nfinal) place(kv.second);
  for (auto& kv : plan.band2L) place(kv.second);
  for (auto& kv : plan.tiny2L) place(kv.second);
  for (auto& kv : plan.nwalkL) place(kv.second);
  for (auto& kv : plan.nfinalL) place(kv.second);
  place(plan.factor);
  plan.zero_off = align_up(off);
  off = plan.zero_off + kZeroBytes;
  plan.plan_bytes = align_up(off);
  plan.total_bytes = plan.plan_bytes + scr;

  if (ws_base != nullptr) {
    char* scr_base = ws_base + plan.plan_bytes;
    auto rebase = [&](auto*& ptr) {
      using P = std::remove_reference_t<decltype(ptr)>;
      ptr = reinterpret_cast<P>(scr_base + reinterpret_cast<uintptr_t>(ptr));
    };
    for (int i = 0; i < n; ++i) {
      DevTensor& d = plan.dev[i];
      if (d.factored) {
        rebase(d.Rn); rebase(d.rfac); rebase(d.RRn); rebase(d.rrfac);
        rebase(d.Cn); rebase(d.cfac); rebase(d.CRn); rebase(d.crfac);
        rebase(d.partU); rebase(d.partW);
        if (d.mode2d) {
          if (!ts[i].res_row_partial) {  // workspace offsets (caller buffers are absolute)
            if (!d.v2d) rebase(d.t2row);
            rebase(d.t2col);
          }
        } else {
          rebase(d.partRes);
        }
        rebase(d.rsum); rebase(d.rrsum); rebase(d.esum);
      }
      rebase(d.clip_part);
      rebase(d.clip);
      if (!d.mode2d) {
        rebase(d.nest);
        rebase(d.nrec);
        rebase(d.nsum);
        rebase(d.nbsum);
        rebase(d.nchain);
      }
    }
    plan.blob.assign(plan.plan_bytes, 0);
    std::memcpy(plan.blob.data(), plan.dev.data(), sizeof(DevTensor) * size_t(n));
    auto put = [&](const WorkList& wl) {
      std::memcpy(plan.blob.data() + wl.tids_off, wl.tids.data(), wl.tids.size() * 4);
      std::memcpy(plan.blob.data() + wl.wstart_off, wl.wstart.data(), wl.wstart.size() * 8);
    };
    for (auto& kv : plan.band) put(kv.second);
    for (auto& kv : plan.bandN) put(kv.second);
    for (auto& kv : plan.band2dw) put(kv.second);
    for (auto& kv : plan.band2) put(kv.second);
    for (auto& kv : plan.tiny1) put(kv.second);
    for (auto& kv : plan.tiny2) put(kv.second);
    for (auto& kv : plan.tiles2d_v) put(kv.second);
    for (auto& kv : plan.tiles2d) put(kv.second);
    for (auto& kv : plan.param2d_v) put(kv.second);
    for (auto& kv : plan.param2d_b) put(kv.second);
    for (auto& kv : plan.param2d) put(kv.second);
    put(plan.res2d);
    for (auto& kv : plan.upd) put(kv.second);
    for (auto& kv : plan.updb) put(kv.second);
    for (auto& kv : plan.vecB) put(kv.second);
    for (auto& kv : plan.vecA) put(kv.second);
    for (auto& kv : plan.vecAn) put(kv.second);
    for (auto& kv : plan.generic) put(kv.second);
    put(plan.nest_w);
    put(plan.nest_n);
    for (auto& kv : plan.nseg2d) put(kv.second);
    for (auto& kv : plan.nseg) put(kv.second);
    put(plan.nbsum);
    for (auto& kv : plan.nfix) put(kv.second);
    for (auto& kv : plan.nwalk) put(kv.second);
    for (auto& kv : plan.nfinal) put(kv.second);
    for (auto& kv : plan.band2L) put(kv.second);
    for (auto& kv : plan.tiny2L) put(kv.second);
    for (auto& kv : plan.nwalkL) put(kv.second);
    for (auto& kv : plan.nfinalL) put(kv.second);
    put(plan.factor);
  }
  return CAME8_OK;
}

uint64_t fnv1a(const uint8_t* p, size_t n) {
  uint64_t h = 1469598103934665603ull;
  for (size_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 1099511628211ull;
  }
  return h;
}

// Plan uploads per (workspace address, caller's workspace tag).  A tag names one allocation of
// the workspace by its owner; a freed-and-reallocated workspace at the same address gets a new
// tag, so a stale entry can never match memory that was reused in between.  Tag 0 never reuses.
struct CacheEntry {
  uint64_t hash = 0;
  size_t bytes = 0;
  std::vector<uint8_t> keep;  // source of the last upload, alive until `done` has fired
  hipEvent_t done = nullptr;
  // the launch plan last built for this workspace and the inputs it was built from: a call with the
  // same descriptors, block size and workspace reuses it without planning again
  std::vector<uint8_t> inputs;
  std::shared_ptr<const Plan> plan;
};

// The inputs a plan depends on, as bytes: the descriptor count, the block size, the workspace
// address (the plan holds pointers into the workspace) and the descriptors themselves.
std::vector<uint8_t> plan_inputs(const came8_tensor* ts, int32_t n, int32_t B, const void* ws) {
  const size_t nb = size_t(std::max(n, 0)) * sizeof(came8_tensor);
  std::vector<uint8_t> v(24 + sizeof(void*) + nb);
  const int64_t head[3] = {n, B, current_device()};  // band sizes depend on the device
  std::memcpy(v.data(), head, 24);
  std::memcpy(v.data() + 24, &ws, sizeof(void*));
  if (nb) std::memcpy(v.data() + 24 + sizeof(void*), ts, nb);
  return v;
}
std::mutex g_cache_mu;
std::map<std::pair<const void*, uint64_t>, CacheEntry> g_cache;

void drop_entry(CacheEntry& ce) {
  if (ce.done) {
    (void)hipEventSynchronize(ce.done);
    (void)hipEventDestroy(ce.done);
    ce.done = nullptr;
  }
  ce.keep.clear();
  ce.keep.shrink_to_fit();
}

Hp make_hp(const came8_hparams& h) {
  Hp hp{};
  hp.b1 = float(h.beta1);
  hp.a1 = float(1.0 - h.beta1);
  hp.b2 = float(h.beta2);
  hp.a2 = float(1.0 - h.beta2);
  hp.b3 = float(h.beta3);
  hp.a3 = float(1.0 - h.beta3);
  hp.eps0 = float(h.eps0);
  hp.eps1 = float(h.eps1);
  hp.awd = float(-h.weight_decay * h.lr);
  hp.awd_bf16 = round_to_bf16(hp.awd);
  hp.awd_f16 = round_to_f16(hp.awd);
  hp.alr = float(-h.lr);
  hp.thr = float(h.clip_threshold);
  hp.wd = h.weight_decay != 0.0 ? 1 : 0;
  // 8bit2d: the reference computes these in float (came_kernels.cu:91, 2623, 2678)
  hp.a1f = 1.0f - float(h.beta1);
  hp.a2f = 1.0f - float(h.beta2);
  hp.a3f = 1.0f - float(h.beta3);
  const float lr_wd = float(h.lr) * float(h.weight_decay);
  hp.wdfac = 1.0f - lr_wd;
  hp.fp16u = (h.flags & CAME8_FLAG_FP16_UPDATE) ? 1 : 0;
  hp.noW = (h.flags & CAME8_FLAG_EXACT_NORM) ? 0 : 1;
  hp.B = h.block_size;
  hp.log2B = log2_or_minus1(h.block_size);
  if (hp.log2B >= 0) {
    hp.mB = 1;
    hp.sB = uint32_t(hp.log2B);
  } else {
    magic_div(h.block_size, hp.mB, hp.sB);
  }
  return hp;
}

// ---------------------------------------------------------------------------
// kernel-variant dispatch
// ---------------------------------------------------------------------------
// band-pass kernels are instantiated in came8_band.hip (one translation unit per family)
BandFn band_fn(int gdt, bool pass2, int V, int K, int TPB, int st, int ua, int ms) {
  switch (gdt) {
    case CAME8_F32: return pass2 ? band_fn_F32_p2(V, K, TPB, st, ua, ms) : band_fn_F32_p1(V, K, TPB, st, ua, ms);
    case CAME8_BF16: return pass2 ? band_fn_BF16_p2(V, K, TPB, st, ua, ms) : band_fn_BF16_p1(V, K, TPB, st, ua, ms);
    case CAME8_F16: return pass2 ? band_fn_F16_p2(V, K, TPB, st, ua, ms) : band_fn_F16_p1(V, K, TPB, st, ua, ms);
    default: return nullptr;
  }
}

using GenFn = void (*)(const DevTensor*, const int32_t*, const int64_t*, int, Hp);

template <typename TP, typename TG>
constexpr GenFn k_fact_pass3_q8 = k_fact_pass3<TP, TG, false>;
template <typename TP, typename TG>
constexpr GenFn k_fact_pass3_f32st = k_fact_pass3<TP, TG, true>;
template <typename TP, typename TG>
constexpr GenFn k_fact_pass3b_q8 = k_fact_pass3b<TP, TG, false>;
template <typename TP, typename TG>
constexpr GenFn k_fact_pass3b_f32st = k_fact_pass3b<TP, TG, true>;

#define CAME8_TYPE_SWITCH2(KERNEL, pdt, gdt, out)                                       \
  do {                                                                                  \
    out = nullptr;                                                                      \
    if (pdt == CAME8_F32 && gdt == CAME8_F32) out = KERNEL<F32, F32>;                   \
    if (pdt == CAME8_F32 && gdt == CAME8_BF16) out = KERNEL<F32, BF16>;                 \
    if (pdt == CAME8_F32 && gdt == CAME8_F16) out = KERNEL<F32, F16>;                   \
    if (pdt == CAME8_BF16 && gdt == CAME8_F32) out = KERNEL<BF16, F32>;                 \
    if (pdt == CAME8_BF16 && gdt == CAME8_BF16) out = KERNEL<BF16, BF16>;               \
    if (pdt == CAME8_BF16 && gdt == CAME8_F16) out = KERNEL<BF16, F16>;                 \
    if (pdt == CAME8_F16 && gdt == CAME8_F32) out = KERNEL<F16, F32>;                   \
    if (pdt == CAME8_F16 && gdt == CAME8_BF16) out = KERNEL<F16, BF16>;                 \
    if (pdt == CAME8_F16 && gdt == CAME8_F16) out = KERNEL<F16, F16>;                   \
  } while (0)

// KERNEL<TP, TG, fp32 states>
#define CAME8_TYPE_SWITCH3(KERNEL, pdt, gdt, st, out)            \
  do {                                                           \
    if (st) {                                                    \
      CAME8_TYPE_SWITCH2(KERNEL##_f32st, pdt, gdt, out);         \
    } else {                                                     \
      CAME8_TYPE_SWITCH2(KERNEL##_q8, pdt, gdt, out);            \
    }                                                            \
  } while (0)

#define CAME8_TYPE_SWITCH1(KERNEL, gdt, out)           \
  do {                                                 \
    out = nullptr;                                     \
    if (gdt == CAME8_F32) out = KERNEL<F32>;           \
    if (gdt == CAME8_BF16) out = KERNEL<BF16>;         \
    if (gdt == CAME8_F16) out = KERNEL<F16>;           \
  } while (0)

// The segment-record and record-rebuild kernels of a work-list key 3 * grad type + chunk form.
#define CAME8_NORM_FN(NAME, KERNEL)                                          \
  GenFn NAME(int key) {                                                      \
    switch (key) {                                                           \
      case 3 * CAME8_F32 + kNormAny: return KERNEL<F32, kNormAny>;           \
      case 3 * CAME8_F32 + kNormRows: return KERNEL<F32, kNormRows>;         \
      case 3 * CAME8_F32 + kNormVec: return KERNEL<F32, kNormVec>;           \
      case 3 * CAME8_BF16 + kNormAny: return KERNEL<BF16, kNormAny>;         \
      case 3 * CAME8_BF16 + kNormRows: return KERNEL<BF16, kNormRows>;       \
      case 3 * CAME8_BF16 + kNormVec: return KERNEL<BF16, kNormVec>;         \
      case 3 * CAME8_F16 + kNormAny: return KERNEL<F16, kNormAny>;           \
      case 3 * CAME8_F16 + kNormRows: return KERNEL<F16, kNormRows>;         \
      case 3 * CAME8_F16 + kNormVec: return KERNEL<F16, kNormVec>;           \
      default: return nullptr;                                               \
    }                                                                        \
  }
CAME8_NORM_FN(norm_seg_fn, k_norm_seg)
// k_norm_seg2d of a work-list key 3 * grad type + chunk form (kNormVec or kNormRows)
GenFn norm_seg2d_fn(int key) {
  switch (key) {
    case 3 * CAME8_F32 + kNormVec: return k_norm_seg2d<F32, kNormVec>;
    case 3 * CAME8_F32 + kNormRows: return k_norm_seg2d<F32, kNormRows>;
    case 3 * CAME8_BF16 + kNormVec: return k_norm_seg2d<BF16, kNormVec>;
    case 3 * CAME8_BF16 + kNormRows: return k_norm_seg2d<BF16, kNormRows>;
    case 3 * CAME8_F16 + kNormVec: return k_norm_seg2d<F16, kNormVec>;
    case 3 * CAME8_F16 + kNormRows: return k_norm_seg2d<F16, kNormRows>;
    default: return nullptr;
  }
}
CAME8_NORM_FN(norm_fix_fn, k_norm_fix)
#undef CAME8_NORM_FN

// Workgroups per launch, at most: a launch of more work items loops over them (grid stride).  One
// workgroup per item where possible: a workgroup that loops waits out each item's first loads itself,
// while fresh workgroups start as others finish.  Pass 3 over C4's 822 000 band items: 10.37 ms with
// 16384 workgroups, 10.19 with 65536, 9.9 with one per item (C5 4.53 -> 4.19 ms, c4_2d 15.80 -> 15.64).
constexpr int64_t kMaxGrid = int64_t(1) << 20;

unsigned grid_for(int64_t work, int64_t per_block = 1) {
  const int64_t blocks = ceil_div(std::max<int64_t>(work, 1), per_block);
  return unsigned(std::min<int64_t>(blocks, kMaxGrid));
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(CAME8_EHIP, std::string("came8: launch of ") + what + " failed: " + hipGetErrorString(e));
  return CAME8_OK;
}

// ---------------------------------------------------------------------------
// optional per-launch device timing (HIP events on the launch stream)
// ---------------------------------------------------------------------------
const char* const kPhaseNames[] = {"pass1", "vec_passA", "row_mean", "factor_blocks", "clip", "norm_est",
                                   "pass2", "row_mean_res", "factor_blocks_res", "pass3", "vec_passB",
                                   "generic_update", "tiles2d", "res_rows2d", "param2d", "norm_bsum",
                                   "norm_seg", "norm_walk", "norm_final", "norm_fix"};
constexpr int kNumPhases = sizeof(kPhaseNames) / sizeof(kPhaseNames[0]);
enum Phase { PH_PASS1, PH_VECA, PH_ROWMEAN, PH_FACTOR, PH_CLIP, PH_NORM_EST, PH_PASS2, PH_ROWMEAN_RES,
             PH_FACTOR_RES, PH_PASS3, PH_VECB, PH_GENERIC, PH_TILES2D, PH_RES2D, PH_PARAM2D, PH_NORM_BSUM,
             PH_NORM_SEG, PH_NORM_WALK, PH_NORM_FINAL, PH_NORM_FIX };

struct Pending {
  int phase;
  hipEvent_t a, b;
  double bytes;
};
struct Profiler {
  std::mutex mu;
  bool on = false;
  std::vector<Pending> pending;
  std::vector<hipEvent_t> pool;
  int64_t launches[kNumPhases] = {};
  double total_ms[kNumPhases] = {};
  double bytes[kNumPhases] = {};
};
Profiler& prof() {
  static Profiler p;
  return p;
}

hipEvent_t take_event(Profiler& p) {
  if (!p.pool.empty()) {
    hipEvent_t e = p.pool.back();
    p.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Records an event before the launch and, in the destructor, after it.
struct PhaseTimer {
  hipEvent_t a = nullptr, b = nullptr;
  int phase;
  double bytes;
  hipStream_t stream;
  bool active = false;
  PhaseTimer(int ph, double alg_bytes, hipStream_t s) : phase(ph), bytes(alg_bytes), stream(s) {
    Profiler& p = prof();
    std::lock_guard<std::mutex> lk(p.mu);
    if (!p.on) return;
    a = take_event(p);
    b = take_event(p);
    if (a && b && hipEventRecord(a, stream) == hipSuccess) active = true;
  }
  ~PhaseTimer() {
    if (!active) return;
    Profiler& p = prof();
    std::lock_guard<std::mutex> lk(p.mu);
    if (hipEventRecord(b, stream) == hipSuccess) p.pending.push_back(Pending{phase, a, b, bytes});
  }
};

// A second queue for the launches of one pass.  The launches of a pass (its kernel variants, the tiny
// and 1-D kernels) work on disjoint tensors; spread over the caller's stream and a side stream they
// may overlap, so that a variant whose workgroups leave CU slots free (the 512-thread pass 1 over
// 11008-wide rows: one workgroup per CU) shares the device with the next one instead of queueing
// before it.  One side stream per (device, caller stream), created on first use and kept; not used
// while the caller's stream is capturing, nor by came8_step_static (which allocates nothing).
struct SideQueue {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
// One side stream and two events per (device, caller stream).  Those not in use by a step are idle; at
// most kMaxIdleSideQueues idle ones are kept: when a new one is needed beyond that, the least recently
// used idle one is released once its work has completed.
constexpr size_t kMaxIdleSideQueues = 16;
struct SideEntry {
  SideQueue q;
  uint64_t last = 0;  // the step that last took it
  int users = 0;      // steps holding it now
};
std::mutex g_side_mu;
std::map<std::pair<int, hipStream_t>, SideEntry> g_side;
uint64_t g_side_tick = 0;

void destroy_side(SideQueue& q) {
  if (q.s) {
    (void)hipStreamSynchronize(q.s);
    (void)hipStreamDestroy(q.s);
  }
  if (q.fork) (void)hipEventDestroy(q.fork);
  if (q.join) (void)hipEventDestroy(q.join);
  q = SideQueue{};
}

// A step's hold on its side stream (released when the step's launches are queued).
struct SideLease {
  std::pair<int, hipStream_t> key{-1, nullptr};
  bool held = false;
  SideLease() = default;
  SideLease(const SideLease&) = delete;
  SideLease& operator=(const SideLease&) = delete;
  ~SideLease() {
    if (!held) return;
    std::lock_guard<std::mutex> lk(g_side_mu);
    auto it = g_side.find(key);
    if (it != g_side.end()) --it->second.users;
  }
};

int side_queue(hipStream_t caller, SideQueue* out, SideLease* lease) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(CAME8_EHIP, "came8_step: no current HIP device");
  const auto key = std::make_pair(dev, caller);
  std::lock_guard<std::mutex> lk(g_side_mu);
  auto it = g_side.find(key);
  if (it == g_side.end()) {
    size_t idle = 0;
    auto lru = g_side.end();
    for (auto e = g_side.begin(); e != g_side.end(); ++e) {
      if (e->second.users) continue;
      ++idle;
      if (lru == g_side.end() || e->second.last < lru->second.last) lru = e;
    }
    if (idle >= kMaxIdleSideQueues) {
      destroy_side(lru->second.q);
      g_side.erase(lru);
    }
    SideEntry ent;
    if (hipStreamCreateWithFlags(&ent.q.s, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ent.q.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ent.q.join, hipEventDisableTiming) != hipSuccess) {
      const hipError_t e = hipGetLastError();
      destroy_side(ent.q);
      return fail(CAME8_EHIP, std::string("came8_step: creating the side stream failed: ") + hipGetErrorString(e));
    }
    it = g_side.emplace(key, ent).first;
  }
  ++it->second.users;
  it->second.last = ++g_side_tick;
  lease->key = key;
  lease->held = true;
  *out = it->second.q;
  return CAME8_OK;
}

// Side streams kept now (idle and in use), for tests.
size_t side_queue_count() {
  std::lock_guard<std::mutex> lk(g_side_mu);
  return g_side.size();
}

// The queue of each launch of a pass: with at least kSideMinLaunches launches in the pass, the first
// on the caller's stream and each later one on whichever of the two has fewer algorithmic bytes
// queued in this pass; else all on the caller's stream.  (Two or three launches gained nothing: the
// first fills the device and the next one's workgroups only start in its tail, while the fork and
// join cost 20-50 us on the small C1 and C2 steps; C5's 13-14 launches per pass gained 0.47 ms.)
// The side stream first waits for everything before the pass on the caller's stream (fork, recorded
// when the pass begins, so that the side's first launch can start with the pass's first one);
// finish() makes the caller's stream wait for the side stream's launches (join).
constexpr size_t kSideMinLaunches = 4;
constexpr size_t kSideMinNormLaunches = 3;  // the clip-norm record and rebuild kernels: C5 11.25 -> 10.87 ms
struct PassQueues {
  hipStream_t main;
  SideQueue side;
  bool can_side, use_side = false;
  double load[2] = {0.0, 0.0};
  bool forked = false;
  bool pending = false;  // the side stream holds work queued outside a pass (the long-chain group)
  PassQueues(hipStream_t m, const SideQueue& s, bool on) : main(m), side(s), can_side(on) {}
  ~PassQueues() { (void)finish(); }  // an early return still leaves the caller's stream after the side's work
  PassQueues(const PassQueues&) = delete;
  PassQueues& operator=(const PassQueues&) = delete;
  void begin(size_t launches, size_t min_launches = kSideMinLaunches) {
    use_side = can_side && launches >= min_launches;
    // a failed record leaves the pass on the caller's stream alone
    if (use_side && hipEventRecord(side.fork, main) != hipSuccess) {
      (void)hipGetLastError();
      use_side = false;
    }
  }
  int pick(double bytes, hipStream_t* out) {
    const int k = (use_side && load[1] < load[0]) ? 1 : 0;
    load[k] += bytes;
    if (k == 1 && !forked) {
      if (hipStreamWaitEvent(side.s, side.fork, 0) != hipSuccess)
        return fail(CAME8_EHIP, "came8_step: fork to the side stream failed");
      forked = true;
    }
    *out = k ? side.s : main;
    return CAME8_OK;
  }
  // Fork the side stream now, for work queued on it outside a pass; the next finish() joins it.
  int fork_now() {
    if (hipEventRecord(side.fork, main) != hipSuccess || hipStreamWaitEvent(side.s, side.fork, 0) != hipSuccess)
      return fail(CAME8_EHIP, "came8_step: fork to the side stream failed");
    pending = true;
    return CAME8_OK;
  }
  int finish() {
    load[0] = load[1] = 0.0;
    if (!forked && !pending) return CAME8_OK;
    forked = pending = false;
    if (hipEventRecord(side.join, side.s) != hipSuccess || hipStreamWaitEvent(main, side.join, 0) != hipSuccess)
      return fail(CAME8_EHIP, "came8_step: join of the side stream failed");
    return CAME8_OK;
  }
};

double elem_bytes(int dt) { return dt == CAME8_F32 ? 4.0 : 2.0; }

// Algorithmic bytes of one launch: every operand the kernel must touch, counted once.
double alg_bytes(const Plan& plan, const WorkList& wl, const came8_tensor* ts, int phase, bool wd = false) {
  double tot = 0.0;
  for (int32_t i : wl.tids) {
    const DevTensor& d = plan.dev[i];
    const double N = double(d.N), sg = elem_bytes(ts[i].grad_dtype), sp = elem_bytes(ts[i].param_dtype);
    const double nbm = double(d.nbm);
    const double mb = d.fp32st ? 4.0 : 1.0;  // momentum bytes per element
    const double vb = d.fp32st ? 4.0 : 1.0;  // 1-D second-moment bytes per element
    switch (phase) {
      case PH_PASS1: tot += N * sg + double(d.P * d.R) + 4.0 * double(d.nbr); break;              // g, old row codes
      case PH_PASS2: tot += N * (sg + mb) + (d.fp32st ? 0.0 : 4.0 * nbm); break;                  // g, m
      case PH_PASS3: tot += N * (sg + 2.0 * sp + 2.0 * mb) + (d.fp32st ? 0.0 : 8.0 * nbm); break;  // g, p rw, m rw
      case PH_VECA: tot += N * (sg + vb) + (d.fp32st ? 0.0 : 4.0 * nbm); break;                   // g, v
      case PH_VECB: tot += N * (sg + 2.0 * sp + 2.0 * (mb + vb)) + (d.fp32st ? 0.0 : 16.0 * nbm); break;
      case PH_GENERIC:
        tot += d.factored ? N * (sg + 2.0 * sp + 2.0) + 8.0 * nbm : N * (sg + 2.0 * sp + 4.0) + 16.0 * nbm;
        break;
      case PH_TILES2D:  // g, m rw, tile scales rw, column tile sums written (+ row tile sums, scalar form)
        tot += N * (sg + 2.0) + 8.0 * double(d.tr) * double(d.tc) + 4.0 * double(d.C) * d.tr +
               (d.v2d ? 0.0 : 4.0 * double(d.R) * d.tc);
        break;
      case PH_RES2D:  // row tile sums, residual row codes and scales, new row states
        tot += 4.0 * double(d.R) * d.tc + double(d.R) + 4.0 * double(d.nbr) + 4.0 * double(d.R);
        break;
      case PH_PARAM2D:  // m, tile scales, p rw (weight decay folded in)
        tot += N * (1.0 + 2.0 * sp) + 4.0 * double(d.tr) * double(d.tc);
        (void)wd;
        break;
      case PH_NORM_SEG: tot += N * sg; break;  // g (the factors come from cache)
      case PH_FACTOR: case PH_FACTOR_RES:  // one row + one column state: codes rw, scales rw
        tot += 2.0 * double(d.P * d.R + d.P * d.C) + 8.0 * double(d.nbr + d.nbc);
        break;
      default: break;
    }
  }
  return tot;
}

}  // namespace

// ---------------------------------------------------------------------------
// the static scratch of came8_step_static: a workspace that is part of the library's code object, so
// that a step needs no allocation by anyone.  Each GPU the library runs on holds its own copy (at its
// own address) until the process ends.  In host code `scratch` names a host-side stand-in; the device
// address comes from hipGetSymbolAddress, once per device, and only that address is ever used.
// ---------------------------------------------------------------------------
constexpr size_t kStaticScratchBytes = size_t(32) << 20;
constexpr uint64_t kStaticScratchTag = 0x5354415449435343ull;  // the plan-cache tag of the static scratch
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::map<int, void*> g_scratch_ptr;  // device -> address of that device's scratch

int static_scratch(void** out) {
  const int dev = current_device();
  if (dev < 0) return fail(CAME8_EHIP, "came8_step_static: no current HIP device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it == g_scratch_ptr.end()) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(CAME8_EHIP, std::string("came8_step_static: hipGetSymbolAddress of the static scratch failed: ") +
                                  hipGetErrorString(e));
    it = g_scratch_ptr.emplace(dev, ptr).first;
  }
  *out = it->second;
  return CAME8_OK;
}
}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* came8_version(void) { return "came8-mi355x 0.1 (gfx950)"; }
int came8_abi_version(void) { return CAME8_ABI_VERSION; }
int came8_side_stream_count(void) { return int(side_queue_count()); }
const char* came8_last_error(void) { return g_last_error.c_str(); }

int came8_workspace_size(const came8_tensor* tensors, int32_t n_tensors, int32_t block_size, size_t* bytes) {
  if (!bytes) return fail(CAME8_EINVAL, "came8_workspace_size: bytes is NULL");
  // the size of a descriptor set already sized is remembered (callers ask on every step)
  static std::mutex mu;
  static std::map<std::vector<uint8_t>, size_t> sized;
  const std::vector<uint8_t> k = plan_inputs(tensors, n_tensors, block_size, nullptr);
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = sized.find(k);
    if (it != sized.end()) {
      *bytes = it->second;
      return CAME8_OK;
    }
  }
  Plan plan;
  const int rc = build_plan(tensors, n_tensors, block_size, nullptr, plan);
  if (rc != CAME8_OK) return rc;
  *bytes = plan.total_bytes;
  std::lock_guard<std::mutex> lk(mu);
  if (sized.size() >= 64) sized.clear();
  sized[k] = plan.total_bytes;
  return CAME8_OK;
}

int came8_release_workspace(const void* workspace) {
  std::lock_guard<std::mutex> lk(g_cache_mu);
  for (auto it = g_cache.begin(); it != g_cache.end();) {
    if (it->first.first == workspace) {
      drop_entry(it->second);
      it = g_cache.erase(it);
    } else {
      ++it;
    }
  }
  return CAME8_OK;
}

int came8_step(const came8_tensor* tensors, int32_t n_tensors, const came8_hparams* hp_in, void* workspace,
               size_t workspace_bytes, uint64_t workspace_tag, void* stream_ptr) {
  if (!hp_in) return fail(CAME8_EINVAL, "came8_step: hparams is NULL");
  if (n_tensors == 0) return CAME8_OK;
  const came8_hparams& h = *hp_in;
  if (!(h.lr > 0.0)) return fail(CAME8_EINVAL, "came8_step: lr must be > 0");
  if (!(h.clip_threshold > 0.0)) return fail(CAME8_EINVAL, "came8_step: clip_threshold must be > 0");
  if (!workspace) return fail(CAME8_EINVAL, "came8_step: workspace is NULL");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  int rc = CAME8_OK;
  const auto key = std::make_pair(static_cast<const void*>(workspace), workspace_tag);
  std::vector<uint8_t> inputs;
  if (workspace_tag) inputs = plan_inputs(tensors, n_tensors, h.block_size, workspace);
  std::shared_ptr<const Plan> cached;
  if (workspace_tag) {
    std::lock_guard<std::mutex> lk(g_cache_mu);
    auto it = g_cache.find(key);
    if (it != g_cache.end() && it->second.plan && it->second.inputs == inputs) cached = it->second.plan;
  }
  std::shared_ptr<Plan> built;
  if (!cached) {
    // building and uploading a plan copies from host memory and synchronises on the previous upload:
    // neither belongs in a graph
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) {
      (void)hipGetLastError();
      cap = hipStreamCaptureStatusNone;
    }
    if (cap != hipStreamCaptureStatusNone)
      return fail(CAME8_EINVAL, "came8_step: the stream is capturing and no launch plan exists for these tensors and "
                                "this workspace; run one step (or a CAME8_FLAG_PLAN_ONLY call) before capture");
    built = std::make_shared<Plan>();
    rc = build_plan(tensors, n_tensors, h.block_size, static_cast<char*>(workspace), *built);
    if (rc != CAME8_OK) return rc;
  }
  const Plan& plan = cached ? *cached : *built;
  if (workspace_bytes < plan.total_bytes)
    return fail(CAME8_ESPACE, "came8_step: workspace has " + std::to_string(workspace_bytes) + " bytes, needs " +
                                  std::to_string(plan.total_bytes));
  if (built) {
    const uint64_t hsh = fnv1a(built->blob.data(), built->blob.size());
    std::lock_guard<std::mutex> lk(g_cache_mu);
    CacheEntry& ce = g_cache[key];
    ce.inputs.clear();  // set again below once this plan is the one uploaded
    ce.plan.reset();
    if (workspace_tag == 0 || ce.hash != hsh || ce.bytes != built->blob.size()) {
      drop_entry(ce);  // the previous upload from this entry has completed before its source is replaced
      ce.keep = std::move(built->blob);
      hipError_t e = hipMemcpyAsync(workspace, ce.keep.data(), ce.keep.size(), hipMemcpyHostToDevice, stream);
      if (e == hipSuccess) e = hipEventCreateWithFlags(&ce.done, hipEventDisableTiming);
      if (e == hipSuccess) e = hipEventRecord(ce.done, stream);
      if (e != hipSuccess) {
        drop_entry(ce);
        g_cache.erase(key);
        return fail(CAME8_EHIP, std::string("came8_step: plan upload failed: ") + hipGetErrorString(e));
      }
      ce.hash = hsh;
      ce.bytes = ce.keep.size();
    }
    built->blob.clear();  // uploaded (or already on the device): the launches need only the offsets
    built->blob.shrink_to_fit();
    if (workspace_tag) {
      ce.inputs = std::move(inputs);
      ce.plan = built;
    }
  }
  if (h.flags & CAME8_FLAG_PLAN_ONLY) return CAME8_OK;
  // the side stream: neither under capture (a captured step keeps one queue) nor for the static entry
  SideQueue side;
  SideLease lease;  // outlives pq, whose destructor may still join the side stream
  bool use_side = workspace_tag != kStaticScratchTag;
  if (use_side) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) {
      (void)hipGetLastError();
      cap = hipStreamCaptureStatusActive;  // unknown: stay on one queue
    }
    use_side = cap == hipStreamCaptureStatusNone;
  }
  if (use_side && (rc = side_queue(stream, &side, &lease)) != CAME8_OK) return rc;
  PassQueues pq(stream, side, use_side);
  hipStream_t ls = stream;  // the queue of the next launch
  Hp hp = make_hp(h);
  const char* base = static_cast<const char*>(workspace);
  hp.zeros = base + plan.zero_off;
  const DevTensor* dT = reinterpret_cast<const DevTensor*>(base);
  auto tids = [&](const WorkList& wl) { return reinterpret_cast<const int32_t*>(base + wl.tids_off); };
  auto wst = [&](const WorkList& wl) { return reinterpret_cast<const int64_t*>(base + wl.wstart_off); };
  const dim3 blk(kThreads);
  const bool exact_norm = (h.flags & CAME8_FLAG_EXACT_NORM) != 0;
  const bool fastB = fast_block(h.block_size);

  // the chain walks and per-tensor clips of one group of tensors, on queue q
  auto launch_walk = [&](const std::map<int, WorkList>& walks, const std::map<int, WorkList>& finals,
                         hipStream_t q) -> int {
    using FinFn = void (*)(const DevTensor*, const int32_t*, int, Hp);
    int r;
    for (auto& kv : walks) {
      const WorkList& wl = kv.second;
      GenFn fn;
      CAME8_TYPE_SWITCH1(k_norm_walk, kv.first, fn);
      PhaseTimer pt(PH_NORM_WALK, 0.0, q);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), dim3(kNormWalkThreads), 0, q, dT, tids(wl), wst(wl),
                         int(wl.tids.size()), hp);
      if ((r = check_launch("norm_walk")) != CAME8_OK) return r;
    }
    for (auto& kv : finals) {
      const WorkList& wl = kv.second;
      FinFn fn;
      CAME8_TYPE_SWITCH1(k_norm_final, kv.first, fn);
      PhaseTimer pt(PH_NORM_FINAL, 0.0, q);
      hipLaunchKernelGGL(fn, dim3(grid_for(int64_t(wl.tids.size()), kThreads)), blk, 0, q, dT, tids(wl),
                         int(wl.tids.size()), hp);
      if ((r = check_launch("norm_final")) != CAME8_OK) return r;
    }
    return CAME8_OK;
  };
  // P2 of one group of factored tensors: through the pass's queues, or all on queue q
  auto launch_pass2 = [&](const std::map<BandKey, WorkList>& bands, const std::map<int, WorkList>& tinies,
                          bool via_pq, hipStream_t q) -> int {
    int r;
    for (auto& kv : bands) {
      const BandKey& k = kv.first;
      const WorkList& wl = kv.second;
      const BandFn fn = band_fn(k.gdt, true, k.V, k.K, k.TPB, k.st, k.ua, k.ms);
      if (!fn) return fail(CAME8_EINVAL, "came8_step: no band kernel for this variant");
      const double ab = alg_bytes(plan, wl, tensors, PH_PASS2);
      if (!via_pq) ls = q;
      else if ((r = pq.pick(ab, &ls)) != CAME8_OK) return r;
      PhaseTimer pt(PH_PASS2, ab, ls);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), dim3(k.TPB), 0, ls, dT, tids(wl), wst(wl),
                         int(wl.tids.size()), hp);
      if ((r = check_launch("pass2")) != CAME8_OK) return r;
    }
    for (auto& kv : tinies) {
      const WorkList& wl = kv.second;
      GenFn fn;
      CAME8_TYPE_SWITCH1(k_tiny_pass2, kv.first, fn);
      const double ab = alg_bytes(plan, wl, tensors, PH_PASS2);
      if (!via_pq) ls = q;
      else if ((r = pq.pick(ab, &ls)) != CAME8_OK) return r;
      PhaseTimer pt(PH_PASS2, ab, ls);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, ls, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((r = check_launch("tiny_pass2")) != CAME8_OK) return r;
    }
    return CAME8_OK;
  };
  bool split = false;  // the long-chain group runs on the side stream (set by the clip-norm section)

  // ---- P1 and 1-D pass A ----
  // the default clip mode's pass 1 keeps no column sums of g^2/R_i (k_fact_pass1n), except for the
  // 8bit2d tensors, whose clip is formed from them
  const std::map<BandKey, WorkList>& band1 = exact_norm ? plan.band : plan.bandN;
  const std::map<int, WorkList>& vecA = exact_norm ? plan.vecA : plan.vecAn;
  pq.begin(band1.size() + plan.band2dw.size() + plan.tiny1.size() + vecA.size());
  for (const auto* lists : {&band1, &plan.band2dw}) {
    for (auto& kv : *lists) {
      const BandKey& k = kv.first;
      const WorkList& wl = kv.second;
      const BandFn fn = band_fn(k.gdt, false, k.V, k.K, k.TPB, k.st, k.ua, k.ms);
      if (!fn) return fail(CAME8_EINVAL, "came8_step: no band kernel for this variant");
      const double ab = alg_bytes(plan, wl, tensors, PH_PASS1);
      if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
      PhaseTimer pt(PH_PASS1, ab, ls);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), dim3(k.TPB), 0, ls, dT, tids(wl), wst(wl),
                         int(wl.tids.size()), hp);
      if ((rc = check_launch("pass1")) != CAME8_OK) return rc;
    }
  }
  for (auto& kv : plan.tiny1) {
    const WorkList& wl = kv.second;
    GenFn fn;
    CAME8_TYPE_SWITCH1(k_tiny_pass1, kv.first, fn);
    const double ab = alg_bytes(plan, wl, tensors, PH_PASS1);
    if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
    { PhaseTimer pt(PH_PASS1, ab, ls);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, ls, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
    if ((rc = check_launch("tiny_pass1")) != CAME8_OK) return rc; }
  }
  for (auto& kv : vecA) {
    const WorkList& wl = kv.second;
    GenFn fn;
    CAME8_TYPE_SWITCH1(k_vec_passA, kv.first, fn);
    const double ab = alg_bytes(plan, wl, tensors, PH_VECA);
    if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
    { PhaseTimer pt(PH_VECA, ab, ls);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, ls, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
    if ((rc = check_launch("vec_passA")) != CAME8_OK) return rc; }
  }
  if ((rc = pq.finish()) != CAME8_OK) return rc;
  const bool any_fact = !plan.factor.tids.empty();
  if (any_fact) {
    const WorkList& fb = plan.factor;
    { PhaseTimer pt(PH_FACTOR, alg_bytes(plan, fb, tensors, PH_FACTOR), stream);
    hipLaunchKernelGGL(k_factor_blocks<false>, dim3(grid_for(fb.total())), blk, 0, stream, dT, tids(fb), wst(fb),
                       int(fb.tids.size()), hp);
    if ((rc = check_launch("factor_blocks")) != CAME8_OK) return rc; }
  }
  // ---- clip divisor ----
  if (!exact_norm) {  // the update norm in the reference's order (came8_norm.h)
    using EstFn = void (*)(const DevTensor*, const int32_t*, const int64_t*, int, Hp);
    if (!plan.nest_w.tids.empty()) {
      const WorkList& wl = plan.nest_w;
      PhaseTimer pt(PH_NORM_EST, 0.0, stream);
      hipLaunchKernelGGL(k_norm_est<true>, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl),
                         int(wl.tids.size()), hp);
      if ((rc = check_launch("norm_est")) != CAME8_OK) return rc;
    }
    if (!plan.nest_n.tids.empty()) {
      const WorkList& wl = plan.nest_n;
      PhaseTimer pt(PH_NORM_EST, 0.0, stream);
      EstFn fn = k_norm_est<false>;
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((rc = check_launch("norm_est")) != CAME8_OK) return rc;
    }
    pq.begin(plan.nseg2d.size() + plan.nseg.size(), kSideMinNormLaunches);
    for (auto& kv : plan.nseg2d) {
      const WorkList& wl = kv.second;
      const GenFn fn = norm_seg2d_fn(kv.first);
      if (fn == nullptr) return fail(CAME8_EINVAL, "came8_step: no norm kernel for this variant");
      int64_t cmax = 0;  // LDS for the widest matrix of the launch (+ 8 factors for the row form)
      for (int32_t ti : wl.tids) cmax = std::max(cmax, plan.dev[ti].C);
      const int64_t lds = cmax + (kv.first % 3 == kNormRows ? 8 : 0);
      const double ab = alg_bytes(plan, wl, tensors, PH_NORM_SEG);
      if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
      PhaseTimer pt(PH_NORM_SEG, ab, ls);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, size_t(lds) * 4, ls, dT, tids(wl), wst(wl),
                         int(wl.tids.size()), hp);
      if ((rc = check_launch("norm_seg2d")) != CAME8_OK) return rc;
    }
    for (auto& kv : plan.nseg) {
      const WorkList& wl = kv.second;
      const GenFn fn = norm_seg_fn(kv.first);
      if (fn == nullptr) return fail(CAME8_EINVAL, "came8_step: no norm kernel for this variant");
      const double ab = alg_bytes(plan, wl, tensors, PH_NORM_SEG);
      if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
      PhaseTimer pt(PH_NORM_SEG, ab, ls);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, ls, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((rc = check_launch("norm_seg")) != CAME8_OK) return rc;
    }
    if ((rc = pq.finish()) != CAME8_OK) return rc;
    if (!plan.nbsum.tids.empty()) {
      const WorkList& wl = plan.nbsum;
      PhaseTimer pt(PH_NORM_BSUM, 0.0, stream);
      hipLaunchKernelGGL(k_norm_bsum<>, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl),
                         int(wl.tids.size()));
      if ((rc = check_launch("norm_bsum")) != CAME8_OK) return rc;
    }
    pq.begin(plan.nfix.size(), kSideMinNormLaunches);
    for (auto& kv : plan.nfix) {
      const WorkList& wl = kv.second;
      const GenFn fn = norm_fix_fn(kv.first);
      if (fn == nullptr) return fail(CAME8_EINVAL, "came8_step: no norm kernel for this variant");
      int64_t lds = 0;  // column factors of the widest tensor that k_norm_seg2d takes (+ 8 for the row form)
      for (int32_t ti : wl.tids)
        if (plan.dev[ti].nseg0 > 0) lds = std::max(lds, plan.dev[ti].C + (kv.first % 3 == kNormRows ? 8 : 0));
      // (no algorithmic bytes: balanced by work items)
      if ((rc = pq.pick(double(wl.total()), &ls)) != CAME8_OK) return rc;
      PhaseTimer pt(PH_NORM_FIX, 0.0, ls);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, size_t(lds) * 4, ls, dT, tids(wl), wst(wl),
                         int(wl.tids.size()), hp);
      if ((rc = check_launch("norm_fix")) != CAME8_OK) return rc;
    }
    if ((rc = pq.finish()) != CAME8_OK) return rc;
    // the long-chain group walks on the side stream, then takes its clip and its pass 2 there, while the
    // other tensors do the same on the caller's stream; the join comes before the residual factors
    split = plan.walk_split && use_side;
    if (split) {
      if ((rc = pq.fork_now()) != CAME8_OK) return rc;
      if ((rc = launch_walk(plan.nwalkL, plan.nfinalL, side.s)) != CAME8_OK) return rc;
      if ((rc = launch_pass2(plan.band2L, plan.tiny2L, false, side.s)) != CAME8_OK) return rc;
    } else if ((rc = launch_walk(plan.nwalkL, plan.nfinalL, stream)) != CAME8_OK) {
      return rc;
    }
    if ((rc = launch_walk(plan.nwalk, plan.nfinal, stream)) != CAME8_OK) return rc;
  }
  const bool any2d = !plan.tiles2d.empty() || !plan.tiles2d_v.empty();
  if (exact_norm || any2d) {  // reference order: only the 8bit2d tensors take this divisor
    PhaseTimer pt(PH_CLIP, 0.0, stream);
    hipLaunchKernelGGL(k_clip<>, dim3(grid_for(n_tensors)), blk, 0, stream, dT, int(n_tensors), int(!exact_norm), hp);
    if ((rc = check_launch("clip")) != CAME8_OK) return rc;
  }
  // ---- P2, residual factors ----
  if (any_fact) {
    const bool withL = !split;  // else the long-chain group's pass 2 is queued on the side stream already
    pq.begin(plan.band2.size() + plan.tiny2.size() + (withL ? plan.band2L.size() + plan.tiny2L.size() : 0));
    if (split)
      for (auto& kv : plan.band2L) pq.load[1] += alg_bytes(plan, kv.second, tensors, PH_PASS2);
    if ((rc = launch_pass2(plan.band2, plan.tiny2, true, stream)) != CAME8_OK) return rc;
    if (withL && (rc = launch_pass2(plan.band2L, plan.tiny2L, true, stream)) != CAME8_OK) return rc;
    for (auto& kv : plan.tiles2d_v) {
      const WorkList& wl = kv.second;
      GenFn fn;
      CAME8_TYPE_SWITCH1(k_2d_rows, kv.first, fn);
      { PhaseTimer pt(PH_TILES2D, alg_bytes(plan, wl, tensors, PH_TILES2D), stream);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((rc = check_launch("tiles2d")) != CAME8_OK) return rc; }
    }
    for (auto& kv : plan.tiles2d) {
      const WorkList& wl = kv.second;
      GenFn fn;
      CAME8_TYPE_SWITCH1(k_2d_tiles, kv.first, fn);
      { PhaseTimer pt(PH_TILES2D, alg_bytes(plan, wl, tensors, PH_TILES2D), stream);
      hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((rc = check_launch("tiles2d")) != CAME8_OK) return rc; }
    }
    if (!plan.res2d.tids.empty()) {
      const WorkList& wl = plan.res2d;
      PhaseTimer pt(PH_RES2D, alg_bytes(plan, wl, tensors, PH_RES2D), stream);
      hipLaunchKernelGGL(k_2d_res_rows<>, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl),
                         int(wl.tids.size()), hp);
      if ((rc = check_launch("res_rows2d")) != CAME8_OK) return rc;
    }
    if ((rc = pq.finish()) != CAME8_OK) return rc;
    const WorkList& fb = plan.factor;
    { PhaseTimer pt(PH_FACTOR_RES, alg_bytes(plan, fb, tensors, PH_FACTOR_RES), stream);
    hipLaunchKernelGGL(k_factor_blocks<true>, dim3(grid_for(fb.total())), blk, 0, stream, dT, tids(fb), wst(fb),
                       int(fb.tids.size()), hp);
    if ((rc = check_launch("factor_blocks_res")) != CAME8_OK) return rc; }
  }
  // ---- P3 and 1-D pass B ----
  for (auto& kv : plan.param2d_v) {
    const WorkList& wl = kv.second;
    GenFn fn;
    CAME8_TYPE_SWITCH1(k_2d_param_v, kv.first, fn);
    { PhaseTimer pt(PH_PARAM2D, alg_bytes(plan, wl, tensors, PH_PARAM2D, h.weight_decay != 0.0), stream);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
    if ((rc = check_launch("param2d")) != CAME8_OK) return rc; }
  }
  for (auto& kv : plan.param2d_b) {
    const WorkList& wl = kv.second;
    GenFn fn;
    CAME8_TYPE_SWITCH1(k_2d_param_b, kv.first, fn);
    { PhaseTimer pt(PH_PARAM2D, alg_bytes(plan, wl, tensors, PH_PARAM2D, h.weight_decay != 0.0), stream);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
    if ((rc = check_launch("param2d")) != CAME8_OK) return rc; }
  }
  for (auto& kv : plan.param2d) {
    const WorkList& wl = kv.second;
    GenFn fn;
    CAME8_TYPE_SWITCH1(k_2d_param, kv.first, fn);
    { PhaseTimer pt(PH_PARAM2D, alg_bytes(plan, wl, tensors, PH_PARAM2D, h.weight_decay != 0.0), stream);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
    if ((rc = check_launch("param2d")) != CAME8_OK) return rc; }
  }
  if (fastB) {
    pq.begin(plan.upd.size() + plan.updb.size() + plan.vecB.size());
    for (auto& kv : plan.upd) {
      const WorkList& wl = kv.second;
      GenFn fn;
      CAME8_TYPE_SWITCH3(k_fact_pass3, kv.first.pdt, kv.first.gdt, kv.first.st, fn);
      const double ab = alg_bytes(plan, wl, tensors, PH_PASS3);
      if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
      { PhaseTimer pt(PH_PASS3, ab, ls);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, ls, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((rc = check_launch("pass3")) != CAME8_OK) return rc; }
    }
    for (auto& kv : plan.updb) {
      const WorkList& wl = kv.second;
      GenFn fn;
      CAME8_TYPE_SWITCH3(k_fact_pass3b, kv.first.pdt, kv.first.gdt, kv.first.st, fn);
      const double ab = alg_bytes(plan, wl, tensors, PH_PASS3);
      if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
      { PhaseTimer pt(PH_PASS3, ab, ls);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, ls, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((rc = check_launch("pass3")) != CAME8_OK) return rc; }
    }
    for (auto& kv : plan.vecB) {
      const WorkList& wl = kv.second;
      GenFn fn;
      CAME8_TYPE_SWITCH2(k_vec_passB, kv.first.pdt, kv.first.gdt, fn);
      const double ab = alg_bytes(plan, wl, tensors, PH_VECB);
      if ((rc = pq.pick(ab, &ls)) != CAME8_OK) return rc;
      { PhaseTimer pt(PH_VECB, ab, ls);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, ls, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
      if ((rc = check_launch("vec_passB")) != CAME8_OK) return rc; }
    }
    if ((rc = pq.finish()) != CAME8_OK) return rc;
  }
  // every tensor when the block size is not a power of two in [8, 2048]; otherwise only those whose
  // per-matrix momentum blocks end inside a matrix
  for (auto& kv : plan.generic) {
    const WorkList& wl = kv.second;
    GenFn fn;
    CAME8_TYPE_SWITCH2(k_generic_update, kv.first.pdt, kv.first.gdt, fn);
    { PhaseTimer pt(PH_GENERIC, alg_bytes(plan, wl, tensors, PH_GENERIC), stream);
    hipLaunchKernelGGL(fn, dim3(grid_for(wl.total())), blk, 0, stream, dT, tids(wl), wst(wl), int(wl.tids.size()), hp);
    if ((rc = check_launch("generic_update")) != CAME8_OK) return rc; }
  }
  return CAME8_OK;
}

int came8_step_static(const came8_tensor* tensors, int32_t n_tensors, const came8_hparams* hp, void* stream) {
  if (!hp) return fail(CAME8_EINVAL, "came8_step_static: hparams is NULL");
  if (n_tensors == 0) return CAME8_OK;
  void* ws = nullptr;
  int rc = static_scratch(&ws);
  if (rc != CAME8_OK) return rc;
  size_t need = 0;
  if ((rc = came8_workspace_size(tensors, n_tensors, hp->block_size, &need)) != CAME8_OK) return rc;
  if (need > kStaticScratchBytes)
    return fail(CAME8_ESPACE, "came8_step_static: these tensors need " + std::to_string(need) +
                                  " bytes of scratch; the static scratch holds " + std::to_string(kStaticScratchBytes) +
                                  " (use came8_step with a workspace of that size)");
  return came8_step(tensors, n_tensors, hp, ws, kStaticScratchBytes, kStaticScratchTag, stream);
}

int came8_profile_enable(int32_t on) {
  Profiler& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  p.on = on != 0;
  return CAME8_OK;
}

int came8_profile_read(came8_phase_stat* out, int32_t max_phases, int32_t* n_phases, int32_t reset) {
  if (!n_phases) return fail(CAME8_EINVAL, "came8_profile_read: n_phases is NULL");
  Profiler& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  for (const Pending& q : p.pending) {
    float ms = 0.0f;
    if (hipEventSynchronize(q.b) != hipSuccess || hipEventElapsedTime(&ms, q.a, q.b) != hipSuccess)
      return fail(CAME8_EHIP, "came8_profile_read: event query failed");
    p.launches[q.phase] += 1;
    p.total_ms[q.phase] += double(ms);
    p.bytes[q.phase] += q.bytes;
    p.pool.push_back(q.a);
    p.pool.push_back(q.b);
  }
  p.pending.clear();
  int32_t k = 0;
  for (int ph = 0; ph < kNumPhases; ++ph) {
    if (p.launches[ph] == 0) continue;
    if (out && k < max_phases) {
      came8_phase_stat& o = out[k];
      std::memset(&o, 0, sizeof(o));
      std::snprintf(o.name, sizeof(o.name), "%s", kPhaseNames[ph]);
      o.launches = p.launches[ph];
      o.total_ms = p.total_ms[ph];
      o.alg_bytes = p.bytes[ph];
    }
    ++k;
  }
  *n_phases = k;
  if (reset) {
    for (int ph = 0; ph < kNumPhases; ++ph) {
      p.launches[ph] = 0;
      p.total_ms[ph] = 0.0;
      p.bytes[ph] = 0.0;
    }
  }
  return CAME8_OK;
}

int came8_read_clip(const void* workspace, uint64_t workspace_tag, int32_t n_tensors, float* out, void* stream_ptr) {
  if (!workspace || !out) return fail(CAME8_EINVAL, "came8_read_clip: null pointer");
  std::shared_ptr<const Plan> plan;
  {
    std::lock_guard<std::mutex> lk(g_cache_mu);
    auto it = g_cache.find(std::make_pair(workspace, workspace_tag));
    if (it != g_cache.end()) plan = it->second.plan;
  }
  if (!plan) return fail(CAME8_EINVAL, "came8_read_clip: no step has run on this workspace and tag");
  if (size_t(std::max(n_tensors, 0)) != plan->dev.size())
    return fail(CAME8_EINVAL, "came8_read_clip: the last step had " + std::to_string(plan->dev.size()) + " tensors");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  hipError_t e = hipStreamSynchronize(stream);
  for (int32_t i = 0; i < n_tensors && e == hipSuccess; ++i)
    e = hipMemcpy(out + i, plan->dev[i].clip, sizeof(float), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return fail(CAME8_EHIP, std::string("came8_read_clip: ") + hipGetErrorString(e));
  return CAME8_OK;
}

int came8_quantize_blockwise(const float* x, int64_t n, int32_t is_signed, int32_t block_size, void* q, float* absmax,
                             void* stream_ptr) {
  if (block_size <= 0) return fail(CAME8_EINVAL, "came8_quantize_blockwise: block_size must be > 0");
  if (n < 0) return fail(CAME8_EINVAL, "came8_quantize_blockwise: n must be >= 0");
  if (!absmax || (n > 0 && (!x || !q))) return fail(CAME8_EINVAL, "came8_quantize_blockwise: null pointer");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const int64_t nb = std::max<int64_t>(1, ceil_div(n, block_size));
  if (is_signed)
    hipLaunchKernelGGL(k_quantize<true>, dim3(grid_for(nb)), dim3(kThreads), 0, stream, x, n, block_size, nb, q, absmax);
  else
    hipLaunchKernelGGL(k_quantize<false>, dim3(grid_for(nb)), dim3(kThreads), 0, stream, x, n, block_size, nb, q, absmax);
  return check_launch("quantize");
}

int came8_dequantize_blockwise(const void* q, const float* absmax, int64_t n, int32_t is_signed, int32_t block_size,
                               float* out, void* stream_ptr) {
  if (block_size <= 0) return fail(CAME8_EINVAL, "came8_dequantize_blockwise: block_size must be > 0");
  if (n < 0) return fail(CAME8_EINVAL, "came8_dequantize_blockwise: n must be >= 0");
  if (n == 0) return CAME8_OK;
  if (!q || !absmax || !out) return fail(CAME8_EINVAL, "came8_dequantize_blockwise: null pointer");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  if (is_signed)
    hipLaunchKernelGGL(k_dequantize<true>, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, stream, q, absmax, n,
                       block_size, out);
  else
    hipLaunchKernelGGL(k_dequantize<false>, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, stream, q, absmax, n,
                       block_size, out);
  return check_launch("dequantize");
}

}  // extern "C"
