// dk_api.hip — the C ABI of libdk_decode (include/dk_decode.h): argument validation,
// launch planning and the two passes.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "dk_args.h"
#include "dk_decode.h"
#include "dk_launch.h"

namespace dk {
namespace {

int hip_fail(hipError_t e, const char* what) {
  return set_error((int)e, "%s: %s", what, hipGetErrorString(e));
}

int current_device(int device) {
  if (device >= 0) return device;
  int d = 0;
  return hipGetDevice(&d) == hipSuccess ? d : -1;
}

// Compute units of `device` (cached; the count never changes for a device).
int cu_count(int device) {
  // per-device cache; calls from several host threads may fill an entry concurrently
  // (with the same value), hence atomics
  static std::atomic<int> cached[64];
  if (device < 0) return -1;
  if (device < 64) {
    const int c = cached[device].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return -1;
  if (device < 64) cached[device].store(n, std::memory_order_relaxed);
  return n;
}

// Trace ranges around the launches, for rocprofv3 --marker-trace: with the environment
// variable DK_TRACE set (to anything but "" or "0") each pass-1 and merge launch is
// wrapped in a roctx range naming the pass, the schedule and the shape. The roctx library
// is opened at the first call that finds DK_TRACE set, so the library does not link it.
struct Roctx {
  int (*push)(const char*) = nullptr;
  int (*pop)() = nullptr;
};

const Roctx& roctx() {
  static const Roctx r = [] {
    Roctx t;
    const char* e = getenv("DK_TRACE");
    if (!e || !*e || (e[0] == '0' && !e[1])) return t;
    for (const char* name : {"librocprofiler-sdk-roctx.so.1", "libroctx64.so.4"}) {
      void* h = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (!h) continue;
      t.push = reinterpret_cast<int (*)(const char*)>(dlsym(h, "roctxRangePushA"));
      t.pop = reinterpret_cast<int (*)()>(dlsym(h, "roctxRangePop"));
      if (t.push && t.pop) break;
      t = Roctx{};
    }
    return t;
  }();
  return r;
}

// A roctx range for the lifetime of the object (nothing when tracing is off).
class TraceRange {
 public:
  template <class... A>
  explicit TraceRange(const char* fmt, A... args) : on_(roctx().push != nullptr) {
    if (!on_) return;
    char buf[160];
    snprintf(buf, sizeof(buf), fmt, args...);
    roctx().push(buf);
  }
  ~TraceRange() {
    if (on_) roctx().pop();
  }
  TraceRange(const TraceRange&) = delete;
  TraceRange& operator=(const TraceRange&) = delete;

 private:
  bool on_;
};

const void* pass1_fn(int dtype, const Plan& pl, int d) {
  return dtype == DK_F16 ? pass1_symbol<F16>(d, pl.heads, pl.waves, pl.mfma, pl.kv8, pl.balanced)
                         : pass1_symbol<BF16>(d, pl.heads, pl.waves, pl.mfma, pl.kv8, pl.balanced);
}

// Resident pass-1 workgroups per compute unit (occupancy calculator).
int resident_groups(int dtype, const Plan& pl, int d) {
  const void* fn = pass1_fn(dtype, pl, d);
  int blocks = 0;
  if (!fn || hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, pl.waves * 64, 0) !=
                 hipSuccess || blocks <= 0)
    blocks = 1;
  return blocks;
}

int explicit_split(const Problem& p, int device) {
  Problem q = p;
  q.split = 1;
  const Plan pl = make_plan(q);
  const int cus = cu_count(device);
  if (cus <= 0) return hip_fail(hipErrorNoDevice, "compute-unit count");
  const int64_t units = (int64_t)p.batch * pl.pairs_per_seq;
  const int64_t avg = p.batch > 0 ? p.num_indices / p.batch : 0;
  return choose_split(units, (int64_t)cus * resident_groups(p.dtype, pl, p.head_dim), avg,
                      pl.waves);
}

// Explicit split that split_kv == 0 runs with a sliding window (whose pages bound every
// sequence): as many splits of the window's pages as fill the device, down to what
// `ws_bytes` of workspace holds (1: one pass).
int window_split(const Problem& p, int cus, size_t ws_bytes) {
  Problem q = p;
  q.split = 1;
  const Plan p1 = make_plan(q);
  const int64_t avg = p.batch > 0 ? p.num_indices / p.batch : 0;
  const int64_t win_pages = p.opt.window / kPageSize + 2;
  int s = choose_split((int64_t)p.batch * p1.pairs_per_seq,
                       (int64_t)cus * resident_groups(p.dtype, p1, p.head_dim),
                       std::min(avg, win_pages), p1.waves);
  for (; s > 1; --s) {
    size_t o, m, l, total;
    partials_layout_rows(split_rows(p.batch, p.hq, s), p.head_dim, &o, &m, &l, &total);
    if (total <= ws_bytes) break;
  }
  return s;
}

// Wavefronts per compute unit the balanced schedule keeps resident. Two measured best on
// MI355X at every decode shape tried with rows of 256 bytes or more (each wavefront keeps
// two pages of loads in flight), also with 8-16 heads on the MFMA q.k path; four with
// narrower rows (fp8 cache, or D = 64) or 8 q heads on the VALU path (twice the work per
// page).
int waves_per_cu(const Problem& p, const Plan& pl, int hp = 1) {
  if (p.opt.waves_per_cu) return p.opt.waves_per_cu;
  if (hp > 1) return kGroupedWavesPerCU;
  return p.narrow_rows() || (pl.heads >= 8 && !pl.mfma) ? kDefaultWavesPerCUNarrow
                                                        : kDefaultWavesPerCU;
}

// 64-byte kv-head rows (fp8 at D = 64)
bool row64(const Problem& p) { return (int64_t)p.head_dim * p.kv_esize() == 64; }

// Kv heads per workgroup of the balanced schedule (1 = one). Rows of at most
// kNarrowRowBytes per kv head and token: the workgroup serves kGroupedKvHeads neighbouring
// kv heads of the same pages (2 if the kv-head count is not a multiple of it), two
// wavefronts each, so their row segments of each token are fetched together; 64-byte rows
// take kGroupedKvHeadsRow64 of one wavefront each when the kv-head count allows. Not with
// user-set wave counts, nor for problems the plan hint shows to be small (fewer than
// kGroupedMinUnitsPerCU (page, head chunk) units per CU), where it measured slower.

int grouped_kv_heads(const Problem& p, const Plan& pl, int cus) {
  if (p.split != 0 || !p.narrow_rows() || p.opt.waves_per_group || p.opt.waves_per_cu) return 1;
  const int64_t hint = p.opt.max_pages_per_seq;
  if (hint > 0 &&
      (int64_t)p.batch * hint * pl.pairs_per_seq < (int64_t)kGroupedMinUnitsPerCU * cus)
    return 1;
  if (row64(p) && p.hkv % kGroupedKvHeadsRow64 == 0) return kGroupedKvHeadsRow64;
  if (p.hkv % kGroupedKvHeads == 0) return kGroupedKvHeads;
  return p.hkv % 2 == 0 ? 2 : 1;
}

// Wavefronts per kv head of a grouped workgroup of hp kv heads.
int grouped_waves(const Problem& p, int hp) {
  return row64(p) && hp == kGroupedKvHeadsRow64 ? kGroupedWavesRow64 : kGroupedWavesPerKvHead;
}

// Workgroups of the balanced grid: about waves_per_cu wavefronts per compute unit, a
// whole number of workgroups per range (pairs_per_seq / hp of them), at most kMaxWaves
// wavefronts.
int64_t balanced_groups(const Problem& p, const Plan& pl, int cus, int hp = 1) {
  const int64_t hc = pl.pairs_per_seq / hp;
  const int64_t block = (int64_t)pl.waves * hp;
  const int64_t max_groups = std::max<int64_t>(hc, kMaxWaves / block / hc * hc);
  const int64_t groups = std::max<int64_t>(1, (int64_t)cus * waves_per_cu(p, pl, hp) / block);
  return std::min(max_groups, std::max(hc, (groups + hc / 2) / hc * hc));
}

// Whether one workgroup per (sequence, head chunk) with pl's wavefronts per workgroup fits
// in the balanced grid of the same shape, and no sequence (plan hint) is longer than a
// balanced workgroup's share of pages: then one pass finishes no later and needs no merge.
// The plan hint shows near-uniform lengths: the longest sequence (hint pages) within 1/32 of
// the mean (num_indices / batch). 128-bit products: the hint is the caller's.
bool near_uniform(const Problem& p, int64_t hint) {
  return (__int128)hint * p.batch * 32 <= (__int128)p.num_indices * 33;
}

bool one_pass_fits(const Problem& p, const Plan& pl, int cus, int64_t hint) {
  const int64_t groups = balanced_groups(p, pl, cus);
  const int64_t pairs = (int64_t)p.batch * pl.pairs_per_seq;
  const int64_t per_group = groups / pl.pairs_per_seq;   // workgroups per head chunk
  const int64_t share = (p.num_indices + per_group - 1) / per_group;
  return pairs <= groups && hint <= share;
}

// A uniform batch (the longest sequence within 1/32 of the mean, by the plan hint) whose
// (sequence, head chunk) pairs are a whole multiple of kOnePassPairsPerCU per CU: one pass
// beats the balanced schedule and its merge there, at one wavefront per workgroup (two at
// exactly that many pairs, i.e. 8 wavefronts per CU). 32/8/128 fp16 unless noted, us,
// automatic (balanced) vs one pass: pairs 4 per CU, B=128 ctx 2048 / 4096 / 8192: 175.1 vs
// 170.8, 342.9 vs 331.2, 665.9 vs 651.8; 8 per CU, B=256 ctx 1024 / 2048 / 4096: 179.3 vs
// 173.2, 340.5 vs 337.8, 661.9 vs 658.1 (bf16 ctx 1024 180.0 vs 173.8, 64/8 190.9 vs
// 174.4, 16/8 178.9 vs 169.7); 12 per CU (B=384 ctx 1024) 270.5 vs 260.2; 16, 24 and 32
// per CU (B=512 ctx 1024, 768 and 1024 ctx 512): 355.4 vs 346.3, 295.7 vs 278.3, 397.3 vs
// 373.4. Other counts stay balanced: 3, 5, 6, 6.25 and 10 per CU measured 1-18 % slower
// or equal in one pass (B=96 ctx 4096, B=160 and 192 ctx 2048, B=200 and 320 ctx 1024).
// A uniform batch of short sequences (at most kShortOnePassPages pages, the longest within
// 1/32 of the mean) with CUs/4 to CUs (sequence, head chunk) pairs: one pass at 4
// wavefronts per workgroup, which needs no merge kernel and leaves each wavefront a chain
// of at most 8 pages. 32/8/128 fp16, us, automatic (balanced + merge) vs one pass at 4 / 2
// wavefronts per workgroup: B=8 ctx 256 13.4 vs 11.9 / 12.2, ctx 512 14.4 vs 13.9 / 17.5;
// B=16 ctx 256 14.6 vs 12.3 / 12.6, ctx 512 17.8 vs 14.6 / 17.9; at ctx 1024 the balanced
// schedule is faster (B=8 17.6 vs 20.5, B=16 22.2 vs 21.9 / 25.6), and so it is with fewer
// pairs (B=2 ctx 512: 12.8 vs 13.5).
bool short_uniform_pairs(const Problem& p, const Plan& pl, int cus, int64_t hint) {
  const int64_t pairs = (int64_t)p.batch * pl.pairs_per_seq;
  return hint <= kShortOnePassPages && 4 * pairs >= cus && pairs <= cus &&
         near_uniform(p, hint);
}

// The same over an fp8 cache at D = 128 (128-byte rows), at any pair count from CUs/4 up:
// one pass, at 4 wavefronts per workgroup below 8 pairs per CU and at one from there
// (0: not such a batch). 32/8/128, fp16 q, us, automatic (balanced + merge, grouped kv
// heads) vs one pass at 4 / 1 wavefronts per workgroup: B=8 ctx 256 14.6 vs 11.3 / 16.4,
// ctx 512 15.5 vs 14.0 / 25.4; B=16 ctx 256 15.7 vs 11.6 / 16.4, ctx 512 17.2 vs 14.2 /
// 25.6; B=64 ctx 256 22.6 vs 16.1 / 17.5, ctx 512 28.9 vs 22.1 / 27.0; B=128 ctx 256 30.7
// vs 24.4 / 25.9, ctx 512 37.7 vs 35.4 / 41.5; B=256 ctx 256 45.2 vs 41.9 / 38.5, ctx 512
// 67.1 vs 62.7 / 65.4; B=512 ctx 256 80.8 vs 75.0 / 61.2, ctx 512 125.5 vs 116.1 / 105.5;
// B=1024 ctx 256 156.8 vs 140.5 / 121.7. At ctx 1024 the balanced schedule stays faster
// (B=256 105.8 vs 109.2 / 119.9).
int short_uniform_fp8_waves(const Problem& p, const Plan& pl, int cus, int64_t hint) {
  const int64_t pairs = (int64_t)p.batch * pl.pairs_per_seq;
  if (hint > kShortOnePassPages || 4 * pairs < cus || !near_uniform(p, hint))
    return 0;
  return pairs < 8 * (int64_t)cus ? 4 : 1;
}

// The same at D = 64 (16-bit rows of 128 bytes, fp8 rows of 64): one pass at 4
// wavefronts per workgroup for CUs/4 to 2 * CUs pairs. 32/8/64, us, automatic (balanced +
// merge, grouped kv heads where the rows are narrow) vs one pass at 4 / 1 wavefronts per
// workgroup: fp16 B=16 ctx 256 13.1 vs 10.7 / 14.1, ctx 512 15.0 vs 11.9 / 20.0; B=64 ctx
// 256 19.0 vs 14.4 / 15.2, ctx 512 23.1 vs 18.5 / 21.8; fp8 B=16 ctx 256 14.2 vs 10.4 /
// 14.3, ctx 512 15.7 vs 12.3 / 21.3; B=64 ctx 256 20.0 vs 14.4 / 15.2, ctx 512 25.4 vs 19.6
// / 22.9. At 8 pairs per CU it is mixed (B=256 ctx 256 / 512: fp16 34.9 vs 32.6 / 31.8,
// 54.9 vs 52.7 / 54.9; fp8 32.8 vs 31.1 / 32.8, 45.3 vs 52.7 / 56.2), so not there.
bool short_uniform_d64(const Problem& p, const Plan& pl, int cus, int64_t hint) {
  const int64_t pairs = (int64_t)p.batch * pl.pairs_per_seq;
  return hint <= kShortOnePassPages && 4 * pairs >= cus && pairs <= 2 * (int64_t)cus &&
         near_uniform(p, hint);
}

bool uniform_many_pairs(const Problem& p, const Plan& pl, int cus, int64_t hint) {
  const int64_t pairs = (int64_t)p.batch * pl.pairs_per_seq;
  const int64_t unit = (int64_t)kOnePassPairsPerCU * cus;
  return unit > 0 && pairs >= unit && pairs % unit == 0 &&
         near_uniform(p, hint);
}

// Wavefronts per workgroup of the one-pass kernel that split_kv == 0 runs, or 0 for the
// balanced schedule. Forced by options.schedule; else only with the max_pages_per_seq
// hint, when one pass fits (one_pass_fits) at the default wavefronts per workgroup, or, for
// 256-byte rows (16-bit caches at D = 128) with the default wave counts, at one wavefront
// per workgroup: twice the workgroups at the same wavefronts per CU, so that uniform
// batches of up to twice the CUs' (sequence, kv head) pairs run without the merge (B=64
// ctx 4096, us, balanced vs one pass NW=1: 32/8 161.2 vs 160.0, bf16 161.9 vs 160.3, 64/8
// 177.9 vs 165.3; B=64 ctx 8192 317.4 vs 314.4; slower where the pairs do not fill the
// CUs evenly, e.g. B=48 127.2 vs 148.1, which the share condition excludes, and over
// narrow rows, e.g. fp8 96.1 vs 157.7). With the same rows and wave counts, uniform
// batches of short sequences (short_uniform_pairs) and of many pairs (uniform_many_pairs)
// run one pass too, and over an fp8 cache at D = 128 (short_uniform_fp8_waves) or at
// D = 64 (short_uniform_d64) uniform batches of short sequences. Rows of 128 bytes (fp8
// D = 128 up to 4 q heads per kv head, 16-bit D = 64 up to 8) with sequences of more than
// kNarrowOnePassMaxPages pages stay balanced where that groups kv heads. Pass-1-only calls
// always take the balanced schedule (they return partials).
int auto_one_pass(const Problem& p, const Plan& pl, int cus) {
  if (!p.need_out || p.opt.schedule == 1) return 0;
  if (p.opt.schedule == 2) return pl.waves;
  const int64_t hint = p.opt.max_pages_per_seq;
  const bool auto_waves = !p.opt.waves_per_group && !p.opt.waves_per_cu;
  // D = 64 (rows of 128 or 64 bytes), VALU q.k, default wave counts: short uniform batches
  if (hint > 0 && auto_waves && p.head_dim == 64 && !pl.mfma &&
      pl.waves == kDefaultWavesPerGroupNarrow && short_uniform_d64(p, pl, cus, hint))
    return kDefaultWavesPerGroupNarrow;
  // rows of at most 64 bytes: the balanced schedule with grouped kv heads
  if ((int64_t)p.head_dim * p.kv_esize() <= kGroupedAlwaysRowBytes &&
      grouped_kv_heads(p, pl, cus) > 1)
    return 0;
  if (hint <= 0) return 0;
  // 128-byte rows (16-bit up to 8 q heads per kv head, fp8 up to 4 on the VALU q.k path),
  // sequences of more than kNarrowOnePassMaxPages pages: balanced with grouped kv heads
  // even where one pass fits
  if (auto_waves && (int64_t)p.head_dim * p.kv_esize() == kNarrowRowBytes &&
      (p.kv_esize() == 2 ? pl.heads <= 8 : !pl.mfma && pl.heads <= 4) &&
      hint > kNarrowOnePassMaxPages && grouped_kv_heads(p, pl, cus) > 1)
    return 0;
  if (one_pass_fits(p, pl, cus, hint)) return pl.waves;
  if (auto_waves && pl.waves == kDefaultWavesPerGroup &&
      waves_per_cu(p, pl) == kDefaultWavesPerCU && p.head_dim == 128 && p.kv_esize() == 2) {
    if (short_uniform_pairs(p, pl, cus, hint)) return kDefaultWavesPerGroupNarrow;
    Plan one = pl;
    one.waves = 1;
    if (one_pass_fits(p, one, cus, hint)) return 1;
    if (uniform_many_pairs(p, pl, cus, hint))
      return (int64_t)p.batch * pl.pairs_per_seq == (int64_t)kOnePassPairsPerCU * cus ? 2 : 1;
  }
  // fp8 cache at D = 128 (128-byte rows), VALU q.k, default wave counts
  if (auto_waves && p.head_dim == 128 && p.kv_esize() == 1 && !pl.mfma &&
      pl.waves == kDefaultWavesPerGroupNarrow)
    return short_uniform_fp8_waves(p, pl, cus, hint);
  return 0;
}

// The explicit split that split_kv == 0 runs for a uniform batch over 256-byte rows whose
// (sequence, kv head) pairs divide the balanced grid into S >= 2 ranges of at least
// kSplitFillMinPages pages (0: not such a batch, or its partials would not fit ws_bytes).
// Full calls only: the pass-1-only entry point returns the balanced schedule's partials.
int auto_split_fill(const Problem& p, const Plan& pl, int cus, size_t ws_bytes) {
  const int64_t hint = p.opt.max_pages_per_seq;
  const bool auto_waves = !p.opt.waves_per_group && !p.opt.waves_per_cu;
  if (!p.need_out || p.opt.schedule != 0 || hint <= 0 || !auto_waves || pl.mfma ||
      (int64_t)p.head_dim * p.kv_esize() != 256 || pl.waves != kDefaultWavesPerGroup ||
      waves_per_cu(p, pl) != kDefaultWavesPerCU || !near_uniform(p, hint))
    return 0;
  const int64_t pairs = (int64_t)p.batch * pl.pairs_per_seq;
  const int64_t groups = balanced_groups(p, pl, cus);
  if (pairs <= 0 || groups % pairs != 0) return 0;
  const int64_t s = groups / pairs;
  if (s < 2 || s > kMaxSplit || (hint + s - 1) / s < kSplitFillMinPages) return 0;
  size_t o, m, l, total;
  partials_layout_rows(split_rows(p.batch, p.hq, (int)s), p.head_dim, &o, &m, &l, &total);
  return total <= ws_bytes ? (int)s : 0;
}

// Whether a caller's explicit split over 256-byte rows runs 4 wavefronts per workgroup
// (kShortSplitPages): its workgroups are fewer than the CUs; as many as the CUs, streaming
// short runs of pages (the mean sequence's pages per split); or up to twice as many, so
// that all their wavefronts are resident at once (2 per SIMD).
bool short_split_runs(const Problem& p, const Plan& pl, int cus) {
  if (p.split < 1 || pl.balanced || p.opt.waves_per_group || p.opt.waves_per_cu ||
      p.opt.window > 0 || pl.mfma || pl.waves != kDefaultWavesPerGroup ||
      (int64_t)p.head_dim * p.kv_esize() != 256)
    return false;
  const int64_t groups = (int64_t)p.batch * p.hkv * pl.chunks * p.split;
  const int64_t avg = p.num_indices / p.batch;
  const int64_t pps = (avg + p.split - 1) / p.split;
  if (groups > 2 * (int64_t)cus) return false;
  return groups != cus || pps <= kShortSplitPages;
}

}  // namespace

// Validation, planning and both passes; shared by the extern "C" entry points.
int run(Problem p, bool do_merge, void* stream) {
  clear_error();
  const int rc = validate(p);
  if (rc != DK_OK || p.batch == 0) return rc;
  Plan pl = make_plan(p);
  if (!pl.balanced) {
    const int cus = cu_count(current_device(-1));
    if (cus > 0 && short_split_runs(p, pl, cus)) pl.waves = kDefaultWavesPerGroupNarrow;
  }
  int waves_per_pair = 0;   // balanced: workgroups per head chunk
  int seg_cost = 0;         // balanced: pages charged per change of sequence
  int hp = 1;               // balanced: kv heads per workgroup
  if (pl.balanced && p.opt.window > 0) {
    // a sliding window bounds every sequence's pages: explicit splits of the window's
    // pages, as many as fill the device and fit the workspace
    if (!p.need_out)
      return set_error(DK_EUNSUPPORTED, "pass 1 alone with a sliding window needs an explicit "
                                        "split_kv");
    const int dev = current_device(-1);
    const int cus = cu_count(dev);
    if (cus <= 0) return hip_fail(hipErrorNoDevice, "compute-unit count");
    p.split = window_split(p, cus, p.workspace_bytes);
    pl = make_plan(p);
  }
  if (pl.balanced) {
    const int dev = current_device(-1);
    const int cus = cu_count(dev);
    if (cus <= 0) return hip_fail(hipErrorNoDevice, "compute-unit count");
    if (const int one_pass_waves = auto_one_pass(p, pl, cus)) {
      p.split = 1;
      pl.balanced = false;
      pl.waves = one_pass_waves;
      pl.grid = split_grid(p.batch, p.hkv, 1, pl.chunks);
    } else if (const int s = auto_split_fill(p, pl, cus, p.workspace_bytes)) {
      p.split = s;
      pl = make_plan(p);
    } else {
      hp = grouped_kv_heads(p, pl, cus);
      const int64_t hint = p.opt.max_pages_per_seq;
      const bool auto_waves = !p.opt.waves_per_group && !p.opt.waves_per_cu;
      if (hp > 1) {
        pl.waves = grouped_waves(p, hp);
      } else if (hint > 0 && auto_waves && pl.waves < kDefaultWavesPerGroupNarrow &&
                 (int64_t)p.batch * hint * pl.pairs_per_seq <= (int64_t)kSmallUnitsPerCU * cus) {
        pl.waves = kDefaultWavesPerGroupNarrow;
        p.opt.waves_per_cu = kDefaultWavesPerCUNarrow;
      } else if (hint > 0 && auto_waves && pl.waves > 1) {
        // short sequences: when even the longest is at most 1/kShortSegments of a
        // workgroup's page range, one wavefront per workgroup (same wavefronts per CU)
        const int64_t groups = balanced_groups(p, pl, cus);
        const int64_t per_chunk = std::max<int64_t>(groups / pl.pairs_per_seq, 1);
        const int64_t range = (p.num_indices + per_chunk - 1) / per_chunk;
        if (hint * kShortSegments <= range) pl.waves = 1;
      }
      pl.grid = balanced_groups(p, pl, cus, hp);
      waves_per_pair = (int)(pl.grid / (pl.pairs_per_seq / hp));
      // a ragged batch (plan hint: the longest sequence well above the mean): charge each
      // change of sequence in the range split, so that ranges crossing more sequences get
      // fewer pages (a kernel build of its own)
      if (hint > 0 && p.batch > 1 &&
          hint * (int64_t)p.batch * 4 > p.num_indices * (int64_t)5)
        seg_cost = kSegmentCostPerWave * pl.waves;   // per head's pages (any kv heads per group)
    }
  }
  const bool direct = p.need_out && (p.split == 1 || pl.balanced);
  const int64_t esize = 2;              // q and out
  const int64_t kes = p.kv_esize();     // the cache

  Pass1Args a{};
  a.q = static_cast<const uint8_t*>(p.q);
  a.kv = static_cast<const uint8_t*>(p.kv);
  a.indptr = p.indptr;
  a.indices = p.indices;
  a.last_len = p.last_len;
  // Partials: every call but a full one-pass call (the balanced schedule writes them for
  // the sequences that span several workgroups even when it writes `out` directly; the
  // pass-1-only entry point writes them for split_kv == 1 too).
  const bool need_partials = !(p.need_out && p.split == 1);
  if (need_partials) {
    const int64_t rows = pl.balanced ? balanced_rows(p.batch, p.hq, p.hkv, p.head_dim)
                                     : split_rows(p.batch, p.hq, p.split);
    size_t off_o, off_m, off_l, total;
    partials_layout_rows(rows, p.head_dim, &off_o, &off_m, &off_l, &total);
    uint8_t* ws = static_cast<uint8_t*>(p.workspace);
    a.part_o = reinterpret_cast<float*>(ws + off_o);
    a.part_m = reinterpret_cast<float*>(ws + off_m);
    a.part_l = reinterpret_cast<float*>(ws + off_l);
  }
  a.out = static_cast<uint8_t*>(p.out);
  a.q_b = p.st.q_b * esize;
  a.q_h = p.st.q_h * esize;
  a.kv_p = p.st.kv_p * kes;
  a.o_b = p.st.o_b * esize;
  a.o_h = p.st.o_h * esize;
  // V slice of a page: kv_r further in the combined cache, or the same offset in the
  // separate V cache
  a.kv_v = p.v ? (int64_t)((const uint8_t*)p.v - (const uint8_t*)p.kv) : p.st.kv_r * kes;
  a.kv_s = (int32_t)(p.st.kv_s * kes);
  a.kv_h = (int32_t)(p.st.kv_h * kes);
  a.batch = p.batch;
  a.hq = p.hq;
  a.hkv = p.hkv;
  a.group = pl.group;
  a.chunks = pl.chunks;
  a.per = pl.per;
  a.window = p.opt.window;
  a.split = std::max(p.split, 1);
  a.num_indices = (int32_t)p.num_indices;
  a.num_pages = (uint32_t)std::min<int64_t>(p.num_pages, (int64_t)1 << 31);
  // bytes from a kv head's K (or V) slice base that its rows reach (validated < 2^31)
  a.page_extent = (uint32_t)(((int64_t)(kPageSize - 1) * p.st.kv_s + p.head_dim) * kes);
  a.direct = direct ? 1 : 0;
  a.ranges = waves_per_pair;
  a.seg_cost = pl.balanced ? seg_cost : 0;
  const bool kv8 = pl.kv8;
  const float k_scale = kv8 && p.opt.k_scale != 0.f ? p.opt.k_scale : 1.f;
  const float score_scale =
      k_scale * (p.opt.sm_scale != 0.f ? p.opt.sm_scale : 1.f / sqrtf((float)p.head_dim));
  a.kscale = kLog2e * score_scale;
  // soft-capped scores: log2(e) * cap * tanh(q.k * score_scale / cap)
  a.cap_in = p.opt.logit_cap > 0.f ? score_scale / p.opt.logit_cap : 0.f;
  a.cap_out = p.opt.logit_cap > 0.f ? kLog2e * p.opt.logit_cap : 0.f;
  a.vscale = kv8 && p.opt.v_scale != 0.f ? p.opt.v_scale : 1.f;
  a.sinks = p.need_out ? p.opt.sinks : nullptr;   // partials (pass 1 alone) stay plain
  // every launch that can store partials has them (or the library is inconsistent)
  if ((pl.balanced || !direct) && (!a.part_o || !a.part_m || !a.part_l))
    return set_error(DK_EWORKSPACE, "internal: partials not assigned for this schedule");

  Pass1Launch L;
  L.d = p.head_dim;
  L.heads = pl.heads;
  L.waves = pl.waves;
  L.mfma = pl.mfma;
  L.balanced = pl.balanced;
  L.kv8 = pl.kv8;
  L.hp = hp;
  L.cost = a.seg_cost > 0;
  L.grid = (int)pl.grid;
  if (pl.balanced && pl.chunks > 1) {
    // the chunks of a (range, kv-head group) unit sit kXcds workgroup ids apart: whole
    // rounds
    const int64_t units = (int64_t)(p.hkv / hp) * waves_per_pair;
    L.grid = (int)((units + kXcds - 1) / kXcds * kXcds * pl.chunks);
  }
  L.stream = static_cast<hipStream_t>(stream);
  hipError_t e;
  {
    TraceRange tr("dk_pass1 %s B=%d Hq=%d Hkv=%d D=%d split=%d grid=%d waves=%d",
                  pl.balanced ? "balanced" : (p.split == 1 ? "one-pass" : "split"), p.batch,
                  p.hq, p.hkv, p.head_dim, p.split, L.grid, L.waves * L.hp);
    e = p.dtype == DK_F16 ? launch_pass1<F16>(a, L) : launch_pass1<BF16>(a, L);
  }
  if (e != hipSuccess) return hip_fail(e, "pass-1 launch");

  if (do_merge && p.split != 1) {
    MergeArgs m{};
    m.po = a.part_o;
    m.pm = a.part_m;
    m.pl = a.part_l;
    m.out = a.out;
    m.o_b = a.o_b;
    m.o_h = a.o_h;
    m.batch = p.batch;
    m.hq = p.hq;
    m.split = a.split;
    m.indptr = p.indptr;
    m.num_indices = a.num_indices;
    m.pairs_per_seq = pl.pairs_per_seq;
    m.heads = pl.heads;
    m.group = pl.group;
    m.per = pl.per;
    m.chunks = pl.chunks;
    m.hkv = p.hkv;
    m.waves_per_pair = waves_per_pair;
    m.seg_cost = a.seg_cost;
    m.sinks = a.sinks;
    TraceRange tr("dk_merge %s B=%d Hq=%d D=%d", pl.balanced ? "balanced" : "split",
                  p.batch, p.hq, p.head_dim);
    e = p.dtype == DK_F16 ? launch_merge<F16>(m, p.head_dim, pl.balanced, L.stream)
                          : launch_merge<BF16>(m, p.head_dim, pl.balanced, L.stream);
    if (e != hipSuccess) return hip_fail(e, "merge launch");
  }
  return DK_OK;
}

}  // namespace dk

// ---------------------------------------------------------------- static scratch
// Device memory of dk_decode_attention_noalloc: every GPU the library runs on holds one
// copy of this array until the process ends. In host code `scratch` is only a handle for
// the runtime; its device address on the current GPU comes from hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[DK_STATIC_SCRATCH_BYTES];

namespace dk {
namespace {

// Device address of `scratch` on `device` (the current device), looked up once per device
// with hipGetSymbolAddress; nullptr (and *err set) if the lookup fails.
void* scratch_ptr(int device, hipError_t* err) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  *err = hipSuccess;
  if (device < 0 || device >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
      return nullptr;
    }
    ptrs[device] = p;
  }
  return ptrs[device];
}

}  // namespace
}  // namespace dk

// ---------------------------------------------------------------- C ABI
using dk::Problem;

static Problem make_problem(const void* q, const void* kv, const void* v, const int32_t* indptr,
                            const int32_t* indices, const int32_t* last_len, void* out,
                            void* ws, size_t ws_bytes, int32_t batch, int32_t hq, int32_t hkv,
                            int32_t d, int32_t page, int64_t num_pages, int64_t num_indices,
                            int32_t dtype, const dk_strides* st, int32_t split,
                            const dk_options* opts, bool need_out) {
  Problem p;
  p.q = q;
  p.kv = kv;
  p.v = v;
  p.indptr = indptr;
  p.indices = indices;
  p.last_len = last_len;
  p.out = out;
  p.workspace = ws;
  p.workspace_bytes = ws_bytes;
  p.batch = batch;
  p.hq = hq;
  p.hkv = hkv;
  p.head_dim = d;
  p.page_size = page;
  p.num_pages = num_pages;
  p.num_indices = num_indices;
  p.dtype = dtype;
  if (st) p.st = *st;
  p.split = split;
  if (opts) p.opt = *opts;
  p.need_out = need_out;
  return p;
}

extern "C" {

int dk_abi_version(void) { return DK_ABI_VERSION; }

const char* dk_last_error(void) { return dk::last_error(); }

size_t dk_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t split_kv) {
  return dk::workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, split_kv);
}

int dk_partials_layout(int32_t batch, int32_t num_q_heads, int32_t head_dim, int32_t split_kv,
                       size_t* off_o, size_t* off_m, size_t* off_l, size_t* total) {
  dk::clear_error();
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || split_kv <= 0 || !off_o || !off_m ||
      !off_l || !total)
    return dk::set_error(DK_EINVAL, "dk_partials_layout: bad argument");
  dk::partials_layout_rows(dk::split_rows(batch, num_q_heads, split_kv), head_dim, off_o, off_m,
                           off_l, total);
  return DK_OK;
}

int dk_choose_split(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                    int32_t dtype, int64_t avg_pages_per_seq, int32_t device) {
  dk::clear_error();
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      (dtype != DK_F16 && dtype != DK_BF16) || avg_pages_per_seq < 0 ||
      avg_pages_per_seq > INT32_MAX || (int64_t)batch * num_q_heads > dk::kMaxRows)
    return dk::set_error(DK_EINVAL, "dk_choose_split: bad argument");
  Problem p;
  p.batch = batch;
  p.hq = num_q_heads;
  p.hkv = num_kv_heads;
  p.head_dim = head_dim;
  p.dtype = dtype;
  p.num_indices = avg_pages_per_seq * (int64_t)batch;
  p.split = 1;
  const int dev = dk::current_device(device);
  if (dev < 0) return dk::hip_fail(hipErrorNoDevice, "dk_choose_split");
  return dk::explicit_split(p, dev);
}

int dk_plan_schedule(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     int64_t num_indices, int32_t dtype, int32_t split_kv,
                     const dk_options* opts, int32_t device) {
  dk::clear_error();
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256) || split_kv < 0 ||
      split_kv > dk::kMaxSplit || num_indices < 0 || (dtype != DK_F16 && dtype != DK_BF16) ||
      (int64_t)batch * num_q_heads > dk::kMaxRows)
    return dk::set_error(DK_EINVAL, "dk_plan_schedule: bad argument");
  if (split_kv != 0) return split_kv;
  Problem p;
  p.batch = batch;
  p.hq = num_q_heads;
  p.hkv = num_kv_heads;
  p.head_dim = head_dim;
  p.num_indices = num_indices;
  p.dtype = dtype;
  if (opts) p.opt = *opts;
  if (p.opt.schedule < 0 || p.opt.schedule > 2)
    return dk::set_error(DK_EINVAL, "options.schedule must be 0, 1 or 2; got %d", p.opt.schedule);
  const int dev = dk::current_device(device);
  const int cus = dk::cu_count(dev);
  if (cus <= 0) return dk::hip_fail(hipErrorNoDevice, "dk_plan_schedule");
  if (p.opt.window > 0)   // explicit splits of the window, in the default workspace
    return dk::window_split(p, cus, dk::workspace_bytes(batch, num_q_heads, num_kv_heads,
                                                        head_dim, 0));
  const dk::Plan pl = dk::make_plan(p);
  if (dk::auto_one_pass(p, pl, cus) > 0) return 1;
  return dk::auto_split_fill(p, pl, cus,
                             dk::workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, 0));
}

int dk_decode_attention_ex(const void* q, const void* kv_data, const int32_t* kv_indptr,
                           const int32_t* kv_indices, const int32_t* kv_last_page_len,
                           void* out, void* workspace, size_t workspace_bytes, int32_t batch,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t page_size, int64_t num_pages, int64_t num_indices,
                           int32_t dtype, const dk_strides* strides, int32_t split_kv,
                           const dk_options* opts, void* hip_stream) {
  dk::clear_error();
  if (!strides) return dk::set_error(DK_ENULL, "strides must be non-NULL");
  Problem p = make_problem(q, kv_data, nullptr, kv_indptr, kv_indices, kv_last_page_len, out,
                           workspace,
                           workspace_bytes, batch, num_q_heads, num_kv_heads, head_dim,
                           page_size, num_pages, num_indices, dtype, strides, split_kv, opts,
                           true);
  return dk::run(p, true, hip_stream);
}

int dk_decode_attention_noalloc(const void* q, const void* kv_data, const int32_t* kv_indptr,
                                const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                void* out, int32_t batch, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                int64_t num_pages, int64_t num_indices, int32_t dtype,
                                const dk_strides* strides, int32_t split_kv,
                                const dk_options* opts, void* hip_stream) {
  dk::clear_error();
  if (!strides) return dk::set_error(DK_ENULL, "strides must be non-NULL");
  // the scratch this call needs, checked before any device call
  const size_t need =
      dk::workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim, split_kv);
  if (need > (size_t)DK_STATIC_SCRATCH_BYTES)
    return dk::set_error(DK_EWORKSPACE,
                         "dk_decode_attention_noalloc: this call needs %zu bytes of scratch, "
                         "more than the %u of the library's static scratch; use "
                         "dk_decode_attention_ex with a workspace",
                         need, (unsigned)DK_STATIC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0 && batch > 0) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return dk::hip_fail(e, "dk_decode_attention_noalloc: current device");
    ws = dk::scratch_ptr(dev, &e);
    if (!ws) return dk::hip_fail(e, "dk_decode_attention_noalloc: static scratch address");
  }
  Problem p = make_problem(q, kv_data, nullptr, kv_indptr, kv_indices, kv_last_page_len, out,
                           ws, ws ? (size_t)DK_STATIC_SCRATCH_BYTES : 0, batch, num_q_heads,
                           num_kv_heads, head_dim, page_size, num_pages, num_indices, dtype,
                           strides, split_kv, opts, true);
  return dk::run(p, true, hip_stream);
}

int dk_decode_attention_kv(const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* kv_indptr, const int32_t* kv_indices,
                           const int32_t* kv_last_page_len, void* out, void* workspace,
                           size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                           int64_t num_pages, int64_t num_indices, int32_t dtype,
                           const dk_strides* strides, int32_t split_kv, const dk_options* opts,
                           void* hip_stream) {
  dk::clear_error();
  if (!strides) return dk::set_error(DK_ENULL, "strides must be non-NULL");
  if (batch > 0 && (!k_cache || !v_cache))
    return dk::set_error(DK_ENULL, "k_cache and v_cache must be non-NULL");
  Problem p = make_problem(q, k_cache, v_cache, kv_indptr, kv_indices, kv_last_page_len, out,
                           workspace, workspace_bytes, batch, num_q_heads, num_kv_heads,
                           head_dim, page_size, num_pages, num_indices, dtype, strides, split_kv,
                           opts, true);
  return dk::run(p, true, hip_stream);
}

int dk_decode_attention(const void* q, const void* kv_data, const int32_t* kv_indptr,
                        const int32_t* kv_indices, const int32_t* kv_last_page_len, void* out,
                        void* workspace, size_t workspace_bytes, int32_t batch,
                        int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t page_size, int64_t num_pages, int64_t num_indices,
                        int32_t dtype, const dk_strides* strides, int32_t split_kv,
                        void* hip_stream) {
  return dk_decode_attention_ex(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, out,
                                workspace, workspace_bytes, batch, num_q_heads, num_kv_heads,
                                head_dim, page_size, num_pages, num_indices, dtype, strides,
                                split_kv, nullptr, hip_stream);
}

int dk_decode_partials(const void* q, const void* kv_data, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* kv_last_page_len,
                       void* workspace, size_t workspace_bytes, int32_t batch,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       int32_t page_size, int64_t num_pages, int64_t num_indices, int32_t dtype,
                       const dk_strides* strides, int32_t split_kv, const dk_options* opts,
                       void* hip_stream) {
  dk::clear_error();
  if (!strides) return dk::set_error(DK_ENULL, "strides must be non-NULL");
  Problem p = make_problem(q, kv_data, nullptr, kv_indptr, kv_indices, kv_last_page_len, nullptr,
                           workspace, workspace_bytes, batch, num_q_heads, num_kv_heads,
                           head_dim, page_size, num_pages, num_indices, dtype, strides,
                           split_kv, opts, false);
  return dk::run(p, false, hip_stream);
}

int dk_merge_partials(const void* workspace, size_t workspace_bytes, void* out, int32_t batch,
                      int32_t num_q_heads, int32_t head_dim, int32_t dtype, int64_t o_b,
                      int64_t o_h, int32_t split_kv, void* hip_stream) {
  dk::clear_error();
  if (batch < 0 || num_q_heads <= 0 || split_kv < 1 || split_kv > dk::kMaxSplit ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      (dtype != DK_F16 && dtype != DK_BF16) || o_b < 0 || o_h < 0)
    return dk::set_error(DK_EINVAL, "dk_merge_partials: bad argument");
  if (batch == 0) return DK_OK;
  if (!workspace || !out) return dk::set_error(DK_ENULL, "workspace and out must be non-NULL");
  // the partials are read as float vectors from 256-byte aligned arrays
  if (((uintptr_t)workspace % 256) != 0)
    return dk::set_error(DK_EWORKSPACE, "workspace must be 256-byte aligned");
  if ((int64_t)batch * num_q_heads > dk::kMaxRows)
    return dk::set_error(DK_EINVAL, "dk_merge_partials: batch*num_q_heads too large");
  if (!dk::extent_ok(batch, o_b, num_q_heads, o_h, head_dim, 2))
    return dk::set_error(DK_EUNSUPPORTED,
                         "dk_merge_partials: out strides must be below 2^40 elements and span "
                         "less than 2^62 bytes");
  size_t off_o, off_m, off_l, need;
  dk::partials_layout_rows(dk::split_rows(batch, num_q_heads, split_kv), head_dim, &off_o,
                           &off_m, &off_l, &need);
  if (workspace_bytes < need)
    return dk::set_error(DK_EWORKSPACE, "workspace of %zu bytes required, %zu given", need,
                         workspace_bytes);
  const uint8_t* ws = static_cast<const uint8_t*>(workspace);
  dk::MergeArgs m{};
  m.po = reinterpret_cast<const float*>(ws + off_o);
  m.pm = reinterpret_cast<const float*>(ws + off_m);
  m.pl = reinterpret_cast<const float*>(ws + off_l);
  m.out = static_cast<uint8_t*>(out);
  m.o_b = o_b * 2;
  m.o_h = o_h * 2;
  m.batch = batch;
  m.hq = num_q_heads;
  m.split = split_kv;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  hipError_t e = dtype == DK_F16 ? dk::launch_merge<dk::F16>(m, head_dim, false, st)
                                 : dk::launch_merge<dk::BF16>(m, head_dim, false, st);
  if (e != hipSuccess) return dk::hip_fail(e, "merge launch");
  return DK_OK;
}

}  // extern "C"
