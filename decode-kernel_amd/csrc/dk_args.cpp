// Host-only argument checking for libdk_decode (compiled with g++, no HIP).
//
// The checks mirror the reference's TORCH_CHECKs (src/cuda_/attention_ext.cu:506-509,
// 549-552: dtype, page_size == 16, split range, head_dim dispatch at :532-535) and the
// layout invariants that need no device read (src/layout.md:171-178: H_q divisible by
// H_kv; q/kv dtype agreement is implied by the single `dtype`). Invariants that need
// device data (kv_indptr[-1] == len(kv_indices), last_page_len in [1, P]) are the Python
// layer's optional `validate` step; the kernels clamp those values instead.
#include "dk_args.h"

#include <stdarg.h>
#include <stdio.h>

#include <cmath>

#include <algorithm>
#include <string>

namespace dk {

namespace {
thread_local std::string g_error;

bool valid_shape(int32_t batch, int32_t hq, int32_t hkv, int32_t d) {
  return batch >= 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && (d == 64 || d == 128 || d == 256);
}
}  // namespace

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

void clear_error() { g_error.clear(); }

const char* last_error() { return g_error.c_str(); }

int valu_head_cap(int head_dim) { return head_dim >= 256 ? 4 : 8; }

bool qk_on_mfma(int qk_path, int group, int head_dim, bool kv8) {
  // automatic: MFMA beyond 4 q heads per kv head, and for fp8 at D = 256. Measured at B=32
  // ctx 8192, best schedule, VALU vs MFMA q.k, us: fp16 D=128 32/32 633 vs 640, 16/8 163
  // vs 165, 32/8 159 vs 164, 40/8 173 vs 169, 56/8 171 vs 169, 64/8 170 vs 170 (balanced
  // 182 vs 174); D=64 32/8 93 vs 95, 40/8 108 vs 95; bf16 32/8 158 vs 165; fp8 64/8 156
  // vs 93, D=256 16/4 131 vs 103.
  return qk_path == 1 || (qk_path == 0 && (group > 4 || (kv8 && head_dim >= 256)));
}

HeadChunks head_chunks(int group, int head_dim, bool mfma) {
  // VALU q.k: at most 8 heads (4 at D = 256; 8 would spill registers). MFMA q.k: up to 16,
  // one per MFMA column, in the same registers at any head count
  const int cap = mfma ? 16 : valu_head_cap(head_dim);
  HeadChunks h;
  const int c0 = (group + cap - 1) / cap;
  h.per = (group + c0 - 1) / c0;
  h.chunks = (group + h.per - 1) / h.per;
  h.heads = 1;
  while (h.heads < h.per) h.heads <<= 1;
  return h;
}

bool extent_ok(int64_t n0, int64_t s0, int64_t n1, int64_t s1, int64_t last, int64_t esize) {
  // 128-bit products, so that no stride can wrap the bound
  if (s0 < 0 || s1 < 0 || s0 >= kMaxStride || s1 >= kMaxStride) return false;
  const __int128 ext = ((__int128)std::max<int64_t>(n0, 1) - 1) * s0 +
                       ((__int128)std::max<int64_t>(n1, 1) - 1) * s1 + last;
  return ext * esize < ((__int128)1 << 62);
}

bool pool_ok(int64_t num_pages, const dk_strides& s, int64_t kv_r, int32_t hkv, int32_t head_dim,
             int64_t esize) {
  const int64_t st[] = {s.kv_p, kv_r, s.kv_s, s.kv_h};
  for (int64_t v : st)
    if (v < 0 || v >= kMaxStride) return false;
  const __int128 last = ((__int128)std::max<int64_t>(num_pages, 1) - 1) * s.kv_p + kv_r +
                        (__int128)(kPageSize - 1) * s.kv_s + (__int128)(hkv - 1) * s.kv_h +
                        head_dim;
  return last * esize < ((__int128)1 << 62);
}

void partials_layout_rows(int64_t rows, int32_t head_dim, size_t* off_o, size_t* off_m,
                          size_t* off_l, size_t* total) {
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  *off_o = 0;
  *off_m = up((size_t)rows * (size_t)head_dim * sizeof(float));
  *off_l = *off_m + up((size_t)rows * sizeof(float));
  *total = *off_l + (size_t)rows * sizeof(float);
}

int64_t split_rows(int32_t batch, int32_t hq, int32_t split) {
  return (int64_t)batch * hq * split;
}

int64_t balanced_rows(int32_t batch, int32_t hq, int32_t hkv, int32_t head_dim) {
  // Enough rows for either q.k path (the path is an option of the call). Pass 1 writes
  // slot rows (hc * (Wg + batch) + j + b) * heads for head chunk hc < HC = hkv * chunks and
  // range j < Wg, so it needs HC * (Wg + batch) * heads rows. The grid holds at most
  // kMaxWaves wavefronts, i.e. HC * Wg <= kMaxWaves, except when HC alone exceeds that
  // and the grid falls back to one range per head chunk (Wg = 1): hence max(kMaxWaves, HC).
  int64_t rows = 0;
  for (bool mfma : {false, true}) {
    const HeadChunks h = head_chunks(hq / hkv, head_dim, mfma);
    const int64_t hc = (int64_t)hkv * h.chunks;
    rows = std::max<int64_t>(rows, (std::max<int64_t>(kMaxWaves, hc) + batch * hc) * h.heads);
  }
  return rows;
}

size_t workspace_bytes(int32_t batch, int32_t hq, int32_t hkv, int32_t head_dim, int32_t split) {
  if (!valid_shape(batch, hq, hkv, head_dim) || split < 0 || split > kMaxSplit || batch == 0 ||
      split == 1 || (int64_t)batch * hq > kMaxRows)
    return 0;
  const int64_t rows = split == 0 ? balanced_rows(batch, hq, hkv, head_dim)
                                  : split_rows(batch, hq, split);
  size_t o, m, l, total;
  partials_layout_rows(rows, head_dim, &o, &m, &l, &total);
  return total;
}

int choose_split(int64_t units, int64_t slots, int64_t avg_pages_per_seq, int waves) {
  if (units <= 0) return 1;
  // Enough workgroups to fill every resident slot once (one round), but no split so fine
  // that a wavefront gets fewer than ~4 pages.
  int64_t s = (slots + units - 1) / units;
  const int64_t max_s = std::max<int64_t>(1, avg_pages_per_seq / (4 * (int64_t)std::max(waves, 1)));
  s = std::max<int64_t>(1, std::min(s, max_s));
  return (int)std::min<int64_t>(s, 4096);
}

int64_t split_grid(int32_t batch, int32_t hkv, int32_t split, int chunks) {
  const int64_t units = (int64_t)batch * hkv * split;
  return chunks == 1 ? units : (units + kXcds - 1) / kXcds * kXcds * chunks;
}

Plan make_plan(const Problem& p) {
  Plan pl;
  pl.group = p.hq / p.hkv;
  // q.k on the VALU by default: its full-row K loads stream faster than the MFMA path's
  // 64-byte row segments on the NHD layout (measured for both fp16 and bf16); groups too
  // large for one VALU chunk take the MFMA path, which holds 16 heads per wavefront
  pl.mfma = qk_on_mfma(p.opt.qk_path, p.hq / p.hkv, p.head_dim,
                       p.opt.kv_dtype == DK_KV_FP8_E4M3);
  const HeadChunks hc = head_chunks(pl.group, p.head_dim, pl.mfma);
  pl.heads = hc.heads;
  pl.per = hc.per;
  pl.chunks = hc.chunks;
  pl.pairs_per_seq = p.hkv * pl.chunks;
  const bool kv8 = p.opt.kv_dtype == DK_KV_FP8_E4M3;
  pl.waves = p.opt.waves_per_group ? p.opt.waves_per_group
                                   : (p.narrow_rows() || (pl.heads >= 8 && !pl.mfma)
                                          ? kDefaultWavesPerGroupNarrow
                                          : kDefaultWavesPerGroup);
  pl.kv8 = kv8;
  pl.balanced = p.split == 0;
  pl.grid = pl.balanced ? 0 : split_grid(p.batch, p.hkv, std::max(p.split, 1), pl.chunks);
  return pl;
}

int validate(const Problem& p) {
  if (p.batch < 0) return set_error(DK_EINVAL, "batch must be >= 0, got %d", p.batch);
  if (p.hq <= 0 || p.hkv <= 0)
    return set_error(DK_EINVAL, "num_q_heads and num_kv_heads must be >= 1 (got %d, %d)",
                     p.hq, p.hkv);
  if (p.hq % p.hkv != 0)
    return set_error(DK_EINVAL,
                     "num_q_heads (%d) must be divisible by num_kv_heads (%d)", p.hq, p.hkv);
  if (p.head_dim != 64 && p.head_dim != 128 && p.head_dim != 256)
    return set_error(DK_EINVAL, "head_dim must be 64, 128, or 256; got %d", p.head_dim);
  if (p.page_size != kPageSize)
    return set_error(DK_EINVAL, "page_size must be 16 for the HIP kernel; got %d",
                     p.page_size);
  if (p.dtype != DK_F16 && p.dtype != DK_BF16)
    return set_error(DK_EINVAL, "dtype must be DK_F16 (0) or DK_BF16 (1); got %d", p.dtype);
  if (p.split < 0) return set_error(DK_EINVAL, "split_kv must be >= 0; got %d", p.split);
  if (p.split > kMaxSplit)
    return set_error(DK_EINVAL, "split_kv must be <= %d; got %d", kMaxSplit, p.split);
  if (p.num_indices < 0 || p.num_indices > INT32_MAX)
    return set_error(DK_EINVAL, "num_indices must be in [0, 2^31); got %lld",
                     (long long)p.num_indices);
  if (p.num_pages < 0) return set_error(DK_EINVAL, "num_pages must be >= 0");
  if (p.num_indices > 0 && p.num_pages == 0)
    return set_error(DK_EINVAL, "kv_indices is non-empty but the page pool is empty");
  const dk_options& o = p.opt;
  if (o.qk_path < 0 || o.qk_path > 2)
    return set_error(DK_EINVAL, "options.qk_path must be 0, 1 or 2; got %d", o.qk_path);
  if (o.waves_per_group != 0 && o.waves_per_group != 1 && o.waves_per_group != 2 &&
      o.waves_per_group != 4)
    return set_error(DK_EINVAL, "options.waves_per_group must be 0, 1, 2 or 4; got %d",
                     o.waves_per_group);
  if (o.waves_per_cu < 0 || o.waves_per_cu > 32)
    return set_error(DK_EINVAL, "options.waves_per_cu must be in [0, 32]; got %d", o.waves_per_cu);
  if (o.schedule < 0 || o.schedule > 2)
    return set_error(DK_EINVAL, "options.schedule must be 0, 1 or 2; got %d", o.schedule);
  if (o.max_pages_per_seq < 0)
    return set_error(DK_EINVAL, "options.max_pages_per_seq must be >= 0; got %d",
                     o.max_pages_per_seq);
  // a negative scale would turn the kernels' -inf masking of dead tokens into +inf
  if (!std::isfinite(o.sm_scale) || o.sm_scale < 0.f)
    return set_error(DK_EINVAL,
                     "options.sm_scale must be finite and >= 0 (0 = 1/sqrt(head_dim)); got %g",
                     (double)o.sm_scale);
  if (o.kv_dtype != DK_KV_SAME && o.kv_dtype != DK_KV_FP8_E4M3)
    return set_error(DK_EINVAL, "options.kv_dtype must be DK_KV_SAME or DK_KV_FP8_E4M3; got %d",
                     o.kv_dtype);
  if (!std::isfinite(o.k_scale) || !std::isfinite(o.v_scale) || o.k_scale < 0 ||
      o.v_scale < 0)
    return set_error(DK_EINVAL, "options.k_scale and v_scale must be finite and >= 0");
  if (o.kv_dtype == DK_KV_SAME && (o.k_scale != 0.f || o.v_scale != 0.f))
    return set_error(DK_EINVAL, "options.k_scale and v_scale apply to an fp8 cache only");
  if (o.window < 0)
    return set_error(DK_EINVAL, "options.window must be >= 0 (0 = the whole sequence); got %d",
                     o.window);
  if (!std::isfinite(o.logit_cap) || o.logit_cap < 0)
    return set_error(DK_EINVAL, "options.logit_cap must be finite and >= 0 (0 = off)");
  for (int r : o.reserved)
    if (r != 0) return set_error(DK_EINVAL, "options.reserved must be zero");
  if (((uintptr_t)o.sinks % alignof(float)) != 0)
    return set_error(DK_EINVAL, "options.sinks must be a 4-byte aligned device array");
  if (p.batch == 0) return DK_OK;   // nothing to do; pointers may be anything

  if (!p.q || !p.kv || !p.indptr || !p.last_len)
    return set_error(DK_ENULL, "q, kv_data, kv_indptr and kv_last_page_len must be non-NULL");
  if (p.num_indices > 0 && !p.indices)
    return set_error(DK_ENULL, "kv_indices must be non-NULL");
  if (p.need_out && !p.out) return set_error(DK_ENULL, "out must be non-NULL");

  // Strides: non-negative, and every 16-byte vector access aligned. Row loads of K/V are
  // up to 16 bytes wide (8 elements), so page/row/head strides and the base must be
  // multiples of 8 elements; q rows are loaded the same way.
  // With a separate V cache the K->V stride kv_r is unused.
  const dk_strides& s = p.st;
  const int64_t kv_r = p.v ? 0 : s.kv_r;
  const int64_t all[] = {s.q_b, s.q_h, s.kv_p, kv_r, s.kv_s, s.kv_h, s.o_b, s.o_h};
  for (int64_t v : all)
    if (v < 0) return set_error(DK_EINVAL, "strides must be non-negative");
  // Every byte offset formed from the strides (here, in the launch arguments and in the
  // kernels) must fit int64: strides below kMaxStride elements, and the last element of q,
  // out and the page pool below 2^62 bytes, bounded in 128-bit arithmetic.
  for (int64_t v : all)
    if (v >= kMaxStride)
      return set_error(DK_EUNSUPPORTED, "strides must be below 2^40 elements; got %lld",
                       (long long)v);
  if (!extent_ok(p.batch, s.q_b, p.hq, s.q_h, p.head_dim, 2) ||
      (p.need_out && !extent_ok(p.batch, s.o_b, p.hq, s.o_h, p.head_dim, 2)) ||
      !pool_ok(p.num_pages, s, kv_r, p.hkv, p.head_dim, p.kv_esize()))
    return set_error(DK_EUNSUPPORTED, "q, out or kv_data spans 2^62 bytes or more");
  const int64_t esize = p.kv_esize();
  auto aligned16 = [](int64_t elems, int64_t es) { return (elems * es) % 16 == 0; };
  if (!aligned16(s.q_b, 2) || !aligned16(s.q_h, 2) || !aligned16(s.kv_p, esize) ||
      !aligned16(kv_r, esize) || !aligned16(s.kv_s, esize) || !aligned16(s.kv_h, esize))
    return set_error(DK_EUNSUPPORTED,
                     "q and kv_data strides must be multiples of 16 bytes (8 fp16/bf16 or 16 "
                     "fp8 elements); pass contiguous tensors");
  if (((uintptr_t)p.q % 16) != 0 || ((uintptr_t)p.kv % 16) != 0 ||
      ((uintptr_t)p.v % 16) != 0)
    return set_error(DK_EUNSUPPORTED, "q and the K/V caches must be 16-byte aligned");
  // Offsets inside one page slice (all kv heads' rows of K, or of V) are 32-bit.
  const int64_t in_page = ((int64_t)(kPageSize - 1) * s.kv_s + (int64_t)(p.hkv - 1) * s.kv_h +
                           p.head_dim) * esize;
  if (in_page >= ((int64_t)1 << 31))
    return set_error(DK_EUNSUPPORTED, "kv_data page extent exceeds 2 GiB");

  // bounds the products below (grid, partial rows) well inside int64
  if ((int64_t)p.batch * p.hq > kMaxRows)
    return set_error(DK_EINVAL, "batch*num_q_heads too large");
  const Plan plan = make_plan(p);
  if (plan.grid > INT32_MAX)
    return set_error(DK_EINVAL, "grid too large: batch*kv_heads*split = %lld workgroups",
                     (long long)plan.grid);
  // Two passes and the pass-1-only entry point write fp32 partials.
  if (p.split != 1 || !p.need_out) {
    size_t req, o, m, l;
    partials_layout_rows(p.split == 0 ? balanced_rows(p.batch, p.hq, p.hkv, p.head_dim)
                                      : split_rows(p.batch, p.hq, p.split),
                         p.head_dim, &o, &m, &l, &req);
    if (!p.workspace || p.workspace_bytes < req)
      return set_error(DK_EWORKSPACE, "workspace of %zu bytes required, %zu given", req,
                       p.workspace_bytes);
    if (((uintptr_t)p.workspace % 256) != 0)
      return set_error(DK_EWORKSPACE, "workspace must be 256-byte aligned");
  }
  return DK_OK;
}

}  // namespace dk
