// Host-only argument checking, workspace layout and launch planning for libdk_decode.
// No HIP in this header or in dk_args.cpp: it is compiled with g++ and exercised on
// machines without a GPU.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "dk_decode.h"

namespace dk {

constexpr int kPageSize = 16;        // tokens per page (reference: PAGE_SIZE=16, attention_ext.cu:509)
constexpr int kMaxWaves = 2048;      // upper bound on the balanced pass-1 grid (wavefronts)
constexpr int64_t kMaxStride = (int64_t)1 << 40;   // element strides accepted (exclusive)
constexpr int kMaxSplit = 4096;                      // split_kv accepted (inclusive)
constexpr int64_t kMaxRows = INT32_MAX / 4;          // batch * num_q_heads accepted
constexpr int kXcds = 8;             // MI355X: the dispatcher deals workgroups to 8 XCDs in turn
constexpr int kDefaultWavesPerCU = 2;
constexpr int kDefaultWavesPerGroup = 2;
// Rows of at most 128 bytes per kv head (fp8 at D <= 128, fp16/bf16 at D = 64) carry half
// the bytes of a page for about the same per-token arithmetic, and 8 q heads per
// wavefront on the VALU q.k path double the arithmetic per byte: then one wavefront per
// SIMD is needed to keep HBM busy (measured at B=32 ctx=8192 with 4 wavefronts per group
// vs 2: fp8 D=128 93 vs 162 us; fp16 D=64 92 vs 122; 64 q / 8 kv heads at D=128, VALU,
// 172 vs 254). On the MFMA q.k path (K staged through LDS) 8-16 heads keep the 2/2
// defaults: 64/8 one pass 165.5 vs 169.9, balanced 168 vs 174; 28/4 balanced 92.6 vs
// 97.5)
constexpr int kDefaultWavesPerCUNarrow = 4;
constexpr int kDefaultWavesPerGroupNarrow = 4;
constexpr int kNarrowRowBytes = 128;
// Balanced schedule over a small problem (the plan hint bounds it at this many (page, head
// chunk) units per compute unit or fewer): the narrow-row wave counts, so each wavefront
// streams half the pages and the call ends one page round trip sooner (B=1 and B=4 at ctx
// 4096, 32/8/128 fp16: 16.2 -> 15.1 and 23.3 -> 22.4 us; at 128 units per CU or 64 with
// one sequence of 32768 tokens, two wavefronts stay faster)
constexpr int kSmallUnitsPerCU = 32;
// Balanced schedule over many short sequences (the plan hint: the longest is at most
// 1/kShortSegments of a workgroup's page range, so a workgroup walks through several
// sequences): one wavefront per workgroup, so a change of sequence needs no workgroup
// combine (B=32*k, ctx 8192/k, 32/8/128 unless noted, balanced, NW=1 vs the default,
// us: B=128 ctx 2048 166 vs 174, B=256 ctx 1024 176 vs 185, 64/8 B=256 ctx 1024 188 vs
// 204, 16/4 93 vs 99; sequences of 1/2 to 1/4 of a range, or ragged, ~1 % either way)
constexpr int kShortSegments = 4;
// Uniform batches over 256-byte rows whose (sequence, head chunk) pairs are a whole
// multiple of this many per CU run one pass (measured in dk_api.hip, uniform_many_pairs)
constexpr int kOnePassPairsPerCU = 4;
// ... and uniform batches of sequences of at most this many pages with CUs/4 to CUs pairs
// run one pass at 4 wavefronts per workgroup (dk_api.hip, short_uniform_pairs)
constexpr int kShortOnePassPages = 32;
// Rows of 128 bytes (an fp8 cache at D = 128 up to 4 q heads per kv head, on the VALU q.k
// path; a 16-bit one at D = 64 up to 8, 64/8 on the MFMA path) take the balanced schedule
// with grouped kv heads (an even kv-head count) for sequences longer than this many pages
// even where one pass fits: grouped kv heads with 2 pages in flight outrun one pass there
// (fp8 at 8 q heads per kv head, on the MFMA path with 4 pages in flight, does not: 64/8
// ctx 8192 one pass 91.8-92.1 vs balanced 92.2-92.3). Uniform B=32 (B=16 at
// 32/16, B=8 at 32/32), 32/8, fp16 q unless noted, us, one pass vs balanced:
//   fp8 D=128: ctx 4096 50.7-51.0 vs 51.4-51.5, 5120 60.9-61.0 vs 61.6-61.9, 6144
//   71.9-72.1 vs 70.3-70.4, 8192 92.2 vs 90.3-90.9 (bf16 q 92.4-92.5 vs 90.6-91.1; 8/8
//   93.3 vs 88.1; 16/8 92.9 vs 88.8-89.0; 24/8 92.1 vs 90.2-90.3; 32/16 91.1-91.3 vs
//   88.6-88.7; 32/32 91.2-91.4 vs 86.9-87.6; 8/2 B=128 96.4 vs 93.3-93.6; 24/6 B=42
//   91.9-92.3 vs 91.4-91.7), 12288 133.5-134.2 vs 129.0-129.5, 16384 175.1 vs
//   166.8-167.3, 32768 339.2-342.0 vs 337.0-337.3;
//   16-bit D=64: ctx 4096 49.0-49.3 vs 48.9, 5120 59.0-59.1 vs 59.3-59.4, 6144 70.2-70.5
//   vs 68.0-68.1, 8192 91.3-91.4 vs 88.1 (bf16 91.1-91.4 vs 87.8-87.9; 8/8 90.7-91.2 vs
//   86.8-86.9; 16/8 92.0-92.4 vs 87.1-87.3; 64/8 92.5-92.6 vs 89.1-89.2; 32/16 91.7-92.2
//   vs 86.8; 32/32 89.8-90.8 vs 85.8-86.0), 12288 134.4-134.9 vs 126.7-126.9, 16384
//   177.9 vs 164.1-164.3.
// An odd kv-head count, which the balanced schedule does not group, stays one pass (fp8
// 12/3 B=85 ctx 8192 93.1-93.5 vs 94.0-94.3).
constexpr int kNarrowOnePassMaxPages = 352;
// A uniform batch over 256-byte rows (16-bit D = 128, VALU q.k, default wave counts) whose
// (sequence, kv head) pairs divide the balanced grid into S >= 2 equal page ranges of at
// least this many pages runs the explicit split S instead: the same ranges on a grid of the
// same size, streamed faster over such long runs (32/8/128, us, balanced vs split S: B=16
// ctx 65536 (S=2, 2048 pages) 631.9-634.0 vs 609.8-611.3, B=4 ctx 131072 bf16 (S=8, 1024)
// 314.5-315.8 vs 308.7-308.8; shorter ranges stay balanced: B=16 ctx 16384 (512)
// 158.5-160.5 vs 159.6-160.0, B=8 ctx 32768 (512) 158.3-159.2 vs 159.5-160.4, B=1 ctx
// 131072 bf16 (256) 84.3-84.5 vs 85.1-85.2, B=2 ctx 65536 (256) 84.4-84.7 vs 84.8-84.9).
constexpr int kSplitFillMinPages = 1024;
// An explicit split_kv over 256-byte rows (16-bit D = 128, VALU q.k, default wave counts)
// runs 4 wavefronts per workgroup instead of 2 when its workgroups are fewer than the CUs,
// up to twice as many (all 4-wavefront workgroups then resident at once, 2 per SIMD), or
// exactly as many and streaming at most this many pages each: each wavefront's chain of
// pages is half as long. 32/8/128 fp16 unless noted, us, 2 vs 4 wavefronts (workgroups,
// pages per split): fewer than the CUs: B=2 ctx 512 split 4 (64, 8) 12.4-12.5 vs 11.2 (bf16
// the same; 8/8 heads 10.7 vs 9.9), split 1 (16, 32) 15.7 vs 11.8; B=8 ctx 512 split 1 (64,
// 32) 15.9 vs 12.3; B=1 ctx 4096 split 1 (8, 256) 73.7 vs 49.1, split 8 (64, 32) 18.9 vs
// 15.2-15.3, split 16 (128, 16) 14.1 vs 13.8; B=4 ctx 4096 split 4 (128, 64) 27.0 vs 23.2;
// B=8 ctx 1024 split 2 (128, 32) 19.3 vs 16.1; as many: B=4 ctx 4096 split 8 (256, 32)
// 20.4-20.5 vs 19.6, but B=16 ctx 4096 split 2 (256, 128) 48.4 vs 49.2-49.3, B=1 ctx 32768
// bf16 split 32 (256, 64) 29.3-29.4 vs 30.6 and the metric shape's one pass (256, 512) stay
// at 2; twice as many: B=4 ctx 4096 split 16 (512, 16) 21.6 vs 20.8, B=16 ctx 1024 split 4
// (512, 16) 21.6 vs 20.6, B=32 ctx 1024 split 2 (512, 32) 33.4 vs 29.8, B=32 ctx 2048
// split 2 (512, 64) 53.5 vs 50.3, ctx 4096 (512, 128) 98.9-99.3 vs 91.3-91.5, ctx 8192
// (512, 256) 184.5-184.7 vs 171.6-172.0, B=64 ctx 512 split 1 (512, 32) 30.5 vs 26.7;
// more (a second round of workgroups at 4): B=64 ctx 2048 split 2 (1024, 64) 92.0-92.8 vs
// 94.5, ctx 4096 (1024, 128) 173.3-173.7 vs 175.1-175.9.
constexpr int kShortSplitPages = 32;
// Balanced schedule over a ragged batch: a change of sequence costs a workgroup about 3 us
// (its reduction, combine, stores and pipeline refill), which at two wavefronts per
// workgroup is the time of ~10 pages (C4, B=128 ctx U[128, 8192]: workgroups crossing 3 / 5
// / 7 sequences ended at 323.6 / 331.0 / 336.7 us); the range split charges each sequence
// start this many pages per wavefront of the workgroup.
#ifndef DK_SEGMENT_COST_PER_WAVE
#define DK_SEGMENT_COST_PER_WAVE 5
#endif
constexpr int kSegmentCostPerWave = DK_SEGMENT_COST_PER_WAVE;
// Balanced schedule over narrow rows: 4 neighbouring kv heads per workgroup, 2 wavefronts
// each, one such workgroup per CU (64- and 128-byte row segments 512 B or 1 KB apart
// stream far better when the segments of neighbouring heads are fetched together). B=32
// ctx 8192, balanced before -> after, us: fp8 D=64 96 -> 64, fp8 D=128 97 -> 94, fp16
// D=64 96 -> 91; fp8 D=128 B=64 184 -> 172; but B=4 ctx 8192 fp8 25.4 -> 26.7 (hence
// kGroupedMinUnitsPerCU). With rows of at most kGroupedAlwaysRowBytes the automatic
// schedule takes it over one pass (fp8 D=64: 64 vs 94 us); wider narrow rows keep the
// one-pass choice (fp8 D=128 95 vs 94, D=64 bf16 ctx 2048 29 vs 33 us).
// 64-byte rows (fp8 D=64) with a multiple of 8 kv heads: all 8 heads of a token row (512
// contiguous bytes) per workgroup, one wavefront each (same wavefronts per CU). Against 4
// heads x 2 wavefronts, us: B=32 ctx 8192 61.1 -> 59.7, ragged B=128 121.0 -> 118.6, B=64
// ctx 4096 61.6 -> 60.2, 16/8 58.7 -> 56.7, B=4 ctx 32768 36.8 -> 37.0; over 128-byte rows
// 8 x 1 measured no faster or slower (fp16 D=64 ctx 8192 88.3 -> 89.4, fp8 D=128 ragged
// 192.6-199.7 -> 202.8-203.3). A build may set other groupings with the macros below (2, 4
// or 8 kv heads, 1 or 2 wavefronts each).
#ifndef DK_GROUPED_KV_HEADS
#define DK_GROUPED_KV_HEADS 4
#endif
#ifndef DK_GROUPED_WAVES_PER_KV_HEAD
#define DK_GROUPED_WAVES_PER_KV_HEAD 2
#endif
#ifndef DK_GROUPED_KV_HEADS_ROW64
#define DK_GROUPED_KV_HEADS_ROW64 8
#endif
#ifndef DK_GROUPED_WAVES_ROW64
#define DK_GROUPED_WAVES_ROW64 1
#endif
constexpr int kGroupedKvHeads = DK_GROUPED_KV_HEADS;
constexpr int kGroupedWavesPerKvHead = DK_GROUPED_WAVES_PER_KV_HEAD;
constexpr int kGroupedKvHeadsRow64 = DK_GROUPED_KV_HEADS_ROW64;
constexpr int kGroupedWavesRow64 = DK_GROUPED_WAVES_ROW64;
constexpr int kGroupedWavesPerCU = 8;
constexpr int kGroupedMinUnitsPerCU = 128;
constexpr int kGroupedAlwaysRowBytes = 64;

// Everything a launch needs that is known on the host.
struct Problem {
  const void* q = nullptr;
  const void* kv = nullptr;      // K cache (or the combined NHD cache)
  const void* v = nullptr;       // separate V cache (same strides as K), or null
  const int32_t* indptr = nullptr;
  const int32_t* indices = nullptr;
  const int32_t* last_len = nullptr;
  void* out = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  int32_t batch = 0, hq = 0, hkv = 0, head_dim = 0, page_size = 0, dtype = 0;
  int64_t num_pages = 0, num_indices = 0;
  int32_t kv_esize() const { return opt.kv_dtype == DK_KV_FP8_E4M3 ? 1 : 2; }
  // a kv head's row of one token is at most kNarrowRowBytes
  bool narrow_rows() const { return (int64_t)head_dim * kv_esize() <= kNarrowRowBytes; }
  dk_strides st{};
  int32_t split = 0;          // 0: balanced persistent mode; >= 1: explicit split
  bool need_out = true;       // false for the pass-1-only entry point
  dk_options opt{};
};

// Launch shape derived from a problem.
// A GQA group of `group` q heads is processed in `chunks` chunks of `per` consecutive q
// heads (the last may hold fewer), each by a wavefront built for `heads` (the power of two
// >= per; at most 8 with VALU q.k (4 at D = 256), 16 with MFMA q.k) whose surplus heads
// are masked. One chunk whenever the
// group fits, so every page is read once per kv head (e.g. 5, 6 or 7 q heads per kv head).
struct HeadChunks {
  int per = 1, chunks = 1, heads = 1;
};
HeadChunks head_chunks(int group, int head_dim, bool mfma);
// q.k path of a call: qk_path 1 / 2 force MFMA / VALU; 0 takes the VALU path unless the
// group exceeds 8 heads (4 at D = 256 or over an fp8 cache) or the cache is fp8 at D = 256
bool qk_on_mfma(int qk_path, int group, int head_dim, bool kv8);

struct Plan {
  int group = 0;       // hq / hkv
  int heads = 0;       // q heads a wavefront is built for (1, 2, 4 or 8)
  int per = 0;         // q heads per chunk (<= heads)
  int chunks = 0;      // ceil(group / per)
  int pairs_per_seq = 0;   // hkv * chunks
  int waves = 0;       // wavefronts per workgroup
  bool mfma = false;   // q.k on MFMA (default: VALU dot2)
  bool balanced = false;
  bool kv8 = false;    // fp8 cache
  int64_t grid = 0;    // workgroups of pass 1 (balanced: filled in from the device)
};

// Workgroups of the explicit-split kernel for `split` splits: one per (sequence, kv head,
// split, head chunk); with several head chunks the count is padded to whole rounds of
// kXcds so that a pair's chunks can sit kXcds ids apart (one XCD).
int64_t split_grid(int32_t batch, int32_t hkv, int32_t split, int chunks);

// Records a message for dk_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char* last_error();

// Validates every host-visible argument (shapes, dtype, strides, alignment, workspace,
// split) without touching device memory. Returns DK_OK or a negative code.
int validate(const Problem& p);

Plan make_plan(const Problem& p);

// Heads per wavefront for a GQA group size (largest power of two <= 8, or <= 4 for
// head_dim 256, that divides the group).


// fp32 partials: `rows` rows of head_dim floats + m + l, each array 256-byte aligned.
void partials_layout_rows(int64_t rows, int32_t head_dim, size_t* off_o, size_t* off_m,
                          size_t* off_l, size_t* total);
// Rows of partials each mode writes: explicit split S -> batch*hq*S; balanced ->
// (max(kMaxWaves, pairs_per_seq) + batch*pairs_per_seq) * heads.
int64_t split_rows(int32_t batch, int32_t hq, int32_t split);
// Whether the last element of an array of n0 x n1 rows (strides s0, s1 elements, `last`
// elements in the final row) lies below 2^62 bytes, the strides below kMaxStride.
bool extent_ok(int64_t n0, int64_t s0, int64_t n1, int64_t s1, int64_t last, int64_t esize);
// The same for a page pool: the last element of its last page (num_pages pages kv_p apart,
// V kv_r after K, 16 token rows kv_s apart, hkv heads kv_h apart, head_dim elements) below
// 2^62 bytes, every stride below kMaxStride.
bool pool_ok(int64_t num_pages, const dk_strides& s, int64_t kv_r, int32_t hkv, int32_t head_dim,
             int64_t esize);
int64_t balanced_rows(int32_t batch, int32_t hq, int32_t hkv, int32_t head_dim);
// Workspace of dk_decode_attention: split 1 -> 0, split > 1 -> explicit partials,
// split 0 -> balanced partials. 0 on invalid shapes.
size_t workspace_bytes(int32_t batch, int32_t hq, int32_t hkv, int32_t head_dim, int32_t split);

// Explicit split count for `units` workgroups per split and `slots` resident workgroups.
int choose_split(int64_t units, int64_t slots, int64_t avg_pages_per_seq, int waves);

}  // namespace dk
