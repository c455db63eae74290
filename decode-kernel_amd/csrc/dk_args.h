// Host-only argument checking, workspace layout and split choice for libdk_decode.
// No HIP in this header or in dk_args.cpp: it is compiled with g++ and exercised on
// machines without a GPU.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "dk_decode.h"

namespace dk {

constexpr int kPageSize = 16;   // tokens per page (reference: PAGE_SIZE=16, attention_ext.cu:509)

// Everything a launch needs that is known on the host.
struct Problem {
  const void* q = nullptr;
  const void* kv = nullptr;
  const int32_t* indptr = nullptr;
  const int32_t* indices = nullptr;
  const int32_t* last_len = nullptr;
  void* out = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  int32_t batch = 0, hq = 0, hkv = 0, head_dim = 0, page_size = 0, dtype = 0;
  int64_t num_pages = 0, num_indices = 0;
  dk_strides st{};
  int32_t split = 0;
  bool need_out = true;       // false for the pass-1-only entry point
  dk_options opt{};
};

// Derived launch shape.
struct Plan {
  int group = 0;       // hq / hkv
  int heads = 0;       // q heads handled by one workgroup (1, 2, 4 or 8)
  int chunks = 0;      // group / heads
  int waves = 0;       // wavefronts per workgroup
  bool mfma = true;    // q.k on MFMA (false: VALU dot2)
  int64_t pass1_groups = 0;
};

// Records a message for dk_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
const char* last_error();

// Validates every host-visible argument (shapes, dtype, strides, alignment, workspace,
// split) without touching device memory. Returns DK_OK or a negative code.
int validate(const Problem& p);

// Plan for a validated problem with split >= 1.
Plan make_plan(const Problem& p);

// Bytes of the fp32 partials for `split` >= 1 splits; workspace_bytes is that for
// split > 1 and 0 for the single-pass split == 1.
size_t partials_bytes(int32_t batch, int32_t hq, int32_t head_dim, int32_t split);
size_t workspace_bytes(int32_t batch, int32_t hq, int32_t head_dim, int32_t split);
void partials_layout(int32_t batch, int32_t hq, int32_t head_dim, int32_t split,
                     size_t* off_o, size_t* off_m, size_t* off_l);

// Split count for `units` = batch * hkv * chunks workgroups per split, given
// `slots` = compute units * resident workgroups per unit.
int choose_split(int64_t units, int64_t slots, int64_t avg_pages_per_seq, int waves);

// Heads per workgroup for a GQA group size (largest power of two <= 8, or <= 4 for
// head_dim 256, that divides the group).
int heads_per_group(int group, int head_dim);

}  // namespace dk
