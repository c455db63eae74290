// dk_paging.hip — page tables for the decode path (C ABI in include/dk_decode.h):
// dk_build_page_table from a token-slot map, dk_expand_page_table from a table of larger
// pages.
//
// Serving frameworks (SGLang's ReqToTokenPool) keep, per request, the cache slot of every
// token: req_to_token[req][t]. With a paged allocator of 16-token pages, token t of a
// request sits at slot 16 * page + t % 16, so the page of the request's p-th 16-token
// chunk is req_to_token[req][16 p] / 16. This kernel writes the CSR page table of
// src/layout.md (kv_indptr, kv_indices, kv_last_page_len) for a batch of requests on the
// device, so a decode step needs no host round trip.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "dk_args.h"
#include "dk_decode.h"

namespace dk {
namespace {

constexpr int kThreads = 256;

struct PageTableArgs {
  const int32_t* req_to_token;
  int64_t req_stride;          // elements between requests' rows
  const int32_t* req_pool_indices;
  const int32_t* seq_lens;
  int32_t batch;
  int32_t* kv_indptr;
  int32_t* kv_indices;
  int64_t capacity;            // entries kv_indices can hold
  int32_t* kv_last_page_len;
};

__device__ __forceinline__ int pages_of(int32_t len) {
  return len > 0 ? (len + kPageSize - 1) / kPageSize : 0;
}

// One workgroup per request b: its first page index is the sum of the page counts of
// requests 0..b-1 (recomputed per workgroup: batch is at most a few thousand).
__global__ __launch_bounds__(kThreads) void dk_page_table(PageTableArgs a) {
  __shared__ int64_t partial[kThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  // int64: a batch of long requests can hold more than 2^31 pages in total
  int64_t sum = 0;
  for (int j = tid; j < b; j += kThreads) sum += pages_of(a.seq_lens[j]);
  // workgroup sum: wavefront butterfly, then across the four wavefronts through LDS
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if ((tid & 63) == 0) partial[tid >> 6] = sum;
  __syncthreads();
  int64_t start = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) start += partial[w];

  const int32_t len = a.seq_lens[b];
  const int n = pages_of(len);
  if (tid == 0) {
    if (b == 0) a.kv_indptr[0] = 0;
    // the true offsets (writes past the capacity are dropped), saturated at int32's range
    a.kv_indptr[b + 1] = (int32_t)min(start + n, (int64_t)INT32_MAX);
    a.kv_last_page_len[b] = n > 0 ? len - (n - 1) * kPageSize : 0;
  }
  const int32_t* row = a.req_to_token + (int64_t)a.req_pool_indices[b] * a.req_stride;
  for (int p = tid; p < n; p += kThreads) {
    const int64_t at = start + p;
    if (at >= a.capacity) break;
    a.kv_indices[at] = row[(int64_t)p * kPageSize] / kPageSize;
  }
}

struct ExpandArgs {
  const int32_t* indptr;       // (batch + 1) over pages of `sub` 16-token sub-pages
  const int32_t* indices;
  const int32_t* last_len;     // tokens in each sequence's last page, in [0, 16 * sub]
  int32_t batch;
  int32_t sub;                 // 16-token sub-pages per page (page_size / 16)
  int32_t mult;                // sub-page ids per page id (page stride / sub-page stride)
  int32_t num_pages;           // pages of the pool (ids outside [0, num_pages) are invalid)
  int32_t num_indices;         // entries of indices (indptr clamped to it)
  int32_t* out_indptr;
  int32_t* out_indices;
  int64_t capacity;            // entries out_indices can hold
  int32_t* out_last;
};

// 16-token sub-pages of sequence b: every page but the last holds `sub`, the last
// ceil(last / 16); none without pages.
__device__ __forceinline__ int sub_pages_of(const ExpandArgs& a, int b, int* np_out,
                                            int* last_out) {
  const int s0 = min(max(a.indptr[b], 0), a.num_indices);
  const int s1 = min(max(a.indptr[b + 1], s0), a.num_indices);
  const int np = s1 - s0;
  const int last = min(max(a.last_len[b], 0), a.sub * kPageSize);
  *np_out = np;
  *last_out = last;
  return np > 0 ? (np - 1) * a.sub + (last + kPageSize - 1) / kPageSize : 0;
}

// One workgroup per sequence b: its first output entry is the sum of the sub-page counts
// of sequences 0..b-1 (recomputed per workgroup, as dk_page_table does). Sub-page j of
// page id p is id p * mult + j; an invalid page id becomes INT32_MAX, which the decode
// kernels treat as they treat any id past the pool.
__global__ __launch_bounds__(kThreads) void dk_expand_pages(ExpandArgs a) {
  __shared__ int64_t partial[kThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  int np, last;
  // int64: sequences whose kv_indptr ranges overlap (not a valid table, but clamped, not
  // refused) can add up to more sub-pages than int32 holds
  int64_t sum = 0;
  for (int j = tid; j < b; j += kThreads) sum += sub_pages_of(a, j, &np, &last);
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if ((tid & 63) == 0) partial[tid >> 6] = sum;
  __syncthreads();
  int64_t start = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) start += partial[w];

  const int n = sub_pages_of(a, b, &np, &last);
  if (tid == 0) {
    if (b == 0) a.out_indptr[0] = 0;
    // saturated at the capacity, so that the rewritten table never points past its
    // entries (a valid table's total is at most the capacity)
    a.out_indptr[b + 1] = (int32_t)min(start + n, a.capacity);
    // the last sub-page's tokens: the last page's remainder, or a full sub-page when the
    // last page holds none (last_len 0 ends the sequence at the page before)
    const int rem = last - ((last + kPageSize - 1) / kPageSize - 1) * kPageSize;
    a.out_last[b] = n == 0 ? 0 : (last == 0 ? kPageSize : rem);
  }
  const int s0 = min(max(a.indptr[b], 0), a.num_indices);
  for (int t = tid; t < n; t += kThreads) {
    const int64_t at = start + t;
    if (at >= a.capacity) break;
    const int p = t / a.sub, j = t % a.sub;
    const int32_t pid = a.indices[s0 + p];
    a.out_indices[at] = pid >= 0 && pid < a.num_pages
                            ? (int32_t)((int64_t)pid * a.mult + j) : INT32_MAX;
  }
}

}  // namespace
}  // namespace dk

extern "C" int dk_expand_page_table(const int32_t* kv_indptr, const int32_t* kv_indices,
                                    const int32_t* kv_last_page_len, int32_t batch,
                                    int32_t page_size, int32_t pages_mult, int64_t num_pages,
                                    int64_t num_indices, int32_t* out_indptr,
                                    int32_t* out_indices, int64_t capacity,
                                    int32_t* out_last_page_len, void* hip_stream) {
  dk::clear_error();
  if (batch < 0 || capacity < 0 || num_pages < 0 || num_indices < 0)
    return dk::set_error(DK_EINVAL,
                         "dk_expand_page_table: negative batch, capacity, pages or indices");
  if (page_size <= 0 || page_size % dk::kPageSize != 0)
    return dk::set_error(DK_EINVAL, "page_size must be a positive multiple of 16; got %d",
                         page_size);
  const int32_t sub = page_size / dk::kPageSize;
  if (pages_mult < sub)
    return dk::set_error(DK_EINVAL,
                         "pages_mult (%d) must be at least page_size / 16 (%d): sub-pages of "
                         "different pages would share ids", pages_mult, sub);
  if (num_indices > INT32_MAX)
    return dk::set_error(DK_EINVAL, "num_indices must be < 2^31");
  if (num_pages > INT32_MAX)
    return dk::set_error(DK_EINVAL, "num_pages must be < 2^31 (page ids are int32)");
  // the rewritten table's offsets (at most num_indices * sub entries) are int32
  if (num_indices * (int64_t)sub > (int64_t)INT32_MAX)
    return dk::set_error(DK_EINVAL, "num_indices * page_size / 16 sub-pages exceed 2^31");
  // every valid sub-page id, (num_pages - 1) * pages_mult + sub - 1, must fit in int32
  if (num_pages > 0 && (num_pages - 1) * (int64_t)pages_mult + sub > (int64_t)INT32_MAX)
    return dk::set_error(DK_EINVAL, "num_pages * pages_mult exceeds 2^31 sub-page ids");
  if (batch == 0) return DK_OK;
  if (!kv_indptr || !kv_last_page_len || !out_indptr || !out_last_page_len ||
      (num_indices > 0 && !kv_indices) || (capacity > 0 && !out_indices))
    return dk::set_error(DK_ENULL, "dk_expand_page_table: NULL pointer");
  dk::ExpandArgs a{kv_indptr, kv_indices, kv_last_page_len, batch, sub, pages_mult,
                   (int32_t)std::min<int64_t>(num_pages, INT32_MAX), (int32_t)num_indices,
                   out_indptr, out_indices, capacity, out_last_page_len};
  void* args[] = {&a};
  const hipError_t e = hipLaunchKernel((const void*)dk::dk_expand_pages, dim3(batch),
                                       dim3(dk::kThreads), args, 0,
                                       static_cast<hipStream_t>(hip_stream));
  if (e != hipSuccess)
    return dk::set_error((int)e, "page-table expansion launch: %s", hipGetErrorString(e));
  return DK_OK;
}

extern "C" int dk_build_page_table(const int32_t* req_to_token, int64_t req_stride,
                                   const int32_t* req_pool_indices, const int32_t* seq_lens,
                                   int32_t batch, int32_t page_size, int32_t* kv_indptr,
                                   int32_t* kv_indices, int64_t capacity,
                                   int32_t* kv_last_page_len, void* hip_stream) {
  dk::clear_error();
  if (batch < 0 || req_stride < 0 || capacity < 0)
    return dk::set_error(DK_EINVAL, "dk_build_page_table: negative batch, stride or capacity");
  // row offsets req_pool_indices[b] * req_stride (int32 index) must fit int64
  if (req_stride >= dk::kMaxStride)
    return dk::set_error(DK_EUNSUPPORTED, "req_stride must be below 2^40 elements; got %lld",
                         (long long)req_stride);
  if (page_size != dk::kPageSize)
    return dk::set_error(DK_EINVAL, "page_size must be 16; got %d", page_size);
  if (batch == 0) return DK_OK;
  if (!req_to_token || !req_pool_indices || !seq_lens || !kv_indptr || !kv_last_page_len ||
      (capacity > 0 && !kv_indices))
    return dk::set_error(DK_ENULL, "dk_build_page_table: NULL pointer");
  dk::PageTableArgs a{req_to_token, req_stride, req_pool_indices, seq_lens, batch,
                      kv_indptr, kv_indices, capacity, kv_last_page_len};
  void* args[] = {&a};
  const hipError_t e = hipLaunchKernel((const void*)dk::dk_page_table, dim3(batch),
                                       dim3(dk::kThreads), args, 0,
                                       static_cast<hipStream_t>(hip_stream));
  if (e != hipSuccess)
    return dk::set_error((int)e, "page-table launch: %s", hipGetErrorString(e));
  return DK_OK;
}
