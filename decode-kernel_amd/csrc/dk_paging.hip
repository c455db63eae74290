// dk_paging.hip — page tables for the decode path from a token-slot map (C ABI in
// include/dk_decode.h: dk_build_page_table).
//
// Serving frameworks (SGLang's ReqToTokenPool) keep, per request, the cache slot of every
// token: req_to_token[req][t]. With a paged allocator of 16-token pages, token t of a
// request sits at slot 16 * page + t % 16, so the page of the request's p-th 16-token
// chunk is req_to_token[req][16 p] / 16. This kernel writes the CSR page table of
// src/layout.md (kv_indptr, kv_indices, kv_last_page_len) for a batch of requests on the
// device, so a decode step needs no host round trip.
#include <hip/hip_runtime.h>
#include <stdint.h>

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
  __shared__ int partial[kThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  int sum = 0;
  for (int j = tid; j < b; j += kThreads) sum += pages_of(a.seq_lens[j]);
  // workgroup sum: wavefront butterfly, then across the four wavefronts through LDS
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if ((tid & 63) == 0) partial[tid >> 6] = sum;
  __syncthreads();
  int start = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) start += partial[w];

  const int32_t len = a.seq_lens[b];
  const int n = pages_of(len);
  if (tid == 0) {
    if (b == 0) a.kv_indptr[0] = 0;
    a.kv_indptr[b + 1] = start + n;
    a.kv_last_page_len[b] = n > 0 ? len - (n - 1) * kPageSize : 0;
  }
  const int32_t* row = a.req_to_token + (int64_t)a.req_pool_indices[b] * a.req_stride;
  for (int p = tid; p < n; p += kThreads) {
    const int64_t at = (int64_t)start + p;
    if (at < a.capacity) a.kv_indices[at] = row[(int64_t)p * kPageSize] / kPageSize;
  }
}

}  // namespace
}  // namespace dk

extern "C" int dk_build_page_table(const int32_t* req_to_token, int64_t req_stride,
                                   const int32_t* req_pool_indices, const int32_t* seq_lens,
                                   int32_t batch, int32_t page_size, int32_t* kv_indptr,
                                   int32_t* kv_indices, int64_t capacity,
                                   int32_t* kv_last_page_len, void* hip_stream) {
  dk::clear_error();
  if (batch < 0 || req_stride < 0 || capacity < 0)
    return dk::set_error(DK_EINVAL, "dk_build_page_table: negative batch, stride or capacity");
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
