// probe_launch_floor.hip — what a small decode call's fixed costs are on MI355X.
//
// Not part of the library: a standalone program for the measurement recorded in
// profiles/launch_floor_probe.md. It times, with HIP events after a 1 GiB fill (the
// bench's cache flush), kernels of 256 workgroups x 256 threads that
//   A: read kernel arguments, then kv_indptr[0] and kv_indptr[batch], then one page id,
//      then that 8 KB page (three dependent memory trips after the arguments), as pass 1
//      of the balanced schedule does before its first page arrives;
//   B: the same, issuing the page-id and page loads first on the guess kv_indptr[0] = 0,
//      kv_indptr[batch] = num_indices, checked afterwards (one trip fewer);
//   C: B with the arguments as leading scalars, preloaded into SGPRs at wave launch
//      (-mllvm -amdgpu-kernarg-preload-count=16): no argument trip either;
//   D: A with preloaded arguments;
//   E: one store per thread and nothing else;
//   F: no kernel (the two events alone).
// If the dependent trips cost time, A > B > C > E.
//
// Build and run (one MI355X):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang \
//       -packed-fp32-ops -mllvm -amdgpu-kernarg-preload-count=16 \
//       decode-kernel_amd/csrc/probe_launch_floor.hip -o /tmp/probe_launch_floor
//   /tmp/probe_launch_floor
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <vector>

#define CK(x)                                                                   \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
      return 1;                                                                 \
    }                                                                           \
  } while (0)

typedef unsigned u4 __attribute__((ext_vector_type(4)));
struct Args {
  const int* indptr;
  const int* idx;
  const u4* kv;
  float* out;
  int batch, nidx, pages;
};

__device__ __forceinline__ int ldc(const int* p, int i) {
  return ((const __attribute__((address_space(4))) int*)p)[i];
}
// one page of the range this workgroup would stream first: page id, then 8 KB of it
__device__ __forceinline__ float first_page(const Args& a, int base, int P) {
  const int L = (P + (int)gridDim.x - 1) / (int)gridDim.x;
  const int u = min((int)blockIdx.x * L, P - 1);
  int pid = __builtin_amdgcn_readfirstlane(ldc(a.idx, base + u));
  pid = (unsigned)pid < (unsigned)a.pages ? pid : 0;
  const u4* pg = a.kv + (size_t)pid * 512 + threadIdx.x;
  const u4 v0 = __builtin_nontemporal_load(pg), v1 = __builtin_nontemporal_load(pg + 256);
  return (float)(v0[0] ^ v0[1] ^ v1[2] ^ v1[3]);
}
__device__ __forceinline__ float guessed(const Args& a) {
  float x = first_page(a, 0, a.nidx);
  asm volatile("" ::: "memory");   // the guessed loads are issued before the check
  const int base = ldc(a.indptr, 0), P = ldc(a.indptr, a.batch) - base;
  if (base != 0 || P != a.nidx) x = first_page(a, base, P);
  return x;
}
__device__ __forceinline__ float in_order(const Args& a) {
  const int base = ldc(a.indptr, 0), P = ldc(a.indptr, a.batch) - base;
  return first_page(a, base, P);
}

extern "C" __global__ void probe_a(Args a) { a.out[blockIdx.x * 256 + threadIdx.x] = in_order(a); }
extern "C" __global__ void probe_b(Args a) { a.out[blockIdx.x * 256 + threadIdx.x] = guessed(a); }
extern "C" __global__ void probe_c(const int* indptr, const int* idx, const u4* kv, int nidx,
                                   int pages, int batch, float* out) {
  out[blockIdx.x * 256 + threadIdx.x] = guessed(Args{indptr, idx, kv, out, batch, nidx, pages});
}
extern "C" __global__ void probe_d(const int* indptr, const int* idx, const u4* kv, int nidx,
                                   int pages, int batch, float* out) {
  out[blockIdx.x * 256 + threadIdx.x] = in_order(Args{indptr, idx, kv, out, batch, nidx, pages});
}
extern "C" __global__ void probe_e(float* out) { out[blockIdx.x * 256 + threadIdx.x] = 1.f; }
__global__ void fill(u4* p, size_t n) {
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    p[i] = u4{(unsigned)i, 1u, 2u, 3u};
}

int main() {
  const int pages = 4096, batch = 1, nidx = 2048;
  u4 *kv, *fl;
  int *indptr, *idx;
  float* out;
  CK(hipMalloc(&kv, (size_t)pages * 8192));
  CK(hipMalloc(&fl, 1ull << 30));
  CK(hipMalloc(&indptr, 8));
  CK(hipMalloc(&idx, nidx * 4));
  CK(hipMalloc(&out, 256 * 256 * 4));
  std::vector<int> h(nidx);
  for (int i = 0; i < nidx; ++i) h[i] = (i * 7919) % pages;
  const int hp[2] = {0, nidx};
  CK(hipMemcpy(idx, h.data(), nidx * 4, hipMemcpyHostToDevice));
  CK(hipMemcpy(indptr, hp, 8, hipMemcpyHostToDevice));
  CK(hipMemset(kv, 1, (size_t)pages * 8192));
  hipStream_t s;
  CK(hipStreamCreate(&s));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  const Args a{indptr, idx, kv, out, batch, nidx, pages};
  const char* names[] = {"A arguments, kv_indptr, page id, page",
                         "B page id and page on a checked guess",
                         "C B with preloaded arguments",
                         "D A with preloaded arguments",
                         "E one store", "F no kernel (events only)"};
  for (int rep = 0; rep < 2; ++rep)
    for (int k = 0; k < 6; ++k) {
      std::vector<float> t;
      for (int it = 0; it < 80; ++it) {
        fill<<<2048, 256, 0, s>>>(fl, (1ull << 30) / 16);
        CK(hipEventRecord(e0, s));
        if (k == 0) probe_a<<<256, 256, 0, s>>>(a);
        if (k == 1) probe_b<<<256, 256, 0, s>>>(a);
        if (k == 2) probe_c<<<256, 256, 0, s>>>(indptr, idx, kv, nidx, pages, batch, out);
        if (k == 3) probe_d<<<256, 256, 0, s>>>(indptr, idx, kv, nidx, pages, batch, out);
        if (k == 4) probe_e<<<256, 256, 0, s>>>(out);
        CK(hipEventRecord(e1, s));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        if (it >= 20) t.push_back(ms * 1000);
      }
      std::sort(t.begin(), t.end());
      printf("%-40s p50 %6.2f us  p10 %6.2f  p90 %6.2f\n", names[k], t[t.size() / 2],
             t[t.size() / 10], t[t.size() * 9 / 10]);
    }
  CK(hipDeviceSynchronize());
  return 0;
}
