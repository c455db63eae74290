// probe_gather_pattern.hip -- a standalone read probe of the K/V gather patterns (not part
// of libdk_decode; dk_build.py does not compile it). It streams a 16,384-page pool in the
// metric shape's page-table order with a given segment per wave and bytes per lane and
// XORs the words, so its time is the load pattern's alone. Build and run on the GPU:
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang \
//       -packed-fp32-ops decode-kernel_amd/csrc/probe_gather_pattern.hip -o /tmp/probe_gather \
//       && /tmp/probe_gather
// Pool: NP pages of 32 rows (16 K + 16 V) x ROW bytes, random page table of B sequences x
// P pages. A wave reads one `seg`-byte segment of each row of its pages (seg = one kv
// head's fp8 D=128 row = 128 B, or two neighbouring heads = 256 B), `bpl` bytes per lane,
// 4 pages in flight; NWH waves per workgroup interleave the pages of 1/SPLIT of a
// sequence. (Loads are issued 4 pages at a time and then consumed, so absolute rates are
// below the pipelined kernel's; compare cases with each other.)
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
#include <algorithm>
#include <random>
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e), __LINE__); return 1; } } while (0)

template <int BPL, int NI>
__global__ void gather(const unsigned char* __restrict__ pool, const int* __restrict__ table,
                       int P, int nseg, int seg, int nwh, int split, long row, unsigned* out) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int g = blockIdx.x;
  const int h = g % nseg; g /= nseg;
  const int sp = g % split; const int b = g / split;
  const int lpr = seg / BPL, rpl = 64 / lpr;
  const int r0 = lane / lpr, cb = (lane % lpr) * BPL;
  const long page_bytes = 32L * row;
  const int per = (P + split - 1) / split;
  const int p0 = sp * per, p1 = min(p0 + per, P);
  unsigned acc = 0;
  const int* tb = table + (long)b * P;
  for (int p = p0 + w; p < p1; p += 4 * nwh) {
    unsigned v[4][NI][BPL / 4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int pp = min(p + u * nwh, p1 - 1);
      const unsigned char* base = pool + (long)__builtin_amdgcn_readfirstlane(tb[pp]) * page_bytes
                                  + (long)h * seg + cb;
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const long off = (long)(r0 + i * rpl) * row;
        if constexpr (BPL == 16) {
          const u32x4 x = __builtin_nontemporal_load((const u32x4*)(base + off));
          v[u][i][0] = x.x; v[u][i][1] = x.y; v[u][i][2] = x.z; v[u][i][3] = x.w;
        } else {
          const u32x2 x = __builtin_nontemporal_load((const u32x2*)(base + off));
          v[u][i][0] = x.x; v[u][i][1] = x.y;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int k = 0; k < BPL / 4; ++k) acc ^= v[u][i][k];
  }
  if (acc == 0x9e3779b9u) out[0] = acc;
}

int main() {
  printf("gather pattern probe start\n"); fflush(stdout);
  const int B = 32, P = 512, NP = B * P;
  const size_t pool_bytes = 1ull << 30, flush_bytes = 1ull << 30;
  unsigned char *pool, *fl; int* table; unsigned* out;
  CK(hipMalloc(&pool, pool_bytes)); CK(hipMalloc(&fl, flush_bytes)); CK(hipMalloc(&out, 4));
  CK(hipMemset(pool, 1, pool_bytes));
  std::vector<int> t(NP); for (int i = 0; i < NP; ++i) t[i] = i;
  std::mt19937 rng(1); std::shuffle(t.begin(), t.end(), rng);
  CK(hipMalloc(&table, NP * 4)); CK(hipMemcpy(table, t.data(), NP * 4, hipMemcpyHostToDevice));
  hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
  struct C { const char* what; long row; int seg, bpl, nwh, split; };
  std::vector<C> cases = {
    {"fp8 D=128, 1 head/wave, 8 B/lane (the kernel)", 1024, 128, 8, 4, 1},
    {"fp8 D=128, 1 head/wave, 16 B/lane", 1024, 128, 16, 4, 1},
    {"fp8 D=128, 2 heads/wave, 16 B/lane, split 2", 1024, 256, 16, 4, 2},
    {"fp8 D=128, 2 heads/wave, 16 B/lane, 8 waves", 1024, 256, 16, 8, 1},
    {"fp8 D=128, 2 heads/wave, 16 B/lane, 4 waves", 1024, 256, 16, 4, 1},
    {"fp8 D=128, 4 heads/wave, 16 B/lane, split 4", 1024, 512, 16, 4, 4},
    {"fp8 D=128, 2 heads/wave, 16 B/lane, split 2, 2 waves", 1024, 256, 16, 2, 2},
    {"fp16 D=128 (metric), 1 head/wave, 16 B/lane, 2 waves", 2048, 256, 16, 2, 1},
    {"fp16 D=64, 1 head/wave, 8 B/lane, 4 waves (C5 rows)", 1024, 128, 8, 4, 1},
    {"fp16 D=64, 2 heads/wave, 16 B/lane, split 2", 1024, 256, 16, 4, 2},
  };
  for (int rep = 0; rep < 2; ++rep)
  for (const C& c : cases) {
    const int nseg = (int)(c.row / c.seg);
    const double bytes = (double)NP * 32 * c.row;
    const int lpr = c.seg / c.bpl, ni = 32 / (64 / lpr);
    const int grid = B * nseg * c.split, blk = 64 * c.nwh;
    auto launch = [&]() {
#define L(BPL, NI) gather<BPL, NI><<<grid, blk>>>(pool, table, P, nseg, c.seg, c.nwh, c.split, c.row, out)
      if (c.bpl == 16 && ni == 4) L(16, 4);
      else if (c.bpl == 16 && ni == 8) L(16, 8);
      else if (c.bpl == 16 && ni == 16) L(16, 16);
      else if (c.bpl == 16 && ni == 2) L(16, 2);
      else if (c.bpl == 8 && ni == 8) L(8, 8);
      else if (c.bpl == 8 && ni == 4) L(8, 4);
      else { printf("no instance bpl %d ni %d\n", c.bpl, ni); }
    };
    std::vector<float> ts;
    for (int it = 0; it < 33; ++it) {
      CK(hipMemsetAsync(fl, it & 0xff, flush_bytes));
      CK(hipEventRecord(e0)); launch(); CK(hipEventRecord(e1)); CK(hipEventSynchronize(e1));
      float ms; CK(hipEventElapsedTime(&ms, e0, e1)); if (it >= 3) ts.push_back(ms * 1e3f);
    }
    std::sort(ts.begin(), ts.end());
    const float p50 = ts[ts.size() / 2];
    printf("%-58s grid %4d x %2d waves: p50 %7.1f us  %5.2f TB/s\n", c.what, grid, c.nwh, p50,
           bytes / (p50 * 1e-6) / 1e12);
    fflush(stdout);
  }
  CK(hipDeviceSynchronize());
  printf("gather pattern probe end\n");
  return 0;
}
