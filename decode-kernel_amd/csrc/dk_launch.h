// dk_launch.h — host-side selection and launch of the decode kernels for one element type.
// dk_{f16,bf16}[_kv8][_mfma].hip instantiate the per-head_dim symbol tables (see the end
// of this file); dk_api.hip dispatches to them.
#pragma once

#include <hip/hip_runtime.h>

#include "dk_kernels.h"

namespace dk {

struct Pass1Launch {
  int d = 128, heads = 4, waves = 4;   // head_dim, q heads per workgroup, waves per workgroup
  bool mfma = false, balanced = false;
  bool kv8 = false;                    // fp8 (E4M3) cache
  int hp = 1;                          // balanced: kv heads per workgroup (waves each)
  bool cost = false;                   // balanced: the range split charging sequence starts
  int grid = 0;
  hipStream_t stream = nullptr;
};

// Kernel symbol for (head_dim, heads, waves, mode, kv heads per workgroup) with q.k on the
// matrix cores (M) or the VALU, over a 16-bit cache and over an fp8 cache; nullptr if not
// instantiated.
template <class T, bool M>
const void* pass1_symbol_16(int d, int heads, int waves, bool balanced, int hp, bool cost);
template <class T, bool M>
const void* pass1_symbol_kv8(int d, int heads, int waves, bool balanced, int hp, bool cost);
template <class T>
const void* merge_symbol(int d, bool balanced, bool cost = false);

template <class T>
const void* pass1_symbol(int d, int heads, int waves, bool mfma, bool kv8, bool balanced,
                         int hp = 1, bool cost = false) {
  if (kv8)
    return mfma ? pass1_symbol_kv8<T, true>(d, heads, waves, balanced, hp, cost)
                : pass1_symbol_kv8<T, false>(d, heads, waves, balanced, hp, cost);
  return mfma ? pass1_symbol_16<T, true>(d, heads, waves, balanced, hp, cost)
              : pass1_symbol_16<T, false>(d, heads, waves, balanced, hp, cost);
}

template <class T>
hipError_t launch_pass1(const Pass1Args& a, const Pass1Launch& L) {
  const void* fn =
      pass1_symbol<T>(L.d, L.heads, L.waves, L.mfma, L.kv8, L.balanced, L.hp, L.cost);
  if (!fn) return hipErrorInvalidDeviceFunction;
  Pass1Args arg = a;
  void* args[] = {&arg};
  return hipLaunchKernel(fn, dim3(L.grid), dim3(L.waves * L.hp * 64), args, 0, L.stream);
}

template <class T>
hipError_t launch_merge(const MergeArgs& m, int d, bool balanced, hipStream_t stream) {
  const void* fn = merge_symbol<T>(d, balanced, balanced && m.seg_cost > 0);
  if (!fn) return hipErrorInvalidDeviceFunction;
  MergeArgs arg = m;
  void* args[] = {&arg};
  const int rows = m.batch * m.hq;
  return hipLaunchKernel(fn, dim3((rows + 3) / 4), dim3(256), args, 0, stream);
}

// ---- symbol tables (instantiated per element type and cache type)
template <class T, int D, int G, int NW, bool M, bool KV8>
const void* pass1_sym(bool balanced, int hp, bool cost) {
  if (!balanced)
    return hp == 1 ? reinterpret_cast<const void*>(&dk_pass1_split<T, D, G, NW, M, KV8>)
                   : nullptr;
  if (hp == 1)
    return cost ? reinterpret_cast<const void*>(&dk_pass1_balanced<T, D, G, NW, M, KV8, 1, true>)
                : reinterpret_cast<const void*>(&dk_pass1_balanced<T, D, G, NW, M, KV8, 1>);
  // several kv heads per workgroup: rows of at most kNarrowRowBytes, kGroupedWavesPerKvHead
  // wavefronts each (2 kv heads when the kv-head count is no multiple of kGroupedKvHeads);
  // 64-byte rows: kGroupedKvHeadsRow64 kv heads of kGroupedWavesRow64 wavefronts
  constexpr int rb = D * (KV8 ? 1 : 2);
  if constexpr (rb <= kNarrowRowBytes && NW == kGroupedWavesPerKvHead) {
    if (hp == 2)
      return cost ? reinterpret_cast<const void*>(&dk_pass1_balanced<T, D, G, NW, M, KV8, 2, true>)
                  : reinterpret_cast<const void*>(&dk_pass1_balanced<T, D, G, NW, M, KV8, 2>);
    if constexpr (kGroupedKvHeads != 2) {
      if (hp == kGroupedKvHeads)
        return cost ? reinterpret_cast<const void*>(
                          &dk_pass1_balanced<T, D, G, NW, M, KV8, kGroupedKvHeads, true>)
                    : reinterpret_cast<const void*>(
                          &dk_pass1_balanced<T, D, G, NW, M, KV8, kGroupedKvHeads>);
    }
  }
  if constexpr (rb == 64 && NW == kGroupedWavesRow64) {
    if (hp == kGroupedKvHeadsRow64)
      return cost ? reinterpret_cast<const void*>(
                        &dk_pass1_balanced<T, D, G, NW, M, KV8, kGroupedKvHeadsRow64, true>)
                  : reinterpret_cast<const void*>(
                        &dk_pass1_balanced<T, D, G, NW, M, KV8, kGroupedKvHeadsRow64>);
  }
  return nullptr;
}

template <class T, int D, int G, bool M, bool KV8>
const void* pass1_sym_w(int waves, bool balanced, int hp, bool cost) {
  switch (waves) {
    case 1: return pass1_sym<T, D, G, 1, M, KV8>(balanced, hp, cost);
    case 2: return pass1_sym<T, D, G, 2, M, KV8>(balanced, hp, cost);
    case 4: return pass1_sym<T, D, G, 4, M, KV8>(balanced, hp, cost);
    default: return nullptr;
  }
}

template <class T, int D, bool M, bool KV8>
const void* pass1_sym_g(int heads, int waves, bool balanced, int hp, bool cost) {
  switch (heads) {
    case 1: return pass1_sym_w<T, D, 1, M, KV8>(waves, balanced, hp, cost);
    case 2: return pass1_sym_w<T, D, 2, M, KV8>(waves, balanced, hp, cost);
    case 4: return pass1_sym_w<T, D, 4, M, KV8>(waves, balanced, hp, cost);
    case 8:
      // 8 heads at D = 256 on the VALU path do not fit a wavefront's registers; the MFMA
      // path holds up to 16 heads in the same registers
      if constexpr (D <= 128 || M) return pass1_sym_w<T, D, 8, M, KV8>(waves, balanced, hp, cost);
      return nullptr;
    case 16:
      if constexpr (M) return pass1_sym_w<T, D, 16, M, KV8>(waves, balanced, hp, cost);
      return nullptr;
    default: return nullptr;
  }
}

template <class T, bool M, bool KV8>
const void* pass1_symbol_t(int d, int heads, int waves, bool balanced, int hp, bool cost) {
  switch (d) {
    case 64: return pass1_sym_g<T, 64, M, KV8>(heads, waves, balanced, hp, cost);
    case 128: return pass1_sym_g<T, 128, M, KV8>(heads, waves, balanced, hp, cost);
    case 256: return pass1_sym_g<T, 256, M, KV8>(heads, waves, balanced, hp, cost);
    default: return nullptr;
  }
}

template <class T, bool M>
const void* pass1_symbol_16(int d, int heads, int waves, bool balanced, int hp, bool cost) {
  return pass1_symbol_t<T, M, false>(d, heads, waves, balanced, hp, cost);
}

template <class T, bool M>
const void* pass1_symbol_kv8(int d, int heads, int waves, bool balanced, int hp, bool cost) {
  return pass1_symbol_t<T, M, true>(d, heads, waves, balanced, hp, cost);
}

template <class T, int D>
const void* merge_symbol_d(bool balanced, bool cost) {
  if (!balanced) return reinterpret_cast<const void*>(&dk_merge_split<T, D>);
  return cost ? reinterpret_cast<const void*>(&dk_merge_balanced<T, D, true>)
              : reinterpret_cast<const void*>(&dk_merge_balanced<T, D>);
}

template <class T>
const void* merge_symbol(int d, bool balanced, bool cost) {
  switch (d) {
    case 64: return merge_symbol_d<T, 64>(balanced, cost);
    case 128: return merge_symbol_d<T, 128>(balanced, cost);
    case 256: return merge_symbol_d<T, 256>(balanced, cost);
    default: return nullptr;
  }
}

// The kernels of one (element type, cache type, q.k path, head_dim) are instantiated by
// one translation unit: dk_{f16,bf16}[_kv8][_mfma].hip compiled once per head_dim
// (-DDK_HEAD_DIM=64 / 128 / 256), so the 24 units compile in parallel. Everything else
// (the dispatch above, the merge kernels) is instantiated where it is used (dk_api.hip).
#define DK_DECLARE_TABLE(T, D, M, KV8) \
  extern template const void* pass1_sym_g<T, D, M, KV8>(int, int, bool, int, bool);
#define DK_DECLARE_TABLES_D(T, D)      \
  DK_DECLARE_TABLE(T, D, false, false) \
  DK_DECLARE_TABLE(T, D, true, false)  \
  DK_DECLARE_TABLE(T, D, false, true)  \
  DK_DECLARE_TABLE(T, D, true, true)
#define DK_DECLARE_TABLES(T) \
  DK_DECLARE_TABLES_D(T, 64) \
  DK_DECLARE_TABLES_D(T, 128) \
  DK_DECLARE_TABLES_D(T, 256)
DK_DECLARE_TABLES(F16)
DK_DECLARE_TABLES(BF16)
#undef DK_DECLARE_TABLES
#undef DK_DECLARE_TABLES_D
#undef DK_DECLARE_TABLE

}  // namespace dk
