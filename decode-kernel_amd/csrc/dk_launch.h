// dk_launch.h — host-side selection and launch of the decode kernels for one element type.
// dk_f16.hip and dk_bf16.hip instantiate these templates (compiled in parallel);
// dk_api.hip calls them.
#pragma once

#include <hip/hip_runtime.h>

#include "dk_kernels.h"

namespace dk {

struct Pass1Launch {
  int d = 128, heads = 4, waves = 4;   // head_dim, q heads per workgroup, waves per workgroup
  bool mfma = false, balanced = false;
  bool kv8 = false;                    // fp8 (E4M3) cache
  int grid = 0;
  hipStream_t stream = nullptr;
};

// Kernel symbol for (head_dim, heads, waves, path, mode) over a 16-bit cache, and over an
// fp8 cache (VALU q.k only); nullptr if not instantiated.
template <class T>
const void* pass1_symbol(int d, int heads, int waves, bool mfma, bool balanced);
template <class T>
const void* pass1_symbol_kv8(int d, int heads, int waves, bool balanced);
template <class T>
const void* merge_symbol(int d, bool balanced);

template <class T>
hipError_t launch_pass1(const Pass1Args& a, const Pass1Launch& L) {
  const void* fn = L.kv8 ? (L.mfma ? nullptr : pass1_symbol_kv8<T>(L.d, L.heads, L.waves, L.balanced))
                         : pass1_symbol<T>(L.d, L.heads, L.waves, L.mfma, L.balanced);
  if (!fn) return hipErrorInvalidDeviceFunction;
  Pass1Args arg = a;
  void* args[] = {&arg};
  return hipLaunchKernel(fn, dim3(L.grid), dim3(L.waves * 64), args, 0, L.stream);
}

template <class T>
hipError_t launch_merge(const MergeArgs& m, int d, bool balanced, hipStream_t stream) {
  const void* fn = merge_symbol<T>(d, balanced);
  if (!fn) return hipErrorInvalidDeviceFunction;
  MergeArgs arg = m;
  void* args[] = {&arg};
  const int rows = m.batch * m.hq;
  return hipLaunchKernel(fn, dim3((rows + 3) / 4), dim3(256), args, 0, stream);
}

// ---- symbol tables (instantiated per element type and cache type)
template <class T, int D, int G, int NW, bool M, bool KV8>
const void* pass1_sym(bool balanced) {
  return balanced ? reinterpret_cast<const void*>(&dk_pass1_balanced<T, D, G, NW, M, KV8>)
                  : reinterpret_cast<const void*>(&dk_pass1_split<T, D, G, NW, M, KV8>);
}

template <class T, int D, int G, int NW, bool KV8>
const void* pass1_sym_m(bool mfma, bool balanced) {
  if constexpr (KV8) {
    return mfma ? nullptr : pass1_sym<T, D, G, NW, false, true>(balanced);
  } else {
    return mfma ? pass1_sym<T, D, G, NW, true, false>(balanced)
                : pass1_sym<T, D, G, NW, false, false>(balanced);
  }
}

template <class T, int D, int G, bool KV8>
const void* pass1_sym_w(int waves, bool mfma, bool balanced) {
  switch (waves) {
    case 1: return pass1_sym_m<T, D, G, 1, KV8>(mfma, balanced);
    case 2: return pass1_sym_m<T, D, G, 2, KV8>(mfma, balanced);
    case 4: return pass1_sym_m<T, D, G, 4, KV8>(mfma, balanced);
    default: return nullptr;
  }
}

template <class T, int D, bool KV8>
const void* pass1_sym_g(int heads, int waves, bool mfma, bool balanced) {
  switch (heads) {
    case 1: return pass1_sym_w<T, D, 1, KV8>(waves, mfma, balanced);
    case 2: return pass1_sym_w<T, D, 2, KV8>(waves, mfma, balanced);
    case 4: return pass1_sym_w<T, D, 4, KV8>(waves, mfma, balanced);
    case 8:
      if constexpr (D <= 128) return pass1_sym_w<T, D, 8, KV8>(waves, mfma, balanced);
      return nullptr;
    default: return nullptr;
  }
}

template <class T, bool KV8>
const void* pass1_symbol_t(int d, int heads, int waves, bool mfma, bool balanced) {
  switch (d) {
    case 64: return pass1_sym_g<T, 64, KV8>(heads, waves, mfma, balanced);
    case 128: return pass1_sym_g<T, 128, KV8>(heads, waves, mfma, balanced);
    case 256: return pass1_sym_g<T, 256, KV8>(heads, waves, mfma, balanced);
    default: return nullptr;
  }
}

template <class T>
const void* pass1_symbol(int d, int heads, int waves, bool mfma, bool balanced) {
  return pass1_symbol_t<T, false>(d, heads, waves, mfma, balanced);
}

template <class T>
const void* pass1_symbol_kv8(int d, int heads, int waves, bool balanced) {
  return pass1_symbol_t<T, true>(d, heads, waves, false, balanced);
}

template <class T>
const void* merge_symbol(int d, bool balanced) {
  switch (d) {
    case 64: return balanced ? reinterpret_cast<const void*>(&dk_merge_balanced<T, 64>)
                             : reinterpret_cast<const void*>(&dk_merge_split<T, 64>);
    case 128: return balanced ? reinterpret_cast<const void*>(&dk_merge_balanced<T, 128>)
                              : reinterpret_cast<const void*>(&dk_merge_split<T, 128>);
    case 256: return balanced ? reinterpret_cast<const void*>(&dk_merge_balanced<T, 256>)
                              : reinterpret_cast<const void*>(&dk_merge_split<T, 256>);
    default: return nullptr;
  }
}

// Explicit instantiation declarations (definitions in dk_f16.hip / dk_bf16.hip and
// dk_f16_kv8.hip / dk_bf16_kv8.hip).
extern template const void* pass1_symbol<F16>(int, int, int, bool, bool);
extern template const void* pass1_symbol<BF16>(int, int, int, bool, bool);
extern template const void* pass1_symbol_kv8<F16>(int, int, int, bool);
extern template const void* pass1_symbol_kv8<BF16>(int, int, int, bool);
extern template const void* merge_symbol<F16>(int, bool);
extern template const void* merge_symbol<BF16>(int, bool);

}  // namespace dk
