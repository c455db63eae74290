// dk_append.hip — the cache write before a decode step (C ABI in include/dk_decode.h:
// dk_append_kv).
//
// For every sequence b the new token is the last one the page table describes: page
// kv_indices[kv_indptr[b+1] - 1], slot kv_last_page_len[b] - 1 (the caller has grown the
// table first, as a paged allocator does). Its K row (rotated) and V row are written there
// for every kv head, and q (optional) is rotated in place, all with rotary position
// embedding at the token's position:
//   rotate-half pairs (i, i + D/2) (Llama / GPT-NeoX) or interleaved pairs (2i, 2i + 1)
//   (GPT-J), angle = position * inv_freq[i], y0 = x0 cos - x1 sin, y1 = x1 cos + x0 sin,
// computed in fp32 and rounded once to the cache type. inv_freq carries any frequency
// scaling (e.g. Llama 3's); without it the rows are copied unrotated. An fp8 (OCP E4M3)
// cache stores RNE(clamp(x / scale, -448, 448)) of each fp32 value x (NaN stays NaN).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>

#include "dk_args.h"
#include "dk_decode.h"

namespace dk {
namespace {

constexpr int kAppendThreads = 256;

struct AppendArgs {
  uint8_t* q;                 // may be null
  const uint8_t* k_new;
  const uint8_t* v_new;
  uint8_t* k_cache;
  int64_t v_off;              // bytes from a K row to the V row of the same slot
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_len;
  const int32_t* positions;   // may be null: position = tokens in the sequence - 1
  const float* inv_freq;      // may be null: no rotation
  int64_t q_b, q_h, n_b, n_h, kv_p, kv_s, kv_h;   // bytes
  int32_t batch, hq, hkv, d, num_indices, rope_style;
  uint32_t num_pages;
  float k_scale, v_scale;     // fp8 cache: stored = value / scale
};

template <class E>
struct Elem;
template <>
struct Elem<_Float16> {
  static constexpr int kBytes = 2;
  static __device__ float load(const uint8_t* p) { return (float)*(const _Float16*)p; }
  __device__ void store(uint8_t* p, float x) const { *(_Float16*)p = (_Float16)x; }
};
template <>
struct Elem<__bf16> {
  static constexpr int kBytes = 2;
  static __device__ float load(const uint8_t* p) { return (float)*(const __bf16*)p; }
  __device__ void store(uint8_t* p, float x) const { *(__bf16*)p = (__bf16)x; }
};

typedef short short2_t __attribute__((ext_vector_type(2)));

// OCP E4M3 store of x / scale: round to nearest even, clamped to +-448 (the largest
// finite value) so that no finite input becomes NaN; NaN stays NaN.
struct Fp8Store {
  static constexpr int kBytes = 1;
  float scale;
  __device__ void store(uint8_t* p, float x) const {
    float y = x / scale;
    y = y != y ? y : fminf(fmaxf(y, -448.f), 448.f);
    const short2_t r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(short2_t{0, 0}, y, 0.f, 1.f, false);
    *p = (uint8_t)(r[0] & 0xff);
  }
};

__device__ __forceinline__ void pair_of(int i, int half, int style, int* i0, int* i1) {
  if (style == 0) {
    *i0 = i;
    *i1 = i + half;
  } else {
    *i0 = 2 * i;
    *i1 = 2 * i + 1;
  }
}

// Rows of `heads` heads from src (head h at src + h * s_h) rotated into dst (dst + h * d_h,
// elements stored by `out`); src and dst may alias (q in place: each pair is read before
// it is written by one thread).
template <class E, class Out>
__device__ void rotate_rows(uint8_t* dst, int64_t d_h, const uint8_t* src, int64_t s_h, int heads,
                            int d, int style, const float* inv_freq, float pos, Out out) {
  const int half = d / 2;
  for (int idx = threadIdx.x; idx < heads * half; idx += kAppendThreads) {
    const int h = idx / half, i = idx % half;
    int i0, i1;
    pair_of(i, half, style, &i0, &i1);
    const float x0 = Elem<E>::load(src + h * s_h + 2 * i0);
    const float x1 = Elem<E>::load(src + h * s_h + 2 * i1);
    float y0 = x0, y1 = x1;
    if (inv_freq) {
      float s, c;
      sincosf(pos * inv_freq[i], &s, &c);
      y0 = x0 * c - x1 * s;
      y1 = x1 * c + x0 * s;
    }
    out.store(dst + h * d_h + Out::kBytes * i0, y0);
    out.store(dst + h * d_h + Out::kBytes * i1, y1);
  }
}

template <class E, bool KV8>
__global__ __launch_bounds__(kAppendThreads) void dk_append_kv_kernel(AppendArgs a) {
  const int b = blockIdx.x;
  const int s0 = min(max(a.indptr[b], 0), a.num_indices);
  const int s1 = min(max(a.indptr[b + 1], 0), a.num_indices);
  if (s1 <= s0) return;                        // a sequence without pages has no slot
  uint32_t page = (uint32_t)a.indices[s1 - 1];
  page = page < a.num_pages ? page : 0u;
  const int slot = min(max(a.last_len[b] - 1, 0), kPageSize - 1);
  const float pos = a.positions ? (float)a.positions[b] : (float)((s1 - s0 - 1) * kPageSize + slot);
  uint8_t* krow = a.k_cache + (int64_t)page * a.kv_p + (int64_t)slot * a.kv_s;
  const uint8_t* kn = a.k_new + (int64_t)b * a.n_b;
  const uint8_t* vn = a.v_new + (int64_t)b * a.n_b;
  uint8_t* vrow = krow + a.v_off;
  if constexpr (KV8) {
    rotate_rows<E>(krow, a.kv_h, kn, a.n_h, a.hkv, a.d, a.rope_style, a.inv_freq, pos,
                   Fp8Store{a.k_scale});
    const Fp8Store vs{a.v_scale};
    for (int idx = threadIdx.x; idx < a.hkv * a.d; idx += kAppendThreads) {
      const int h = idx / a.d, i = idx % a.d;
      vs.store(vrow + h * a.kv_h + i, Elem<E>::load(vn + h * a.n_h + 2 * i));
    }
  } else {
    rotate_rows<E>(krow, a.kv_h, kn, a.n_h, a.hkv, a.d, a.rope_style, a.inv_freq, pos,
                   Elem<E>{});
    for (int idx = threadIdx.x; idx < a.hkv * a.d; idx += kAppendThreads) {
      const int h = idx / a.d, i = idx % a.d;
      *(uint16_t*)(vrow + h * a.kv_h + 2 * i) = *(const uint16_t*)(vn + h * a.n_h + 2 * i);
    }
  }
  if (a.q && a.inv_freq) {
    uint8_t* qb = a.q + (int64_t)b * a.q_b;
    rotate_rows<E>(qb, a.q_h, qb, a.q_h, a.hq, a.d, a.rope_style, a.inv_freq, pos, Elem<E>{});
  }
}

}  // namespace
}  // namespace dk

static int append_impl(void* q, const void* k_new, const void* v_new, int64_t new_b,
                       int64_t new_h, void* k_cache, void* v_cache,
                       const int32_t* kv_indptr, const int32_t* kv_indices,
                       const int32_t* kv_last_page_len, const int32_t* positions,
                       const float* inv_freq, int32_t rope_style, int32_t batch,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       int32_t page_size, int64_t num_pages, int64_t num_indices,
                       int32_t dtype, bool kv8, float k_scale, float v_scale,
                       const dk_strides* strides, void* hip_stream) {
  dk::clear_error();
  if (!strides) return dk::set_error(DK_ENULL, "strides must be non-NULL");
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 ||
      head_dim > 1024)
    return dk::set_error(DK_EINVAL, "dk_append_kv: bad batch / head counts / head_dim");
  if (page_size != dk::kPageSize)
    return dk::set_error(DK_EINVAL, "page_size must be 16; got %d", page_size);
  if (dtype != DK_F16 && dtype != DK_BF16)
    return dk::set_error(DK_EINVAL, "dtype must be DK_F16 or DK_BF16; got %d", dtype);
  if (kv8 && (!(k_scale > 0.f) || !(v_scale > 0.f) || !std::isfinite(k_scale) ||
              !std::isfinite(v_scale)))
    return dk::set_error(DK_EINVAL, "k_scale and v_scale must be finite and > 0");
  if (rope_style != 0 && rope_style != 1)
    return dk::set_error(DK_EINVAL, "rope_style must be 0 (rotate half) or 1 (interleaved)");
  if (num_indices < 0 || num_indices > INT32_MAX || num_pages < 0)
    return dk::set_error(DK_EINVAL, "dk_append_kv: bad num_indices / num_pages");
  if (num_indices > 0 && num_pages == 0)
    return dk::set_error(DK_EINVAL, "kv_indices is non-empty but the page pool is empty");
  const dk_strides& s = *strides;
  if (new_b < 0 || new_h < 0 || s.q_b < 0 || s.q_h < 0 || s.kv_p < 0 || s.kv_s < 0 ||
      s.kv_h < 0 || (!v_cache && s.kv_r < 0))
    return dk::set_error(DK_EINVAL, "strides must be non-negative");
  // every byte offset formed from the strides must fit int64 (bounded in 128-bit arithmetic)
  const int64_t kes_ = kv8 ? 1 : 2;
  if (!dk::extent_ok(batch, s.q_b, num_q_heads, s.q_h, head_dim, 2) ||
      !dk::extent_ok(batch, new_b, num_kv_heads, new_h, head_dim, 2) ||
      !dk::pool_ok(num_pages, s, v_cache ? 0 : s.kv_r, num_kv_heads, head_dim, kes_))
    return dk::set_error(DK_EUNSUPPORTED,
                         "strides must be below 2^40 elements and q, the new rows and the cache "
                         "must span less than 2^62 bytes");
  if (batch == 0) return DK_OK;
  if (!k_new || !v_new || !k_cache || !kv_indptr || !kv_last_page_len ||
      (num_indices > 0 && !kv_indices))
    return dk::set_error(DK_ENULL, "dk_append_kv: NULL pointer");
  dk::AppendArgs a{};
  a.q = static_cast<uint8_t*>(q);
  a.k_new = static_cast<const uint8_t*>(k_new);
  a.v_new = static_cast<const uint8_t*>(v_new);
  a.k_cache = static_cast<uint8_t*>(k_cache);
  const int64_t kes = kv8 ? 1 : 2;   // cache element bytes
  a.v_off = v_cache ? (int64_t)(static_cast<uint8_t*>(v_cache) - static_cast<uint8_t*>(k_cache))
                    : s.kv_r * kes;
  a.indptr = kv_indptr;
  a.indices = kv_indices;
  a.last_len = kv_last_page_len;
  a.positions = positions;
  a.inv_freq = inv_freq;
  a.q_b = s.q_b * 2;
  a.q_h = s.q_h * 2;
  a.n_b = new_b * 2;
  a.n_h = new_h * 2;
  a.kv_p = s.kv_p * kes;
  a.kv_s = s.kv_s * kes;
  a.kv_h = s.kv_h * kes;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.batch = batch;
  a.hq = num_q_heads;
  a.hkv = num_kv_heads;
  a.d = head_dim;
  a.num_indices = (int32_t)num_indices;
  a.rope_style = rope_style;
  a.num_pages = (uint32_t)std::min<int64_t>(num_pages, (int64_t)1 << 31);
  void* args[] = {&a};
  const void* fn =
      kv8 ? (dtype == DK_F16 ? (const void*)dk::dk_append_kv_kernel<_Float16, true>
                             : (const void*)dk::dk_append_kv_kernel<__bf16, true>)
          : (dtype == DK_F16 ? (const void*)dk::dk_append_kv_kernel<_Float16, false>
                             : (const void*)dk::dk_append_kv_kernel<__bf16, false>);
  const hipError_t e = hipLaunchKernel(fn, dim3(batch), dim3(dk::kAppendThreads), args, 0,
                                       static_cast<hipStream_t>(hip_stream));
  if (e != hipSuccess) return dk::set_error((int)e, "append launch: %s", hipGetErrorString(e));
  return DK_OK;
}

extern "C" int dk_append_kv(void* q, const void* k_new, const void* v_new, int64_t new_b,
                            int64_t new_h, void* k_cache, void* v_cache,
                            const int32_t* kv_indptr, const int32_t* kv_indices,
                            const int32_t* kv_last_page_len, const int32_t* positions,
                            const float* inv_freq, int32_t rope_style, int32_t batch,
                            int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t page_size, int64_t num_pages, int64_t num_indices,
                            int32_t dtype, const dk_strides* strides, void* hip_stream) {
  return append_impl(q, k_new, v_new, new_b, new_h, k_cache, v_cache, kv_indptr, kv_indices,
                     kv_last_page_len, positions, inv_freq, rope_style, batch, num_q_heads,
                     num_kv_heads, head_dim, page_size, num_pages, num_indices, dtype, false,
                     0.f, 0.f, strides, hip_stream);
}

extern "C" int dk_append_kv_fp8(void* q, const void* k_new, const void* v_new, int64_t new_b,
                                int64_t new_h, void* k_cache, void* v_cache,
                                const int32_t* kv_indptr, const int32_t* kv_indices,
                                const int32_t* kv_last_page_len, const int32_t* positions,
                                const float* inv_freq, int32_t rope_style, int32_t batch,
                                int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t page_size, int64_t num_pages, int64_t num_indices,
                                int32_t dtype, float k_scale, float v_scale,
                                const dk_strides* strides, void* hip_stream) {
  return append_impl(q, k_new, v_new, new_b, new_h, k_cache, v_cache, kv_indptr, kv_indices,
                     kv_last_page_len, positions, inv_freq, rope_style, batch, num_q_heads,
                     num_kv_heads, head_dim, page_size, num_pages, num_indices, dtype, true,
                     k_scale, v_scale, strides, hip_stream);
}
