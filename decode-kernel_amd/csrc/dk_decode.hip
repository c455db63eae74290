// dk_decode.hip — split-KV paged decode attention for CDNA4 (gfx950, wave64).
//
// Pass 1 (dk_pass1): one workgroup per (sequence, kv head, split); its NW wavefronts take
// the split's pages round-robin. A wavefront owns one 16-token page at a time:
//   * K rows arrive as 16-byte non-temporal loads laid out as the A operand of
//     v_mfma_f32_16x16x32_{f16,bf16} (lane l: token l%16, 8 dims per MFMA), so S^T = K.Q^T
//     lands with lane (r = l/16, c = l%16) holding the scores of tokens 4r..4r+3 for q head
//     (c mod 4) of the GQA group — every K element is read once and serves all G heads.
//   * V rows arrive as 16-byte loads with lane (r, c) holding tokens 4r..4r+3, dims
//     c*D/16 .. c*D/16 + D/16 - 1 (each 16-lane row of the wave reads whole 256-B rows).
//   * Online softmax in fp32 with exp2 (v_exp_f32); the running reference max is only
//     moved when a score exceeds it by more than 2^8 (a wave-uniform branch), so the
//     accumulators are rescaled a handful of times per split instead of every page.
//   * P.V is a VALU fma per (token, head, dim); each lane's p for the other heads of the
//     group comes from its quad neighbours through DPP quad_perm.
//   The next page is loaded while the current one is computed (two register buffers).
//   At the end the 4 lane rows are summed with permlane16/32 swaps and the NW
//   wavefronts are merged through LDS. With one split the workgroup writes the
//   normalised output directly; otherwise it writes fp32 partials (O unnormalised, m, l)
//   with the semantics of the reference's decode_attn_partition_kernel
//   (src/cuda_/attention_ext.cu:207-349, scratch contract src/layout.md:142-167).
// Pass 2 (dk_merge): one wavefront per (sequence, q head) merges the split partials with
//   the log-sum-exp identity (reference decode_attn_reduce_kernel,
//   src/cuda_/attention_ext.cu:363-406).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dk_args.h"
#include "dk_decode.h"

namespace dk {
namespace {

using u32 = uint32_t;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kPage = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kEmptyM = -1e9f;        // partial_m of an empty split (attention_ext.cu:254)
constexpr float kMinit = -1e30f;        // running reference before the first score
constexpr float kSlack = 8.0f;          // log2 headroom before the reference max moves
constexpr float kNegInf = -__builtin_inff();

// ---------------------------------------------------------------- element types
struct F16 {
  static __device__ __forceinline__ float lo(u32 w) {
    return (float)__builtin_bit_cast(f16x2, w)[0];
  }
  static __device__ __forceinline__ float hi(u32 w) {
    return (float)__builtin_bit_cast(f16x2, w)[1];
  }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(u32 a, u32 b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b),
                                  c, false);
  }
  static __device__ __forceinline__ void store(uint8_t* p, float x) {
    *reinterpret_cast<_Float16*>(p) = (_Float16)x;
  }
};

struct BF16 {
  static __device__ __forceinline__ float lo(u32 w) { return __builtin_bit_cast(float, w << 16); }
  static __device__ __forceinline__ float hi(u32 w) {
    return __builtin_bit_cast(float, w & 0xffff0000u);
  }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(u32 a, u32 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  static __device__ __forceinline__ void store(uint8_t* p, float x) {
    *reinterpret_cast<__bf16*>(p) = (__bf16)x;
  }
};

// ---------------------------------------------------------------- cross-lane helpers
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  // bound_ctrl: every pattern used here reads an existing lane, so no "old" value is
  // needed (and no zeroing move is emitted for it).
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
// Value of lane (4*(l/4) + Q): DPP quad_perm [Q,Q,Q,Q].
template <int Q>
__device__ __forceinline__ float quad_bcast(float x) {
  return dpp<Q * 0x55>(x);
}
// Rotate right by N lanes inside each row of 16: DPP row_ror:N.
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return dpp<0x120 + N>(x);
}
// (v[l], v[l ^ 16]) and (v[l], v[l ^ 32]) through the gfx950 permlane swaps; both lanes
// of a pair get the operands in the same order, so sums are bitwise identical.
__device__ __forceinline__ float sum_xor16(float x) {
  const u32 v = __builtin_bit_cast(u32, x);
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return __builtin_bit_cast(float, (u32)r[0]) + __builtin_bit_cast(float, (u32)r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const u32 v = __builtin_bit_cast(u32, x);
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __builtin_bit_cast(float, (u32)r[0]) + __builtin_bit_cast(float, (u32)r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
  const u32 v = __builtin_bit_cast(u32, x);
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return fmaxf(__builtin_bit_cast(float, (u32)r[0]), __builtin_bit_cast(float, (u32)r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const u32 v = __builtin_bit_cast(u32, x);
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__builtin_bit_cast(float, (u32)r[0]), __builtin_bit_cast(float, (u32)r[1]));
}
// Max over all lanes whose column c = l%16 agrees modulo GQ (every lane holding the
// same q head of a head set), result in all of them.
template <int GQ>
__device__ __forceinline__ float allmax_head(float x) {
  if constexpr (GQ == 1) {
    x = fmaxf(x, row_ror<1>(x));
    x = fmaxf(x, row_ror<2>(x));
  } else if constexpr (GQ == 2) {
    x = fmaxf(x, row_ror<2>(x));
  }
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<8>(x));
  return max_xor32(max_xor16(x));
}
// Sum over the 16 lanes of a row (result in all of them).
__device__ __forceinline__ float row_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += row_ror<4>(x);
  x += row_ror<8>(x);
  return x;
}
__device__ __forceinline__ float wave_sum(float x) { return sum_xor32(sum_xor16(row_sum(x))); }
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<8>(x));
  return max_xor32(max_xor16(x));
}
__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

// ---------------------------------------------------------------- streaming loads
__device__ __forceinline__ u32x4 ld_nt16(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld_nt8(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
// NWORDS consecutive 32-bit words from p (NWORDS in {2, 4, 8}).
template <int NWORDS>
__device__ __forceinline__ void ld_words(u32* dst, const uint8_t* p) {
  if constexpr (NWORDS == 2) {
    const u32x2 v = ld_nt8(p);
    dst[0] = v[0];
    dst[1] = v[1];
  } else {
#pragma unroll
    for (int k = 0; k < NWORDS / 4; ++k) {
      const u32x4 v = ld_nt16(p + 16 * k);
      dst[4 * k + 0] = v[0];
      dst[4 * k + 1] = v[1];
      dst[4 * k + 2] = v[2];
      dst[4 * k + 3] = v[3];
    }
  }
}
template <int NWORDS>
__device__ __forceinline__ void ld_words_cached(u32* dst, const uint8_t* p) {
#pragma unroll
  for (int k = 0; k < NWORDS; ++k) dst[k] = reinterpret_cast<const u32*>(p)[k];
}

// ---------------------------------------------------------------- pass 1
struct Pass1Args {
  const uint8_t* q;
  const uint8_t* kv;
  const int32_t* indptr;
  const int32_t* indices;
  const int32_t* last_len;
  float* part_o;
  float* part_m;
  float* part_l;
  uint8_t* out;
  int64_t q_b, q_h, kv_p, o_b, o_h;   // bytes
  int32_t kv_r, kv_s, kv_h;           // bytes
  int32_t hq, hkv, group, chunks, split;
  int32_t num_indices;
  uint32_t num_pages;                 // clamp bound for page ids (min(num_pages, 2^31))
  int32_t direct;                     // 1: split == 1, write normalised output
  float kscale;                       // log2(e) / sqrt(head_dim)
};

// Resident wavefronts per SIMD the register allocator is held to: two page buffers of
// D/4 words each, G*D/16 accumulators and the q operand must fit without spilling.
template <int D, int G>
constexpr int min_waves_per_simd() {
  return D >= 256 ? 1 : (D * G >= 1024 ? 2 : 3);
}

template <class T, int D, int G, int NW, bool MFMA>
__global__ __launch_bounds__(NW * 64, (min_waves_per_simd<D, G>())) void dk_pass1(Pass1Args a) {
  constexpr int GQ = G < 4 ? G : 4;   // heads per MFMA column set
  constexpr int NS = G / GQ;          // column sets (G = 8 -> 2)
  constexpr int DPL = D / 16;         // V dims per lane
  constexpr int VWT = DPL / 2;        // V words per token per lane
  constexpr int KW = D / 8;           // K words per lane per page (both q.k paths)
  constexpr int VW = 4 * VWT;         // V words per lane per page
  constexpr int NMF = D / 32;         // MFMAs per head set per page

  __shared__ float sm_acc[NW][G][D];
  __shared__ float sm_m[NW][G], sm_mt[NW][G], sm_l[NW][G];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane >> 4, c = lane & 15;

  int t = blockIdx.x;
  const int hc = t % a.chunks;
  t /= a.chunks;
  const int kvh = t % a.hkv;
  t /= a.hkv;
  const int s = t % a.split;
  const int b = t / a.split;

  int seq0 = a.indptr[b], seq1 = a.indptr[b + 1];
  seq0 = min(max(seq0, 0), a.num_indices);
  seq1 = min(max(seq1, seq0), a.num_indices);
  const int npages = seq1 - seq0;
  const int pps = (npages + a.split - 1) / a.split;          // attention_ext.cu:249-252
  const int p0 = min(s * pps, npages);
  const int n = max(min(p0 + pps, npages) - p0, 0);
  const int valid_last = min(max(a.last_len[b], 0), kPage);
  const int qh0 = kvh * a.group + hc * G;

  // ---- q operand (loaded once)
  const uint8_t* qbase = a.q + (int64_t)b * a.q_b + (int64_t)qh0 * a.q_h;
  u32 qw[NS][KW];   // MFMA: Q^T column (head s*GQ + c%GQ), dims 32i + 8*r16 .. +7
  u32 qv[G][VWT];   // VALU: head h, dims c*DPL .. +DPL-1
  if constexpr (MFMA) {
#pragma unroll
    for (int ss = 0; ss < NS; ++ss) {
      const uint8_t* qp = qbase + (int64_t)(ss * GQ + c % GQ) * a.q_h + 16 * r16;
#pragma unroll
      for (int i = 0; i < NMF; ++i) ld_words_cached<4>(&qw[ss][4 * i], qp + 64 * i);
    }
  } else {
#pragma unroll
    for (int h = 0; h < G; ++h)
      ld_words_cached<VWT>(qv[h], qbase + (int64_t)h * a.q_h + 2 * DPL * c);
  }

  // ---- per-lane byte offsets inside a page (the same every page)
  const uint8_t* kvh_base = a.kv + (int64_t)kvh * a.kv_h;
  const u32 koff = MFMA ? (u32)(c * a.kv_s + 16 * r16) : (u32)(4 * r16 * a.kv_s + 2 * DPL * c);
  const u32 voff = (u32)(a.kv_r + 4 * r16 * a.kv_s + 2 * DPL * c);
  const u32 tok_s = (u32)a.kv_s;

  // ---- running state
  float acc[G][DPL];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[h][j] = 0.f;
  float mref[NS], mtrue[NS], lsum[NS];
#pragma unroll
  for (int ss = 0; ss < NS; ++ss) {
    mref[ss] = kMinit;
    mtrue[ss] = kNegInf;
    lsum[ss] = 0.f;
  }

  // pages of this wavefront: j = w + NW*k, k < nk
  const int nk = n > w ? (n - w + NW - 1) / NW : 0;
  const int32_t* ids = a.indices + seq0 + p0 + w;
  const int last_k = (npages - 1 - p0 - w) % NW == 0 ? (npages - 1 - p0 - w) / NW : -1;

  // Page id of wave page k and its base address.
  // readfirstlane keeps ids and page addresses in scalar registers (they are uniform).
  auto page_id = [&](int k) -> u32 {
    const u32 pid = (u32)__builtin_amdgcn_readfirstlane(ids[NW * k]);
    return pid < a.num_pages ? pid : 0u;
  };
  auto page_ptr = [&](u32 pid) -> const uint8_t* { return kvh_base + (int64_t)pid * a.kv_p; };
  auto load_page = [&](u32 (&kb)[KW], u32 (&vb)[VW], const uint8_t* pg) {
    if constexpr (MFMA) {
#pragma unroll
      for (int i = 0; i < NMF; ++i) ld_words<4>(&kb[4 * i], pg + koff + 64 * i);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) ld_words<VWT>(&kb[r * VWT], pg + koff + r * tok_s);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) ld_words<VWT>(&vb[r * VWT], pg + voff + r * tok_s);
  };

  auto compute_page = [&](const u32 (&kb)[KW], u32 (&vb)[VW], int k) {
    // S^T scores: sc[ss][r] = q_{head ss*GQ + c%GQ} . k_{token 4*r16 + r}
    float sc[NS][4];
    if constexpr (MFMA) {
#pragma unroll
      for (int ss = 0; ss < NS; ++ss) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
          const u32x4 av = {kb[4 * i], kb[4 * i + 1], kb[4 * i + 2], kb[4 * i + 3]};
          const u32x4 bv = {qw[ss][4 * i], qw[ss][4 * i + 1], qw[ss][4 * i + 2],
                            qw[ss][4 * i + 3]};
          d = T::mfma(av, bv, d);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[ss][r] = d[r];
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float part[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float x = 0.f;
#pragma unroll
          for (int q = 0; q < VWT; ++q) x = T::dot2(kb[r * VWT + q], qv[h][q], x);
          part[h] = row_sum(x);
        }
#pragma unroll
        for (int ss = 0; ss < NS; ++ss) {
          float v = part[ss * GQ];
#pragma unroll
          for (int g = 1; g < GQ; ++g) v = (c % GQ == g) ? part[ss * GQ + g] : v;
          sc[ss][r] = v;
        }
      }
    }
    // last page of the sequence: tokens >= valid are masked (select, never multiply, so
    // stale or NaN bytes in the page tail cannot reach the output)
    if (k == last_k && valid_last < kPage) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (4 * r16 + r >= valid_last) {
#pragma unroll
          for (int ss = 0; ss < NS; ++ss) sc[ss][r] = kNegInf;
#pragma unroll
          for (int q = 0; q < VWT; ++q) vb[r * VWT + q] = 0u;
        }
      }
    }
    // online softmax (log2 domain)
    float x[NS][4], mx[NS];
    bool need = false;
#pragma unroll
    for (int ss = 0; ss < NS; ++ss) {
#pragma unroll
      for (int r = 0; r < 4; ++r) x[ss][r] = sc[ss][r] * a.kscale;
      mx[ss] = fmaxf(fmaxf(x[ss][0], x[ss][1]), fmaxf(x[ss][2], x[ss][3]));
      mtrue[ss] = fmaxf(mtrue[ss], mx[ss]);
      need |= mx[ss] > mref[ss] + kSlack;
    }
    if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
      for (int ss = 0; ss < NS; ++ss) {
        const float mn = allmax_head<GQ>(fmaxf(mref[ss], mx[ss]));
        const float al = __builtin_amdgcn_exp2f(mref[ss] - mn);
        lsum[ss] *= al;
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
          float ab = al;
          if constexpr (GQ > 1) {
            if (g == 0) ab = quad_bcast<0>(al);
            if (g == 1) ab = quad_bcast<1>(al);
            if (g == 2) ab = quad_bcast<2>(al);
            if (g == 3) ab = quad_bcast<3>(al);
          }
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[ss * GQ + g][j] *= ab;
        }
        mref[ss] = mn;
      }
    }
    float p[NS][4];
#pragma unroll
    for (int ss = 0; ss < NS; ++ss) {
#pragma unroll
      for (int r = 0; r < 4; ++r) p[ss][r] = __builtin_amdgcn_exp2f(x[ss][r] - mref[ss]);
      lsum[ss] += (p[ss][0] + p[ss][1]) + (p[ss][2] + p[ss][3]);
    }
    // P.V
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float vf[DPL];
#pragma unroll
      for (int q = 0; q < VWT; ++q) {
        vf[2 * q] = T::lo(vb[r * VWT + q]);
        vf[2 * q + 1] = T::hi(vb[r * VWT + q]);
      }
#pragma unroll
      for (int ss = 0; ss < NS; ++ss) {
#pragma unroll
        for (int g = 0; g < GQ; ++g) {
          float pb = p[ss][r];
          if constexpr (GQ > 1) {
            if (g == 0) pb = quad_bcast<0>(p[ss][r]);
            if (g == 1) pb = quad_bcast<1>(p[ss][r]);
            if (g == 2) pb = quad_bcast<2>(p[ss][r]);
            if (g == 3) pb = quad_bcast<3>(p[ss][r]);
          }
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[ss * GQ + g][j] = fmaf(pb, vf[j], acc[ss * GQ + g][j]);
        }
      }
    }
  };

  // ---- page loop: the next page's loads are in flight while the current page is
  // computed. The steady-state loop has no early exit (pages k, k+1, k+2 all exist), so
  // the hardware wait counters see the same pending loads on every path into the loop
  // head and only wait for the page about to be used; the last one or two pages are
  // peeled off after it.
  u32 ka[KW], va[VW], kb2[KW], vb2[VW];
  if (nk > 0) {
    load_page(ka, va, page_ptr(page_id(0)));
    int k = 0;
    for (; k + 2 < nk; k += 2) {
      load_page(kb2, vb2, page_ptr(page_id(k + 1)));
      compute_page(ka, va, k);
      load_page(ka, va, page_ptr(page_id(k + 2)));
      compute_page(kb2, vb2, k + 1);
    }
    if (k + 1 < nk) {
      load_page(kb2, vb2, page_ptr(page_id(k + 1)));
      compute_page(ka, va, k);
      compute_page(kb2, vb2, k + 1);
    } else {
      compute_page(ka, va, k);
    }
  }

  // ---- reduce the wavefront's four lane rows
#pragma unroll
  for (int ss = 0; ss < NS; ++ss) {
    lsum[ss] = sum_xor32(sum_xor16(lsum[ss]));
    mtrue[ss] = allmax_head<GQ>(mtrue[ss]);
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[h][j] = sum_xor32(sum_xor16(acc[h][j]));

#pragma unroll
  for (int h = 0; h < G; ++h) {
    if (h % 4 == r16) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) sm_acc[w][h][c * DPL + j] = acc[h][j];
    }
  }
  if (r16 == 0 && c < GQ) {
#pragma unroll
    for (int ss = 0; ss < NS; ++ss) {
      sm_m[w][ss * GQ + c] = mref[ss];
      sm_mt[w][ss * GQ + c] = mtrue[ss];
      sm_l[w][ss * GQ + c] = lsum[ss];
    }
  }
  __syncthreads();

  // ---- merge the wavefronts and write
  for (int idx = threadIdx.x; idx < G * D; idx += NW * 64) {
    const int h = idx / D, d = idx % D;
    float mt = kNegInf;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) mt = fmaxf(mt, sm_mt[ww][h]);
    float L = 0.f, O = 0.f;
    const bool empty = !(mt > kNegInf);
    if (!empty) {
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float f = __builtin_amdgcn_exp2f(sm_m[ww][h] - mt);
        L += sm_l[ww][h] * f;
        O += sm_acc[ww][h][d] * f;
      }
    }
    const int qh = qh0 + h;
    if (a.direct) {
      const float o = L > 0.f ? O / L : 0.f;
      T::store(a.out + (int64_t)b * a.o_b + (int64_t)qh * a.o_h + 2 * d, o);
    } else {
      const int64_t row = ((int64_t)b * a.hq + qh) * a.split + s;
      a.part_o[row * D + d] = empty ? 0.f : O;
      if (d == 0) {
        a.part_m[row] = empty ? kEmptyM : mt * kLn2;
        a.part_l[row] = L;
      }
    }
  }
}

// ---------------------------------------------------------------- pass 2
template <class T, int D>
__global__ __launch_bounds__(256) void dk_merge(const float* __restrict__ po,
                                                const float* __restrict__ pm,
                                                const float* __restrict__ pl, uint8_t* out,
                                                int64_t o_b, int64_t o_h, int32_t hq,
                                                int32_t rows, int32_t split) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* m = pm + (int64_t)row * split;
  const float* l = pl + (int64_t)row * split;
  float M = kNegInf;
  for (int ss = lane; ss < split; ss += 64) M = fmaxf(M, m[ss]);
  M = wave_max(M);
  float accv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) accv[e] = 0.f;
  float L = 0.f;
  for (int s0 = 0; s0 < split; s0 += 64) {
    const int ss = s0 + lane;
    float wgt = 0.f;
    if (ss < split) {
      wgt = __builtin_amdgcn_exp2f((m[ss] - M) * kLog2e);
      L += wgt * l[ss];
    }
    const int cnt = min(64, split - s0);
    const float* o = po + ((int64_t)row * split + s0) * D + lane * E;
    for (int k = 0; k < cnt; ++k) {
      const float wk = readlane_f(wgt, k);
      if constexpr (E == 1) {
        accv[0] = fmaf(wk, o[(int64_t)k * D], accv[0]);
      } else if constexpr (E == 2) {
        const f32x2 v = *reinterpret_cast<const f32x2*>(o + (int64_t)k * D);
        accv[0] = fmaf(wk, v[0], accv[0]);
        accv[1] = fmaf(wk, v[1], accv[1]);
      } else {
        const f32x4 v = *reinterpret_cast<const f32x4*>(o + (int64_t)k * D);
#pragma unroll
        for (int e = 0; e < 4; ++e) accv[e] = fmaf(wk, v[e], accv[e]);
      }
    }
  }
  L = wave_sum(L);
  const int b = row / hq, qh = row % hq;
  uint8_t* op = out + (int64_t)b * o_b + (int64_t)qh * o_h + 2 * lane * E;
#pragma unroll
  for (int e = 0; e < E; ++e) T::store(op + 2 * e, L > 0.f ? accv[e] / L : 0.f);
}

// ---------------------------------------------------------------- host side
struct Launch {
  Pass1Args a;
  int grid;
  hipStream_t stream;
};

template <class T, int D, int G, int NW, bool MFMA>
hipError_t launch_pass1_t(const Launch& L) {
  hipLaunchKernelGGL((dk_pass1<T, D, G, NW, MFMA>), dim3(L.grid), dim3(NW * 64), 0, L.stream,
                     L.a);
  return hipGetLastError();
}

template <class T, int D, int G, int NW>
hipError_t launch_pass1_m(const Launch& L, bool mfma) {
  return mfma ? launch_pass1_t<T, D, G, NW, true>(L) : launch_pass1_t<T, D, G, NW, false>(L);
}

template <class T, int D, int G>
hipError_t launch_pass1_w(const Launch& L, int waves, bool mfma) {
  switch (waves) {
    case 1: return launch_pass1_m<T, D, G, 1>(L, mfma);
    case 2: return launch_pass1_m<T, D, G, 2>(L, mfma);
    default: return launch_pass1_m<T, D, G, 4>(L, mfma);
  }
}

template <class T, int D>
hipError_t launch_pass1_g(const Launch& L, int heads, int waves, bool mfma) {
  switch (heads) {
    case 1: return launch_pass1_w<T, D, 1>(L, waves, mfma);
    case 2: return launch_pass1_w<T, D, 2>(L, waves, mfma);
    case 4: return launch_pass1_w<T, D, 4>(L, waves, mfma);
    default:
      if constexpr (D <= 128) return launch_pass1_w<T, D, 8>(L, waves, mfma);
      return hipErrorInvalidValue;
  }
}

template <class T>
hipError_t launch_pass1_d(const Launch& L, int d, int heads, int waves, bool mfma) {
  switch (d) {
    case 64: return launch_pass1_g<T, 64>(L, heads, waves, mfma);
    case 128: return launch_pass1_g<T, 128>(L, heads, waves, mfma);
    default: return launch_pass1_g<T, 256>(L, heads, waves, mfma);
  }
}

template <class T>
hipError_t launch_merge_t(int d, const float* po, const float* pm, const float* pl,
                          uint8_t* out, int64_t o_b, int64_t o_h, int hq, int rows, int split,
                          hipStream_t st) {
  const dim3 grid((rows + 3) / 4), block(256);
  switch (d) {
    case 64:
      hipLaunchKernelGGL((dk_merge<T, 64>), grid, block, 0, st, po, pm, pl, out, o_b, o_h, hq,
                         rows, split);
      break;
    case 128:
      hipLaunchKernelGGL((dk_merge<T, 128>), grid, block, 0, st, po, pm, pl, out, o_b, o_h, hq,
                         rows, split);
      break;
    default:
      hipLaunchKernelGGL((dk_merge<T, 256>), grid, block, 0, st, po, pm, pl, out, o_b, o_h, hq,
                         rows, split);
      break;
  }
  return hipGetLastError();
}

int hip_fail(hipError_t e, const char* what) {
  return set_error((int)e, "%s: %s", what, hipGetErrorString(e));
}

// Resident pass-1 workgroups per compute unit for this problem's kernel, from the
// occupancy calculator (cached per (dtype, head_dim, heads, waves, path)).
int resident_groups(int dtype, int d, int heads, int waves, bool mfma) {
  const void* fn = nullptr;
#define DK_FN(T_, D_, G_, W_, M_) reinterpret_cast<const void*>(&dk_pass1<T_, D_, G_, W_, M_>)
#define DK_PICK_W(T_, D_, G_)                                                               \
  fn = waves == 1 ? (mfma ? DK_FN(T_, D_, G_, 1, true) : DK_FN(T_, D_, G_, 1, false))       \
       : waves == 2 ? (mfma ? DK_FN(T_, D_, G_, 2, true) : DK_FN(T_, D_, G_, 2, false))     \
                    : (mfma ? DK_FN(T_, D_, G_, 4, true) : DK_FN(T_, D_, G_, 4, false))
#define DK_PICK_G(T_, D_)                     \
  switch (heads) {                            \
    case 1: DK_PICK_W(T_, D_, 1); break;      \
    case 2: DK_PICK_W(T_, D_, 2); break;      \
    case 4: DK_PICK_W(T_, D_, 4); break;      \
    default: DK_PICK_W(T_, D_, 8); break;     \
  }
#define DK_PICK_G256(T_)                      \
  switch (heads) {                            \
    case 1: DK_PICK_W(T_, 256, 1); break;     \
    case 2: DK_PICK_W(T_, 256, 2); break;     \
    default: DK_PICK_W(T_, 256, 4); break;    \
  }
  if (dtype == DK_F16) {
    if (d == 64) { DK_PICK_G(F16, 64) } else if (d == 128) { DK_PICK_G(F16, 128) } else { DK_PICK_G256(F16) }
  } else {
    if (d == 64) { DK_PICK_G(BF16, 64) } else if (d == 128) { DK_PICK_G(BF16, 128) } else { DK_PICK_G256(BF16) }
  }
#undef DK_PICK_G256
#undef DK_PICK_G
#undef DK_PICK_W
#undef DK_FN
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, waves * 64, 0) != hipSuccess ||
      blocks <= 0)
    blocks = 1;
  return blocks;
}

int cu_count(int device) {
  static int cached[64] = {0};
  if (device < 0) {
    if (hipGetDevice(&device) != hipSuccess) return -1;
  }
  if (device < 64 && cached[device] > 0) return cached[device];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return -1;
  if (device < 64) cached[device] = n;
  return n;
}

int auto_split(const Problem& p, int device) {
  Problem q = p;
  q.split = 1;
  const Plan pl = make_plan(q);
  const int cus = cu_count(device);
  if (cus <= 0) return hip_fail(hipGetLastError(), "hipDeviceGetAttribute");
  const int per_cu = resident_groups(p.dtype, p.head_dim, pl.heads, pl.waves, pl.mfma);
  const int64_t units = (int64_t)p.batch * p.hkv * pl.chunks;
  const int64_t avg = p.batch > 0 ? p.num_indices / p.batch : 0;
  return choose_split(units, (int64_t)cus * per_cu, avg, pl.waves);
}

}  // namespace

// Full launch sequence, shared by the extern "C" entry points.
static int dk_run(Problem p, bool do_merge, void* stream) {
  clear_error();
  if (p.split == 0) {
    if (p.batch == 0) return DK_OK;
    const int s = auto_split(p, -1);
    if (s <= 0) return s < 0 ? s : set_error(DK_EINVAL, "split choice failed");
    p.split = s;
  }
  const int rc = validate(p);
  if (rc != DK_OK || p.batch == 0) return rc;
  const Plan pl = make_plan(p);
  const bool direct = p.need_out && p.split == 1;
  const int64_t esize = 2;

  Launch L{};
  Pass1Args& a = L.a;
  a.q = static_cast<const uint8_t*>(p.q);
  a.kv = static_cast<const uint8_t*>(p.kv);
  a.indptr = p.indptr;
  a.indices = p.indices;
  a.last_len = p.last_len;
  size_t off_o = 0, off_m = 0, off_l = 0;
  if (!direct) {
    partials_layout(p.batch, p.hq, p.head_dim, p.split, &off_o, &off_m, &off_l);
    uint8_t* ws = static_cast<uint8_t*>(p.workspace);
    a.part_o = reinterpret_cast<float*>(ws + off_o);
    a.part_m = reinterpret_cast<float*>(ws + off_m);
    a.part_l = reinterpret_cast<float*>(ws + off_l);
  }
  a.out = static_cast<uint8_t*>(p.out);
  a.q_b = p.st.q_b * esize;
  a.q_h = p.st.q_h * esize;
  a.kv_p = p.st.kv_p * esize;
  a.o_b = p.st.o_b * esize;
  a.o_h = p.st.o_h * esize;
  a.kv_r = (int32_t)(p.st.kv_r * esize);
  a.kv_s = (int32_t)(p.st.kv_s * esize);
  a.kv_h = (int32_t)(p.st.kv_h * esize);
  a.hq = p.hq;
  a.hkv = p.hkv;
  a.group = pl.group;
  a.chunks = pl.chunks;
  a.split = p.split;
  a.num_indices = (int32_t)p.num_indices;
  a.num_pages = (uint32_t)(p.num_pages < ((int64_t)1 << 31) ? p.num_pages : ((int64_t)1 << 31));
  a.direct = direct ? 1 : 0;
  a.kscale = kLog2e / sqrtf((float)p.head_dim);
  L.grid = (int)pl.pass1_groups;
  L.stream = static_cast<hipStream_t>(stream);

  hipError_t e = p.dtype == DK_F16
                     ? launch_pass1_d<F16>(L, p.head_dim, pl.heads, pl.waves, pl.mfma)
                     : launch_pass1_d<BF16>(L, p.head_dim, pl.heads, pl.waves, pl.mfma);
  if (e != hipSuccess) return hip_fail(e, "pass-1 launch");
  if (do_merge && !direct) {
    const int rows = p.batch * p.hq;
    e = p.dtype == DK_F16
            ? launch_merge_t<F16>(p.head_dim, a.part_o, a.part_m, a.part_l, a.out, a.o_b, a.o_h,
                                  p.hq, rows, p.split, L.stream)
            : launch_merge_t<BF16>(p.head_dim, a.part_o, a.part_m, a.part_l, a.out, a.o_b,
                                   a.o_h, p.hq, rows, p.split, L.stream);
    if (e != hipSuccess) return hip_fail(e, "merge launch");
  }
  return DK_OK;
}

}  // namespace dk

// ---------------------------------------------------------------- C ABI
using dk::Problem;

static Problem make_problem(const void* q, const void* kv, const int32_t* indptr,
                            const int32_t* indices, const int32_t* last_len, void* out,
                            void* ws, size_t ws_bytes, int32_t batch, int32_t hq, int32_t hkv,
                            int32_t d, int32_t page, int64_t num_pages, int64_t num_indices,
                            int32_t dtype, const dk_strides* st, int32_t split,
                            const dk_options* opts, bool need_out) {
  Problem p;
  p.q = q;
  p.kv = kv;
  p.indptr = indptr;
  p.indices = indices;
  p.last_len = last_len;
  p.out = out;
  p.workspace = ws;
  p.workspace_bytes = ws_bytes;
  p.batch = batch;
  p.hq = hq;
  p.hkv = hkv;
  p.head_dim = d;
  p.page_size = page;
  p.num_pages = num_pages;
  p.num_indices = num_indices;
  p.dtype = dtype;
  if (st) p.st = *st;
  p.split = split;
  if (opts) p.opt = *opts;
  p.need_out = need_out;
  return p;
}

extern "C" {

int dk_abi_version(void) { return DK_ABI_VERSION; }

const char* dk_last_error(void) { return dk::last_error(); }

size_t dk_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                          int32_t split_kv) {
  return dk::workspace_bytes(batch, num_q_heads, head_dim, split_kv);
}

int dk_partials_layout(int32_t batch, int32_t num_q_heads, int32_t head_dim, int32_t split_kv,
                       size_t* off_o, size_t* off_m, size_t* off_l, size_t* total) {
  dk::clear_error();
  if (batch < 0 || num_q_heads <= 0 || head_dim <= 0 || split_kv <= 0 || !off_o || !off_m ||
      !off_l || !total)
    return dk::set_error(DK_EINVAL, "dk_partials_layout: bad argument");
  dk::partials_layout(batch, num_q_heads, head_dim, split_kv, off_o, off_m, off_l);
  *total = dk::partials_bytes(batch, num_q_heads, head_dim, split_kv);
  return DK_OK;
}

int dk_choose_split(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                    int32_t dtype, int64_t avg_pages_per_seq, int32_t device) {
  dk::clear_error();
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      (dtype != DK_F16 && dtype != DK_BF16) || avg_pages_per_seq < 0)
    return dk::set_error(DK_EINVAL, "dk_choose_split: bad argument");
  Problem p;
  p.batch = batch;
  p.hq = num_q_heads;
  p.hkv = num_kv_heads;
  p.head_dim = head_dim;
  p.dtype = dtype;
  p.num_indices = avg_pages_per_seq * (int64_t)(batch > 0 ? batch : 0);
  p.split = 1;
  return dk::auto_split(p, device);
}

int dk_decode_attention_ex(const void* q, const void* kv_data, const int32_t* kv_indptr,
                           const int32_t* kv_indices, const int32_t* kv_last_page_len,
                           void* out, void* workspace, size_t workspace_bytes, int32_t batch,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t page_size, int64_t num_pages, int64_t num_indices,
                           int32_t dtype, const dk_strides* strides, int32_t split_kv,
                           const dk_options* opts, void* hip_stream) {
  if (!strides) return dk::set_error(DK_ENULL, "strides must be non-NULL");
  if (split_kv < 0) return dk::set_error(DK_EINVAL, "split_kv must be >= 0; got %d", split_kv);
  Problem p = make_problem(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, out, workspace,
                           workspace_bytes, batch, num_q_heads, num_kv_heads, head_dim,
                           page_size, num_pages, num_indices, dtype, strides, split_kv, opts,
                           true);
  return dk::dk_run(p, true, hip_stream);
}

int dk_decode_attention(const void* q, const void* kv_data, const int32_t* kv_indptr,
                        const int32_t* kv_indices, const int32_t* kv_last_page_len, void* out,
                        void* workspace, size_t workspace_bytes, int32_t batch,
                        int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t page_size, int64_t num_pages, int64_t num_indices,
                        int32_t dtype, const dk_strides* strides, int32_t split_kv,
                        void* hip_stream) {
  return dk_decode_attention_ex(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, out,
                                workspace, workspace_bytes, batch, num_q_heads, num_kv_heads,
                                head_dim, page_size, num_pages, num_indices, dtype, strides,
                                split_kv, nullptr, hip_stream);
}

int dk_decode_partials(const void* q, const void* kv_data, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* kv_last_page_len,
                       void* workspace, size_t workspace_bytes, int32_t batch,
                       int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                       int32_t page_size, int64_t num_pages, int64_t num_indices, int32_t dtype,
                       const dk_strides* strides, int32_t split_kv, const dk_options* opts,
                       void* hip_stream) {
  if (!strides) return dk::set_error(DK_ENULL, "strides must be non-NULL");
  if (split_kv < 1) return dk::set_error(DK_EINVAL, "split_kv must be >= 1; got %d", split_kv);
  Problem p = make_problem(q, kv_data, kv_indptr, kv_indices, kv_last_page_len, nullptr,
                           workspace, workspace_bytes, batch, num_q_heads, num_kv_heads,
                           head_dim, page_size, num_pages, num_indices, dtype, strides,
                           split_kv, opts, false);
  return dk::dk_run(p, false, hip_stream);
}

int dk_merge_partials(const void* workspace, size_t workspace_bytes, void* out, int32_t batch,
                      int32_t num_q_heads, int32_t head_dim, int32_t dtype, int64_t o_b,
                      int64_t o_h, int32_t split_kv, void* hip_stream) {
  dk::clear_error();
  if (batch < 0 || num_q_heads <= 0 || split_kv < 1 ||
      (head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      (dtype != DK_F16 && dtype != DK_BF16) || o_b < 0 || o_h < 0)
    return dk::set_error(DK_EINVAL, "dk_merge_partials: bad argument");
  if (batch == 0) return DK_OK;
  if (!workspace || !out) return dk::set_error(DK_ENULL, "workspace and out must be non-NULL");
  if ((int64_t)batch * num_q_heads > INT32_MAX)
    return dk::set_error(DK_EINVAL, "dk_merge_partials: batch*num_q_heads too large");
  const size_t need = dk::partials_bytes(batch, num_q_heads, head_dim, split_kv);
  if (workspace_bytes < need)
    return dk::set_error(DK_EWORKSPACE, "workspace of %zu bytes required, %zu given", need,
                         workspace_bytes);
  size_t off_o, off_m, off_l;
  dk::partials_layout(batch, num_q_heads, head_dim, split_kv, &off_o, &off_m, &off_l);
  const uint8_t* ws = static_cast<const uint8_t*>(workspace);
  const int rows = batch * num_q_heads;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const float* po = reinterpret_cast<const float*>(ws + off_o);
  const float* pm = reinterpret_cast<const float*>(ws + off_m);
  const float* pl = reinterpret_cast<const float*>(ws + off_l);
  uint8_t* o = static_cast<uint8_t*>(out);
  hipError_t e = dtype == DK_F16 ? dk::launch_merge_t<dk::F16>(head_dim, po, pm, pl, o, o_b * 2,
                                                               o_h * 2, num_q_heads, rows,
                                                               split_kv, st)
                                 : dk::launch_merge_t<dk::BF16>(head_dim, po, pm, pl, o, o_b * 2,
                                                                o_h * 2, num_q_heads, rows,
                                                                split_kv, st);
  if (e != hipSuccess) return dk::hip_fail(e, "merge launch");
  return DK_OK;
}

}  // extern "C"
