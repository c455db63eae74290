// dk_kernels.h — device code of the split-KV paged decode attention (gfx950, wave64).
//
// A wavefront owns one 16-token page of one kv head at a time. Lane (r, c) with
// r = lane/16, c = lane%16:
//   * V rows: tokens 4r..4r+3, dims c*D/16 .. +D/16-1 (each 16-lane row of the wave reads
//     whole rows: four 256-byte rows per 16-byte load instruction at D = 128).
//   * K rows, VALU q.k path: the same layout as V; each lane forms dot2 partial scores over
//     its dims for its 4 tokens and the G heads of the GQA group, and a reduce-scatter
//     over the row's 16 lanes leaves lane (r, c) with the scores of tokens 4r..4r+3 for
//     q head c mod 4.
//   * K rows, MFMA q.k path (groups above 4 heads): lane l holds token l%16 with 8 dims
//     per v_mfma_f32_16x16x32_{f16,bf16}, so S^T = K.Q^T lands in the same score layout.
//     K is loaded like V (whole rows per instruction) and moved into that layout through
//     a per-wavefront LDS tile (Wave::STAGE); loading the operand layout directly reads
//     64 bytes per row per instruction, which MI355X streams markedly slower.
//   Every K/V element is read once and serves all G heads of its kv head.
//   Online softmax is fp32 in the log2 domain (v_exp_f32); the reference max only moves
//   when a score exceeds it by more than 2^8, so accumulators are rescaled a handful of
//   times per split instead of every page. P.V runs on v_mfma_f32_16x16x16_{f16,bf16}
//   with p split into hi + lo parts of the element type (weights exact to 2^-22 / 2^-16)
//   and B taken from the V registers as loaded. The next pages' loads are in flight while
//   the current page is computed: in registers, or, for 16-bit caches at D = 256 on the
//   VALU q.k path, straight into a per-wavefront LDS ring (stream_lds).
//
// Pass 1, explicit split (dk_pass1_split): one workgroup per (sequence, kv head chunk,
//   split) over ceil(N/S)-page ranges as in the reference partition kernel
//   (src/cuda_/attention_ext.cu:207-349); NW wavefronts take the split's pages round-robin
//   and merge through LDS. With one split it writes the normalised output.
// Pass 1, balanced (dk_pass1_balanced): a persistent grid; the Wg workgroups of each head
//   chunk split the linear (sequence, page) space into Wg equal ranges, so every
//   workgroup streams the same number of pages, uniform or ragged. A workgroup writes the
//   output of a sequence its range covers alone and one partial per other sequence it
//   crosses (slot hc * (Wg + batch) + range + sequence: unique per head chunk). Over narrow
//   rows a workgroup serves HP neighbouring kv heads of the same range.
// Pass 2 (dk_merge_split / dk_merge_balanced): one wavefront per (sequence, q head)
//   merges its partials with the log-sum-exp identity (reference decode_attn_reduce_kernel,
//   src/cuda_/attention_ext.cu:363-406; contract src/layout.md:142-167).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "dk_args.h"   // shared constants (kXcds)

namespace dk {

// f(std::integral_constant<int, i>) for i = 0 .. N-1, each i a compile-time constant
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

using u32 = uint32_t;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

constexpr int kPage = 16;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kEmptyM = -1e9f;        // partial_m of an empty split (attention_ext.cu:254)
constexpr float kMinit = -1e30f;        // running reference before the first score
constexpr float kSlack = 8.0f;          // log2 headroom before the reference max moves
constexpr float kNegInf = -__builtin_inff();

// MFMA q.k with K staged through LDS (see Wave::STAGE); a build may turn it off with
// DK_STAGE_K=0 for comparisons.
#ifndef DK_STAGE_K
#define DK_STAGE_K 1
#endif
// 16-bit caches at D = 256 on the VALU q.k path: pages loaded straight into LDS
// (stream_lds); a build may turn it off with DK_LDS_PAGES=0 for comparisons.
#ifndef DK_LDS_PAGES
#define DK_LDS_PAGES 1
#endif

// ---------------------------------------------------------------- launch arguments
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
  int64_t kv_v;                       // bytes from a K page slice to the V slice of the
                                      // same page (in-page offset, or V cache - K cache)
  int32_t kv_s, kv_h;                 // bytes
  int32_t batch, hq, hkv, group, chunks, split;
  int32_t per;                        // q heads per chunk (the last chunk may have fewer)
  int32_t window;                     // > 0: attend to each sequence's last `window` tokens
                                      // (explicit-split kernel only)
  int32_t num_indices;
  uint32_t num_pages;                 // clamp bound for page ids (min(num_pages, 2^31))
  uint32_t page_extent;               // bytes one kv head's K (or V) rows of a page span (< 2^31)
  int32_t direct;                     // explicit split 1 / balanced: may write the
                                      // normalised output (0: partials only)
  int32_t ranges;                     // balanced: workgroups (page ranges) per head chunk
  float kscale;                       // log2(e) * softmax scale (* K dequant scale)
  float cap_in, cap_out;              // logit soft-cap: x = cap_out * tanh(q.k * cap_in)
                                      // (cap_out == 0: off, x = q.k * kscale)
  float vscale;                       // V dequant scale (1 unless the cache is fp8)
  int32_t seg_cost;                   // balanced, COST build: pages a change of sequence is
                                      // charged in the range split
  const float* sinks;                 // attention sinks: one fp32 logit per q head, or null
};

struct MergeArgs {
  const float* po;
  const float* pm;
  const float* pl;
  uint8_t* out;
  int64_t o_b, o_h;                   // bytes
  int32_t batch, hq, split;           // explicit split
  const int32_t* indptr;              // balanced: recompute each pair's slots
  int32_t num_indices, pairs_per_seq, heads, waves_per_pair;
  int32_t group, per, chunks, hkv;    // balanced: q head -> (head chunk, slot row)
  int32_t seg_cost;                   // balanced: pass 1's seg_cost (0: equal page ranges)
  const float* sinks;                 // attention sinks: one fp32 logit per q head, or null
};

// ---------------------------------------------------------------- element types
struct F16 {
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
  // two fp8 (E4M3) values, bytes 2*HI and 2*HI+1 of w, widened exactly to an f16 pair
  template <bool HI>
  static __device__ __forceinline__ u32 from_fp8(u32 w) {
    return __builtin_bit_cast(u32, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
  static __device__ __forceinline__ f32x4 mfma_pv(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ u32 pack2(float x0, float x1, float* r0, float* r1) {
    const f16x2 h = __builtin_convertvector(f32x2{x0, x1}, f16x2);
    *r0 = (float)h[0];
    *r1 = (float)h[1];
    return __builtin_bit_cast(u32, h);
  }
};

struct BF16 {
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot2(u32 a, u32 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
  template <bool HI>
  static __device__ __forceinline__ u32 from_fp8(u32 w) {
    return __builtin_bit_cast(u32, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  }
  // C += A.B with A 16x16 (rows: lane%16, k: 4 per lane), B 16x16 (k: 4 per lane, cols:
  // lane%16), 4 bf16 per lane in two words each
  static __device__ __forceinline__ f32x4 mfma_pv(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, a),
                                                     __builtin_bit_cast(bf16x4, b), c, 0, 0, 0);
  }
  // (bf16(x0), bf16(x1)) rounded to nearest, and the fp32 values they stand for
  static __device__ __forceinline__ u32 pack2(float x0, float x1, float* r0, float* r1) {
    const bf16x2 h = __builtin_convertvector(f32x2{x0, x1}, bf16x2);
    *r0 = (float)h[0];
    *r1 = (float)h[1];
    return __builtin_bit_cast(u32, h);
  }
  static __device__ __forceinline__ void store(uint8_t* p, float x) {
    *reinterpret_cast<__bf16*>(p) = (__bf16)x;
  }
};

// ---------------------------------------------------------------- cross-lane helpers
template <int CTRL>
__device__ __forceinline__ u32 dpp_u(u32 x) {
  // bound_ctrl: every pattern used here reads an existing lane, so no "old" value is
  // needed (and no zeroing move is emitted for it).
  return (u32)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xf, 0xf, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, dpp_u<CTRL>(__builtin_bit_cast(u32, x)));
}
// Value of lane 4*(l/4) + Q: DPP quad_perm [Q,Q,Q,Q].
template <int Q>
__device__ __forceinline__ float quad_bcast(float x) { return dpp<Q * 0x55>(x); }
template <int Q>
__device__ __forceinline__ u32 quad_bcast_u(u32 x) { return dpp_u<Q * 0x55>(x); }
// Runtime-indexed (but compile-time unrolled) quad broadcast.
__device__ __forceinline__ float quad_bcast_i(float x, int q) {
  return q == 0 ? quad_bcast<0>(x) : q == 1 ? quad_bcast<1>(x) : q == 2 ? quad_bcast<2>(x)
                                                                        : quad_bcast<3>(x);
}
template <int N>
__device__ __forceinline__ float row_ror(float x) { return dpp<0x120 + N>(x); }
__device__ __forceinline__ float xor1(float x) { return dpp<0xB1>(x); }   // quad_perm [1,0,3,2]
__device__ __forceinline__ float xor2(float x) { return dpp<0x4E>(x); }   // quad_perm [2,3,0,1]

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
// Max over all lanes whose column c = l%16 agrees modulo GQ (the lanes holding one q head
// of a head set), result in all of them.
template <int GQ>
__device__ __forceinline__ float allmax_head(float x) {
  if constexpr (GQ == 16) return max_xor32(max_xor16(x));   // head = lane column
  if constexpr (GQ == 1) {
    x = fmaxf(x, xor1(x));
    x = fmaxf(x, xor2(x));
  } else if constexpr (GQ == 2) {
    x = fmaxf(x, xor2(x));
  }
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<8>(x));
  return max_xor32(max_xor16(x));
}
__device__ __forceinline__ float row_sum(float x) {
  x += xor1(x);
  x += xor2(x);
  x += row_ror<4>(x);
  x += row_ror<8>(x);
  return x;
}
__device__ __forceinline__ float wave_sum(float x) { return sum_xor32(sum_xor16(row_sum(x))); }
__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, xor1(x));
  x = fmaxf(x, xor2(x));
  x = fmaxf(x, row_ror<4>(x));
  x = fmaxf(x, row_ror<8>(x));
  return max_xor32(max_xor16(x));
}
__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// ---------------------------------------------------------------- memory helpers
// Page tables are read through the constant address space: the kernels never write
// them, and this lets every uniform read stay a scalar load even after stores.
template <class X>
__device__ __forceinline__ X ld_const(const X* p, int64_t i) {
  return ((const __attribute__((address_space(4))) X*)p)[i];
}

// Buffer resource of one page slice: base address, no stride, `extent` bytes in range
// (out-of-range lanes read 0). gfx9-family descriptor word 3.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const uint8_t* base, u32 extent) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)extent, 0x00020000);
}
// Buffer-load cache policy of the K/V pages: non-temporal (nt, bit 1; streamed once). A
// build may set another policy word with DK_LOAD_POLICY (bit 0 sc0, bit 4 sc1) for
// comparisons.
#ifndef DK_LOAD_POLICY
#define DK_LOAD_POLICY 2
#endif
constexpr int kBufNT = DK_LOAD_POLICY;

// NWORDS consecutive words at base + voff + soff (NWORDS in {2, 4, 8}), streaming.
template <int NWORDS>
__device__ __forceinline__ void ld_buf(u32* dst, __amdgpu_buffer_rsrc_t r, u32 voff, u32 soff) {
  if constexpr (NWORDS == 1) {
    dst[0] = (u32)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, kBufNT);
  } else if constexpr (NWORDS == 2) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, kBufNT));
    dst[0] = v[0];
    dst[1] = v[1];
  } else {
#pragma unroll
    for (int k = 0; k < NWORDS / 4; ++k) {
      const u32x4 v = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(voff + 16 * k), (int)soff, kBufNT));
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
template <int N>
__device__ __forceinline__ void st_floats(float* p, const float* v) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int k = 0; k < N / 4; ++k)
      reinterpret_cast<f32x4*>(p)[k] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
  } else {
#pragma unroll
    for (int k = 0; k < N; ++k) p[k] = v[k];
  }
}

// Clamped CSR range of sequence b (so that no access leaves kv_indices).
__device__ __forceinline__ int seq_begin(const Pass1Args& a, int b) {
  return min(max(ld_const(a.indptr, b), 0), a.num_indices);
}

// tanh(y) = 1 - 2 / (e^(2y) + 1): saturates to +-1 for large |y| (e^(2y) overflowing to
// infinity or underflowing to 0); absolute error a few float ulps
__device__ __forceinline__ float tanh_approx(float y) {
  const float e = __builtin_amdgcn_exp2f(y * (2.f * kLog2e));
  return 1.f - 2.f * __builtin_amdgcn_rcpf(e + 1.f);
}

// ---------------------------------------------------------------- per-wavefront decoder
// T: element type of q and out (and of the cache unless KV8); KV8: the cache holds fp8
// (E4M3) values, widened to T in registers after the loads.
template <class T, int D, int G, bool MFMA, bool KV8 = false>
struct Wave {
  // WIDE (q.k on MFMA with 8 or 16 heads): the MFMA's 16 columns are 16 distinct q heads,
  // so lane (r16, c) holds the scores of head c and the P.V accumulators of heads
  // 4*r16 .. 4*r16+3; registers do not grow with G. Otherwise every lane row holds all
  // G heads (columns repeat the GQ heads of a set).
  static constexpr bool WIDE = MFMA && G >= 8;
  static constexpr int GQ = WIDE ? 16 : (G < 4 ? G : 4);   // heads per column set
  static constexpr int NS = WIDE ? 1 : G / GQ;             // column sets (G = 8 -> 2)
  static constexpr int AH = WIDE ? 4 : G;                  // heads held in acc
  static constexpr int HEADS = G;                          // q heads per wavefront
  static constexpr bool MF = MFMA;                         // q.k on the matrix cores
  static constexpr int DPL = D / 16;         // V (and VALU-path K) dims per lane
  static constexpr int VWT = DPL / 2;        // words per token per lane
  static constexpr int KW = D / 8;           // K words per lane per page (both paths)
  static constexpr int VW = 4 * VWT;         // V words per lane per page
  static constexpr int NMF = D / 32;         // MFMAs per head set per page
  static constexpr int KB = KV8 ? D / 16 : KW;   // words of a page buffer as loaded (K)
  static constexpr int VB = KV8 ? D / 16 : VW;   // (V)
  static constexpr int EB = KV8 ? 1 : 2;         // bytes per cache element
  // MFMA q.k: 16-byte K loads per lane, token c, bytes 16*r16 + 64*i of the row; an fp8
  // load holds the dims of two MFMAs (D/64 loads), a 16-bit load those of one (D/32)
  static constexpr int NKL = KV8 ? D / 64 : NMF;
  // STAGE (MFMA q.k): K is loaded like V -- lane (r16, c) takes bytes c*RB/16 .. of tokens
  // 4*r16 .. 4*r16+3, so every load instruction reads whole rows -- then written to this
  // wavefront's LDS tile and read back in the MFMA layout above (token c, 16-byte chunk
  // 4*i + r16). Loading the MFMA layout directly reads 64-byte row segments per
  // instruction, which HBM serves markedly slower. Chunk k of token t sits at chunk
  // position k ^ (t & SWZ) of LDS row t, so neither the writes (one token per 16 lanes)
  // nor the reads (16 tokens per 16 lanes) put two lanes of a 16-lane group on one bank.
  // Not for fp8 at D = 256, whose wavefronts already need all 256 registers and measured
  // slower staged.
  static constexpr bool STAGE = MFMA && (DK_STAGE_K != 0) && !(KV8 && D >= 256);
  static constexpr int RB = D * EB;                       // bytes per K row
  static constexpr int NCH = RB / 16;                     // 16-byte chunks per row
  static constexpr int SWZ = (NCH < 16 ? NCH : 16) - 1;
  static constexpr int STAGE_BYTES = STAGE ? kPage * RB : 0;
  // LDS pages (stream_lds): a page slot holds the K rows then the V rows of one kv head,
  // row-major, as the 1 KB buffer-load-to-LDS instructions write them
  static constexpr int LDS_PAGE = 2 * kPage * RB;
  static constexpr int LDS_LOADS = kPage * RB / 1024;   // instructions per K (or V) slice

  int r16, c;
  uint8_t* kst;           // STAGE: this wavefront's K tile in LDS (STAGE_BYTES)
  int hv;                 // valid q heads of this chunk (<= G); heads hv.. are masked
  u32 koff, voff, tok_s, extent;
  int64_t kv_v;
  float kscale, vscale, cap_in, cap_out;
  u32 qw[MFMA ? NS : 1][MFMA ? KW : 1];      // MFMA: Q^T column s*GQ + c%GQ, the dims of
                                             // the K operand of MFMA i (see q_dim0)
  u32 qv[MFMA ? 1 : G][MFMA ? 1 : VWT];      // VALU: head h, dims c*DPL..
  float acc[AH][DPL];     // after reduce_rows: head h (WIDE: head 4*r16 + h), dim c*DPL + j
  f32x4 cv[NS][DPL];      // while pages stream: the P.V accumulators as MFMA C vectors,
                          // element g = head ss*GQ + g of dim c*DPL + j
  float mref[NS], mtrue[NS], lsum[NS];

  __device__ __forceinline__ void init(const Pass1Args& a) {
    const int lane = threadIdx.x & 63;
    r16 = lane >> 4;
    c = lane & 15;
    tok_s = (u32)a.kv_s;
    koff = MFMA && !STAGE ? (u32)(c * a.kv_s + 16 * r16) : (u32)(4 * r16 * a.kv_s + EB * DPL * c);
    voff = (u32)(4 * r16 * a.kv_s + EB * DPL * c);
    extent = a.page_extent;
    kv_v = a.kv_v;
    kscale = a.kscale;
    cap_in = a.cap_in;
    cap_out = a.cap_out;
    vscale = a.vscale;
  }

  // MFMA q.k: first of the 8 dims lane row r16 supplies to MFMA i (k = 8*r16..8*r16+7).
  // 16-bit cache: load i holds dims 32i + 8r16 .. +7. fp8 cache: load j = i/2 holds dims
  // 64j + 16r16 .. +15, widened in order, so MFMA 2j takes the first 8 and 2j+1 the rest.
  __device__ __forceinline__ int q_dim0(int i) const {
    return KV8 ? 64 * (i >> 1) + 16 * r16 + 8 * (i & 1) : 32 * i + 8 * r16;
  }

  // q rows of the chunk's valid heads starting at qbase (q_h bytes apart); the rows of
  // masked heads (h >= hv) are zero and never read.
  __device__ __forceinline__ void load_q(const uint8_t* qbase, int64_t q_h) {
    if constexpr (MFMA) {
#pragma unroll
      for (int ss = 0; ss < NS; ++ss) {
        const int h = ss * GQ + c % GQ;
        const uint8_t* qp = qbase + (int64_t)h * q_h;
#pragma unroll
        for (int i = 0; i < KW; ++i) qw[ss][i] = 0u;
        if (h < hv) {
#pragma unroll
          for (int i = 0; i < NMF; ++i) ld_words_cached<4>(&qw[ss][4 * i], qp + 2 * q_dim0(i));
        }
      }
    } else {
#pragma unroll
      for (int h = 0; h < G; ++h) {
#pragma unroll
        for (int q = 0; q < VWT; ++q) qv[h][q] = 0u;
        if (h < hv) ld_words_cached<VWT>(qv[h], qbase + (int64_t)h * q_h + 2 * DPL * c);
      }
    }
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int ss = 0; ss < NS; ++ss)
#pragma unroll
      for (int j = 0; j < DPL; ++j) cv[ss][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ss = 0; ss < NS; ++ss) {
      mref[ss] = kMinit;
      mtrue[ss] = kNegInf;
      lsum[ss] = 0.f;
    }
  }

  // pg: base of this kv head's slice of a page (page base + kvh * kv_h). Buffer loads:
  // the address is the page base (scalar) + a per-lane offset + a per-row scalar offset.
  // live == false: a zero-extent descriptor, the loads return zeros without touching memory
  __device__ __forceinline__ void load_page(u32 (&kb)[KB], u32 (&vb)[VB], const uint8_t* pg,
                                            bool live = true) const {
    const u32 ext = live ? extent : 0u;
    const __amdgpu_buffer_rsrc_t rk = page_rsrc(pg, ext);
    const __amdgpu_buffer_rsrc_t rv = page_rsrc(pg + kv_v, ext);
    constexpr int TW = KB / 4;   // words per token per lane as loaded
    if constexpr (MFMA && !STAGE) {
#pragma unroll
      for (int i = 0; i < NKL; ++i) ld_buf<4>(&kb[4 * i], rk, koff, 64 * i);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) ld_buf<TW>(&kb[r * TW], rk, koff, r * tok_s);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) ld_buf<TW>(&vb[r * TW], rv, voff, r * tok_s);
  }

  // K and V rows of a page straight into the LDS slot: instruction i writes bytes
  // i*1024.. of the slot's K (V) part, lane L bytes 16L..16L+15, i.e. token
  // i*TPI + L/(64/TPI), 16-byte chunk L%(64/TPI) of its row. Every lane loads 16 bytes and
  // every instruction reads whole rows: 8 rows of 128 bytes (16-bit D = 64, fp8 D = 128),
  // 16 of 64 bytes (fp8 D = 64), 4 of 256 or 2 of 512.
  // live == false: a zero-extent descriptor (no memory access; the slot gets zeros).
  __device__ __forceinline__ void lds_load_page(uint8_t* slot, const uint8_t* pg,
                                                bool live = true) const {
    static_assert(RB >= 64 && RB <= 1024 && 1024 % RB == 0, "rows of 64 to 1024 bytes");
    constexpr int TPI = 1024 / RB, LPR = 64 / TPI;   // tokens per instruction, lanes per row
    const u32 ext = live ? extent : 0u;
    const __amdgpu_buffer_rsrc_t rk = page_rsrc(pg, ext);
    const __amdgpu_buffer_rsrc_t rv = page_rsrc(pg + kv_v, ext);
    const int lane = threadIdx.x & 63;
    const u32 voff = (u32)(lane / LPR) * tok_s + (u32)(lane % LPR) * 16u;
#pragma unroll
    for (int i = 0; i < LDS_LOADS; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void*)(slot + i * 1024), 16, (int)voff,
          (int)(i * TPI * tok_s), 0, kBufNT);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void*)(slot + LDS_PAGE / 2 + i * 1024), 16,
          (int)voff, (int)(i * TPI * tok_s), 0, kBufNT);
    }
  }

  // A page of the LDS slot into the VALU layout's registers (tokens 4*r16 .. 4*r16+3,
  // bytes c*RB/16 .. of each row) and the lgkmcnt wait, in one asm block (outputs
  // early-clobber, so none shares a register with the address). Written in asm because a
  // compiler-visible LDS read after the LDS-bound buffer loads makes hipcc wait for all of
  // them (vmcnt(0)), which would serialise the ring; the waits for those loads are
  // stream_lds's. Rows of RB bytes give each lane RB/16 bytes per token: 4 (ds_read_b32),
  // 8 (b64), 16 (b128) or 32 (two b128).
  __device__ __forceinline__ void lds_read_page(const uint8_t* slot, u32 (&kb)[KB],
                                                u32 (&vb)[VB]) const {
    static_assert(KB == VB && KB == RB / 16 && LDS_PAGE == 32 * RB,
                  "a page slot of K rows then V rows, RB / 16 bytes per lane and token");
    const u32 base = (u32)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)(
        slot + 4 * r16 * RB + c * (RB / 16));
    if constexpr (RB == 512) {
      lds_read_512(base, kb, vb);
    } else if constexpr (RB == 256) {
      u32x4 k[4], v[4];
      asm volatile(
          "ds_read_b128 %0, %8 offset:0\n\t"
          "ds_read_b128 %1, %8 offset:256\n\t"
          "ds_read_b128 %2, %8 offset:512\n\t"
          "ds_read_b128 %3, %8 offset:768\n\t"
          "ds_read_b128 %4, %8 offset:4096\n\t"
          "ds_read_b128 %5, %8 offset:4352\n\t"
          "ds_read_b128 %6, %8 offset:4608\n\t"
          "ds_read_b128 %7, %8 offset:4864\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(v[0]), "=&v"(v[1]),
            "=&v"(v[2]), "=&v"(v[3])
          : "v"(base)
          : "memory");
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kb[4 * i + e] = k[i][e];
          vb[4 * i + e] = v[i][e];
        }
    } else if constexpr (RB == 128) {
      u32x2 k[4], v[4];
      asm volatile(
          "ds_read_b64 %0, %8 offset:0\n\t"
          "ds_read_b64 %1, %8 offset:128\n\t"
          "ds_read_b64 %2, %8 offset:256\n\t"
          "ds_read_b64 %3, %8 offset:384\n\t"
          "ds_read_b64 %4, %8 offset:2048\n\t"
          "ds_read_b64 %5, %8 offset:2176\n\t"
          "ds_read_b64 %6, %8 offset:2304\n\t"
          "ds_read_b64 %7, %8 offset:2432\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(v[0]), "=&v"(v[1]),
            "=&v"(v[2]), "=&v"(v[3])
          : "v"(base)
          : "memory");
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          kb[2 * i + e] = k[i][e];
          vb[2 * i + e] = v[i][e];
        }
    } else {
      static_assert(RB == 64, "rows of 64, 128, 256 or 512 bytes");
      u32 k[4], v[4];
      asm volatile(
          "ds_read_b32 %0, %8 offset:0\n\t"
          "ds_read_b32 %1, %8 offset:64\n\t"
          "ds_read_b32 %2, %8 offset:128\n\t"
          "ds_read_b32 %3, %8 offset:192\n\t"
          "ds_read_b32 %4, %8 offset:1024\n\t"
          "ds_read_b32 %5, %8 offset:1088\n\t"
          "ds_read_b32 %6, %8 offset:1152\n\t"
          "ds_read_b32 %7, %8 offset:1216\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(v[0]), "=&v"(v[1]),
            "=&v"(v[2]), "=&v"(v[3])
          : "v"(base)
          : "memory");
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kb[i] = k[i];
        vb[i] = v[i];
      }
    }
  }

  // lds_read_page for 512-byte rows (16-bit caches at D = 256): 16 ds_read_b128
  __device__ __forceinline__ void lds_read_512(u32 base, u32 (&kb)[KB], u32 (&vb)[VB]) const {
    u32x4 k[8], v[8];
    asm volatile(
        "ds_read_b128 %0, %16 offset:0\n\t"
        "ds_read_b128 %1, %16 offset:16\n\t"
        "ds_read_b128 %2, %16 offset:512\n\t"
        "ds_read_b128 %3, %16 offset:528\n\t"
        "ds_read_b128 %4, %16 offset:1024\n\t"
        "ds_read_b128 %5, %16 offset:1040\n\t"
        "ds_read_b128 %6, %16 offset:1536\n\t"
        "ds_read_b128 %7, %16 offset:1552\n\t"
        "ds_read_b128 %8, %16 offset:8192\n\t"
        "ds_read_b128 %9, %16 offset:8208\n\t"
        "ds_read_b128 %10, %16 offset:8704\n\t"
        "ds_read_b128 %11, %16 offset:8720\n\t"
        "ds_read_b128 %12, %16 offset:9216\n\t"
        "ds_read_b128 %13, %16 offset:9232\n\t"
        "ds_read_b128 %14, %16 offset:9728\n\t"
        "ds_read_b128 %15, %16 offset:9744\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(k[4]), "=&v"(k[5]),
          "=&v"(k[6]), "=&v"(k[7]), "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]),
          "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
        : "v"(base)
        : "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kb[4 * i + e] = k[i][e];
        vb[4 * i + e] = v[i][e];
      }
  }

  // STAGE: the K words of a page as loaded (row layout) -> the MFMA layout, through LDS
  __device__ __forceinline__ void stage_k(const u32 (&kb)[KB], u32 (&km)[KB]) const {
    constexpr int TB = RB / 16;   // bytes per token per lane as loaded (4, 8, 16 or 32)
    constexpr int TW = TB / 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * r16 + r;
      uint8_t* row = kst + t * RB;
      if constexpr (TB >= 16) {
#pragma unroll
        for (int h = 0; h < TB / 16; ++h) {
          const int k = c * (TB / 16) + h;
          *reinterpret_cast<u32x4*>(row + ((k ^ (t & SWZ)) << 4)) =
              u32x4{kb[r * TW + 4 * h], kb[r * TW + 4 * h + 1], kb[r * TW + 4 * h + 2],
                    kb[r * TW + 4 * h + 3]};
        }
      } else {
        const int k = (c * TB) >> 4, o = (c * TB) & 15;
        uint8_t* dst = row + ((k ^ (t & SWZ)) << 4) + o;
        if constexpr (TB == 8)
          *reinterpret_cast<u32x2*>(dst) = u32x2{kb[2 * r], kb[2 * r + 1]};
        else
          *reinterpret_cast<u32*>(dst) = kb[r];
      }
    }
    const uint8_t* row = kst + c * RB;
#pragma unroll
    for (int i = 0; i < NCH / 4; ++i) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(row + (((4 * i + r16) ^ (c & SWZ)) << 4));
#pragma unroll
      for (int e = 0; e < 4; ++e) km[4 * i + e] = v[e];
    }
  }

  // One loaded page: K staged into the MFMA layout (STAGE); fp8 buffers are widened to T
  // pairs (word u of a token's fp8 dims 4u..4u+3 becomes words 2u, 2u+1); then compute_page.
  template <bool CAP>
  __device__ __forceinline__ void consume(const u32 (&kb)[KB], u32 (&vb)[VB], int valid) {
    if constexpr (STAGE) {
      u32 km[KB];
      stage_k(kb, km);
      consume_loaded<CAP>(km, vb, valid);
    } else {
      consume_loaded<CAP>(kb, vb, valid);
    }
  }

  template <bool CAP>
  __device__ __forceinline__ void consume_loaded(const u32 (&kb)[KB], u32 (&vb)[VB], int valid) {
    if constexpr (KV8) {
      u32 kw[KW], vw[VW];
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        kw[2 * i] = T::template from_fp8<false>(kb[i]);
        kw[2 * i + 1] = T::template from_fp8<true>(kb[i]);
        vw[2 * i] = T::template from_fp8<false>(vb[i]);
        vw[2 * i + 1] = T::template from_fp8<true>(vb[i]);
      }
      compute_page<CAP>(kw, vw, valid);
    } else {
      compute_page<CAP>(kb, vb, valid);
    }
  }

  // Scores of tokens 4*r16 + r for head ss*GQ + c%GQ from per-lane partials of the G
  // heads over this lane's dims: reduce-scatter over the low column bits (the head),
  // all-reduce over the rest.
  __device__ __forceinline__ float scatter_scores(const float (&part)[GQ], int r) const {
    (void)r;
    if constexpr (GQ == 4) {
      const bool b0 = c & 1, b1 = c & 2;
      const float k0 = b0 ? part[1] : part[0], s0 = b0 ? part[0] : part[1];
      const float k1 = b0 ? part[3] : part[2], s1 = b0 ? part[2] : part[3];
      const float w0 = k0 + xor1(s0), w1 = k1 + xor1(s1);   // heads {b0, 2+b0}
      float x = (b1 ? w1 : w0) + xor2(b1 ? w0 : w1);        // head 2*b1 + b0
      x += row_ror<4>(x);
      x += row_ror<8>(x);
      return x;
    } else if constexpr (GQ == 2) {
      const bool b0 = c & 1;
      float x = (b0 ? part[1] : part[0]) + xor1(b0 ? part[0] : part[1]);
      x += xor2(x);
      x += row_ror<4>(x);
      x += row_ror<8>(x);
      return x;
    } else {
      return row_sum(part[0]);
    }
  }

  // One page: scores, online softmax, P.V. valid = hi | lo << 8 masks the tokens outside
  // [lo, hi) (a full page: valid == 16).
  // CAP: logit soft-capping on (a separate instantiation, so uncapped calls carry no
  // trace of it)
  template <bool CAP>
  __device__ __forceinline__ void compute_page(const u32 (&kb)[KW], u32 (&vb)[VW], int valid) {
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
#pragma unroll
        for (int ss = 0; ss < NS; ++ss) {
          float part[GQ];
#pragma unroll
          for (int g = 0; g < GQ; ++g) {
            float x = 0.f;
#pragma unroll
            for (int q = 0; q < VWT; ++q) x = T::dot2(kb[r * VWT + q], qv[ss * GQ + g][q], x);
            part[g] = x;
          }
          sc[ss][r] = scatter_scores(part, r);
        }
      }
    }
    // `valid` = hi | lo << 8: tokens [lo, hi) of the page are attended. Others (the tail
    // of a sequence's last page, or before a sliding window's first token) are masked by
    // selection (never by multiplying), so stale or NaN bytes cannot reach the output
    if (valid != kPage) {
      const int hi = valid & 0xff, lo = valid >> 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool dead = 4 * r16 + r >= hi || 4 * r16 + r < lo;
#pragma unroll
        for (int ss = 0; ss < NS; ++ss) sc[ss][r] = dead ? kNegInf : sc[ss][r];
#pragma unroll
        for (int q = 0; q < VWT; ++q) vb[r * VWT + q] = dead ? 0u : vb[r * VWT + q];
      }
    }
    // online softmax (log2 domain)
    float x[NS][4], mx[NS];
#pragma unroll
    for (int ss = 0; ss < NS; ++ss)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[ss][r] = sc[ss][r] * kscale;
    if constexpr (CAP) {
      // soft-capped scores (masked tokens stay -inf)
#pragma unroll
      for (int ss = 0; ss < NS; ++ss)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          x[ss][r] = sc[ss][r] > kNegInf ? cap_out * tanh_approx(sc[ss][r] * cap_in) : kNegInf;
    }
    bool need = false;
#pragma unroll
    for (int ss = 0; ss < NS; ++ss) {
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
        f32x4 ab4 = {0.f, 0.f, 0.f, 0.f};
        if constexpr (WIDE) {
#pragma unroll
          for (int i = 0; i < 4; ++i) ab4[i] = col_value(al, i);
        } else {
#pragma unroll
          for (int g = 0; g < GQ; ++g) ab4[g] = GQ > 1 ? quad_bcast_i(al, g) : al;
        }
#pragma unroll
        for (int j = 0; j < DPL; ++j) cv[ss][j] *= ab4;
        mref[ss] = mn;
      }
    }
    float p[NS][4];
#pragma unroll
    for (int ss = 0; ss < NS; ++ss)
#pragma unroll
      for (int r = 0; r < 4; ++r) p[ss][r] = __builtin_amdgcn_exp2f(x[ss][r] - mref[ss]);

    {
      // P.V on MFMA (v_mfma_f32_16x16x16_{f16,bf16}): C[head][dim] += P[head][token]
      // V[token][dim] over the page's 16 tokens. The lane holding the scores of tokens
      // 4r..4r+3 for head c mod GQ is exactly A's row c, k = 4r..4r+3; B (V) is the
      // lane's own 4 tokens of one dim, paired by v_perm. p enters as hi + lo (p - hi) in
      // the element type, so the weights keep 22 (fp16) / 16 (bf16) significant bits;
      // l sums the fp32 p. C row i of every lane row is head i: no reduction across
      // lane rows is needed afterwards.
      u32x2 ah[NS], al[NS];
#pragma unroll
      for (int ss = 0; ss < NS; ++ss) {
        lsum[ss] += (p[ss][0] + p[ss][1]) + (p[ss][2] + p[ss][3]);
        float h0, h1, h2, h3, e;
        const u32 w01 = T::pack2(p[ss][0], p[ss][1], &h0, &h1);
        const u32 w23 = T::pack2(p[ss][2], p[ss][3], &h2, &h3);
        ah[ss] = u32x2{w01, w23};
        al[ss] = u32x2{T::pack2(p[ss][0] - h0, p[ss][1] - h1, &e, &e),
                       T::pack2(p[ss][2] - h2, p[ss][3] - h3, &e, &e)};
      }
#pragma unroll
      for (int q = 0; q < VWT; ++q) {
        const u32 v0 = vb[q], v1 = vb[VWT + q], v2 = vb[2 * VWT + q], v3 = vb[3 * VWT + q];
        const u32x2 blo = {__builtin_amdgcn_perm(v1, v0, 0x05040100u),
                           __builtin_amdgcn_perm(v3, v2, 0x05040100u)};
        const u32x2 bhi = {__builtin_amdgcn_perm(v1, v0, 0x07060302u),
                           __builtin_amdgcn_perm(v3, v2, 0x07060302u)};
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int j = 2 * q + half;
          const u32x2 b = half ? bhi : blo;
#pragma unroll
          for (int ss = 0; ss < NS; ++ss) {
            cv[ss][j] = T::mfma_pv(ah[ss], b, cv[ss][j]);
            cv[ss][j] = T::mfma_pv(al[ss], b, cv[ss][j]);
          }
        }
      }
    }
  }

  // Sum lsum over the four lane rows, exact max over the lanes of each head, and unpack
  // the P.V accumulators into acc.
  __device__ __forceinline__ void reduce_rows() {
#pragma unroll
    for (int ss = 0; ss < NS; ++ss) {
      lsum[ss] = sum_xor32(sum_xor16(lsum[ss]));
      mtrue[ss] = allmax_head<GQ>(mtrue[ss]);
    }
    // the MFMA P.V already summed over all tokens of every lane row
    if constexpr (WIDE) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[i][j] = cv[0][j][i] * vscale;
    } else {
#pragma unroll
      for (int ss = 0; ss < NS; ++ss)
#pragma unroll
        for (int g = 0; g < GQ; ++g)
#pragma unroll
          for (int j = 0; j < DPL; ++j) acc[ss * GQ + g][j] = cv[ss][j][g] * vscale;
    }
  }

  // WIDE: a per-head value x that lives in lane column h (lsum, mref, mtrue of head h),
  // fetched for this lane row's head 4*r16 + i (all lanes must take part)
  __device__ __forceinline__ float col_value(float x, int i) const {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                         (16 * r16 + 4 * r16 + i) << 2, __builtin_bit_cast(int, x)));
  }

  // After reduce_rows every lane holds every head's sums. Lane row r16 stores heads
  // 4k + r16 (k < ceil(G/4)); the value of that head is picked with selects on r16, never
  // by indexing acc with a lane-dependent value (which would move acc to scratch memory).
  static constexpr int KR = (G + 3) / 4;   // heads stored per lane row

  // acc[4K + r16][j]. K is a template argument and each candidate passes through an
  // empty asm, so that the compiler cannot fold the selects into one load from a
  // lane-dependent (or loop-dependent) address of acc.
  template <int K>
  __device__ __forceinline__ float row_head(int j) const {
    float v = acc[4 * K][j];
    __asm__("" : "+v"(v));
#pragma unroll
    for (int t = 1; t < 4; ++t)
      if (4 * K + t < G) {
        float o = acc[4 * K + t][j];
        __asm__("" : "+v"(o));
        v = r16 == t ? o : v;
      }
    return v;
  }

  // per-head-set value x[ss] of head 4K + r16 (head h sits in set h / GQ at quad lane
  // h % GQ), selected the same way
  template <int K>
  __device__ __forceinline__ float row_head_scalar(const float (&x)[NS]) const {
    float v = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int h = 4 * K + t;
      if (h < G) {
        float xt = GQ > 1 ? quad_bcast_i(x[h / GQ], h % GQ) : x[h / GQ];
        __asm__("" : "+v"(xt));
        v = r16 == t ? xt : v;
      }
    }
    return v;
  }

  // After reduce_rows: rescale to the exact maximum and store the partial of the G
  // heads, head h at row row0 + h * hstride of part_o (D floats) / part_m / part_l
  // (reference semantics: m = max score in natural units or -1e9 if nothing was seen,
  // l = sum exp(s - m), O = sum exp(s - m) V).
  __device__ __forceinline__ void store_partial(const Pass1Args& a, int64_t row0, int64_t hstride) {
    float f[NS];
#pragma unroll
    for (int ss = 0; ss < NS; ++ss)
      f[ss] = mtrue[ss] > kNegInf ? __builtin_amdgcn_exp2f(mref[ss] - mtrue[ss]) : 0.f;
    if constexpr (WIDE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * r16 + i;
        const float fh = col_value(f[0], i);
        if (h < hv) {
          float v[DPL];
#pragma unroll
          for (int j = 0; j < DPL; ++j) v[j] = acc[i][j] * fh;
          st_floats<DPL>(a.part_o + (row0 + h * hstride) * D + c * DPL, v);
        }
      }
      if (r16 == 0 && c < hv) {
        const int64_t r = row0 + (int64_t)c * hstride;
        const bool seen = mtrue[0] > kNegInf;
        a.part_m[r] = seen ? mtrue[0] * kLn2 : kEmptyM;
        a.part_l[r] = lsum[0] * f[0];
      }
    } else {
      static_for<KR>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int h = 4 * k + r16;
        const float fh = row_head_scalar<k>(f);
        if (h < hv) {
          float v[DPL];
#pragma unroll
          for (int j = 0; j < DPL; ++j) v[j] = row_head<k>(j) * fh;
          st_floats<DPL>(a.part_o + (row0 + h * hstride) * D + c * DPL, v);
        }
      });
      if (r16 == 0 && c < GQ) {
#pragma unroll
        for (int ss = 0; ss < NS; ++ss) {
          if (ss * GQ + c >= hv) continue;
          const int64_t r = row0 + (int64_t)(ss * GQ + c) * hstride;
          const bool seen = mtrue[ss] > kNegInf;
          a.part_m[r] = seen ? mtrue[ss] * kLn2 : kEmptyM;
          a.part_l[r] = lsum[ss] * f[ss];
        }
      }
    }
  }

  // After reduce_rows: normalised output of the G heads (q head h at out + h * o_h). With
  // attention sinks (sink: the group's first q head's logit, else null) the denominator
  // of head h has one more term, e^{sink[h]}: 2^(sink[h] log2(e) - mref) relative to the
  // head's reference max (+inf, hence a zero output, when the head saw no token).
  __device__ __forceinline__ void store_output(uint8_t* out, int64_t o_h,
                                               const float* sink = nullptr) {
    if constexpr (WIDE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * r16 + i;
        float L = col_value(lsum[0], i);
        if (sink) {
          const float mr = col_value(mref[0], i);
          if (h < hv) L += __builtin_amdgcn_exp2f(sink[h] * kLog2e - mr);
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        if (h < hv) {
#pragma unroll
          for (int j = 0; j < DPL; ++j)
            T::store(out + (int64_t)h * o_h + 2 * (c * DPL + j), acc[i][j] * inv);
        }
      }
    } else {
      static_for<KR>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int h = 4 * k + r16;
        float L = row_head_scalar<k>(lsum);
        if (sink) {
          const float mr = row_head_scalar<k>(mref);
          if (h < hv) L += __builtin_amdgcn_exp2f(sink[h] * kLog2e - mr);
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        if (h < hv) {
#pragma unroll
          for (int j = 0; j < DPL; ++j)
            T::store(out + (int64_t)h * o_h + 2 * (c * DPL + j), row_head<k>(j) * inv);
        }
      });
    }
  }
};

// Pages kept in flight ahead of the one being computed (prefetch_depth below); a build may
// set another depth for 16-bit caches (DK_PREFETCH_DEPTH) or fp8 ones (DK_PREFETCH_DEPTH_KV8).
#ifndef DK_PREFETCH_DEPTH
#define DK_PREFETCH_DEPTH 0
#endif
#ifndef DK_PREFETCH_DEPTH_KV8
#define DK_PREFETCH_DEPTH_KV8 0
#endif
// Pages in flight per wavefront. An fp8 page is half the bytes of a 16-bit one, so the
// fp8 path keeps twice the pages in flight for the same bytes (and the same registers).
// (A 16-bit cache at D = 64 measured no faster with 4 pages than with 2.) BAL: the
// balanced kernel; there an fp8 cache with at most 4 q heads per kv head keeps 2 pages in
// flight, like a 16-bit one, and loads its first page before the sequence search (fp8
// 32/8/128, ctx 8192 unless noted, us, 4 -> 2 pages; kv heads grouped per workgroup: B=16
// 54.6 -> 51.3, B=4 ctx 32768 54.6 -> 51.1, B=256 ctx 1024 103.3 -> 96.4, B=128 ctx 2048
// 92.7 -> 90.5, B=64 171.2 -> 168.3, ragged B=128 199.6-200.4 -> 193.4-199.0; one kv head
// per workgroup: B=4 24.4 -> 22.8, B=1 ctx 32768 24.3 -> 22.8, B=1 ctx 4096 14.0 -> 12.3,
// D=64 B=2 ctx 16384 21.9 -> 20.7;
// 8 q heads on the VALU path spill with it). The one-pass / explicit-split kernel keeps 4
// on the VALU q.k path (metric shape 92.2 vs 93.0 with 2). MF: q.k on the matrix cores
// (more than 4 q heads per kv head), where an fp8 cache keeps 2 pages in flight in either
// kernel (32/8/128 B=32 ctx 8192 but for the heads, us, 4 -> 2 pages: 64/8 one pass 92.2
// -> 91.5, balanced 92.1 -> 90.7-90.8; 128/8 one pass 93.1-93.3 -> 92.3-92.5, balanced
// 95.1 -> 93.5-93.7; 64/8 ragged B=128 198.1-203.5 -> 201.9-202.2).
template <int D, bool KV8, bool BAL = false, int G = 1, bool MF = false>
constexpr int prefetch_depth() {
  if constexpr (KV8) {
    if constexpr (DK_PREFETCH_DEPTH_KV8 != 0) return DK_PREFETCH_DEPTH_KV8;
    else if constexpr (D <= 128 && (MF || (BAL && G <= 4))) return 2;
    else return D <= 128 ? 4 : 2;
  } else {
    return DK_PREFETCH_DEPTH ? DK_PREFETCH_DEPTH : (D <= 128 ? 2 : 1);
  }
}

// Resident wavefronts per SIMD the register allocator is held to: the page buffers
// (D/8 words per page for 16-bit elements, D/16 for fp8), G*D/16 accumulators and the q
// operand must fit without spilling.
template <int D, int G, bool KV8>
constexpr int min_waves_per_simd() {
  constexpr int buffer_words = (prefetch_depth<D, KV8>() + 1) * (KV8 ? D / 16 : D / 8);
  return (D >= 256 || buffer_words > 3 * 128 / 8) ? 1 : (D * G >= 1024 ? 1 : 2);
}

// Pages [first, first + n) of one (sequence, kv head), streamed through register buffers:
// while page k is computed, the loads of the next DEPTH pages are in flight. The
// steady-state loop has no early exit and issues its loads unconditionally, so the wait
// counters at its head see the same pending loads on every path and only wait for the
// page about to be used; the last pages are peeled off after it. Buffer 0 must already
// hold (or be loading) page 0; page(i) is the base address of page i, valid(i) its valid
// token count.
//
// GATED (DEPTH 2): page 1's loads are issued only when there is a page 1. The compiler's
// wait counts at the loop head then merge the path without them, so the first compute of
// every round of three pages waits until the second page has landed too, and the next
// loads go out later: at most about two pages in flight instead of three. Measured on
// MI355X (µs per call, fp16 32/8/128): one pass at B=32 ctx 8192 157.3 gated vs 162.0
// not; the balanced schedule at the same shape 160.8 vs 158.6, ragged B=128 350.4 vs
// 343.8, B=16 ctx 4096 51.9 vs 50.7, B=256 ctx 1024 175.7 vs 181.6. So the one-pass /
// explicit-split kernel streams gated and the balanced kernel does not.
template <int DEPTH, bool CAP, bool GATED, class W, class PageFn, class ValidFn>
__device__ __forceinline__ void stream_pages(W& wv, u32 (&ka)[W::KB], u32 (&va)[W::VB],
                                             int n, PageFn page, ValidFn valid) {
  u32 kb[W::KB], vb[W::VB];
  if constexpr (DEPTH == 1) {
    int k = 0;
    for (; k + 2 < n; k += 2) {
      wv.load_page(kb, vb, page(k + 1));
      wv.template consume<CAP>(ka, va, valid(k));
      wv.load_page(ka, va, page(k + 2));
      wv.template consume<CAP>(kb, vb, valid(k + 1));
    }
    if (k + 1 < n) {
      wv.load_page(kb, vb, page(k + 1));
      wv.template consume<CAP>(ka, va, valid(k));
      wv.template consume<CAP>(kb, vb, valid(k + 1));
    } else if (k < n) {
      wv.template consume<CAP>(ka, va, valid(k));
    }
  } else {
    u32 kc[W::KB], vc[W::VB];
    if constexpr (GATED) {
      if (n > 1) wv.load_page(kb, vb, page(1));
    } else {
      wv.load_page(kb, vb, page(n > 1 ? 1 : 0), n > 1);   // zero extent without a page 1
    }
    int k = 0;
    for (; k + 4 < n; k += 3) {
      wv.load_page(kc, vc, page(k + 2));
      wv.template consume<CAP>(ka, va, valid(k));
      wv.load_page(ka, va, page(k + 3));
      wv.template consume<CAP>(kb, vb, valid(k + 1));
      wv.load_page(kb, vb, page(k + 4));
      wv.template consume<CAP>(kc, vc, valid(k + 2));
    }
    const int r = n - k;   // 1..4 pages left; buffers a, b hold pages k, k+1
    if (r >= 3) wv.load_page(kc, vc, page(k + 2));
    if (r >= 1) wv.template consume<CAP>(ka, va, valid(k));
    if (r >= 4) wv.load_page(ka, va, page(k + 3));
    if (r >= 2) wv.template consume<CAP>(kb, vb, valid(k + 1));
    if (r >= 3) wv.template consume<CAP>(kc, vc, valid(k + 2));
    if (r >= 4) wv.template consume<CAP>(ka, va, valid(k + 3));
  }
}

// Ring of DEPTH + 1 page buffers for any DEPTH: buffer j % (DEPTH + 1) holds page j. Every
// step issues one page's loads and computes another, so the wait counters see the same
// pending loads on every path; steps past the last page load with a zero-extent
// descriptor (no memory access) and skip the compute.
template <int DEPTH, bool CAP, class W, class PageFn, class ValidFn>
__device__ __forceinline__ void stream_ring(W& wv, int n, PageFn page, ValidFn valid) {
  constexpr int NB = DEPTH + 1;
  u32 kb[NB][W::KB], vb[NB][W::VB];
#pragma unroll
  for (int j = 0; j < DEPTH; ++j) wv.load_page(kb[j], vb[j], page(min(j, n - 1)), j < n);
  for (int k = 0; k < n; k += NB) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int ld = k + j + DEPTH;
      wv.load_page(kb[(j + DEPTH) % NB], vb[(j + DEPTH) % NB], page(min(ld, n - 1)), ld < n);
      if (k + j < n) wv.template consume<CAP>(kb[j], vb[j], valid(k + j));
    }
  }
}

// Pages straight into LDS: a ring of DEPTH + 1 page slots per wavefront (`ring`,
// DEPTH + 1 slots of W::LDS_PAGE bytes); while page k is read and computed, the loads of
// the next DEPTH pages are in flight without holding registers. hipcc does not order the
// loads' LDS writes before later LDS reads, so each step waits explicitly: the wavefront's
// only vector-memory operations here are these loads, 2 * LDS_LOADS per page, so when
// at most DEPTH pages' worth are outstanding, page k has landed. Steps past the last page
// load with a zero-extent descriptor (no memory access) into a slot already consumed, so
// every step waits for the same count; all are drained before returning.
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int DEPTH, bool CAP, class W, class PageFn, class ValidFn>
__device__ __forceinline__ void stream_lds(W& wv, uint8_t* ring, int n, PageFn page,
                                           ValidFn valid) {
  constexpr int NB = DEPTH + 1;
  constexpr int PER = 2 * W::LDS_LOADS;
#pragma unroll
  for (int j = 0; j < DEPTH; ++j) wv.lds_load_page(ring + j * W::LDS_PAGE, page(min(j, n - 1)), j < n);
  for (int k = 0; k < n; ++k) {
    const int ld = k + DEPTH;
    wv.lds_load_page(ring + (ld % NB) * W::LDS_PAGE, page(min(ld, n - 1)), ld < n);
    wait_vmem<PER * DEPTH>();
    u32 kb[W::KB], vb[W::VB];
    wv.lds_read_page(ring + (k % NB) * W::LDS_PAGE, kb, vb);
    wv.template consume<CAP>(kb, vb, valid(k));
  }
  wait_vmem<0>();
}

// Whether a kernel streams its pages through LDS (stream_lds), on the VALU q.k path (GROUPED:
// a balanced kernel serving several kv heads per workgroup; NW: the workgroup's wavefronts):
//  * 16-bit caches at D = 256 (512-byte rows), at most 2 wavefronts per workgroup (64 KB of
//    ring each);
//  * fp8 caches at D = 64 (64-byte rows) in the grouped balanced kernels: 16-byte lane loads
//    (16 rows per instruction) instead of 4-byte ones, 2 pages in flight, the workgroup's
//    rings within DK_LDS_NARROW_BUDGET bytes (against the register ring, us: ragged B=128
//    ctx U[128, 8192] 129.4 -> 123.1, B=32 ctx 2048 28.0 -> 26.9, ctx 8192 63.8 -> 63.3;
//    depth 1, 3, 5 and 7 measured slower than 2, and the one-pass kernels over short
//    sequences 3 % slower with the ring).
// Build switches for comparisons (all measured slower): DK_LDS_NARROW=0 turns the fp8 D = 64
// case off, DK_LDS_NARROW=2 extends it to every row of at most 128 bytes (16-bit D = 64,
// fp8 D = 128) in any kernel, DK_LDS_256=1 to 256-byte rows (16-bit D = 128, fp8 D = 256);
// DK_LDS_DEPTH / DK_LDS_DEPTH_NARROW set the pages in flight (at D = 256, 2 measured the
// same as 3).
#ifndef DK_LDS_DEPTH
#define DK_LDS_DEPTH 3
#endif
#ifndef DK_LDS_DEPTH_NARROW
#define DK_LDS_DEPTH_NARROW 2
#endif
#ifndef DK_LDS_NARROW
#define DK_LDS_NARROW 1
#endif
#ifndef DK_LDS_256
#define DK_LDS_256 0
#endif
#ifndef DK_LDS_NARROW_BUDGET
#define DK_LDS_NARROW_BUDGET 65536
#endif
#ifndef DK_LDS_GROUPED_ROW          // grouped kernels: the ring over rows of at most this
#define DK_LDS_GROUPED_ROW 64       // many bytes
#endif
template <int D, bool KV8>
constexpr int lds_depth() {
  return D * (KV8 ? 1 : 2) <= kNarrowRowBytes ? DK_LDS_DEPTH_NARROW : DK_LDS_DEPTH;
}
template <int D, bool KV8, bool MFMA, int NW, bool GROUPED = false>
constexpr bool lds_pages() {
  constexpr int rb = D * (KV8 ? 1 : 2);
  if (!DK_LDS_PAGES || MFMA) return false;
  if (rb == 512) return !KV8 && NW <= 2;
  if (rb == 256) return DK_LDS_256 && NW <= 2;
  if (rb > kNarrowRowBytes) return false;
  const bool on = DK_LDS_NARROW >= 2 || (DK_LDS_NARROW == 1 && GROUPED && rb <= DK_LDS_GROUPED_ROW);
  return on && NW * (lds_depth<D, KV8>() + 1) * 2 * kPage * rb <= DK_LDS_NARROW_BUDGET;
}

// ---------------------------------------------------------------- workgroup combine
// LDS scratch for merging the NW wavefronts of a workgroup.
template <int G, int D, int NW>
struct CombineSmem {
  float acc[NW][G][D];
  float m[NW][G], mt[NW][G], l[NW][G];
};

// After every wavefront's reduce_rows: the result of the NW wavefronts that share one kv
// head (w = this wavefront among them, tid = this thread among their NW * 64) for its G
// heads, written normalised to out (head h at out + h * o_h) when `direct`, otherwise as a
// partial with head h at row prow0 + h * phstride. Every wavefront of the workgroup calls
// it the same number of times (it holds workgroup barriers). qh0: the first q head (for
// the attention sinks of the normalised output).
template <class T, int D, int G, int NW, class WV>
__device__ __forceinline__ void combine_store(WV& wv, CombineSmem<G, D, (NW > 1 ? NW : 1)>& sm,
                                              const Pass1Args& a, bool direct, uint8_t* out,
                                              int64_t o_h, int64_t prow0, int64_t phstride,
                                              int w, int tid, int qh0) {
  constexpr int DPL = WV::DPL, NS = WV::NS, GQ = WV::GQ;
  const float* sink = a.sinks ? a.sinks + qh0 : nullptr;
  if constexpr (NW == 1) {
    (void)w;
    (void)tid;
    if (direct) wv.store_output(out, o_h, sink);
    else wv.store_partial(a, prow0, phstride);
  } else {
    if constexpr (WV::WIDE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * wv.r16 + i;
        if (h < G) {
#pragma unroll
          for (int j = 0; j < DPL; ++j) sm.acc[w][h][wv.c * DPL + j] = wv.acc[i][j];
        }
      }
    } else {
      static_for<WV::KR>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const int h = 4 * k + wv.r16;
        if (h < G) {
#pragma unroll
          for (int j = 0; j < DPL; ++j)
            sm.acc[w][h][wv.c * DPL + j] = wv.template row_head<k>(j);
        }
      });
    }
    if (wv.r16 == 0 && wv.c < GQ) {
#pragma unroll
      for (int ss = 0; ss < NS; ++ss) {
        if (ss * GQ + wv.c >= G) continue;
        sm.m[w][ss * GQ + wv.c] = wv.mref[ss];
        sm.mt[w][ss * GQ + wv.c] = wv.mtrue[ss];
        sm.l[w][ss * GQ + wv.c] = wv.lsum[ss];
      }
    }
    __syncthreads();
    for (int idx = tid; idx < wv.hv * D; idx += NW * 64) {
      const int h = idx / D, d = idx % D;
      float mt = kNegInf;
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) mt = fmaxf(mt, sm.mt[ww][h]);
      float L = 0.f, O = 0.f;
      const bool empty = !(mt > kNegInf);
      if (!empty) {
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
          const float f = __builtin_amdgcn_exp2f(sm.m[ww][h] - mt);
          L += sm.l[ww][h] * f;
          O += sm.acc[ww][h][d] * f;
        }
      }
      if (direct) {
        if (sink) L += __builtin_amdgcn_exp2f(sink[h] * kLog2e - mt);   // +inf when empty
        T::store(out + (int64_t)h * o_h + 2 * d, L > 0.f ? O / L : 0.f);
      } else {
        const int64_t row = prow0 + h * phstride;
        a.part_o[row * D + d] = empty ? 0.f : O;
        if (d == 0) {
          a.part_m[row] = empty ? kEmptyM : mt * kLn2;
          a.part_l[row] = L;
        }
      }
    }
    __syncthreads();   // the LDS is reused by the next segment
  }
}

// Wavefront w of NW streams pages first + w, first + w + NW, ... of a run of n pages
// (through its LDS ring when LDS is set; GATED: see stream_pages).
template <int D, bool KV8, bool CAP, bool LDS, bool GATED, bool BAL = false, class WV,
          class PageFn, class ValidFn>
__device__ __forceinline__ void stream_interleaved(WV& wv, int NW, int w, int n, PageFn page,
                                                   ValidFn valid, uint8_t* ring = nullptr) {
  const int nk = n > w ? (n - w + NW - 1) / NW : 0;
  if (nk > 0) {
    auto pk = [&](int k) { return page(w + NW * k); };
    auto vk = [&](int k) { return valid(w + NW * k); };
    constexpr int depth = prefetch_depth<D, KV8, BAL, WV::HEADS, WV::MF>();
    if constexpr (LDS) {
      stream_lds<lds_depth<D, KV8>(), CAP>(wv, ring, nk, pk, vk);
    } else if constexpr (depth <= 2) {
      u32 ka[WV::KB], va[WV::VB];
      wv.load_page(ka, va, pk(0));
      stream_pages<depth, CAP, GATED>(wv, ka, va, nk, pk, vk);
    } else {
      stream_ring<depth, CAP>(wv, nk, pk, vk);
    }
  }
  (void)ring;
}

// Whether a kernel streams through registers with its first page loaded by the caller
// (stream_loaded below): the register ring of depth <= 2 on the VALU q.k path (16-bit
// caches at D <= 128). (The MFMA q.k path stages K through LDS and has no registers to
// spare for it: two of its kernels spilled.)
template <int D, bool KV8, bool LDS, bool MFMA, bool BAL = false, int G = 1>
constexpr bool first_page_by_caller() {
  return !LDS && !MFMA && prefetch_depth<D, KV8, BAL, G, MFMA>() <= 2;
}

// stream_interleaved with this wavefront's first page (page w of the run) already loading
// into ka / va; the balanced kernel issues that load before it has found the sequence of
// its first segment, and before the previous segment's combine for the others
// (first_page_by_caller kernels only).
template <int D, bool KV8, bool CAP, bool BAL = false, class WV, class PageFn,
          class ValidFn>
__device__ __forceinline__ void stream_loaded(WV& wv, int NW, int w, int n, PageFn page,
                                              ValidFn valid, u32 (&ka)[WV::KB],
                                              u32 (&va)[WV::VB]) {
  const int nk = n > w ? (n - w + NW - 1) / NW : 0;
  if (nk > 0) {
    auto pk = [&](int k) { return page(w + NW * k); };
    auto vk = [&](int k) { return valid(w + NW * k); };
    stream_pages<prefetch_depth<D, KV8, BAL, WV::HEADS, WV::MF>(), CAP, false>(wv, ka, va, nk,
                                                                               pk, vk);
  }
}


// ---------------------------------------------------------------- pass 1, explicit split
template <class T, int D, int G, int NW, bool MFMA, bool KV8>
__global__ __launch_bounds__(NW * 64, (min_waves_per_simd<D, G, KV8>())) void dk_pass1_split(Pass1Args a) {
  using WV = Wave<T, D, G, MFMA, KV8>;
  __shared__ CombineSmem<G, D, (NW > 1 ? NW : 1)> sm;
  __shared__ __attribute__((aligned(16))) uint8_t kst[WV::STAGE ? NW * WV::STAGE_BYTES : 16];
  constexpr bool LDSP = lds_pages<D, KV8, MFMA, NW>();
  constexpr int RING = (lds_depth<D, KV8>() + 1) * WV::LDS_PAGE;
  __shared__ __attribute__((aligned(16))) uint8_t ring[LDSP ? NW * RING : 16];
  WV wv;
  wv.init(a);
  const int w = uniform(threadIdx.x >> 6);
  wv.kst = kst + w * WV::STAGE_BYTES;
  uint8_t* const wring = ring + (LDSP ? w * RING : 0);

  // workgroup -> (head chunk, kv head, split, sequence). The head chunks of one (sequence,
  // kv head, split) read the same pages: they are placed kXcds workgroup ids apart (the
  // dispatcher deals workgroups to the XCDs in turn), so they run on one XCD, close in
  // time, and the later reads of a page can hit that XCD's L2.
  int hc = 0, t = blockIdx.x;
  if (a.chunks > 1) {
    const int x = t % kXcds, y = t / kXcds;
    hc = y % a.chunks;
    t = (y / a.chunks) * kXcds + x;
    if (t >= a.batch * a.hkv * a.split) return;   // padding of the last XCD round
  }
  const int kvh = t % a.hkv;
  t /= a.hkv;
  const int s = t % a.split;
  const int b = t / a.split;

  const int seq0 = seq_begin(a, b);
  const int npages = max(seq_begin(a, b + 1), seq0) - seq0;
  const int valid_last = min(max(ld_const(a.last_len, b), 0), kPage);
  // sliding window: pages from the one holding the window's first token
  int first_page = 0, first_tok = 0;
  if (a.window > 0 && npages > 0) {
    const int t0 = max((npages - 1) * kPage + valid_last - a.window, 0);
    first_page = t0 / kPage;
    first_tok = t0 % kPage;
  }
  const int npw = npages - first_page;
  const int pps = (npw + a.split - 1) / a.split;             // attention_ext.cu:249-252
  const int p0 = first_page + min(s * pps, npw);
  const int n = max(min(p0 + pps, npages) - p0, 0);
  const int qh0 = kvh * a.group + hc * a.per;
  wv.hv = min(a.per, a.group - hc * a.per);

  wv.load_q(a.q + (int64_t)b * a.q_b + (int64_t)qh0 * a.q_h, a.q_h);
  wv.reset();
  const uint8_t* kvh_base = a.kv + (int64_t)kvh * a.kv_h;
  auto page = [&](int i) -> const uint8_t* {
    u32 pid = (u32)uniform(ld_const(a.indices, seq0 + p0 + i));
    pid = pid < a.num_pages ? pid : 0u;
    return kvh_base + (int64_t)pid * a.kv_p;
  };
  // page validity hi | lo << 8: a full page but for the sequence's last page and, with a
  // window starting inside a page, that page
  const int lo_page = first_tok > 0 ? first_page : -1;
  const int enc_last = valid_last | (npages - 1 == lo_page ? first_tok << 8 : 0);
  const int enc_lo = kPage | first_tok << 8;
  auto valid = [&](int i) -> int {
    const int pg = p0 + i;
    return pg == npages - 1 ? enc_last : (pg == lo_page ? enc_lo : kPage);
  };
  if (a.cap_out != 0.f)
    stream_interleaved<D, KV8, true, LDSP, true>(wv, NW, w, n, page, valid, wring);
  else
    stream_interleaved<D, KV8, false, LDSP, true>(wv, NW, w, n, page, valid, wring);
  wv.reduce_rows();
  combine_store<T, D, G, NW>(wv, sm, a, a.direct != 0,
                             a.out + (int64_t)b * a.o_b + (int64_t)qh0 * a.o_h, a.o_h,
                             ((int64_t)b * a.hq + qh0) * a.split + s, a.split, w,
                             (int)threadIdx.x, qh0);
}

// ---------------------------------------------------------------- pass 1, balanced
// Range split of the balanced schedule. A head chunk's units (its pages in sequence order,
// x = 0 .. P-1) carry the cost x + A * seq(x), where seq(x) is the largest b with
// start(b) <= x (start(b) = kv_indptr[b] - kv_indptr[0]): every sequence start is charged
// A pages, what a change of sequence costs a workgroup. The cost space [0, C), C = P +
// A * (batch - 1), is cut into Wg ranges of Lc = ceil(C / Wg); range j holds the units with
// floor(cost / Lc) == j, contiguous since the cost grows with x. With A = 0 these are the
// equal page ranges. The merge kernel finds a sequence's ranges with the same formula.
__device__ __forceinline__ int64_t range_cost_len(int P, int A, int batch, int Wg) {
  const int64_t C = (int64_t)P + (int64_t)A * max(batch - 1, 0);
  return (C + Wg - 1) / Wg;
}

// First unit of the cost interval starting at T (A > 0): the smallest x with
// x + A * seq(x) >= T, or P. *b_out = the largest b with f(b) = start(b) + A * b <= T (the
// sequence holding x, or the last one before it). A search over kv_indptr by one wavefront,
// 64 candidates per step (f grows with b: one step up to 64 sequences, two up to 4096);
// every lane returns the same values.
__device__ __forceinline__ int cost_boundary(const Pass1Args& a, int base, int P, int A,
                                             int64_t T, int* b_out) {
  const int lane = threadIdx.x & 63;
  int lo = 0, S = a.batch;   // the answer is in [lo, lo + S); f(lo) <= T
  while (S > 1) {
    const int st = (S + 63) / 64;
    const bool in = lane * st < S;
    const int bi = min(lo + lane * st, a.batch);   // kv_indptr has batch + 1 entries
    const int64_t fb = (int64_t)(seq_begin(a, bi) - base) + (int64_t)A * bi;
    const int64_t f = in ? fb : INT64_MAX;
    const uint64_t m = __builtin_amdgcn_ballot_w64(f <= T);
    const int k = m ? 63 - __builtin_clzll(m) : 0;   // lane 0 holds f(lo) <= T
    lo += k * st;
    S = min(st, S - k * st);
  }
  const int b = uniform(lo);
  const int sb = seq_begin(a, b) - base;
  const int se = max(seq_begin(a, b + 1) - base, sb);
  const int64_t f = (int64_t)sb + (int64_t)A * b;
  *b_out = b;
  const int64_t x = min((int64_t)sb + max(T - f, (int64_t)0), (int64_t)se);
  return (int)min(max(x, (int64_t)0), (int64_t)P);
}

// Head-major persistent schedule over workgroups. Each of the HC = hkv * chunks head
// chunks (hc = chunk * hkv + kv head) has Wg = a.ranges workgroups; consecutive
// workgroups -- and the XCDs they are dispatched to round-robin -- cover all kv heads of
// the same pages at the same time. The Wg workgroups of a head chunk split its pages in sequence
// order ((b, page) is linear unit seq_begin(b) - seq_begin(0) + page) into Wg ranges of
// equal cost (range_cost_len: equal pages, or with a.seg_cost pages charged per sequence
// start); workgroup j takes range j and its NW wavefronts interleave the pages of each
// segment (maximal run of the range inside one sequence). A sequence covered by a single
// segment is written out directly (when a.direct); otherwise the segment is stored as a
// partial at slot hc * (Wg + batch) + j + b (unique, < HC * (Wg + batch), as the ranges are
// contiguous and ordered) for the merge kernel.
// COST: the build whose range split charges sequence starts (a.seg_cost, ragged batches);
// the other one splits equal pages and carries none of that code.
template <class T, int D, int G, int NW, bool MFMA, bool KV8, int HP, bool COST = false>
__global__ __launch_bounds__(NW * HP * 64, (min_waves_per_simd<D, G, KV8>())) void dk_pass1_balanced(Pass1Args a) {
  using WV = Wave<T, D, G, MFMA, KV8>;
  __shared__ CombineSmem<G, D, (NW > 1 ? NW : 1)> smh[HP];
  __shared__ __attribute__((aligned(16))) uint8_t kst[WV::STAGE ? HP * NW * WV::STAGE_BYTES : 16];
  constexpr bool LDSP = lds_pages<D, KV8, MFMA, NW * HP, (HP > 1)>();
  constexpr int RING = (lds_depth<D, KV8>() + 1) * WV::LDS_PAGE;
  __shared__ __attribute__((aligned(16))) uint8_t ring[LDSP ? HP * NW * RING : 16];
  WV wv;
  wv.init(a);
  const int wa = uniform(threadIdx.x >> 6);   // wavefront of the workgroup
  const int hl = wa / NW, w = wa % NW;        // its kv head among the HP, its rank there
  wv.kst = kst + wa * WV::STAGE_BYTES;
  uint8_t* const wring = ring + (LDSP ? wa * RING : 0);
  auto& sm = smh[hl];
  // workgroup -> (HP head chunks hc, range j): its NW * HP wavefronts serve HP consecutive
  // kv heads (same head chunk) of the same pages, so the HP row segments of each token are
  // read at the same time (narrow rows: HP * 64 or HP * 128 contiguous bytes). Unit
  // u = j * (hkv / HP) + kv-head group: consecutive workgroups cover the kv heads of the
  // same pages. With several head chunks, which all read the unit's pages, the chunks of
  // a unit are placed kXcds workgroup ids apart (the grid is padded to whole rounds), so
  // they run on one XCD and share its L2.
  const int Wg = a.ranges;
  const int hkg = a.hkv / HP;                 // kv-head groups (HP divides hkv)
  int hc, j;
  if (a.chunks > 1) {
    const int x = (int)blockIdx.x % kXcds, y = (int)blockIdx.x / kXcds;
    const int un = (y / a.chunks) * kXcds + x;
    if (un >= hkg * Wg) return;                              // padding of the last round
    j = un / hkg;
    hc = (y % a.chunks) * a.hkv + (un % hkg) * HP + hl;
  } else {
    hc = ((int)blockIdx.x % hkg) * HP + hl;
    j = (int)blockIdx.x / hkg;
  }
  const int base = seq_begin(a, 0);
  const int P = max(seq_begin(a, a.batch) - base, 0);        // pages per head chunk
  const int A = COST ? a.seg_cost : 0;
  int u, u_end, b = 0;   // the range's units [u, u_end); b: the sequence search's result
  int L = 0;             // A == 0: pages per range
  int64_t Lc = 0;        // A > 0: cost per range
  if (A == 0) {
    L = (P + Wg - 1) / Wg;
    if (L <= 0) return;                                      // whole workgroup
    u = (int)min((int64_t)j * L, (int64_t)P);
    u_end = min(u + L, P);
  } else {
    Lc = range_cost_len(P, A, a.batch, Wg);
    if (Lc <= 0) return;
    u = cost_boundary(a, base, P, A, (int64_t)j * Lc, &b);
    int b_end;
    u_end = (int64_t)(j + 1) * Lc >= (int64_t)P + (int64_t)A * max(a.batch - 1, 0)
                ? P : cost_boundary(a, base, P, A, (int64_t)(j + 1) * Lc, &b_end);
  }
  if (u >= u_end) return;

  const int kvh = hc % a.hkv, chunk = hc / a.hkv;
  const int qh0 = kvh * a.group + chunk * a.per;
  wv.hv = min(a.per, a.group - chunk * a.per);
  const uint8_t* kvh_base = a.kv + (int64_t)kvh * a.kv_h;
  auto page_at = [&](int idx) -> const uint8_t* {   // page of kv_indices[idx]
    u32 pid = (u32)uniform(ld_const(a.indices, idx));
    pid = pid < a.num_pages ? pid : 0u;
    return kvh_base + (int64_t)pid * a.kv_p;
  };
  // The range's units are kv_indices[base + u ..]: this wavefront's first page (unit
  // u + w) is known before the sequence it belongs to, so its load is issued now and the
  // binary search and the sequence's bounds (dependent memory trips) run while it is in
  // flight. A range shorter than the wavefront index loads nothing (zero extent); a page
  // loaded for a segment too short to have a page w is not used.
  constexpr bool PRE = first_page_by_caller<D, KV8, LDSP, MFMA, true, G>();
  u32 ka[WV::KB], va[WV::VB];   // unused (and allocated no registers) unless PRE
  if constexpr (PRE) wv.load_page(ka, va, page_at(base + min(u + w, u_end - 1)), u + w < u_end);

  if (A == 0) {
    // sequence containing unit u: the largest b with start(b) <= u (binary search)
    int lo = 0, hi = a.batch - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (seq_begin(a, mid) - base <= u) lo = mid; else hi = mid - 1;
    }
    b = lo;
  }
  // q of that sequence, in flight with its bounds below
  wv.load_q(a.q + (int64_t)b * a.q_b + (int64_t)qh0 * a.q_h, a.q_h);
  int seq0 = seq_begin(a, b);
  int np = max(seq_begin(a, b + 1), seq0) - seq0;
  int pg = u - (seq0 - base);
  if (A != 0 && pg >= np) {
    // the range starts at the next non-empty sequence (its first cost fell in the charge of
    // sequence b's start)
    do {
      ++b;
      seq0 = seq_begin(a, b);
      np = max(seq_begin(a, b + 1), seq0) - seq0;
      pg = u - (seq0 - base);
    } while (pg >= np && b < a.batch - 1);
    wv.load_q(a.q + (int64_t)b * a.q_b + (int64_t)qh0 * a.q_h, a.q_h);
  }
  if (np <= 0 || pg < 0 || pg >= np) return;   // only for a decreasing kv_indptr (invalid)

  // Segment after segment; the next segment's q (and, PRE, this wavefront's first page of
  // it) is loaded before the current segment's reduction and workgroup combine, so its
  // memory latency overlaps that work.
  while (true) {
    const int n = min(np - pg, u_end - u);   // pages of this segment (>= 1)
    wv.reset();
    const int valid_last = min(max(ld_const(a.last_len, b), 0), kPage);
    const int first = pg, cur_seq0 = seq0, cur_np = np, cur_b = b;
    auto page = [&](int i) -> const uint8_t* { return page_at(cur_seq0 + first + i); };
    auto valid = [&](int i) -> int { return first + i == cur_np - 1 ? valid_last : kPage; };
    if constexpr (PRE) {
      // ka / va hold (or are loading) this segment's page w, the range's unit u + w
      if (a.cap_out != 0.f)
        stream_loaded<D, KV8, true, true>(wv, NW, w, n, page, valid, ka, va);
      else
        stream_loaded<D, KV8, false, true>(wv, NW, w, n, page, valid, ka, va);
    } else {
      if (a.cap_out != 0.f)
        stream_interleaved<D, KV8, true, LDSP, false, true>(wv, NW, w, n, page, valid, wring);
      else
        stream_interleaved<D, KV8, false, LDSP, false, true>(wv, NW, w, n, page, valid, wring);
    }

    // the next non-empty sequence of the range, if any
    bool more = false;
    if (u + n < u_end) {
      u += n;
      do {
        ++b;
        seq0 = seq_begin(a, b);
        np = max(seq_begin(a, b + 1), seq0) - seq0;
      } while (np == 0 && b < a.batch - 1);
      more = np > 0;   // np == 0 only for an invalid kv_indptr
      pg = 0;
    }
    if (more) {
      wv.load_q(a.q + (int64_t)b * a.q_b + (int64_t)qh0 * a.q_h, a.q_h);
      if constexpr (PRE)
        wv.load_page(ka, va, page_at(base + min(u + w, u_end - 1)), u + w < u_end);
    }

    wv.reduce_rows();
    // ranges holding this sequence's units (cost = unit + A * sequence)
    const int start = cur_seq0 - base;
    int nslots;
    if (A == 0) {
      nslots = (start + cur_np - 1) / L - start / L + 1;
    } else {
      const int64_t c0 = (int64_t)start + (int64_t)A * cur_b;
      nslots = (int)((c0 + cur_np - 1) / Lc - c0 / Lc + 1);
    }
    combine_store<T, D, G, NW>(wv, sm, a, a.direct != 0 && nslots == 1,
                               a.out + (int64_t)cur_b * a.o_b + (int64_t)qh0 * a.o_h, a.o_h,
                               ((int64_t)hc * (Wg + a.batch) + j + cur_b) * G, 1, w,
                               (int)(threadIdx.x & 63) + 64 * w, qh0);
    if (!more) break;
  }
}

// ---------------------------------------------------------------- pass 2
// Partial k of a row: O at po + k * stride_rows * D, m and l at pm / pl + k * stride_rows.
// One wavefront per row, lanes over the D dims (E = D/64 each). The O loads of the first
// kU slots are issued before the m / l loads and the max, so a row with up to kU slots
// costs one memory round trip; more slots are loaded kV at a time.
template <class T, int D>
__device__ __forceinline__ void merge_row(const MergeArgs& m, int row, const float* po,
                                          const float* pm, const float* pl, int nslots,
                                          int64_t stride_rows) {
  constexpr int E = D / 64;
  constexpr int kU = E <= 2 ? 32 : 16;
  constexpr int kV = 8;   // slots per later batch (rows of more than kU slots)
  typedef float vecE __attribute__((ext_vector_type(E)));
  const int lane = threadIdx.x & 63;
  // slot k's row starts at a wave-uniform address (scalar registers); each lane adds its
  // own 32-bit byte offset, so no slot needs a 64-bit vector address
  const uint32_t lane_off = (uint32_t)(lane * E) * 4u;
  auto o_at = [&](int k) {
    const char* base = reinterpret_cast<const char*>(po + (int64_t)k * stride_rows * D);
    return *reinterpret_cast<const vecE*>(base + lane_off);
  };
  // first batch of O (uniform guards: no load past the row's last slot)
  const int cnt0 = min(nslots, kU);
  vecE v0[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    v0[u] = vecE{};
    if (u < cnt0) v0[u] = o_at(u);
  }
  // the first 64 slots' m and l stay in registers (one slot per lane)
  float pm0 = kNegInf, pl0 = 0.f;
  if (lane < nslots) {
    pm0 = pm[(int64_t)lane * stride_rows];
    pl0 = pl[(int64_t)lane * stride_rows];
  }
  float M = pm0;
  for (int k = lane + 64; k < nslots; k += 64) M = fmaxf(M, pm[(int64_t)k * stride_rows]);
  M = wave_max(M);
  vecE acc = {};
  float L = 0.f;
  for (int k0 = 0; k0 < nslots; k0 += 64) {
    const int k = k0 + lane;
    float wgt = 0.f;
    if (k < nslots) {
      const float mk = k0 == 0 ? pm0 : pm[(int64_t)k * stride_rows];
      const float lk = k0 == 0 ? pl0 : pl[(int64_t)k * stride_rows];
      wgt = __builtin_amdgcn_exp2f((mk - M) * kLog2e);
      L += wgt * lk;
    }
    const int cnt = min(64, nslots - k0);
    int j = 0;
    if (k0 == 0) {
#pragma unroll
      for (int u = 0; u < kU; ++u) acc += readlane_f(wgt, u) * v0[u];   // zero past cnt0
      j = cnt0;
    }
    for (; j + kV <= cnt; j += kV) {
      vecE v[kV];
#pragma unroll
      for (int u = 0; u < kV; ++u) v[u] = o_at(k0 + j + u);
#pragma unroll
      for (int u = 0; u < kV; ++u) acc += readlane_f(wgt, j + u) * v[u];
    }
    for (; j < cnt; ++j) acc += readlane_f(wgt, j) * o_at(k0 + j);
  }
  L = wave_sum(L);
  const int b = row / m.hq, qh = row % m.hq;
  // attention sink of this q head: one more denominator term, e^{sink - M} (+inf, hence a
  // zero output, when no slot saw a token)
  if (m.sinks) L += __builtin_amdgcn_exp2f((m.sinks[qh] - M) * kLog2e);
  uint8_t* op = m.out + (int64_t)b * m.o_b + (int64_t)qh * m.o_h + 2 * lane * E;
#pragma unroll
  for (int e = 0; e < E; ++e) T::store(op + 2 * e, L > 0.f ? acc[e] / L : 0.f);
}

template <class T, int D>
__global__ __launch_bounds__(256) void dk_merge_split(MergeArgs m) {
  const int row = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (row >= m.batch * m.hq) return;
  const int64_t r0 = (int64_t)row * m.split;
  merge_row<T, D>(m, row, m.po + r0 * D, m.pm + r0, m.pl + r0, m.split, 1);
}

// COST: pass 1 ran the charged range split (m.seg_cost); the other build carries none of it.
template <class T, int D, bool COST = false>
__global__ __launch_bounds__(256) void dk_merge_balanced(MergeArgs m) {
  const int row = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (row >= m.batch * m.hq) return;
  const int b = row / m.hq, qh = row % m.hq;
  const int G = m.heads, Wg = m.waves_per_pair;
  auto sb = [&](int bb) { return min(max(ld_const(m.indptr, bb), 0), m.num_indices); };
  const int base = sb(0);
  const int P = max(sb(m.batch) - base, 0);
  const int seq0 = sb(b);
  const int np = max(sb(b + 1), seq0) - seq0;
  const int kvh = qh / m.group, r = qh % m.group;
  const int hc = (r / m.per) * m.hkv + kvh, g = r % m.per;   // chunk-major; slot row g of G
  int nslots = 0;
  int64_t r0 = 0;
  // the ranges of pass 1 that hold this sequence's units (its range split: equal pages, or
  // the charged split's cost)
  int j0 = 0;
  if constexpr (!COST) {
    const int L = (P + Wg - 1) / Wg;
    if (np > 0 && L > 0) {
      const int start = seq0 - base;
      j0 = start / L;
      nslots = (start + np - 1) / L - j0 + 1;
    }
  } else {
    const int64_t Lc = range_cost_len(P, m.seg_cost, m.batch, Wg);
    if (np > 0 && Lc > 0) {
      const int64_t c0 = (int64_t)(seq0 - base) + (int64_t)m.seg_cost * b;
      j0 = (int)(c0 / Lc);
      nslots = (int)((c0 + np - 1) / Lc) - j0 + 1;
    }
  }
  if (nslots > 0) r0 = ((int64_t)hc * (Wg + m.batch) + j0 + b) * G + g;
  if (nslots == 1) return;   // pass 1 wrote this head's output
  // slot k of this pair is r0 + k * G (rows of G heads per slot); none -> zeros
  merge_row<T, D>(m, row, m.po + r0 * D, m.pm + r0, m.pl + r0, nslots, (int64_t)G);
}

}  // namespace dk
