/*
 * dk_decode.h — C ABI of the MI355X (gfx950) split-KV paged decode-attention library
 * (libdk_decode.so).
 *
 * One query token per sequence attends over a paged KV cache in the FlashInfer NHD
 * layout:
 *   q        (batch, num_q_heads, head_dim)                       fp16 | bf16
 *   kv_data  (num_pages, 2, page_size, num_kv_heads, head_dim)    same dtype as q
 *            [:, 0] = K, [:, 1] = V
 *   kv_indptr (batch + 1) int32, kv_indices (kv_indptr[batch]) int32,
 *   kv_last_page_len (batch) int32 in [1, page_size]
 *   out      (batch, num_q_heads, head_dim)                       same dtype as q
 * GQA: q head h reads kv head h / (num_q_heads / num_kv_heads).
 * scale = 1/sqrt(head_dim); softmax state and split partials are fp32.
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers except `strides`, `opts` and the out-parameters
 *     of the size/choice helpers, which are host pointers.
 *   - Strides are in ELEMENTS; the last (head_dim) stride of q, kv_data and out must be 1.
 *   - Work is enqueued on `hip_stream` (a hipStream_t; NULL = the legacy default stream)
 *     and is stream-ordered. No entry point allocates device memory: the caller owns
 *     `out` and `workspace`.
 *   - Return value: 0 on success; < 0 invalid argument (nothing was launched);
 *     > 0 a hipError_t from the launch. dk_last_error() then holds a message
 *     (thread-local, valid until the next call on the same thread).
 *   - Device-side safety: page ids outside [0, num_pages), kv_indptr entries outside
 *     [0, num_indices] and kv_last_page_len outside [0, page_size] are clamped inside
 *     the kernels so that no access leaves the buffers; results for such inputs are
 *     unspecified (the reference does not check them either).
 */
#ifndef DK_DECODE_H
#define DK_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DK_ABI_VERSION 3

/* Element type of q / kv_data / out. The reference is fp16 only
 * (src/cuda_/attention_ext.cu:507,550); bf16 is an extension. */
typedef enum { DK_F16 = 0, DK_BF16 = 1 } dk_dtype;

/* Element type of the KV cache when it differs from q / out (dk_options.kv_dtype):
 * OCP FP8 E4M3 (torch.float8_e4m3fn), dequantised as value * k_scale / v_scale. No
 * counterpart in the reference (fp16 cache only). */
#define DK_KV_SAME 0
#define DK_KV_FP8_E4M3 2

/* Error codes (< 0). */
enum {
  DK_OK = 0,
  DK_EINVAL = -1,      /* bad shape / size / stride / dtype / split value   */
  DK_ENULL = -2,       /* required pointer is NULL                           */
  DK_EWORKSPACE = -3,  /* workspace missing or smaller than dk_workspace_bytes */
  DK_EUNSUPPORTED = -4 /* valid input this build does not implement           */
};

/* Element strides. Replaces the int32 stride marshalling of
 * src/cuda_/attention_ext.cu:577-587 (here int64, so pools > 2^31 elements work). */
typedef struct {
  int64_t q_b, q_h;                /* q (batch, num_q_heads, head_dim)            */
  int64_t kv_p, kv_r, kv_s, kv_h;  /* kv_data (num_pages, 2, page_size, Hkv, D)   */
  int64_t o_b, o_h;                /* out (batch, num_q_heads, head_dim)          */
} dk_strides;

/* Optional tuning knobs (NULL = defaults). No counterpart in the reference, which
 * hard-codes one kernel per extension module (src/cuda_/build.py:256-282). */
typedef struct {
  int32_t qk_path;         /* 0 = automatic: VALU dot2 q.k up to 4 q heads per kv head,
                              MFMA q.k (up to 16 heads per wavefront) beyond and for fp8
                              at D = 256; 1 = MFMA, 2 = VALU; P.V always on MFMA         */
  int32_t waves_per_group; /* 0 = default: 2, or 4 with kv-head rows of <= 128 bytes (fp8,
                              or D = 64) or 8 heads per wavefront on the VALU q.k path;
                              the balanced schedule over such narrow rows serves 4 (or
                              2) neighbouring kv heads per workgroup with 2 wavefronts
                              each, over small problems (plan hint) uses 4, and over many
                              short sequences (plan hint) 1; an explicit split_kv over
                              256-byte rows uses 4 when its workgroups are fewer than the
                              compute units, up to twice as many, or as many with at most
                              32 pages each; else 1, 2 or 4 (then one kv head per
                              workgroup)                                                  */
  int32_t waves_per_cu;    /* wavefronts per compute unit the automatic and balanced
                              schedules aim for (0 = default: 2, or 4 as above, 8 with
                              grouped kv heads)                                           */
  int32_t schedule;        /* split_kv == 0: 0 = automatic, 1 = balanced, 2 = one workgroup
                              per (sequence, kv head) (split_kv == 1)                       */
  int32_t max_pages_per_seq; /* plan hint for split_kv == 0: the most pages any sequence
                              has (from the host copy of kv_indptr), 0 = unknown. With it
                              the automatic schedule runs one pass when that is as short
                              as the balanced one; without it, it always balances.
                              Too small a value affects speed only, never results.       */
  float sm_scale;          /* softmax scale applied to q.k; 0 = 1/sqrt(head_dim), the
                              reference's fixed scale (attention_ext.cu:79-80)             */
  int32_t kv_dtype;        /* DK_KV_SAME (0): the cache has q's type; DK_KV_FP8_E4M3: fp8
                              (strides still in elements, now bytes)                      */
  float k_scale;           /* fp8 cache: K = k_scale * stored value (0 = 1); must be 0
                              for a cache of q's type                                     */
  float v_scale;           /* fp8 cache: V = v_scale * stored value (0 = 1); likewise     */
  float logit_cap;         /* logit soft-capping (Gemma 2 style): each score s = q.k *
                              sm_scale (* k_scale) becomes logit_cap * tanh(s / logit_cap)
                              before the softmax; 0 = off. No counterpart in the reference */
  int32_t window;          /* sliding window: attend to the last `window` tokens of each
                              sequence (the new token and window - 1 before it); 0 = the
                              whole sequence. split_kv 0 then picks explicit splits of the
                              window's pages. No counterpart in the reference             */
  int32_t reserved[1];     /* must be 0                                                     */
  const float* sinks;      /* attention sinks (gpt-oss style): NULL = off, else a device
                              array of num_q_heads fp32 logits; head h's softmax then has
                              one more term, exp(sinks[h]), that takes weight but has no
                              value (out = sum_i e^{s_i} v_i / (sum_i e^{s_i} + e^{sinks[h]}),
                              the scores s_i already scaled and soft-capped). Applied where
                              the output is normalised (one pass, and the merge of
                              decode_attention); dk_decode_partials' partials and
                              dk_merge_partials do not see it. No counterpart in the
                              reference                                                   */
} dk_options;

/* ABI version of the loaded library (DK_ABI_VERSION). */
int dk_abi_version(void);

/* Message for the last non-zero return on this thread ("" if none). */
const char* dk_last_error(void);

/* Bytes of fp32 scratch that dk_decode_attention needs for `split_kv`:
 *   split_kv == 1: 0 (single pass, no scratch);
 *   split_kv  > 1: partial_O (batch, Hq, split, D) + partial_m and partial_l
 *                  (batch, Hq, split), the scratch of src/cuda_/attention_ext.cu:563-568 /
 *                  src/layout.md:142-152;
 *   split_kv == 0: the partials of the balanced schedule (one per workgroup segment).
 * The workspace needs no initialisation; calls that share one must not overlap in time.
 * 0 for an invalid shape. */
size_t dk_workspace_bytes(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t split_kv);

/* Byte offsets of partial_O, partial_m and partial_l inside the workspace and its total
 * size for split_kv >= 1 (layout of src/layout.md:148-152, all fp32, C-contiguous,
 * each array 256-byte aligned). dk_decode_partials needs `total` bytes even for
 * split_kv == 1. Returns 0 or DK_EINVAL. */
int dk_partials_layout(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                       int32_t split_kv, size_t* off_o, size_t* off_m, size_t* off_l,
                       size_t* total);

/* An explicit split count (for split_kv > 1 callers) chosen from occupancy over the
 * device's compute units, for an average of `avg_pages_per_seq` pages per sequence (use
 * num_indices / batch: no device sync). split_kv == 0 needs no choice: it balances work
 * itself. No counterpart in the reference (split_kv is always caller-given there,
 * src/attention.py:32). Returns >= 1, or < 0 on a bad argument / HIP error. */
int dk_choose_split(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                    int32_t head_dim, int32_t dtype, int64_t avg_pages_per_seq,
                    int32_t device);

/* The schedule that dk_decode_attention_ex runs for these arguments on `device` (-1 =
 * current): 1 = one pass (one workgroup per (sequence, kv head), no merge), 0 = balanced
 * schedule + merge, > 1 = that explicit split + merge (with opts->window, the explicit
 * split of the window's pages that a workspace of dk_workspace_bytes(..., 0) allows; for a
 * long uniform batch over 256-byte rows, the split that fills the balanced grid). No
 * counterpart in the reference; for callers that size launches or profile the kernels.
 * Returns < 0 on a bad argument. */
int dk_plan_schedule(int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int64_t num_indices, int32_t dtype, int32_t split_kv,
                     const dk_options* opts, int32_t device);

/* decode_attention: pass 1 (split-KV partials) then pass 2 (log-sum-exp merge).
 *   split_kv == 1: one pass, one workgroup per (sequence, kv head) writing `out` directly
 *                  (no workspace needed);
 *   split_kv  > 1: the reference's partition: one workgroup per (sequence, kv head,
 *                  split) over ceil(pages/split)-page ranges, then the merge;
 *   split_kv == 0: automatic: the balanced schedule (a persistent grid of about
 *                  options.waves_per_cu wavefronts per compute unit whose workgroups each
 *                  stream an equal share of all (sequence, kv head, page) units whatever
 *                  the lengths -- for a batch the plan hint shows to be ragged, equal
 *                  shares of pages plus a charge per sequence start; sequences one
 *                  workgroup covers are written directly, the rest merged), or the
 *                  split_kv == 1 pass when options.max_pages_per_seq
 *                  shows that one workgroup per pair fits that grid and is no longer,
 *                  or (256-byte kv-head rows) that the batch is uniform and its pairs
 *                  are a whole multiple of 4 per compute unit, or that its sequences
 *                  are uniform, at most 32 pages, with CUs/4 to CUs pairs (over an
 *                  fp8 cache at D = 128: CUs/4 pairs or more; at D = 64: CUs/4 to
 *                  2 * CUs pairs, either cache) (otherwise never for kv-head rows
 *                  of <= 64 bytes, which stream faster with grouped kv heads in the
 *                  balanced schedule, nor for 128-byte rows with an even kv-head count
 *                  and sequences of more than 352 pages); or, for a uniform batch over
 *                  256-byte rows whose pairs divide the balanced grid into S >= 2
 *                  ranges of at least 1024 pages, the explicit split S
 *                  (dk_plan_schedule returns S).
 * Replaces decode_attention_split_kv_cuda (src/cuda_/attention_ext.cu:541-609) and
 * decode_attention_naive_cuda (src/cuda_/attention_ext.cu:499-539), i.e. the two
 * functions behind src/attention.py:50-58. Differences: the caller allocates `out`
 * and the workspace; any split_kv >= 0 (the reference allows 1..32); bf16; int64
 * page offsets; explicit stream. */
int dk_decode_attention(const void* q, const void* kv_data, const int32_t* kv_indptr,
                        const int32_t* kv_indices, const int32_t* kv_last_page_len,
                        void* out, void* workspace, size_t workspace_bytes,
                        int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t page_size, int64_t num_pages,
                        int64_t num_indices, int32_t dtype, const dk_strides* strides,
                        int32_t split_kv, void* hip_stream);

/* dk_decode_attention with tuning options (NULL = defaults). */
int dk_decode_attention_ex(const void* q, const void* kv_data, const int32_t* kv_indptr,
                           const int32_t* kv_indices, const int32_t* kv_last_page_len,
                           void* out, void* workspace, size_t workspace_bytes,
                           int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                           int32_t head_dim, int32_t page_size, int64_t num_pages,
                           int64_t num_indices, int32_t dtype, const dk_strides* strides,
                           int32_t split_kv, const dk_options* opts, void* hip_stream);

/* Bytes of the library's static scratch (see dk_decode_attention_noalloc). */
#define DK_STATIC_SCRATCH_BYTES (32u << 20)

/* dk_decode_attention_ex without a workspace argument: the fp32 partials go to a static
 * device array of DK_STATIC_SCRATCH_BYTES (32 MiB) that the library holds on every GPU it
 * runs on until the process ends, and the call allocates nothing (no hipMalloc / hipFree,
 * no allocating library routine). No counterpart in the reference: this is for callers
 * that cannot allocate device memory, e.g. code under HIP graph capture or serving loops
 * that forbid allocation. The caller still passes inputs and `out`. Calls on one GPU share
 * that GPU's scratch: calls that overlap in time on one GPU (different streams, or
 * graphs replayed concurrently) race and give wrong results. Nothing in the scratch needs
 * to start at zero. A call whose dk_workspace_bytes(batch, num_q_heads, num_kv_heads,
 * head_dim, split_kv) exceeds DK_STATIC_SCRATCH_BYTES returns DK_EWORKSPACE before any
 * device call (e.g. the balanced schedule, split_kv 0, at D = 128 and 4 q heads per kv
 * head fits about 1,500 sequences x 8 kv heads). */
int dk_decode_attention_noalloc(const void* q, const void* kv_data, const int32_t* kv_indptr,
                                const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                void* out, int32_t batch, int32_t num_q_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                                int64_t num_pages, int64_t num_indices, int32_t dtype,
                                const dk_strides* strides, int32_t split_kv,
                                const dk_options* opts, void* hip_stream);

/* dk_decode_attention_ex over separate K and V caches, each
 * (num_pages, page_size, num_kv_heads, head_dim) with the same strides (kv_p, kv_s, kv_h;
 * kv_r is ignored): the `(k_cache, v_cache)` form of FlashInfer's paged KV cache that
 * SGLang's token pools hand to attention backends (the pool the reference adapter
 * integration/sglang_backend.py:85-101 forwards). Both caches hold num_pages pages. */
int dk_decode_attention_kv(const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* kv_indptr, const int32_t* kv_indices,
                           const int32_t* kv_last_page_len, void* out, void* workspace,
                           size_t workspace_bytes, int32_t batch, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t page_size,
                           int64_t num_pages, int64_t num_indices, int32_t dtype,
                           const dk_strides* strides, int32_t split_kv, const dk_options* opts,
                           void* hip_stream);

/* CSR page table (kv_indptr, kv_indices, kv_last_page_len as in src/layout.md:27-138) of
 * `batch` requests from a token-slot map: request b is row req_pool_indices[b] of
 * req_to_token (rows req_stride int32 apart), holding seq_lens[b] tokens whose cache slot
 * is 16 * page + position % 16, so page p of the request is req_to_token[row][16 p] / 16.
 * This is the map SGLang's ReqToTokenPool keeps and its attention backends turn into
 * FlashInfer page tables; the reference adapter (integration/sglang_backend.py:85-101)
 * expects the caller to have built them. Writes batch + 1 indptr entries, batch last-page
 * lengths (0 for an empty request) and min(total pages, capacity) indices; size
 * kv_indices for sum(ceil(seq_lens / 16)) (at most (sum(seq_lens) + 15 * batch) / 16).
 * Device pointers; enqueued on hip_stream. No counterpart in the reference. */
int dk_build_page_table(const int32_t* req_to_token, int64_t req_stride,
                        const int32_t* req_pool_indices, const int32_t* seq_lens,
                        int32_t batch, int32_t page_size, int32_t* kv_indptr,
                        int32_t* kv_indices, int64_t capacity, int32_t* kv_last_page_len,
                        void* hip_stream);

/* The page table of a cache with pages of page_size = 16 * s tokens (FlashInfer allows any
 * page size; the reference checks page_size == 16, src/cuda_/attention_ext.cu:508,551)
 * rewritten over its 16-token sub-pages, so the decode entry points (page_size 16) read
 * the same cache in place: sub-page j < s of page id p is id p * pages_mult + j, for a
 * view of the cache whose page stride is that of a sub-page (16 token rows) and
 * pages_mult = (page stride) / (sub-page stride) (2 * s for the combined
 * (num_pages, 2, page_size, Hkv, D) cache, s for separate K / V caches). Sequence b's
 * pages kv_indices[kv_indptr[b] ..) become (pages - 1) * s + ceil(last / 16) sub-pages
 * (last = kv_last_page_len[b] clamped to [0, page_size]); its last sub-page holds the
 * last page's remainder (16 when last is 0 or a multiple of 16). Page ids outside
 * [0, num_pages) become INT32_MAX (past any pool: read as page 0, as the decode kernels
 * treat bad ids). Writes batch + 1 out_indptr entries, batch out_last_page_len entries (0
 * for a sequence without pages) and min(total sub-pages, capacity) out_indices; size
 * out_indices for num_indices * s. Device pointers; enqueued on hip_stream. No
 * counterpart in the reference. */
int dk_expand_page_table(const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* kv_last_page_len, int32_t batch, int32_t page_size,
                         int32_t pages_mult, int64_t num_pages, int64_t num_indices,
                         int32_t* out_indptr, int32_t* out_indices, int64_t capacity,
                         int32_t* out_last_page_len, void* hip_stream);

/* Cache write before a decode step: for every sequence b, the new token is the last one
 * the page table describes (page kv_indices[kv_indptr[b+1] - 1], slot
 * kv_last_page_len[b] - 1; grow the table first). Writes its K row rotated by rotary
 * position embedding and its V row there for all kv heads, and rotates q (optional, NULL
 * to skip) in place. k_new / v_new are (batch, num_kv_heads, head_dim) with element
 * strides new_b, new_h (unit head_dim stride); q and the caches use `strides` (q_b, q_h;
 * kv_p, kv_s, kv_h, and kv_r for the combined cache when v_cache is NULL). Rotation:
 * position = positions[b] (or, when positions is NULL, the token's index in its sequence),
 * angle_i = position * inv_freq[i] for i < head_dim / 2, pairs (i, i + head_dim/2) when
 * rope_style == 0 (Llama / GPT-NeoX) or (2i, 2i + 1) when 1 (GPT-J); fp32 arithmetic,
 * one rounding. inv_freq NULL: rows copied unrotated. A sequence without pages is skipped.
 * No counterpart in the reference, which has no cache write (src/layout.md:41-69 fixes
 * the format written). */
int dk_append_kv(void* q, const void* k_new, const void* v_new, int64_t new_b, int64_t new_h,
                 void* k_cache, void* v_cache, const int32_t* kv_indptr,
                 const int32_t* kv_indices, const int32_t* kv_last_page_len,
                 const int32_t* positions, const float* inv_freq, int32_t rope_style,
                 int32_t batch, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                 int32_t page_size, int64_t num_pages, int64_t num_indices, int32_t dtype,
                 const dk_strides* strides, void* hip_stream);

/* dk_append_kv into an fp8 (OCP E4M3) cache: q, k_new and v_new have type `dtype`
 * (DK_F16 / DK_BF16); each cached element is RNE(clamp(x / scale, -448, 448)) of the
 * fp32 value x (rotated K with k_scale, V with v_scale; both finite and > 0; NaN stays
 * NaN), the inverse of dk_options.k_scale / v_scale in the decode call. Cache strides in
 * elements (= bytes). No counterpart in the reference (fp16 cache only). */
int dk_append_kv_fp8(void* q, const void* k_new, const void* v_new, int64_t new_b,
                     int64_t new_h, void* k_cache, void* v_cache, const int32_t* kv_indptr,
                     const int32_t* kv_indices, const int32_t* kv_last_page_len,
                     const int32_t* positions, const float* inv_freq, int32_t rope_style,
                     int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t page_size, int64_t num_pages,
                     int64_t num_indices, int32_t dtype, float k_scale, float v_scale,
                     const dk_strides* strides, void* hip_stream);

/* Pass 1 only: writes partial_O / partial_m / partial_l for split_kv >= 1 splits into
 * the workspace (layout from dk_partials_layout; partial_m is the split's max of
 * q.k*scale, -1e9 for an empty split, partial_l = sum exp(score - partial_m),
 * partial_O = sum exp(score - partial_m) * V, unnormalised). split_kv == 0 runs the
 * balanced pass 1 into a workspace of dk_workspace_bytes(..., 0) bytes; its partials
 * (one per wavefront segment) have no public layout (this is for timing pass 1).
 * Replaces the partition launch launch_partition_hd (src/cuda_/attention_ext.cu:452-476)
 * with the semantics of decode_attn_partition_kernel (:207-349). `out`-related strides
 * are ignored. */
int dk_decode_partials(const void* q, const void* kv_data, const int32_t* kv_indptr,
                       const int32_t* kv_indices, const int32_t* kv_last_page_len,
                       void* workspace, size_t workspace_bytes,
                       int32_t batch, int32_t num_q_heads, int32_t num_kv_heads,
                       int32_t head_dim, int32_t page_size, int64_t num_pages,
                       int64_t num_indices, int32_t dtype, const dk_strides* strides,
                       int32_t split_kv, const dk_options* opts, void* hip_stream);

/* Pass 2 only: log-sum-exp merge of the workspace partials into `out`
 * (o_b, o_h element strides). Replaces launch_reduce_hd / decode_attn_reduce_kernel
 * (src/cuda_/attention_ext.cu:478-495, :363-406). A (sequence, head) whose splits are
 * all empty gets 0. */
int dk_merge_partials(const void* workspace, size_t workspace_bytes, void* out,
                      int32_t batch, int32_t num_q_heads, int32_t head_dim,
                      int32_t dtype, int64_t o_b, int64_t o_h, int32_t split_kv,
                      void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* DK_DECODE_H */
