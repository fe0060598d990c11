/*
 * dsa_abi.h - C ABI of the MI355X (gfx950) DeepSeek-sparse-attention path.
 *
 * Two operators, each a drop-in for one of the reference's PyTorch modules:
 *   Task1  sparse attention with attention sink      reference/task1_v0_ref.py:5-36
 *   Task2  lightning indexer (RoPE, score, top-k)     reference/task2_v0_ref.py:93-144
 *
 * Conventions shared by every entry point:
 *   - All pointers are device pointers (HBM) except where noted; the caller
 *     owns every buffer. The library never allocates device memory (the one
 *     exception is the static scratch array of dsa_indexer_score_topk_noalloc,
 *     created when the module loads). Its only state between calls is a
 *     per-device cache of the CU count and of the LDS limits already set per
 *     kernel, filled on first use and thread-safe; calls on different streams
 *     may run concurrently.
 *   - Tensors are dense and row-major (C-contiguous) unless a stride argument
 *     says otherwise. bf16 tensors are passed as raw 16-bit words.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Launches
 *     are asynchronous: a return value of DSA_OK means the work was enqueued.
 *   - Every entry point returns DSA_OK (0) or a negative DSA_ERR_* code;
 *     dsa_strerror() turns it into text. Shape checks run on the host before
 *     anything is launched, so an error leaves all outputs untouched.
 */
#ifndef DSA_ABI_H_
#define DSA_ABI_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_ABI_VERSION 4

#define DSA_OK 0
#define DSA_ERR_NULL (-1)        /* a required pointer is NULL */
#define DSA_ERR_SHAPE (-2)       /* sizes are negative or inconsistent */
#define DSA_ERR_UNSUPPORTED (-3) /* valid request this build does not implement */
#define DSA_ERR_LAUNCH (-4)      /* the HIP runtime rejected a launch */
#define DSA_ERR_DEVICE (-5)      /* no usable gfx950 device / attribute query failed */
#define DSA_ERR_ALIGN (-6)       /* a pointer is not 16-byte aligned */
#define DSA_ERR_SCRATCH (-7)     /* request larger than the library's static scratch buffer */

/* Task1 kernel selection (the `variant` argument of dsa_sparse_attn_fwd). */
#define DSA_SA_AUTO 0         /* multiplicity kernel when n_kv <= 32, else gather */
#define DSA_SA_MULTIPLICITY 1 /* per-token kv-index histogram, all scores of a batch's kv block */
#define DSA_SA_GATHER 2       /* gathers the topk rows of every token (any n_kv) */

/* Rounding of the RoPE complex product (the `rope_mode` arguments). */
#define DSA_ROPE_CPU 0        /* torch CPU: re = (a*c) - (b*d), im = (a*d) + (b*c), each product rounded */
#define DSA_ROPE_TORCH_ROCM 1 /* torch-ROCm broadcast mul kernel: contraction depends on the unroll slot */

int dsa_abi_version(void);
const char* dsa_strerror(int code);

/*
 * Task1: out[b,m,h,:] = sum_t softmax_t(scale * q[b,m,h,:] . kv[b,idx_t,:] ; sink_h) kv[b,idx_t,:]
 * where idx_t = topk_idxs[b,m,t] and the softmax denominator includes exp(sink_h - max).
 *
 * Replaces sparse_attn_ref (reference/task1_v0_ref.py:5-24), called from
 * Model.forward (task1_v0_ref.py:35-36); on the Ascend side the same call is
 * ModelNew.forward -> run_fused -> launch_sa_fused
 * (src/task1_sparse_attn.py:746-804,420-429; src/sparse_attn_kernel_mm.asc:310-313).
 *
 *   q          bf16 [b, m, h, d]
 *   kv         bf16 [b, n_kv, d]          shared K = V (MQA over the h heads)
 *   topk_idxs  int32 [b, m, topk]         negative = masked slot (task1_v0_ref.py:8);
 *                                         values >= n_kv are treated as masked
 *   attn_sink  fp32 [h]
 *   out        bf16 [b, m, h, d]
 *   softmax_scale  fp32 value of the reference's head_dim ** -0.5
 * Requirements: d == 128, h % 16 == 0, 1 <= n_kv, topk >= 1; the multiplicity
 * variant also needs n_kv <= 32, the gather variant h <= 128, topk <= 2048,
 * n_kv <= 2^23 and softmax_scale > 0. q/kv/out 16-byte aligned.
 */
int dsa_sparse_attn_fwd(const void* q, const void* kv, const int32_t* topk_idxs,
                        const float* attn_sink, void* out, int64_t b, int64_t m,
                        int64_t h, int64_t d, int64_t n_kv, int64_t topk,
                        float softmax_scale, int32_t variant, void* stream);

/*
 * dsa_sparse_attn_fwd with int64 topk_idxs, the dtype the indexer returns
 * (reference/task2_v0_ref.py:138-143) and sparse_attn_ref accepts as well
 * (task1_v0_ref.py:8-12 indexes with whatever integer tensor it is given). The
 * kernels read the int64 values themselves (no narrowing pass); a value outside
 * [0, n_kv), including any outside the int32 range, is a masked slot.
 */
int dsa_sparse_attn_fwd_i64(const void* q, const void* kv, const int64_t* topk_idxs,
                            const float* attn_sink, void* out, int64_t b, int64_t m,
                            int64_t h, int64_t d, int64_t n_kv, int64_t topk,
                            float softmax_scale, int32_t variant, void* stream);

/*
 * Sparse MLA: Task1 with a key wider than the value (the attention of the DSA layer,
 * configs[4]): one latent kv row is the key (its first d_qk channels) and the value
 * (its first d_v channels):
 *   out[b,m,h,:] = sum_t softmax_t(scale * q[b,m,h,:] . kv[b,idx_t,:d_qk] ; sink_h) kv[b,idx_t,:d_v]
 * Same semantics as sparse_attn_ref (reference/task1_v0_ref.py:5-24, masked slots,
 * sink in the denominator, fp32 softmax, bf16 output), whose K = V = kv is the case
 * d_v = d_qk; the reference has no separate value width, this entry point adds it.
 *
 *   q          bf16 [b, m, h, d_qk]
 *   kv         bf16 [b, n_kv, kv_dim]     rows of kv_dim >= d_qk channels
 *   topk_idxs  int32 [b, m, topk]         negative or >= n_kv = masked slot
 *   attn_sink  fp32 [h]
 *   out        bf16 [b, m, h, d_v]
 * Requirements: d_qk == 576, d_v == 512, h % 16 == 0 with 64 <= h <= 128,
 * topk <= 2048, n_kv <= 2^21, kv_dim % 8 == 0, n_kv * kv_dim * 2 <= 2^32 - 1 (a batch's
 * kv rows are addressed with 32-bit byte offsets), softmax_scale > 0; q/kv/out
 * 16-byte aligned. A -inf sink is allowed; with every slot masked and a -inf sink the
 * output is NaN, as in the reference (its denominator is exp(-inf - (-inf))).
 */
int dsa_sparse_mla_fwd(const void* q, const void* kv, const int32_t* topk_idxs,
                       const float* attn_sink, void* out, int64_t b, int64_t m, int64_t h,
                       int64_t d_qk, int64_t d_v, int64_t kv_dim, int64_t n_kv, int64_t topk,
                       float softmax_scale, void* stream);

/*
 * dsa_sparse_mla_fwd with int64 topk_idxs: the indexer's output (reference/
 * task2_v0_ref.py:138-143, -1 for masked picks) fed to the attention as it is.
 * Values outside [0, n_kv) are masked slots.
 */
int dsa_sparse_mla_fwd_i64(const void* q, const void* kv, const int64_t* topk_idxs,
                           const float* attn_sink, void* out, int64_t b, int64_t m, int64_t h,
                           int64_t d_qk, int64_t d_v, int64_t kv_dim, int64_t n_kv, int64_t topk,
                           float softmax_scale, void* stream);

/*
 * Workspace bytes for dsa_sparse_mla_fwd_ws / _i64_ws: with fewer tokens (b * m)
 * than CUs (decode), each token's slot list is split among several workgroups
 * whose fp32 partial results go to the workspace and are merged by a second
 * kernel. Returns 0 when no split applies (then the _ws calls run the one-pass
 * kernel and need no workspace, also for b * m == 0), DSA_ERR_SHAPE for invalid
 * sizes and DSA_ERR_DEVICE when the device cannot be queried (a negative value is
 * never a size).
 * Same computation as sparse_attn_ref (reference/task1_v0_ref.py:5-24) with
 * v_dim 512; the split changes only the fp32 summation order of the softmax sums.
 */
int64_t dsa_sparse_mla_workspace_bytes(int64_t b, int64_t m, int64_t h, int64_t topk);

/*
 * dsa_sparse_mla_fwd (int32 topk_idxs) / dsa_sparse_mla_fwd_i64 (int64) with a
 * caller-provided device workspace (16-byte aligned) of workspace_bytes: when
 * workspace_bytes >= dsa_sparse_mla_workspace_bytes(b, m, h, topk) > 0 the slot
 * list is split as described there; otherwise the one-pass kernel runs. The
 * workspace may be reused by calls on one stream; calls that overlap on different
 * streams need their own.
 */
int dsa_sparse_mla_fwd_ws(const void* q, const void* kv, const int32_t* topk_idxs,
                          const float* attn_sink, void* out, int64_t b, int64_t m, int64_t h,
                          int64_t d_qk, int64_t d_v, int64_t kv_dim, int64_t n_kv, int64_t topk,
                          float softmax_scale, void* workspace, int64_t workspace_bytes,
                          void* stream);
int dsa_sparse_mla_fwd_i64_ws(const void* q, const void* kv, const int64_t* topk_idxs,
                              const float* attn_sink, void* out, int64_t b, int64_t m, int64_t h,
                              int64_t d_qk, int64_t d_v, int64_t kv_dim, int64_t n_kv,
                              int64_t topk, float softmax_scale, void* workspace,
                              int64_t workspace_bytes, void* stream);

/*
 * Task2 RoPE, in place on the last `rd` channels of every head of q.
 * Replaces apply_rotary_emb(q[..., -rd:], freqs_cis) (reference/task2_v0_ref.py:93-104,131)
 * and the Ascend ix_rope launch (src/indexer_kernel_aiv.asc:19-111; src/task2_indexer.py:1117-1130).
 *
 *   q          bf16 [b, s, h, d], rotated channels are q[..., d-rd:] taken as (re, im) pairs
 *   freqs_cis  complex64 [s, rd/2] as interleaved fp32 (re, im); row t is position start_pos + t,
 *              i.e. the caller passes &freqs_cis[start_pos]
 *   rope_mode  DSA_ROPE_CPU or DSA_ROPE_TORCH_ROCM (which torch rounding to reproduce)
 * Requirements: rd even, 0 < rd <= d, d % 8 == 0.
 */
int dsa_indexer_rope(void* q, const void* freqs_cis, int64_t b, int64_t s, int64_t h,
                     int64_t d, int64_t rd, int32_t rope_mode, void* stream);

/*
 * Task2 score + mask + top-k (the body of Model.forward after the two
 * projections; reference/task2_v0_ref.py:131-143):
 *   w[b,t,h]      = bf16(fp32(wl[b,t,h]) * w_scale)                          (:132)
 *   S[b,t,h,k]    = bf16(q[b,t,h,:] . kv_cache[b,k,:])   fp32 accumulate      (:133)
 *   score[b,t,k]  = bf16( sum_h bf16(relu(S) * w) )      fp32, torch order    (:134)
 *   causal: score[b,t,k] = -inf for k >= (t+1)//ratio                         (:135-137)
 *   out[b,t,:]    = indices of the k_out largest scores, value desc / index asc (:138)
 *   causal: out = -1 where idx >= (t+1)//ratio, else idx + offset; non-causal: idx + offset (:139-143)
 * Replaces the Ascend fused score/top-k kernel launch_ix_fused
 * (src/indexer_kernel_mm.asc:421-436; src/task2_indexer.py:1338-1339).
 *
 *   q          bf16 [b, s, h, d]  projected queries (F.linear output). If `freqs_cis` is
 *              not NULL the RoPE above is applied on the fly (q itself is not written),
 *              which is equivalent to calling dsa_indexer_rope first.
 *   kv_cache   bf16, row k of batch i at kv_cache + i*kv_batch_stride + k*d (elements)
 *   wl         bf16 [b, s, h]      unscaled weights_proj output
 *   out        int64 [b, s, k_out]
 *   n_cand     number of candidate keys T = end_pos // ratio
 *   causal     1 when start_pos == 0 (mask and -1 fill), else 0
 * Requirements: rd as for dsa_indexer_rope (when freqs_cis != NULL), ratio >= 1,
 * 1 <= k_out <= n_cand, and one of
 *   h == 16, d == 64:   n_cand <= 2048, k_out <= 256                (configs[2])
 *   h == 64, d == 128:  n_cand <= 8192, k_out <= 2048 (configs[4]; the 64-head sum is
 *                       added in the order torch-ROCm's reduction uses for b*s*n_cand
 *                       outputs of n_cand candidates: over 1, 2 or 4 threads)
 */
int dsa_indexer_score_topk(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                           const void* wl, float w_scale, const void* freqs_cis,
                           int32_t rope_mode, int64_t* out, int64_t b, int64_t s,
                           int64_t h, int64_t d, int64_t rd, int64_t n_cand, int64_t k_out,
                           int64_t ratio, int32_t causal, int64_t offset, void* stream);

/*
 * Workspace for dsa_indexer_score_topk_ws, in bytes (0: the configuration needs none;
 * DSA_ERR_SHAPE: invalid sizes). For h == 64, d == 128 it is b * s * round_up(n_cand, 4) * 2
 * (one 16-bit order key per token and candidate, rows padded to 8 bytes).
 */
int64_t dsa_indexer_workspace_bytes(int64_t b, int64_t s, int64_t h, int64_t d, int64_t n_cand);

/*
 * dsa_indexer_score_topk with a caller-provided device workspace (16-byte aligned,
 * workspace_bytes as given by dsa_indexer_workspace_bytes). Same results. For
 * h == 64, d == 128 the scores go to the workspace and a second kernel ranks each
 * token's row (faster than the single kernel, which keeps four tokens' keys in LDS);
 * with a smaller or NULL workspace it behaves as dsa_indexer_score_topk. The
 * workspace content is scratch: not read before it is written, not needed afterwards.
 * Replaces the same reference call as dsa_indexer_score_topk (task2_v0_ref.py:131-143).
 */
int dsa_indexer_score_topk_ws(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                              const void* wl, float w_scale, const void* freqs_cis,
                              int32_t rope_mode, int64_t* out, int64_t b, int64_t s,
                              int64_t h, int64_t d, int64_t rd, int64_t n_cand, int64_t k_out,
                              int64_t ratio, int32_t causal, int64_t offset, void* workspace,
                              int64_t workspace_bytes, void* stream);

/*
 * dsa_indexer_score_topk_ws without a caller workspace and without any allocation:
 * the workspace is a static device array of DSA_INDEXER_NOALLOC_MAX_BYTES inside the
 * library (one per device, held from module load until the process ends). Same
 * arguments and results as dsa_indexer_score_topk. Returns DSA_ERR_SCRATCH when
 * dsa_indexer_workspace_bytes(b, s, h, d, n_cand) exceeds that size (64 heads x 128:
 * b * s * round_up(n_cand, 4) <= 8,388,608, e.g. 1024 tokens at 8192 candidates); configurations
 * that need no workspace (16 heads x 64) run as dsa_indexer_score_topk. Calls on one
 * device share the array, so calls that overlap on one device (different streams)
 * race; calls ordered on one stream do not. No hipMalloc/hipFree or other allocating
 * call is made, so it can be used where the caller cannot allocate (inside HIP graph
 * capture, allocation-free serving loops).
 * No counterpart in the reference: an addition for callers that cannot allocate;
 * it computes what dsa_indexer_score_topk does.
 */
#define DSA_INDEXER_NOALLOC_MAX_BYTES (INT64_C(16) << 20)
int dsa_indexer_score_topk_noalloc(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                                   const void* wl, float w_scale, const void* freqs_cis,
                                   int32_t rope_mode, int64_t* out, int64_t b, int64_t s,
                                   int64_t h, int64_t d, int64_t rd, int64_t n_cand,
                                   int64_t k_out, int64_t ratio, int32_t causal, int64_t offset,
                                   void* stream);

/*
 * Task2 score stage alone: writes the bf16 index_score [b, s, n_cand] that the reference
 * hands to topk (reference/task2_v0_ref.py:131-137), with masked entries = -inf in the
 * causal case. Same arguments and requirements as dsa_indexer_score_topk (and, for
 * h == 64, n_cand >= 2: torch reduces a single candidate's heads in another order);
 * `scores` is a device buffer of b*s*n_cand bf16 words. Used to check the rounding chain stage by stage
 * and by callers that want the scores themselves.
 */
int dsa_indexer_scores(const void* q, const void* kv_cache, int64_t kv_batch_stride,
                       const void* wl, float w_scale, const void* freqs_cis, int32_t rope_mode,
                       void* scores, int64_t b, int64_t s, int64_t h, int64_t d, int64_t rd,
                       int64_t n_cand, int64_t ratio, int32_t causal, void* stream);

/*
 * Task2 query projection with RoPE: q = qr . wq^T (the F.linear of the indexer's wq_b,
 * reference/task2_v0_ref.py:129-130 through Linear.forward :81-83) followed by
 * apply_rotary_emb on the last rd channels of every head (:131, :93-104), as one kernel.
 * The product accumulates in fp32 over k in ascending order and rounds once to bf16,
 * which equals torch-ROCm's F.linear at the indexer's shapes for the token counts its
 * GPU test covers (not for every small m: hipBLASLt reduces those in another order).
 *
 *   qr         bf16 [m, k]        m = b * s_len token rows
 *   wq         bf16 [n, k]        n = heads * head_dim
 *   freqs_cis  complex64 [s_len, rd/2] rows of positions start_pos .. (16-byte aligned), or
 *              NULL for no RoPE
 *   rope_mode  DSA_ROPE_TORCH_ROCM or DSA_ROPE_CPU, the rounding rule of the rotation (as for
 *              dsa_indexer_score_topk)
 *   q          bf16 [m, n] output
 * Requirements: k % 32 == 0, n % 256 == 0, head_dim in {64, 128}, (head_dim - rd) % 8 == 0,
 * m * k * 2 and n * k * 2 below 2^32, m % s_len == 0; pointers 16-byte aligned.
 * The drop-in Model uses it for q_lora_rank 256 and rd 32 from 64 tokens (configs[2]:
 * ~19 us against ~26 us for hipBLASLt's F.linear alone) and keeps F.linear + the score
 * kernel's own RoPE below 64 tokens and for other k.
 */
int dsa_indexer_q_proj(const void* qr, const void* wq, const void* freqs_cis, int32_t rope_mode,
                       void* q, int64_t m, int64_t n, int64_t k, int64_t head_dim, int64_t rd,
                       int64_t s_len, void* stream);

/*
 * Fragment packing of the indexer's projection weights for dsa_indexer_projections: a
 * permutation of the same bytes into the order the kernel's registers take them, done
 * once per weight version (the Ascend submission prepares its matmul executors once the
 * same way, src/task2_indexer.py:764-804 prepare_c2).
 *   wq           bf16 [n, k]      wq_b.weight (reference/task2_v0_ref.py:116), k == 256, n % 64 == 0
 *   wproj        bf16 [n_w, dim]  weights_proj.weight (:117), n_w % 16 == 0, dim % 32 == 0
 *   wq_packed    n * k bf16 words; wproj_packed n_w * dim bf16 words
 * Either pair (wq, wq_packed) or (wproj, wproj_packed) may be NULL, NULL. Pointers 16-byte
 * aligned. Layouts: wq_packed fragment f = ((r * 2 + i) * 16 + ks) * 64 + lane (16 bytes)
 * holds wq[64 r + 32 i + lane % 32][16 ks + 8 (lane / 32) .. + 7]; wproj_packed fragment
 * e = (hg * (dim / 32) + ks) * 64 + lane holds wproj[16 hg + lane % 16][32 ks + 8 (lane / 16) .. + 7].
 */
int dsa_indexer_pack_projection_weights(const void* wq, int64_t n, int64_t k, const void* wproj,
                                        int64_t n_w, int64_t dim, void* wq_packed,
                                        void* wproj_packed, void* stream);

/*
 * Both projections of the indexer in one launch (reference/task2_v0_ref.py:129-132):
 *   q  = apply_rotary_emb(qr . wq^T)  on the last rd channels of every head   (:129-131)
 *   wl = x . wproj^T                                                       (:132, before the scale)
 * Replaces the two F.linear calls and the RoPE; the Ascend submission runs weights_proj on a
 * second stream beside the query path (src/task2_indexer.py:805-839 go_c2_ovl, :871-879
 * go_t2); here both run in one grid, with no stream or event calls. Both products
 * accumulate in fp32 over k in ascending order and round once to bf16; RoPE as in
 * dsa_indexer_q_proj. That equals torch-ROCm's F.linear where hipBLASLt runs a kernel
 * without split-k: for wq (k = 256) from 17 tokens up, for weights_proj (k = 1024, 16
 * outputs) only from about 15,400 tokens (below, hipBLASLt sums k over 4 wave groups, which
 * changes ~1.7e-4 of the outputs);
 * the drop-in Model calls this entry point only inside the token range its GPU sweep covers.
 *
 *   qr            bf16 [m, k]      m = b * s_len token rows, k == 256
 *   wq_packed     from dsa_indexer_pack_projection_weights, n = heads * head_dim, n % 256 == 0
 *   freqs_cis     complex64 [s_len, rd/2] rows of positions start_pos .. (16-byte aligned), or NULL
 *   rope_mode     DSA_ROPE_TORCH_ROCM or DSA_ROPE_CPU
 *   q             bf16 [m, n] output (RoPE applied)
 *   x             bf16 [m, dim], dim == 1024
 *   wproj_packed  from dsa_indexer_pack_projection_weights, n_w == 16
 *   wl            bf16 [m, n_w] output (8-byte aligned)
 * Requirements: head_dim == 64, rd == 32 when freqs_cis != NULL, m % s_len == 0,
 * m * n * 2 and m * dim * 2 below 2^32; pointers 16-byte aligned unless stated.
 */
int dsa_indexer_projections(const void* qr, const void* wq_packed, const void* freqs_cis,
                            int32_t rope_mode, void* q, const void* x, const void* wproj_packed,
                            void* wl, int64_t m, int64_t n, int64_t k, int64_t dim, int64_t n_w,
                            int64_t head_dim, int64_t rd, int64_t s_len, void* stream);

/*
 * The indexer's two projections for a few tokens (decode), in one launch, without RoPE
 * (the score kernel applies it): the F.linear calls of reference/task2_v0_ref.py:129
 * (q = qr . wq^T) and :132 (wl = x . wproj^T), Linear.forward :81-83. At the DeepSeek-V3.2
 * sizes (q_lora_rank 1536, dim 7168) and 1..16 tokens, torch-ROCm's hipBLASLt splits k
 * over 4 waves: in every depth block of 128 (q) or 512 (wl), chain c accumulates the
 * c-th quarter in fp32 in ascending k over all blocks, and the four chains are summed as
 * ((c0 + c1) + c2) + c3 and rounded once to bf16. This entry point computes exactly that
 * sum (bit-equal to F.linear on the build the drop-in Model gates it on).
 *   qr     bf16 [m, k_q], k_q == 1536          wq     bf16 [n_q, k_q] (wq_b.weight), n_q % 64 == 0
 *   x      bf16 [m, k_w], k_w == 7168          wproj  bf16 [n_w, k_w] (weights_proj.weight), n_w % 16 == 0
 *   q      bf16 [m, n_q] output                wl     bf16 [m, n_w] output (both 2-byte aligned)
 * 0 <= m <= 16, n_q % 64 == 0; inputs 16-byte aligned, rows contiguous.
 */
int dsa_indexer_decode_projections(const void* qr, const void* wq, const void* x, const void* wproj,
                                   void* q, void* wl, int64_t m, int64_t n_q, int64_t k_q, int64_t n_w,
                                   int64_t k_w, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_ABI_H_ */
