/*
 * lik.h — C ABI of the MI355X (gfx950) MaxSim engine, liblik_hip.so.
 *
 * Every entry point takes raw device pointers, element strides and scalars,
 * launches on the caller's HIP stream, performs no device allocation and no
 * host synchronisation, and returns a status code (LIK_OK == 0, negative on
 * error). Scratch memory, where an entry point needs it, is passed in by the
 * caller; its size comes from the matching *_workspace_size() query. The
 * library keeps no mutable state between calls and reads no environment
 * variables, so every entry point is reentrant; tuning and timing choices
 * travel with the call (lik_launch_opts_t, the *_ex entry points).
 *
 * The reference library (late-interaction-kernels v0.4.5) has no native ABI:
 * its "FFI" is Triton's Python launcher. Each declaration below names the
 * reference launcher whose behaviour it replaces. The Python binding that
 * calls these through ctypes lives in late_interaction_kernels/_lib.py.
 */
#ifndef LIK_H_
#define LIK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* lik_stream_t; /* == hipStream_t */

enum {
  LIK_OK = 0,
  LIK_ERR_INVALID = -1,     /* bad shape / pointer / argument */
  LIK_ERR_UNSUPPORTED = -2, /* shape or dtype outside what the kernels handle */
  LIK_ERR_WORKSPACE = -3,   /* workspace missing or too small */
  LIK_ERR_LAUNCH = -4       /* hipLaunchKernel / hipGetLastError failure */
};

typedef enum {
  LIK_BF16 = 0,
  LIK_F16 = 1,
  LIK_F32 = 2,
  LIK_FP8_E4M3 = 3 /* OCP e4m3fn, torch.float8_e4m3fn */
} lik_dtype_t;

/*
 * A batch of token sequences, either padded or packed:
 *   padded: sequence i, token t at  data + i*stride_n + t*stride_l   (elements)
 *   packed: cu_seqlens != NULL; token t of sequence i at
 *           data + (cu_seqlens[i] + t)*stride_l, length cu_seqlens[i+1]-cu_seqlens[i]
 * The embedding dim is contiguous (stride 1) and each token row starts on a
 * 16-byte boundary; dim*elem_size is a multiple of 16.
 * lengths (optional, padded only): valid length of each sequence (prefix).
 * mask (optional, padded only): int8 keep-flags, mask[i*mask_stride_n + t*mask_stride_l].
 * token_scale (optional, fp8 only): fp32 per-token dequant scale,
 *           token_scale[i*scale_stride_n + t*scale_stride_l]. With both
 *           strides 0 it is one per-tensor scale in device memory, folded
 *           into the score scale in the kernel's epilogue (no host read, so
 *           the call can be captured in a HIP graph).
 */
typedef struct {
  const void* data;
  int32_t dtype;      /* lik_dtype_t */
  int32_t dim;        /* embedding dim d */
  int64_t n;          /* number of sequences */
  int64_t len;        /* padded length (max length for packed input) */
  int64_t stride_n;
  int64_t stride_l;
  const int32_t* cu_seqlens;
  const int32_t* lengths;
  const int8_t* mask;
  int64_t mask_stride_n;
  int64_t mask_stride_l;
  const float* token_scale;
  int64_t scale_stride_n;
  int64_t scale_stride_l;
} lik_seqs_t;

/*
 * Per-call launch options (no counterpart in the reference, whose Triton
 * launcher autotunes and times from Python). Passing NULL, or a zeroed
 * struct, is exactly the plain entry point. The struct is read during the
 * call only; the library keeps no state between calls, so concurrent calls
 * with different options are independent.
 *   col_waves, col_blocks: force the tile kernel's column block (waves per
 *       workgroup W in {1, 4, 8}, 32-column blocks per wave NSUB in
 *       {1, 2, 4}; fp8 at d <= 128 also 4 x 6); 0 = automatic. A
 *       configuration the call cannot use is ignored. Calls whose query
 *       group fits one 32-column block otherwise run a streaming
 *       one-block kernel; a forced block of 4 or 8 waves keeps them on
 *       the tile kernel.
 *   docs_per_wg: documents per workgroup of the tile kernel, 1..512;
 *       0 = automatic (the streaming kernel picks its own).
 *   plaid_variant (lik_plaid_maxsim_ex): 0 automatic, 1 per-lane stream
 *       decode, 2 exact LDS-gather decode (bitwise equal to the tile
 *       kernel), 3 the tile kernel (no stream kernel). lik_plaid_maxsim_qc:
 *       0 automatic, 5 the LDS-staged scan (two queries per wavefront when
 *       there are several) instead of the register-direct one (the automatic
 *       choice for 2-bit residuals and for 4-bit residuals at d <= 64: one
 *       query per wavefront, two with LIK_TOKEN_RECORDS).
 *   timing_start, timing_stop: hipEvent_t or NULL. When both are set, the
 *       call's MaxSim scoring launches carry them in their own dispatches
 *       (hipExtLaunchKernel): timing_start records the start of the first
 *       scoring kernel, timing_stop the end of the last one. That spans both
 *       launches of a doc mask that has holes (the mask-free documents, then
 *       those with holes) but none of the pre-passes (mask summary, row
 *       norms, query-chunk sums), so a caller can time the scoring kernels
 *       alone; no event packet is queued between launches, so a timed call
 *       runs as an untimed one does. A call that launches no scoring kernel
 *       records both events back to back (zero duration).
 */
typedef struct {
  int32_t col_waves;
  int32_t col_blocks;
  int32_t docs_per_wg;
  int32_t plaid_variant;
  void* timing_start;
  void* timing_stop;
} lik_launch_opts_t;

/* flags for lik_maxsim */
#define LIK_NORMALIZE 1u /* per-token L2 normalise Q and D (F.normalize, eps 1e-12) */
#define LIK_KD_LAYOUT 2u /* D holds n = Nq*K docs; query i scores docs [i*K, (i+1)*K) */
#define LIK_NORMALIZE_Q 4u /* normalise query tokens only (docs already unit rows, e.g. decoded PLAID) */
#define LIK_NORMALIZE_D 8u /* normalise doc tokens only (queries pre-normalised, e.g. a projection head) */
#define LIK_BIAS_16 16u /* lik_maxsim_from_hidden: bias holds d_out values of Q's 16-bit dtype, not fp32 */
#define LIK_TOKEN_RECORDS 32u /* lik_plaid_maxsim_qc: token_inv points at lik_plaid_token_t records */

/*
 * score[i, j] = out_scale * sum_{s valid in Q_i} max_{t valid in D_j} <Q_i[s], D_j[t]>
 * with a row whose max ranges over no valid token contributing 0.
 * Cross-product layout: out is [Q->n, D->n]; KD layout: out is [Q->n, D->n / Q->n].
 * out[i*out_stride_q + j*out_stride_d], fp32.
 *
 * Replaces forward.py:_run_forward (forward.py:228-346) launching
 * _maxsim_fwd_kernel (forward.py:45-186) — both the in-batch and the
 * kd_layout variants — varlen.py:_varlen_forward (varlen.py:271-364) and
 * fp8.py:maxsim_inference_fp8's launch of _maxsim_fp8_fwd_kernel
 * (fp8.py:234-422; Q and D fp8, per-tensor scales as token_scale with
 * strides 0 or as out_scale, per-token scales as token_scale).
 */
int lik_maxsim(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale,
               float* out, int64_t out_stride_q, int64_t out_stride_d, void* workspace,
               size_t workspace_bytes, lik_stream_t stream);
size_t lik_maxsim_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags);

/*
 * Training forward: lik_maxsim (out_scale 1) that also writes, for every
 * (query i, doc j, query token s), the index of the doc token that wins the
 * max: argmax[(i * docs + j) * Q->len + s], docs = D->n (cross product) or
 * D->n / Q->n (LIK_KD_LAYOUT); ties go to the lowest doc-token index, and -1
 * marks a row with no valid doc token (it contributes 0). bf16 / f16 / f32
 * padded or packed docs; same masks, flags and workspace as lik_maxsim.
 * Replaces forward.py:_run_forward with save_argmax=True
 * (forward.py:160-182, autograd.py:169-181).
 */
int lik_maxsim_argmax(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float* out,
                      int64_t out_stride_q, int64_t out_stride_d, int32_t* argmax, void* workspace,
                      size_t workspace_bytes, lik_stream_t stream);

/*
 * MaxSim against docs given as hidden states through a linear head, without
 * forming the projected docs: D[j, t] = H[j, t] @ W^T + b, each row L2
 * normalised (x / max(||x||, 1e-12)) with LIK_NORMALIZE_D, rounded to the
 * input dtype, then score[i, j] as lik_maxsim (cross product, out_scale 1).
 * Q: padded [Q->n, Q->len, d_out], already projected (and normalised by the
 * caller if wanted), no mask. H: padded [H->n, H->len, d_model] with its mask
 * and lengths marking the doc tokens that can win. W: [d_out, d_model] with
 * row stride w_stride elements; bias: fp32 [d_out], or with flag LIK_BIAS_16
 * [d_out] in the Q / H dtype (widened to fp32 in the kernel, so the caller
 * needs no conversion pass), or NULL. bf16 / f16 (Q, H
 * and W in one dtype); d_out <= 128; Q->n * Q->len <= 256; d_model, the H
 * strides and w_stride multiples of 8; H and W 16-byte aligned (other shapes:
 * LIK_ERR_UNSUPPORTED, and the caller projects first). argmax (optional)
 * as lik_maxsim_argmax: [(i * H->n + j) * Q->len + s], -1 for no valid token.
 * Workspace: lik_maxsim_from_hidden_workspace_size() bytes.
 * Replaces fused_head.py:_fused_head_forward (fused_head.py:192-259)
 * launching _fused_head_fwd_kernel (fused_head.py:46-189).
 */
int lik_maxsim_from_hidden(const lik_seqs_t* Q, const lik_seqs_t* H, const void* W, int64_t w_stride,
                           const void* bias, uint32_t flags, float* out, int64_t out_stride_q,
                           int64_t out_stride_d, int32_t* argmax, void* workspace, size_t workspace_bytes,
                           lik_stream_t stream);
size_t lik_maxsim_from_hidden_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* H);

/*
 * Backward: given grad[i * grad_ld + j] = dL/dscore[i, j] (fp32) and the
 * argmax of lik_maxsim_argmax, writes grad_q [Q->n, Q->len, dim] and grad_d
 * [D->n, D->len, dim], contiguous, in the dtype of Q and D (accumulated in
 * fp32; every element written, rows that win nothing get 0). grad_d may be
 * null (only grad_q is computed). Either side may be packed (cu_seqlens,
 * ->len = longest sequence): its gradient is then [rows, dim] indexed like
 * the packed input, and only rows cu[0] .. cu[n] are written. Q->mask (keep
 * flags) zeroes the masked query tokens' terms; doc masks / lengths act only
 * through the argmax. A packed side cannot be normalised here. With
 * LIK_NORMALIZE (both sides), LIK_NORMALIZE_Q or LIK_NORMALIZE_D the
 * gradients are taken through x / max(||x||, 1e-12) on those sides. The
 * caller passes lik_maxsim_backward_workspace_size() bytes of workspace
 * (inverse norms, the partial grad_q rows when few query tokens split their
 * docs over several wavefronts, the sorted winner entries when many query
 * tokens share each doc; may be 0).
 * Deterministic: fixed summation order, no atomics.
 * Replaces backward/unified.py:maxsim_backward_unified and
 * backward/lowmem.py:maxsim_backward_lowmem (+ the normalise Jacobian of
 * autograd.py:211-225), and varlen.py:143-263 for packed inputs.
 */
int lik_maxsim_backward(const float* grad, int64_t grad_ld, const lik_seqs_t* Q, const lik_seqs_t* D,
                        const int32_t* argmax, uint32_t flags, void* grad_q, void* grad_d, void* workspace,
                        size_t workspace_bytes, lik_stream_t stream);
size_t lik_maxsim_backward_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags);

/*
 * Pair-list scoring: out[p] = MaxSim(Q_{pair_q[p]}, D_{pair_d[p]}).
 * Replaces score_pairs.py:_scatter_forward / _scatter_fwd_kernel
 * (score_pairs.py:33, launcher score_pairs.py:318).
 */
int lik_maxsim_pairs(const lik_seqs_t* Q, const lik_seqs_t* D, const int32_t* pair_q,
                     const int32_t* pair_d, int64_t num_pairs, uint32_t flags, float* out,
                     lik_stream_t stream);

/*
 * Training forward of pair-list scoring: lik_maxsim_pairs that also writes
 * argmax[p * Q->len + s] (winning doc-token index of query token s in pair
 * p, ties to the lowest index, -1 where the pair has no valid doc token).
 * bf16 / f16 / f32. Replaces score_pairs.py:_scatter_forward(save_argmax=True).
 */
int lik_maxsim_pairs_argmax(const lik_seqs_t* Q, const lik_seqs_t* D, const int32_t* pair_q,
                            const int32_t* pair_d, int64_t num_pairs, uint32_t flags, float* out,
                            int32_t* argmax, lik_stream_t stream);

/*
 * Backward of pair-list scoring: grad[p] = dL/dout[p] (fp32) and the argmax
 * of lik_maxsim_pairs_argmax give grad_q and grad_d laid out like Q and D
 * (padded [n, len, dim] or packed [rows, dim], contiguous, input dtype;
 * grad_d may be null). Pairs with an out-of-range index contribute nothing.
 * No normalise, no KD flag. Needs lik_maxsim_pairs_backward_workspace_size()
 * bytes of workspace (each query's and each doc's pair list, built on the
 * device with a stable radix sort). Deterministic, no atomics.
 * Replaces score_pairs.py:344-420 (_MaxSimScorePairsFn.backward and its
 * grad kernels).
 */
int lik_maxsim_pairs_backward(const float* grad, const lik_seqs_t* Q, const lik_seqs_t* D,
                              const int32_t* pair_q, const int32_t* pair_d, int64_t num_pairs,
                              const int32_t* argmax, uint32_t flags, void* grad_q, void* grad_d,
                              void* workspace, size_t workspace_bytes, lik_stream_t stream);
size_t lik_maxsim_pairs_backward_workspace_size(const lik_seqs_t* Q, const lik_seqs_t* D, int64_t num_pairs);

/*
 * PLAID compressed documents: token t of doc j has centroid code
 * codes[tok] and packed residual bytes residuals[tok*res_stride + 0..packed_dim),
 * tok = cu_seqlens[j] + t (packed) or j*codes_stride_n + t (padded, with
 * lengths[j] valid tokens). Decoded token:
 *   emb[f] = centroids[code*cent_stride + f]
 *          + bucket_weights[(byte[f / (8/nbits)] >> ((f % (8/nbits))*nbits)) & (2^nbits-1)]
 */
typedef struct {
  const int32_t* codes;
  const uint8_t* residuals;
  const int32_t* cu_seqlens; /* packed layout */
  const int32_t* lengths;    /* padded layout: [n] valid lengths */
  int64_t n;                 /* number of docs */
  int64_t max_len;           /* padded length / max doc length */
  int64_t codes_stride_n;    /* padded: codes row stride (tokens) */
  int64_t res_stride_tok;    /* bytes between consecutive tokens' residuals */
  const void* centroids;
  int32_t centroid_dtype; /* LIK_BF16 / LIK_F16 / LIK_F32 */
  int32_t dim;
  int64_t n_centroids;
  int64_t cent_stride; /* elements between centroid rows */
  const float* bucket_weights;
  int32_t n_buckets;
  int32_t nbits; /* 2, 4 or 8 */
} lik_plaid_docs_t;

/*
 * Fused PLAID decode + L2-normalise + MaxSim. out[i*out_stride_q + j*out_stride_d].
 * Replaces plaid.py:_maxsim_residual_forward (plaid.py:404-516, kernel
 * plaid.py:144-300) and plaid.py:maxsim_residual_varlen's launch of
 * _maxsim_residual_varlen_kernel (plaid.py:832-963, kernel plaid.py:684-829).
 */
int lik_plaid_maxsim(const lik_seqs_t* Q, const lik_plaid_docs_t* docs, uint32_t flags, float* out,
                     int64_t out_stride_q, int64_t out_stride_d, lik_stream_t stream);

/*
 * Decode PLAID tokens [tok_begin, tok_end) of `docs`, indexed flat
 * (codes[tok], residuals[tok*res_stride_tok ...]; cu_seqlens / lengths are
 * not used), into rows of out_dtype (LIK_BF16 / LIK_F16):
 * out[(tok - tok_begin)*out_stride + f], L2-normalised per token when flags
 * has LIK_NORMALIZE. The rows are bitwise the ones lik_plaid_maxsim stages
 * in LDS, so decode + lik_maxsim(..., LIK_NORMALIZE_Q) scores exactly like
 * the fused call; that route decodes each doc once instead of once per
 * query block, which wins when many queries share the corpus.
 * Replaces the decode step of plaid.py:_maxsim_residual_varlen_kernel
 * (plaid.py:780-801) and reference.py:124-139,164-167.
 */
int lik_plaid_decode(const lik_plaid_docs_t* docs, int64_t tok_begin, int64_t tok_end, uint32_t flags,
                     int32_t out_dtype, void* out, int64_t out_stride, lik_stream_t stream);

/*
 * Per-token inverse norms of decoded PLAID tokens: inv[tok] =
 * 1 / max(||x_tok||, 1e-12) with x = centroids[code] + bucket weights (fp32,
 * the decode arithmetic of lik_plaid_decode) for tok in [tok_begin,
 * tok_end); inv is indexed by absolute token. Computed once per corpus, it
 * lets lik_plaid_maxsim_qc score normalised tokens without their centroid
 * rows. No counterpart in the reference (its kernels re-decode every token
 * per query, plaid.py:780-801).
 */
int lik_plaid_token_norms(const lik_plaid_docs_t* docs, int64_t tok_begin, int64_t tok_end, float* inv,
                          lik_stream_t stream);

/*
 * A prepared token: its code (docs->codes[tok], as stored) and its inverse
 * norm (as lik_plaid_token_norms computes it). 8 bytes, 8-byte aligned.
 */
typedef struct {
  int32_t code;
  float inv;
} lik_plaid_token_t;

/*
 * The records of tokens [tok_begin, tok_end) (rec indexed by absolute token,
 * 8-byte aligned). With LIK_TOKEN_RECORDS, lik_plaid_maxsim_qc reads a
 * token's code and norm from its record with one load instead of two (the
 * scan is bound by its load instructions; the bytes read are the same). No
 * counterpart in the reference (as lik_plaid_token_norms).
 */
int lik_plaid_token_records(const lik_plaid_docs_t* docs, int64_t tok_begin, int64_t tok_end, lik_plaid_token_t* rec,
                            lik_stream_t stream);

/*
 * Few-query PLAID scoring from centroid scores (up to 64 queries of <= 32
 * tokens, bf16 / f16 query and centroids of the same type, d <= 128): the
 * same scores as lik_plaid_maxsim (plaid.py:832-963; within bf16 rounding:
 * q.c comes from an fp16 table of query-centroid scores, q.r from the MFMA
 * on bucket weights rounded to the query type, both divided by the token's
 * precomputed norm). token_inv (from lik_plaid_token_norms) is required when
 * flags normalise the docs (LIK_NORMALIZE / LIK_NORMALIZE_D) and ignored
 * otherwise; with LIK_TOKEN_RECORDS it is required and points at the
 * lik_plaid_token_t records of every token (lik_plaid_token_records, from
 * the same docs), which then supply the codes as well as the norms. Docs must be packed (docs->cu_seqlens; a lengths-only layout
 * returns LIK_ERR_UNSUPPORTED). The workspace holds the [Q->n, n_centroids,
 * 32] fp16 table (lik_plaid_maxsim_qc_workspace_size bytes): the caller
 * keeps |q.c| below fp16's 65504 (the Python layer routes larger query or
 * centroid norms to lik_plaid_maxsim). Q->len == 0 writes zero scores. opts:
 * docs_per_wg, plaid_variant and the timing events (around the scan kernel)
 * are honoured.
 */
size_t lik_plaid_maxsim_qc_workspace_size(const lik_seqs_t* Q, const lik_plaid_docs_t* docs);
int lik_plaid_maxsim_qc(const lik_seqs_t* Q, const lik_plaid_docs_t* docs, const float* token_inv, uint32_t flags,
                        float* out, int64_t out_stride_q, int64_t out_stride_d, void* workspace,
                        size_t workspace_bytes, const lik_launch_opts_t* opts, lik_stream_t stream);

/*
 * Reverse the bit order inside each of nbytes bytes (in may equal out; both
 * 4-byte aligned). Converts ColBERTv2 / fast-plaid residual bytes (each code's
 * bits least-significant first, packed most-significant-bit first by
 * numpy.packbits) to the little-endian field layout the PLAID kernels read.
 * Replaces the byte_reversed_bits_map lookup of fast-plaid's decompressor
 * (noted at benchmarks/plaid/bench_decompress_maxsim.py:144-149), applied
 * once at index load instead of per decode.
 */
int lik_residual_reverse_bits(const uint8_t* in, uint8_t* out, int64_t nbytes, lik_stream_t stream);

/*
 * PLAID approximate (centroid-only) score: out[b] = sum_{s<Lq} max_{t<len_b} qcs[codes[b,t], s],
 * with out-of-range codes clamped to centroid 0 and an empty doc scoring 0.
 * Replaces plaid.py:plaid_approx_score (plaid.py:82-136, kernel plaid.py:28-79).
 */
int lik_plaid_approx_score(const float* qcs, int64_t n_centroids, int64_t lq, int64_t qcs_stride_c,
                           int64_t qcs_stride_l, const int32_t* codes, int64_t B, int64_t max_len,
                           int64_t codes_stride_b, const int64_t* doc_lengths, float* out,
                           lik_stream_t stream);

/*
 * Chunk top-k merge. For each row r, the candidates are the running list
 * (prev_scores[r*prev_ld + i], prev_idx[r*prev_ld + i]) for i < prev_k, and
 * (scores[r*ld + c], idx_base + c) for c < n. Writes the k best, ordered by
 * score (descending if largest, else ascending) and then by lower index,
 * to out_scores/out_idx[r*out_ld + i]. k <= prev_k + n, k <= 8192,
 * indices < 2^32. For k <= 1024: prev_k <= 1024 and n <= 4096; for larger k:
 * prev_k <= 8192 and n <= 8192. prev may alias out.
 * Replaces the torch.topk + cat + gather merge of topk.py:41-86 /
 * retrieve.py:278-305 with a deterministic tie order (lower index first).
 */
int lik_topk_merge(const float* scores, int64_t rows, int64_t n, int64_t ld, int64_t idx_base,
                   const float* prev_scores, const int64_t* prev_idx, int64_t prev_k,
                   int64_t prev_ld, int64_t k, int largest, float* out_scores, int64_t* out_idx,
                   int64_t out_ld, lik_stream_t stream);

/*
 * Top-k of rows of any width: the same selection and tie rule as
 * lik_topk_merge, but n is unbounded (idx_base + n < 2^32). Rows wider than
 * one slice (4096 scores for k <= 1024, 8192 above) are reduced as a tree of
 * workgroups (slices, then merges of k-key lists) in a workspace of
 * lik_topk_select_workspace_size(rows, n, k) bytes (0 for a single slice).
 * Replaces topk.py:41-86 / retrieve.py:278-305 for an unchunked call
 * (chunk=None): one selection over all Nd scores per query instead of a
 * sequence of per-chunk merges.
 */
size_t lik_topk_select_workspace_size(int64_t rows, int64_t n, int64_t k);
int lik_topk_select(const float* scores, int64_t rows, int64_t n, int64_t ld, int64_t idx_base,
                    const float* prev_scores, const int64_t* prev_idx, int64_t prev_k,
                    int64_t prev_ld, int64_t k, int largest, float* out_scores, int64_t* out_idx,
                    int64_t out_ld, void* workspace, size_t workspace_bytes, lik_stream_t stream);

/*
 * Allocation-free scoring. No counterpart in the reference: this entry point
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). It scores
 * exactly like lik_maxsim (same flags, layouts and outputs; doc-side
 * normalisation stays inside the tile kernel instead of a pre-normalised
 * copy) but takes no workspace: the mask summaries and query-chunk partial
 * sums live in a fixed per-device scratch array of LIK_NOALLOC_SCRATCH_BYTES
 * that the library owns until the process ends. It calls no allocator.
 * A call whose scratch need exceeds that size returns LIK_ERR_WORKSPACE
 * (use lik_maxsim with a workspace instead). Every call on a device shares
 * that device's array, so calls that overlap on one device (different
 * streams, or threads) race; calls on one stream are ordered and safe.
 */
#define LIK_NOALLOC_SCRATCH_BYTES (64u << 20)
int lik_maxsim_noalloc(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale, float* out,
                       int64_t out_stride_q, int64_t out_stride_d, lik_stream_t stream);

/* Library version string and the gfx target it was built for. */
const char* lik_version(void);


/* lik_maxsim / lik_maxsim_workspace_size / lik_plaid_maxsim with launch options. */
int lik_maxsim_ex(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags, float out_scale, float* out,
                  int64_t out_stride_q, int64_t out_stride_d, void* workspace, size_t workspace_bytes,
                  const lik_launch_opts_t* opts, lik_stream_t stream);
size_t lik_maxsim_workspace_size_ex(const lik_seqs_t* Q, const lik_seqs_t* D, uint32_t flags,
                                    const lik_launch_opts_t* opts);
int lik_plaid_maxsim_ex(const lik_seqs_t* Q, const lik_plaid_docs_t* docs, uint32_t flags, float* out,
                        int64_t out_stride_q, int64_t out_stride_d, const lik_launch_opts_t* opts,
                        lik_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LIK_H_ */
