/*
 * pkm_hip.h — C ABI of the MI355X (gfx950) product-key-memory lookup library
 * (libpkm_hip.so).
 *
 * Every entry point:
 *   - takes borrowed device pointers and plain sizes (no framework types);
 *   - writes only into caller-provided outputs / workspace (no allocation);
 *   - enqueues its kernels on `stream` (a hipStream_t passed as void*, NULL =
 *     the null stream) and returns without synchronising;
 *   - returns PKM_OK (0) or a nonzero pkm_status_t; the message of the last
 *     failure on the calling thread is returned by pkm_last_error_string().
 *
 * Index tensors are int64 (torch.long), row-major [bags, bag_size].
 * Indices outside [0, num_rows) do not fault: they read nothing, contribute
 * zero to outputs and get a zero per-sample-weight gradient.
 * pkm_count_invalid_indices() reports how many there are.
 */
#ifndef PKM_HIP_H_
#define PKM_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes (tables, gradients, per-sample weights). */
enum pkm_dtype_t {
  PKM_DTYPE_NONE = -1, /* pointer is NULL: unweighted bag (all weights 1) */
  PKM_DTYPE_F32 = 0,
  PKM_DTYPE_BF16 = 1,
  PKM_DTYPE_F16 = 2
};

enum pkm_status_t {
  PKM_OK = 0,
  PKM_ERR_INVALID_ARGUMENT = 1, /* bad shape, dtype, null pointer, overflow */
  PKM_ERR_UNSUPPORTED = 2,      /* valid request this build has no kernel for */
  PKM_ERR_WORKSPACE = 3,        /* workspace smaller than the size query returned */
  PKM_ERR_HIP = 4               /* a HIP runtime call or kernel launch failed */
};

/* Library version, (major << 16) | minor. */
int pkm_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* pkm_last_error_string(void);

/*
 * Weighted embedding bag, forward (mode "sum").
 *   out[b, :] = sum_{j < bag_size} psw[b, j] * weight[indices[b, j], :]
 * Accumulates in float32 in j order and rounds once to weight's dtype.
 * psw may be NULL (psw_dtype PKM_DTYPE_NONE): all weights are 1.
 * out: [bags, dim] in weight_dtype.
 *
 * Replaces embedding_bag_triton / embedding_bag_k
 *   (pkm/xformer_embeddingbag.py:97-138, fwpkm/xformer_embeddingbag_legacy.py:33-74)
 * and the index_select+sum forward of _XEmbeddingBagFn
 *   (fwpkm/xformer_embeddingbag_grad_wrapper.py:98-103).
 */
int pkm_eb_fwd(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
               const int64_t* indices, const void* psw, int psw_dtype,
               int64_t bags, int64_t bag_size, void* out, void* stream);

/* Workspace bytes pkm_eb_bwd needs for these sizes. */
size_t pkm_eb_bwd_workspace_size(int64_t num_rows, int64_t dim, int64_t bags, int64_t bag_size);

/*
 * Weighted embedding bag, backward. Deterministic (no float atomics; the
 * float32 sums run in a fixed order independent of the launch).
 *   grad_weight[r, :] = sum_{(b,j): indices[b,j] == r} psw[b, j] * grad_out[b, :]
 *       dense [num_rows, dim] in weight_dtype; untouched rows are written as 0.
 *   grad_psw[b, j]    = <weight[indices[b, j], :], grad_out[b, :]>   (float32 dot)
 *       [bags, bag_size] in psw_dtype; not written when psw is NULL.
 * grad_out: [bags, dim] in grad_dtype: weight_dtype, or F32 beside a BF16 /
 * F16 table (read as float32, unrounded, as the reference's kernel widens it,
 * pkm/xformer_embeddingbag.py:322); other combinations return
 * PKM_ERR_UNSUPPORTED (a caller widens a 16-bit gradient to float32 first,
 * which is exact).
 * workspace: device buffer of at least pkm_eb_bwd_workspace_size() bytes.
 * Rows with at least max(257, bags / 16) lookups (a BF16 table and grad_out,
 * dim a multiple of 512) are reduced as dense bf16 matrix products on the
 * matrix cores, their weights merged per bag: float32 sums in a fixed order
 * (deterministic), not in position order as the other rows' are.
 *
 * Replaces embedding_bag_bw_rev_indices
 *   (pkm/xformer_embeddingbag.py:331-386, fwpkm/xformer_embeddingbag_legacy.py:170-227),
 * i.e. count_per_embedding_k + argsort/cumsum + map_embeddings_and_outputs_k
 * + aggregate_gradient_for_embedding_k (pkm/xformer_embeddingbag.py:261-328),
 * and the CPU fallback _embedding_bag_bw_native (legacy:147-167).
 */
int pkm_eb_bwd(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
               const int64_t* indices, const void* psw, int psw_dtype,
               const void* grad_out, int grad_dtype, int64_t bags, int64_t bag_size,
               void* grad_weight, void* grad_psw,
               void* workspace, size_t workspace_bytes, void* stream);

/*
 * pkm_eb_bwd in two steps, so that the part that depends only on the lookups
 * can run early (e.g. during the forward pass, on another stream, beside the
 * gather) and the backward pass keeps only the reduction:
 *   pkm_eb_bwd_prepare  sorts the lookups by row, builds the row offsets, the
 *                       per-lookup metadata (bag, weight) and the row
 *                       kernel's lists in `workspace`. It reads indices and
 *                       psw, not weight or grad_out.
 *   pkm_eb_bwd_prepared runs the reduction (grad_weight, grad_psw) on a
 *                       workspace that pkm_eb_bwd_prepare filled, with the
 *                       same num_rows, dim, weight_dtype, indices, psw, bags
 *                       and bag_size (psw unchanged in between; the caller
 *                       orders the two calls, e.g. with an event).
 * pkm_eb_bwd(args) == pkm_eb_bwd_prepare + pkm_eb_bwd_prepared, bit for bit.
 * Together they replace the same reference code as pkm_eb_bwd (its
 * count/argsort/map steps, pkm/xformer_embeddingbag.py:261-288, are the
 * prepare step; aggregate_gradient_for_embedding_k, :291-328, the reduction).
 */
int pkm_eb_bwd_prepare(int64_t num_rows, int64_t dim, int weight_dtype,
                       const int64_t* indices, const void* psw, int psw_dtype,
                       int64_t bags, int64_t bag_size,
                       void* workspace, size_t workspace_bytes, void* stream);
int pkm_eb_bwd_prepared(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
                        const int64_t* indices, const void* psw, int psw_dtype,
                        const void* grad_out, int grad_dtype, int64_t bags, int64_t bag_size,
                        void* grad_weight, void* grad_psw,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * pkm_eb_bwd that adds into a gradient already in grad_weight instead of
 * overwriting it:
 *   grad_weight[r, :] = grad_weight[r, :] + T(sum_{(b,j): indices[b,j] == r} psw[b, j] * grad_out[b, :])
 * (rounded to the table dtype T once more), rows without lookups unchanged;
 * grad_psw as pkm_eb_bwd. The result equals pkm_eb_bwd into a separate
 * buffer followed by an elementwise add of the two gradients, bit for bit
 * (the sum autograd forms for a table read by two operations), without
 * that add's pass over the table or the zero rows. Needs grad_dtype ==
 * weight_dtype and a row split of 64 lanes (dim >= 256 float32 / 512 16-bit
 * elements, as pkm_eb_bwd's row kernels take it); otherwise
 * PKM_ERR_UNSUPPORTED, nothing enqueued.
 *
 * Replaces the reference's pair of embedding_bag_bw_rev_indices
 * (pkm/xformer_embeddingbag.py:331-386) and autograd's accumulation of the
 * table gradient when the fast-weight module reads a table twice (its
 * retrieval and its update step, fwpkm/fwpkm.py:448, 503-509).
 */
int pkm_eb_bwd_accumulate(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
                          const int64_t* indices, const void* psw, int psw_dtype,
                          const void* grad_out, int grad_dtype, int64_t bags, int64_t bag_size,
                          void* grad_weight, void* grad_psw,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * pkm_eb_bwd without a workspace argument: the same kernels and results
 * (bit-identical outputs), with their workspace in a fixed scratch array of
 * 64 MiB that the library holds on each GPU it runs on until the process ends.
 * It allocates nothing (no hipMalloc / hipFree, no allocating library call).
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). Limits:
 *   - sizes whose pkm_eb_bwd_workspace_size() exceeds 64 MiB are rejected with
 *     PKM_ERR_WORKSPACE (e.g. a 2^18 x 1024 table with 8192 x 64 lookups
 *     needs 34.5 MiB, a 2^20 x 1024 table with 2048 x 256 lookups 40.5 MiB);
 *   - the device current on the calling thread must be the stream's device;
 *   - every call on a GPU shares that GPU's array: calls that overlap on one
 *     GPU (other streams, other threads) race, so serialise them.
 */
int pkm_eb_bwd_noalloc(const void* weight, int64_t num_rows, int64_t dim, int weight_dtype,
                       const int64_t* indices, const void* psw, int psw_dtype,
                       const void* grad_out, int grad_dtype, int64_t bags, int64_t bag_size,
                       void* grad_weight, void* grad_psw, void* stream);

/*
 * Double backward of the embedding bag: the VJP of
 *   grad_weight = EBbwd(indices, a, grad_out)
 * with respect to grad_out and a, given gbar = dLoss/d(grad_weight):
 *   d_grad_out[b, :] = sum_j a[b, j] * gbar[indices[b, j], :]     [bags, dim], grad_dtype
 *   d_a[b, j]        = <gbar[indices[b, j], :], grad_out[b, :]>   [bags, bag_size], a_dtype
 * a may be NULL (unweighted): then d_a is not written.
 * gbar: [num_rows, dim] in gbar_dtype, read in that dtype.
 * grad_out and d_grad_out: [bags, dim] in grad_dtype, which is gbar_dtype or
 * F32 beside a BF16 / F16 gbar (float32 sums in both cases, as the
 * reference's type promotion gives; other combinations return
 * PKM_ERR_UNSUPPORTED).
 *
 * Replaces EmbeddingBagBW.backward (fwpkm/xformer_embeddingbag_grad_wrapper.py:42-74).
 */
int pkm_eb_bwd2(const void* gbar, int64_t num_rows, int64_t dim, int gbar_dtype,
                const int64_t* indices, const void* a, int a_dtype,
                const void* grad_out, int grad_dtype, int64_t bags, int64_t bag_size,
                void* d_grad_out, void* d_a, void* stream);

/*
 * Marginal-entropy address loss of the fast-weight memory and the key
 * table's gradient of it (compute_marginal_entropy / compute_addr_loss,
 * fwpkm/fwpkm.py:117-147, 233-264, differentiated by update_fw with
 * create_graph, fwpkm/fwpkm.py:274-367), and that gradient's derivative
 * along a direction (its double backward).
 *   s1, s2   [num_tokens, heads, n_keys] sub-score matrices (dtype), rows
 *            r = t * heads + h; sel1, sel2 [num_tokens, heads, topk] int64 the
 *            per-half top-k lists of the same retrieval, best first (row r
 *            keeps its entries >= s[r, sel[r, topk - 1]]);
 *   weight   addr_loss_weight: loss = weight * (-H_1 - H_2), H_c = -sum_j
 *            pbar_j log(pbar_j + 1e-8), pbar = mean over rows of the masked
 *            float32 softmax;
 *   batch b = 2h + c (head h, half c), q_t the token's c-th half-query of
 *   head h, k_j key (h, c, j), float32 products (idw only, NULL for dot):
 *     qq [2 heads, num_tokens] |q_t|^2, kk [2 heads, n_keys] |k_j|^2,
 *     dots [2 heads, num_tokens, n_keys] <q_t, k_j>.
 * pkm_me_grad_fwd writes entropy[2] = (H_1, H_2), avec [2, n_keys] (d loss /
 * d P_rj), pbar [2, n_keys], and coef [2 heads, num_tokens, n_keys] float32:
 * idw U_tj = dS_tj / (1e-3 + d2_tj) where d2 = (qq + kk) - 2 dots > 0 (else
 * 0), dot dS_tj, with dS the sub-scores' gradient rounded to dtype; for idw
 * also colsum [2 heads, n_keys] = sum_t U_tj (NULL = not written). The key
 * gradient is then
 *   idw: g[b, j] = 2 (sum_t coef[b, t, j] q_t - k_j colsum[b, j]);
 *   dot: g[b, j] = sum_t coef[b, t, j] q_t.
 * pkm_me_grad_hvp takes, for a direction gbar [2 heads, n_keys, half] (the
 * outer gradient of g), qg [2 heads, num_tokens, n_keys] = <q_t, gbar_j> and
 * (idw) kg [2 heads, n_keys] = <k_j, gbar_j>, with avec and pbar from the
 * forward, and writes the derivative of <gbar, g>: as the sub-scores'
 * gradient d_s1, d_s2 (dtype, every entry; for idw it includes the terms of
 * the form the retrieval's own backward gives a sub-score gradient), and the
 * rest as the rows ul [2 heads, num_tokens, n_keys] float32 (idw U, dot dS),
 * from which
 *   idw: d q_t = 2 sum_j ul[b, t, j] gbar_j,  d k_j = -2 gbar_j colsum_j;
 *   dot: d q_t = sum_j ul[b, t, j] gbar_j.
 * adot [2, n_keys] float32 is scratch. Deterministic.
 * Limits: n_keys <= 1024, topk <= n_keys, num_tokens >= 1.
 * workspace: pkm_me_grad_workspace_size(num_tokens, heads, n_keys) bytes.
 */
size_t pkm_me_grad_workspace_size(int64_t num_tokens, int64_t heads, int64_t n_keys);
int pkm_me_grad_fwd(const void* s1, const void* s2, const int64_t* sel1, const int64_t* sel2, int dtype,
                    int64_t num_tokens, int64_t heads, int64_t n_keys, int64_t topk, int score_type,
                    float weight, const float* qq, const float* kk, const float* dots, float* entropy,
                    float* coef, float* avec, float* pbar, float* colsum, void* workspace,
                    size_t workspace_bytes, void* stream);
int pkm_me_grad_hvp(const void* s1, const void* s2, const int64_t* sel1, const int64_t* sel2, int dtype,
                    int64_t num_tokens, int64_t heads, int64_t n_keys, int64_t topk, int score_type,
                    float weight, const float* qq, const float* kk, const float* kg, const float* dots,
                    const float* qg, const float* avec, const float* pbar, float* adot, void* d_s1,
                    void* d_s2, float* ul, void* workspace, size_t workspace_bytes, void* stream);

/* Sub-key score of pkm_score_topk. */
enum pkm_score_t {
  PKM_SCORE_DOT = 0, /* <q, k> */
  PKM_SCORE_IDW = 1  /* -log(1e-3 + max(|q|^2 + |k|^2 - 2 <q, k>, 0)) */
};

/*
 * Product-key retrieval: sub-key scores, per-half top-knn and the top-knn of
 * the knn x knn cartesian sums, for every (token t, head h).
 *   query: [num_tokens, heads, 2 * half], keys: [2 * heads * n_keys, half]
 *   (key (h, c, i) is row (2h + c) * n_keys + i), both in dtype (F32 or BF16).
 *   s_c[i]          = score(query[t, h, c*half : (c+1)*half], key (h, c, i))
 *                     in float32, rounded to dtype
 *   (v_c, i_c)      = top-knn of s_c, best first
 *   out_scores      = top-knn of dtype(v_0[a] + v_1[b]), best first  [num_tokens*heads, knn], dtype
 *   out_indices     = i_0[a] * n_keys + i_1[b] of those              [num_tokens*heads, knn], int64
 * Optional (NULL = not written):
 *   out_sub_indices1/2 = i_0 / i_1                                    [num_tokens, heads, knn], int64
 *   out_sub_scores1/2  = s_0 / s_1 (every key)                        [num_tokens, heads, n_keys], dtype
 * Equal scores are ordered by the smaller sub-key index (per half) and by
 * the smaller a * knn + b (cartesian); the result is deterministic.
 * Limits: knn <= 64, n_keys a multiple of 64 up to 2048, half a multiple of
 * 32 (BF16) or 16 (F32); query and keys 16-byte aligned.
 *
 * Replaces HashingMemory.get_indices (pkm/memory.py:250-289; score_type DOT,
 * no sub outputs) and FastWeightProductKeyMemory.get_indices +
 * compute_qk_scores (fwpkm/fwpkm.py:853-934; DOT or IDW, all outputs).
 */
int pkm_score_topk(const void* query, const void* keys, int64_t num_tokens, int64_t heads,
                   int64_t n_keys, int64_t half, int64_t knn, int score_type, int dtype,
                   void* out_scores, int64_t* out_indices,
                   int64_t* out_sub_indices1, int64_t* out_sub_indices2,
                   void* out_sub_scores1, void* out_sub_scores2, void* stream);

/*
 * pkm_score_topk with a workspace: the same arguments and results (bit for
 * bit), plus a device buffer of at least
 * pkm_score_topk_workspace_size(heads, n_keys, half, dtype) bytes (the keys'
 * size), 16-byte aligned. Where the tile kernel runs (knn above 32, IDW
 * scores, F32, other half widths), the keys are first copied into it with
 * each block of 16 keys stored chunk-major, so the kernel's key loads read
 * whole cache lines. A NULL or smaller workspace gives pkm_score_topk.
 * Replaces the same reference calls as pkm_score_topk (pkm/memory.py:250-289,
 * fwpkm/fwpkm.py:853-934); the workspace has no counterpart there.
 */
size_t pkm_score_topk_workspace_size(int64_t heads, int64_t n_keys, int64_t half, int dtype);
int pkm_score_topk_ws(const void* query, const void* keys, int64_t num_tokens, int64_t heads,
                      int64_t n_keys, int64_t half, int64_t knn, int score_type, int dtype,
                      void* out_scores, int64_t* out_indices,
                      int64_t* out_sub_indices1, int64_t* out_sub_indices2,
                      void* out_sub_scores1, void* out_sub_scores2,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * Dense gradient of the two sub-score matrices from the gradient of the
 * selected scores (scores[t,h,j] = s_0[i_0] + s_1[i_1], id = i_0 * n_keys + i_1):
 *   d_sub_dense[h, c, t, i] = sum_{j : i_c(indices[t,h,j]) == i} d_scores[t,h,j]
 *                             + d_sub_scores_c[t, h, i]          (when not NULL)
 * float32 sums in j order, rounded once to dtype (F32 or BF16).
 *   indices, d_scores: [num_tokens, heads, knn];  d_sub_scores1/2: [num_tokens, heads, n_keys]
 *   d_sub_dense: [heads, 2, num_tokens, n_keys], fully written; 16-byte aligned.
 * Limits: knn <= 64, n_keys a multiple of 4 up to 2048. Ids outside [0, n_keys^2) are ignored.
 * With it, dq = d_sub_dense[h, c] @ keys_c and dkeys_c = d_sub_dense[h, c]^T @ q_c are
 * plain batched GEMMs.
 *
 * Replaces the autograd backward of topk + gather + expand-add in
 * HashingMemory.get_indices (pkm/memory.py:267-285) and
 * FastWeightProductKeyMemory.get_indices (fwpkm/fwpkm.py:904-921).
 */
int pkm_score_grad_dense(const int64_t* indices, const void* d_scores, int dtype,
                         int64_t num_tokens, int64_t heads, int64_t n_keys, int64_t knn,
                         const void* d_sub_scores1, const void* d_sub_scores2,
                         void* d_sub_dense, void* stream);

/*
 * The idw (distance) factor of a dense sub-score gradient, for the products
 *   dq_b = 2 (U_b @ keys_b - q_b * rowsum_b),  dkeys_b = 2 (U_b^T @ q_b - keys_b * colsum_b):
 *   U[b, t, j]   = dS[b, t, j] / (1e-3 + d2) where d2 = (qq[b, t] + kk[b, j]) - 2 dots[b, t, j] > 0, else 0
 *   rowsum[b, t] = sum_j U[b, t, j],  colsum[b, j] = sum_t U[b, t, j]   (fixed order)
 * dS [batches, tokens, n_keys] in dtype (pkm_score_grad_dense's output, batch
 * b = 2h + c, batches even); qq [batches, tokens] = |q_t|^2, kk [batches,
 * n_keys] = |k_j|^2, dots [batches, tokens, n_keys] = <q_t, k_j>, float32 (the
 * operands of the mm-based distance); U, rowsum, colsum float32, fully
 * written. Limits: n_keys <= 1024, tokens >= 1.
 * workspace: pkm_idw_grad_coef_workspace_size(batches, tokens, n_keys) bytes.
 *
 * Replaces the elementwise part of cdist's autograd backward (compute_mode
 * use_mm_for_euclid_dist) under the idw scores of
 * FastWeightProductKeyMemory.compute_qk_scores (fwpkm/fwpkm.py:863-866).
 */
size_t pkm_idw_grad_coef_workspace_size(int64_t batches, int64_t tokens, int64_t n_keys);
int pkm_idw_grad_coef(const void* dS, int dtype, const float* qq, const float* kk, const float* dots,
                      int64_t batches, int64_t tokens, int64_t n_keys, float* U, float* rowsum, float* colsum,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes pkm_score_grad_sparse needs for these sizes (0 when unsupported). */
size_t pkm_score_grad_sparse_workspace_size(int64_t num_tokens, int64_t heads, int64_t n_keys,
                                            int64_t half, int64_t knn);

/*
 * Gradients of the selected dot-product scores w.r.t. query and keys without
 * the dense sub-score gradient: with dS_c the matrix pkm_score_grad_dense
 * writes (no d_sub_scores),
 *   d_query[t, h, c*half + e] = sum_i dS_c[h, t, i] * keys[(2h + c) n_keys + i, e]
 *   d_keys[(2h + c) n_keys + i, e] = sum_t dS_c[h, t, i] * query[t, h, c*half + e]
 * d_query from the nonzeros of each dS row (a gather of key rows, float32 in
 * order of first occurrence), d_keys on MFMA (float32, summed over fixed
 * token splits in order); both deterministic, rounded once to bfloat16.
 *   query: [num_tokens, heads, 2*half], keys: [2*heads*n_keys, half],
 *   indices, d_scores: [num_tokens, heads, knn].
 *   d_query / d_keys: same shapes as query / keys, fully written; NULL skips one.
 *   query, keys, d_query, d_keys 16-byte aligned.
 * dtype BF16 only. Limits: n_keys a multiple of 128 up to 65535, half a multiple of 16
 * up to 256, knn <= 64. Ids outside [0, n_keys^2) are ignored.
 *
 * Replaces the autograd backward of einsum + topk + gather + expand-add in
 * HashingMemory.get_indices (pkm/memory.py:257-285), score_type DOT.
 */
int pkm_score_grad_sparse(const int64_t* indices, const void* d_scores, int dtype,
                          int64_t num_tokens, int64_t heads, int64_t n_keys, int64_t half, int64_t knn,
                          const void* query, const void* keys, void* d_query, void* d_keys,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * RMS normalisation of the query rows, forward (dtype F32 or BF16 for x,
 * weight and y alike; x, weight, y 16-byte aligned, dim a multiple of 4 / 8):
 *   rstd[i]  = rsqrt(mean_j x[i, j]^2 + eps)                       float32 [rows]
 *   y[i, j]  = dtype(weight[j] * dtype(x[i, j] * rstd[i]))          [rows, dim]
 *
 * Replaces Qwen3RMSNorm.forward of the query network (pkm/memory.py:311,
 * 341-349; transformers' Qwen3RMSNorm: float32 cast, pow, mean, rsqrt, mul,
 * cast back, weight mul).
 */
int pkm_rmsnorm_fwd(const void* x, const void* weight, int64_t rows, int64_t dim, int dtype, float eps, void* y,
                    float* rstd, void* stream);

/*
 * Softmax of the selected scores over each row of 1 to 65536 entries (dtype
 * F32, BF16 or F16 for x, y, dy, dx alike; float32 math; rows of up to 64
 * entries sum in column order, longer rows over 64 lane-strided partial sums
 * combined by a fixed tree):
 *   y[i, j] = dtype(exp(x[i, j] - max_k x[i, k]) / sum_k exp(x[i, k] - max_k x[i, k]))
 * Replaces `F.softmax(scores.float(), dim=-1).type_as(scores)` in
 * HashingMemory.forward (pkm/memory.py:218) and the softmax over heads x
 * top-k of FastWeightProductKeyMemory.score_transform (fwpkm/fwpkm.py:105-115).
 */
int pkm_softmax_fwd(const void* x, int64_t rows, int64_t cols, int dtype, void* y, void* stream);

/*
 * Backward of pkm_softmax_fwd through .float(), softmax and .type_as
 * (pkm/memory.py:218), with the float32 probabilities p recomputed from x:
 *   dx[i, j] = dtype(p_j * (dy[i, j] - sum_k dy[i, k] * p_k))
 */
int pkm_softmax_bwd(const void* dy, const void* x, int64_t rows, int64_t cols, int dtype, void* dx, void* stream);

/*
 * Fast-weight value update of FwPKM in one pass (fwpkm/fwpkm.py:334-365 with
 * update_fw_param at 266-272; optimizer "sgd"). For rows r < num_rows and
 * columns j < dim (dtype F32 or BF16 for values, grad and both outputs;
 * counts int64 [num_rows], the bincount of the step's indices):
 *   scaled_grad[r, j] = dtype(dtype(grad[r, j] * scale) / dtype(max(counts[r], 1)))
 *   c                 = grad_clip ? clamp(scaled_grad[r, j], -1, 1) : scaled_grad[r, j]
 *   new_values[r, j]  = dtype(values - dtype(lr * dtype(c + dtype(weight_decay * values))))
 * every step rounded to dtype in the reference's order, no fused multiply-add.
 * values, grad and the outputs 16-byte aligned; dim a multiple of 4 / 8.
 */
int pkm_fw_sgd_update(const void* values, const void* grad, const int64_t* counts, int64_t num_rows, int64_t dim,
                      int dtype, float scale, float lr, float weight_decay, int grad_clip, void* scaled_grad,
                      void* new_values, void* stream);

/*
 * Backward of pkm_fw_sgd_update: the gradients autograd forms for the
 * reference's p - lr * (clip(gs) + wd * p), gs = grad * scale / count
 * (fwpkm/fwpkm.py:334-365, 266-272), op by op in dtype:
 *   x             = dtype(lr * -d_new_values)
 *   d_values      = dtype(d_new_values + dtype(weight_decay * x))
 *   d             = (grad_clip ? x * [-1 <= scaled_grad <= 1] : x) (+ d_scaled_grad, when not NULL)
 *   d_grad        = dtype(dtype(d / dtype(max(counts, 1))) * scale)
 * d_grad may be NULL: then only d_values is written.
 */
int pkm_fw_sgd_update_bwd(const void* d_new_values, const void* d_scaled_grad, const void* scaled_grad,
                          const int64_t* counts, int64_t num_rows, int64_t dim, int dtype, float scale, float lr,
                          float weight_decay, int grad_clip, void* d_values, void* d_grad, void* stream);

/*
 * Value backward with the fast-weight SGD step in its epilogue: the reduction
 * of pkm_eb_bwd (same workspace, same float32 sums in position order), where
 * each table row, instead of its gradient row, gets the values step of FwPKM's
 * inner update (dtype F32 or BF16 for values, grad_out and both outputs):
 *   g                 = dtype(sum_{(b,j): indices[b,j]==r} psw[b,j] * grad_out[b,:])
 *   scaled_grad[r, :] = dtype(dtype(g * scale) / dtype(max(cnt[r], 1)))    cnt = lookups of row r
 *   c                 = grad_clip ? clamp(scaled_grad, -1, 1) : scaled_grad
 *   new_values[r, :]  = dtype(values - dtype(lr * dtype(c + dtype(weight_decay * values))))
 * with pkm_fw_sgd_update's rounding steps. Every row is written (untouched
 * rows: g = 0). new_values must not overlap values. Optional outputs (NULL =
 * not written): scaled_grad; grad_psw as in pkm_eb_bwd; counts [num_rows]
 * int32 = cnt; row_sumsq [num_rows] float32 = sum over the row of
 * scaled_grad^2 (the squared norm of the scaled gradient is their sum).
 *
 * Replaces, for the values (fwpkm/fwpkm.py:333-365 with update_fw_param,
 * 266-272), the table gradient of autograd.grad(mem_loss, values) through
 * _XEmbeddingBagFn's backward (fwpkm/xformer_embeddingbag_grad_wrapper.py:118-
 * 155) followed by the bincount-normalised SGD step: one pass over the table
 * instead of a gradient write and a second pass.
 */
int pkm_eb_bwd_sgd(const void* values, int64_t num_rows, int64_t dim, int dtype, const int64_t* indices,
                   const void* psw, int psw_dtype, const void* grad_out, int64_t bags, int64_t bag_size,
                   float scale, float lr, float weight_decay, int grad_clip, void* new_values, void* scaled_grad,
                   void* grad_psw, int32_t* counts, float* row_sumsq, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * Double backward through pkm_eb_bwd_sgd's step: pkm_eb_bwd2 whose gathered
 * rows are the gradient of the table gradient that autograd forms through the
 * step from d_new_values (and d_scaled_grad, NULL = none), computed per
 * gathered row (dtype F32 or BF16 for every tensor, counts int32 from
 * pkm_eb_bwd_sgd):
 *   x  = dtype(lr * -d_new_values[r])
 *   d  = grad_clip ? x * [-1 <= scaled_grad[r] <= 1] : x     (+ d_scaled_grad[r], rounded)
 *   gb = dtype(dtype(d / dtype(max(counts[r], 1))) * scale)
 *   d_grad_out[b, :] = sum_j a[b, j] * gb[indices[b, j]]      [bags, dim]
 *   d_a[b, j]        = <gb[indices[b, j]], grad_out[b, :]>    [bags, bag_size], a_dtype
 * The values' own gradient (d_new_values, plus weight_decay's term) is the
 * caller's (pkm_fw_sgd_update_bwd with d_grad NULL when weight_decay != 0).
 *
 * Replaces pkm_fw_sgd_update_bwd's d_grad followed by EmbeddingBagBW.backward
 * (fwpkm/xformer_embeddingbag_grad_wrapper.py:42-74): the dense [K, D]
 * gradient of the table gradient is not materialised.
 */
int pkm_eb_bwd2_sgd(const void* d_new_values, const void* d_scaled_grad, const void* scaled_grad,
                    const int32_t* counts, int64_t num_rows, int64_t dim, int dtype, float scale, float lr,
                    int grad_clip, const int64_t* indices, const void* a, int a_dtype, const void* grad_out,
                    int64_t bags, int64_t bag_size, void* d_grad_out, void* d_a, void* stream);

/* Workspace bytes pkm_column_sum needs for these sizes. */
size_t pkm_column_sum_workspace_size(int64_t rows, int64_t cols);

/*
 * Column sums of a row-major [rows, cols] matrix (dtype and out_dtype F32,
 * BF16 or F16; the workspace 16-byte aligned; rows of whole 16-byte vectors
 * take the vector kernel, any other width one column per thread):
 *   out[j] = out_dtype(sum_i x[i, j])   float32, over fixed row blocks in order
 * (deterministic; up to 32 rows need no workspace). Replaces g.sum(0), the bias
 * gradient autograd forms for the Linear layers of HashingMemory and its query
 * network (pkm/memory.py:147-149, 305), and sums the split-K partials of their
 * weight gradients.
 */
int pkm_column_sum(const void* x, int64_t rows, int64_t cols, int dtype, int out_dtype, void* out, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * SwiLU gating of the value output (dtype F32 or BF16 for every tensor;
 * all 16-byte aligned, n elements each):
 *   a[i] = dtype(s[i] / (1 + exp(-s[i])))      h[i] = dtype(e[i] * a[i])
 * Replaces `output * F.silu(swilu_projection(input))` in HashingMemory.forward
 * (pkm/memory.py:229), float32 math and the same rounding points.
 */
int pkm_swilu_fwd(const void* e, const void* s, int64_t n, int dtype, void* h, void* stream);

/*
 * Backward of pkm_swilu_fwd, the gradients autograd forms through the product
 * and F.silu (pkm/memory.py:229):
 *   de[i] = dtype(dh[i] * a[i])        dm[i] = dtype(dh[i] * e[i])
 *   ds[i] = dtype(dm[i] * sig * (1 + s[i] * (1 - sig))),  sig = 1 / (1 + exp(-s[i]))
 */
int pkm_swilu_bwd(const void* dh, const void* e, const void* s, int64_t n, int dtype, void* de, void* ds,
                  void* stream);

/* Workspace bytes pkm_rmsnorm_bwd needs for these sizes. */
size_t pkm_rmsnorm_bwd_workspace_size(int64_t rows, int64_t dim);

/*
 * Backward of pkm_rmsnorm_fwd, the gradients autograd forms through the
 * reference's op sequence (rstd from the forward):
 *   g[i, j]       = dtype(dy[i, j] * weight[j])
 *   s[i]          = sum_j g[i, j] * x[i, j]                         float32
 *   dx[i, j]      = dtype(g[i, j] * rstd[i] + x[i, j] * (2 / dim) * (-0.5 * s[i] * rstd[i]^3))
 *   dweight[j]    = dtype(sum_i dtype(dy[i, j] * dtype(x[i, j] * rstd[i])))   float32 sum
 * dweight is a deterministic reduction (fixed order over 64-row blocks).
 * workspace: device buffer of at least pkm_rmsnorm_bwd_workspace_size() bytes.
 *
 * Replaces the autograd backward of Qwen3RMSNorm.forward (pkm/memory.py:311).
 */
int pkm_rmsnorm_bwd(const void* dy, const void* x, const void* weight, const float* rstd, int64_t rows, int64_t dim,
                    int dtype, void* dx, void* dweight, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Counts indices outside [0, num_rows) into *count_out (a device int64),
 * which the call overwrites. No counterpart in the reference (its Triton
 * kernels do no bounds check; its CPU path raises from F.embedding_bag,
 * pkm/xformer_embeddingbag.py:436-437): it lets a caller turn bad indices
 * into an error.
 */
int pkm_count_invalid_indices(const int64_t* indices, int64_t n, int64_t num_rows,
                              int64_t* count_out, void* stream);

/*
 * Kernel timing for measurement tools. No counterpart in the reference (it
 * has no FFI); it lets a benchmark time one kernel of a multi-kernel entry
 * point on the stream the kernel runs on.
 * pkm_kernel_timing_begin() turns timing on for the process (every thread:
 * backward passes launch from the autograd engine's thread) and drops earlier
 * records. While it is on, these launches are bracketed by a pair of HIP
 * events recorded on the call's stream (at most 4096 records):
 *   "eb_fwd"       the gather kernel of pkm_eb_fwd;
 *   "eb_bwd2"      the kernel of pkm_eb_bwd2;
 *   "eb_bwd_rows"  the row-reduction kernel of pkm_eb_bwd (after its sort);
 *   "score_topk"   the scoring + per-half top-k kernel of pkm_score_topk
 *                  (not its cartesian kernel).
 * pkm_kernel_timing_read() waits for the records named `kernel` and writes the
 * milliseconds of the first `cap` of them, in call order, to ms_out; *count_out
 * gets their number. pkm_kernel_timing_end() turns timing off and releases the
 * records. Timing is for measurement: each record creates two events.
 */
int pkm_kernel_timing_begin(void);
int pkm_kernel_timing_read(const char* kernel, float* ms_out, int64_t cap, int64_t* count_out);
int pkm_kernel_timing_end(void);

#ifdef __cplusplus
}
#endif

#endif /* PKM_HIP_H_ */
