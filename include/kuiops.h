/*
 * kuiops.h -- C ABI of the MI355X (gfx950) kuiops hot path.
 *
 * Every entry point is a plain C function over device pointers, sizes and a
 * HIP stream passed as `void *` (NULL = the legacy default stream).  Nothing
 * here allocates device memory, synchronises the device or depends on torch:
 * the caller owns every buffer (inputs, outputs and the optional workspace),
 * and all work is enqueued asynchronously on the given stream, so every entry
 * point may be recorded into a HIP graph.
 *
 * Return value: KUIOPS_OK (0) or a negative kuiops_status.  A negative status
 * means nothing was enqueued.  KUIOPS_E_UNSUPPORTED means "shape/dtype outside
 * what the kernels implement" (the caller falls back); KUIOPS_E_INVALID means
 * inconsistent arguments (a bug in the caller).
 *
 * Reference interfaces replaced (panther03/kuiLLM):
 *   - the per-instantiation host launchers `<Module>_<name>(uint32 dims...,
 *     T* ptrs...)` that each pybind wrapper calls
 *     (kuiops/mm/wrapper_mm.cu.j2:15-19, kuiops/addmm/wrapper_addmm.cu.j2:18-24,
 *     kuiops/bmm/wrapper_bmm.cu.j2:16-20, kuiops/softmax/wrapper_softmax.cu.j2:14-16,
 *     kuiops/sdpa/wrapper_sdpa.cu.j2:21-30, kuiops/gather/wrapper_gather.cu.j2:26-32);
 *   - the libtorch glue of the reference's include/kuiops.h:11-36
 *     (sync_current_stream / clone_in / index_to_u32), which has no counterpart
 *     here because nothing is synchronised, cloned or narrowed.
 */
#ifndef KUIOPS_H_
#define KUIOPS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KUIOPS_ABI_VERSION 1

#if defined(__GNUC__)
#define KUIOPS_API __attribute__((visibility("default")))
#else
#define KUIOPS_API
#endif

typedef enum kuiops_status {
    KUIOPS_OK = 0,
    KUIOPS_E_UNSUPPORTED = -1, /* outside the implemented shapes / dtypes   */
    KUIOPS_E_INVALID = -2,     /* inconsistent or null arguments             */
    KUIOPS_E_HIP = -3,         /* a HIP runtime call failed (launch error)   */
    KUIOPS_E_WORKSPACE = -4    /* workspace missing or smaller than queried  */
} kuiops_status;

/* Element types.  Values are part of the ABI. */
typedef enum kuiops_dtype {
    KUIOPS_F32 = 0,
    KUIOPS_F16 = 1,
    KUIOPS_BF16 = 2,
    KUIOPS_F64 = 3,
    KUIOPS_I64 = 4,
    KUIOPS_I32 = 5,
    KUIOPS_I16 = 6,
    KUIOPS_I8 = 7,
    KUIOPS_U8 = 8,
    KUIOPS_BOOL = 9
} kuiops_dtype;

/* Storage of the [K, N] right-hand operand B of a GEMM.
 *   KUIOPS_B_ROW: element (k, n) at B[k * ldb + n]   (row-major [K, N])
 *   KUIOPS_B_COL: element (k, n) at B[n * ldb + k]   (an nn.Linear weight
 *                 [N, K] seen through .t(): K contiguous)                      */
typedef enum kuiops_b_layout { KUIOPS_B_ROW = 0, KUIOPS_B_COL = 1 } kuiops_b_layout;

/* Addend of addmm.
 *   KUIOPS_C_NONE : out = alpha * A@B
 *   KUIOPS_C_FULL : out = beta * Cin[M, N] + alpha * A@B   (Cin row stride ldcin)
 *   KUIOPS_C_ROW  : out = beta * bias[N]   + alpha * A@B   (bias broadcast over rows) */
typedef enum kuiops_c_kind { KUIOPS_C_NONE = 0, KUIOPS_C_FULL = 1, KUIOPS_C_ROW = 2 } kuiops_c_kind;

/* Input stage fused into kuiops_decode_linear (see there). */
typedef enum kuiops_x_kind { KUIOPS_X_PLAIN = 1, KUIOPS_X_RMSNORM = 2, KUIOPS_X_SWIGLU = 3 } kuiops_x_kind;

/* Operation ids for kuiops_query_workspace. */
typedef enum kuiops_op {
    KUIOPS_OP_ADDMM = 1,
    KUIOPS_OP_GEMV_SPLITK = 2,
    KUIOPS_OP_SDPA_DECODE = 3,
    KUIOPS_OP_TOPK = 4,
    KUIOPS_OP_SORT = 5,         /* (m, n, 0): rows x row length */
    KUIOPS_OP_DECODE_ROWS_BATCHED = 6   /* (M, N, K) */
} kuiops_op;

KUIOPS_API int kuiops_abi_version(void);
KUIOPS_API const char *kuiops_status_string(int status);

/* Bytes of workspace the given call needs (0 = none).  Arguments are the
 * leading size arguments of that op:
 *   ADDMM:        a = M, b = N, c = K
 *   GEMV_SPLITK:  a = M, b = N, c = K
 *   SDPA_DECODE:  a = batch * q_heads * q_len, b = kv_len, c = head_dim_v
 *   TOPK:         a = rows, b = row length, c = k
 *   DECODE_ROWS_BATCHED: a = M, b = N, c = K
 * Workspace contents need no initialisation, except GEMV_SPLITK's first
 * 16 KB (arrival counters): zero before the first call, and every call
 * leaves them zero.  Calls that share one workspace must be ordered on one
 * stream.                                                                  */
KUIOPS_API size_t kuiops_query_workspace(int op, int64_t a, int64_t b, int64_t c);

/* ---------------------------------------------------------------- GEMM --
 * C[M, N] = A[M, K] @ B[K, N]
 * Replaces the mm launcher `(M, N, K, A, B, C)` of
 * kuiops/mm/wrapper_mm.cu.j2:15-19 (family gate kuipy/kuiops.py:403-469).
 * in_dtype: BF16, F16 or F32 (A and B share it).  out_dtype: same as
 * in_dtype, or F32 for half inputs.  Accumulation is fp32 (fp64 for F64).
 * A is row-major with row stride lda; B per b_layout; C row stride ldc.    */
KUIOPS_API int kuiops_mm(int64_t M, int64_t N, int64_t K, int in_dtype,
              const void *A, int64_t lda,
              const void *B, int64_t ldb, int b_layout,
              int out_dtype, void *C, int64_t ldc, void *stream);

/* out[M, N] = beta * Cin + alpha * (A @ B), see kuiops_c_kind.
 * Replaces the addmm launcher `(M, K, N, alpha, beta, A, B, C)` of
 * kuiops/addmm/wrapper_addmm.cu.j2:18-24 (gate kuipy/kuiops.py:526-564),
 * extended with the 1-D bias form the reference rejects
 * (kuipy/kuiops.py:540, tests/test_jit_ops.py:82).
 * splits: K-splits (0 = choose).  With splits > 1 fp32 partial tiles go to
 * the workspace and are summed in split order 0..splits-1 (deterministic).
 * `out` may alias Cin (in-place update, as the reference's wrapper does on a
 * clone).                                                                  */
KUIOPS_API int kuiops_addmm(int64_t M, int64_t K, int64_t N, double alpha, double beta,
                 int in_dtype,
                 const void *A, int64_t lda,
                 const void *B, int64_t ldb, int b_layout,
                 const void *Cin, int c_kind, int64_t ldcin,
                 int out_dtype, void *out, int64_t ldo,
                 int splits, void *workspace, size_t workspace_bytes,
                 void *stream);

/* C[b] = A[b] @ B[b] for b < batch (output overwritten, as comb2 in
 * kuiops/bmm/Kuiops.Bmm.fst:10-23).  Replaces the bmm launcher
 * `(Bn, M, K, N, A, B, C)` of kuiops/bmm/wrapper_bmm.cu.j2:16-20
 * (gate kuipy/kuiops.py:481-511).  Batch strides in elements.             */
KUIOPS_API int kuiops_bmm(int64_t batch, int64_t M, int64_t K, int64_t N, int in_dtype,
               const void *A, int64_t stride_a, int64_t lda,
               const void *B, int64_t stride_b, int64_t ldb, int b_layout,
               int out_dtype, void *C, int64_t stride_c, int64_t ldc,
               void *stream);

/* Skinny (decode) GEMM: out[M, N] = x[M, K] @ W[K, N] (+ bias[N]) for
 * 1 <= M <= 64, bf16/f16 in, fp32 accumulate, out_dtype = in or F32.
 * K is split over `splits` work-groups (0 = choose); fp32 partials go to the
 * workspace and are summed in split order (row-major W: by the last work-
 * group of each column strip to finish, K-contiguous W: by a second
 * kernel), so the result is bitwise repeatable.  Requires the workspace of
 * kuiops_query_workspace(KUIOPS_OP_GEMV_SPLITK, M, N, K).  Serves the
 * reference's mm/addmm families at decode shapes, which its gate rejects
 * (`M % 64`, kuipy/kuiops.py:372-374).                                    */
KUIOPS_API int kuiops_gemv_splitk(int64_t M, int64_t N, int64_t K, int in_dtype,
                       const void *x, int64_t ldx,
                       const void *W, int64_t ldw, int w_layout,
                       const void *bias,
                       int out_dtype, void *out, int64_t ldo,
                       int splits, void *workspace, size_t workspace_bytes,
                       void *stream);

/* kuiops_gemv_splitk without a workspace argument: it allocates nothing
 * (no hipMalloc / hipFree, no torch, no allocating library call), so it can
 * be called by code that may not allocate -- under HIP graph capture, in
 * tight serving loops, from harnesses that forbid allocation.  No
 * counterpart in the reference.  Split partials and arrival counters live in
 * a file-scope device array of kuiops_gemv_splitk_noalloc_max_bytes() bytes
 * per GPU (8 MiB), held until the process ends; a shape whose workspace
 * (kuiops_query_workspace) exceeds it returns KUIOPS_E_WORKSPACE.  Every
 * call on one GPU shares that array: calls that overlap on one GPU race.
 * The counters it uses are cleared by a fill kernel at the start of each
 * call.  Same kernels and results as kuiops_gemv_splitk.                 */
KUIOPS_API int kuiops_gemv_splitk_noalloc(int64_t M, int64_t N, int64_t K, int in_dtype,
                       const void *x, int64_t ldx,
                       const void *W, int64_t ldw, int w_layout,
                       const void *bias,
                       int out_dtype, void *out, int64_t ldo,
                       int splits, void *stream);
KUIOPS_API size_t kuiops_gemv_splitk_noalloc_max_bytes(void);

/* ---------------------------------------------------------------- SDPA --
 * Flash-attention forward: O = softmax(scale * Q K^T [+ causal mask]) V,
 * LSE = logsumexp over keys (natural log, fp32, optional: pass NULL).
 * Q (n, hq, l, e), K (n, hkv, s, e), V (n, hkv, s, ev); hq % hkv == 0
 * (grouped-query heads share KV head h / (hq / hkv)).  Every tensor has a
 * contiguous last dim; strides (in elements) are given for dims 0..2 as
 * {batch, head, seq}.  O (n, hq, l, ev) with strides so[3]; LSE contiguous
 * (n, hq, l).  Causal masking follows aten: query i sees keys j <= i (top
 * left aligned; rows with no visible key output 0 and LSE = -inf).
 * dtype BF16 or F16; e == ev, e in {64, 128}.
 * Replaces the SDPA launcher of kuiops/sdpa/wrapper_sdpa.cu.j2:21-30
 * (family kuipy/kuiops.py:627-681), which rejects is_causal.              */
KUIOPS_API int kuiops_sdpa_fwd(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s,
                    int64_t e, int64_t ev, int dtype,
                    const void *Q, const int64_t sq[3],
                    const void *K, const int64_t sk[3],
                    const void *V, const int64_t sv[3],
                    void *O, const int64_t so[3],
                    float *lse, float scale, int causal, void *stream);

/* kuiops_sdpa_fwd with an additive attention bias -- the reference family's
 * own form (kuipy/kuiops.py:627-681: a full (N, H, L, S) bias, which it
 * pre-divides by the scale, :673-676) and the call its app issues,
 * _scaled_dot_product_efficient_attention with a bf16 bias from left-padded
 * batched generation (KERNELS.md:64, infer.py:22-24,102):
 *   O = softmax(scale * Q K^T + bias [+ causal mask]) V.
 * Bias element (b, h, i, j) is at bias + b*sb[0] + h*sb[1] + i*sb[2] + j
 * (stride 0 broadcasts, e.g. one padding mask for every head), in `dtype`;
 * sb[] multiples of 4 and bias 8-byte aligned.  -inf entries mask keys;
 * rows with no visible key output 0 and LSE = -inf.  bias == NULL is
 * kuiops_sdpa_fwd.  scale > 0.                                              */
KUIOPS_API int kuiops_sdpa_fwd_bias(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s,
                         int64_t e, int64_t ev, int dtype,
                         const void *Q, const int64_t sq[3],
                         const void *K, const int64_t sk[3],
                         const void *V, const int64_t sv[3],
                         void *O, const int64_t so[3],
                         float *lse, float scale, int causal,
                         const void *bias, const int64_t sb[3], void *stream);

/* Every other SDPA: bf16 / f16 / fp32 / fp64 Q, K, V (one dtype), head dims
 * e and ev independent and up to 1024, optional additive bias (element
 * (b, h, i, j) at bias + b*sb[0] + h*sb[1] + i*sb[2] + j, the Q dtype, any
 * alignment), causal top-left masking, grouped-query heads; same tensor
 * conventions as kuiops_sdpa_fwd.  score = scale * q.k + bias (aten's
 * order), accumulated in fp32 (fp64 for fp64 inputs); lse (optional, fp32
 * [n, hq, l]) is the natural-log log-sum-exp; rows with no visible key give
 * 0 and -inf.  A SIMT kernel (one wave per query row): the coverage path for
 * what the MFMA kernels do not take.  Replaces the reference's sdpa launcher
 * for its full dtype / shape range (kuiops/sdpa/wrapper_sdpa.cu.j2:21-30,
 * gate kuipy/kuiops.py:640-648).                                            */
KUIOPS_API int kuiops_sdpa_general(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s,
                         int64_t e, int64_t ev, int dtype,
                         const void *Q, const int64_t sq[3],
                         const void *K, const int64_t sk[3],
                         const void *V, const int64_t sv[3],
                         void *O, const int64_t so[3],
                         float *lse, double scale, int causal,
                         const void *bias, const int64_t sb[3], void *stream);

/* Decode attention (l small, typically 1) over a KV cache, split over the
 * key axis; same tensor conventions as kuiops_sdpa_fwd.  Causal masking with
 * l > 1 aligns the queries to the END of the keys (query i sees keys
 * j <= s - l + i), which is what a KV-cache decode step needs; pass
 * causal = 0 for plain full attention.  kv_len (optional, device memory,
 * int32[n]) gives each batch entry's key count s_b <= s, read when the
 * kernel runs: a decode step recorded once in a HIP graph passes s = cache
 * capacity and advances kv_len on the device.  Requires the workspace of
 * kuiops_query_workspace(KUIOPS_OP_SDPA_DECODE, n*hq*l, s, ev), 16-byte
 * aligned, whose first bytes hold the split arrival counters: they must be
 * zero before the first call and every call leaves them zero (calls that
 * share a workspace must not overlap).  One launch: the last split
 * work-group of each query-row group merges the splits.  Rows with no
 * visible key (s = 0, or kv_len[b] = 0) give zero output and lse = -inf;
 * K / V must still be non-null.  Counters sit 64 bytes apart.
 * Replaces the decode use of the reference sdpa launcher
 * (kuiops/sdpa/wrapper_sdpa.cu.j2:21-30), which has no KV-cache form.     */
KUIOPS_API int kuiops_sdpa_decode(int64_t n, int64_t hq, int64_t hkv, int64_t l, int64_t s,
                       int64_t e, int64_t ev, int dtype,
                       const void *Q, const int64_t sq[3],
                       const void *K, const int64_t sk[3],
                       const void *V, const int64_t sv[3],
                       void *O, const int64_t so[3],
                       float *lse, float scale, int causal, const int32_t *kv_len,
                       void *workspace, size_t workspace_bytes, void *stream);

/* ------------------------------------------------------- sampling tail --
 * Row softmax over the last dim of a contiguous [m, n] tensor:
 * Y = exp(X - max) / sum.  in/out dtype F32, BF16, F16 or F64; X and Y may
 * alias (the reference softmaxes a clone in place,
 * kuiops/softmax/wrapper_softmax.cu.j2:8-18, kuipy/kuiops.py:607-610).     */
KUIOPS_API int kuiops_softmax_lastdim(int64_t m, int64_t n, int dtype,
                           const void *X, void *Y, void *stream);

/* Top-k along the last dim of a contiguous [m, n] tensor (aten.topk with
 * dim = -1).  values [m, k] (dtype of X), indices [m, k] int64.
 * Ordering: largest (or smallest) first; NaN counts as larger than every
 * number; equal values are ordered by ascending index, and a tie at the
 * k-th place keeps the lowest indices.  `sorted` = 0 is accepted and also
 * returns sorted output.  1 <= k <= min(n, 1024).  dtype F32, BF16, F16.
 * No reference kernel exists (kuiops/topk/.gitkeep); aten.topk is the
 * reference's result.                                                      */
KUIOPS_API int kuiops_topk_lastdim(int64_t m, int64_t n, int64_t k, int dtype,
                        const void *X, void *values, int64_t *indices,
                        int largest, int sorted,
                        void *workspace, size_t workspace_bytes, void *stream);

/* Greedy decode tail: per row of X[m, n] (n <= 32768), the top-1 of
 * softmax(X) in fp32 -- index[row] and, if prob is non-null, its
 * probability prob[row] -- with the probabilities bitwise equal to
 * kuiops_softmax_lastdim's on the fp32 row when n > 1024 (shorter rows take
 * its one-wave kernel, which sums in another order) and topk's ordering (NaN largest,
 * lowest index on ties); then, when given, history[row * hist_len + pos[row]]
 * = index (positions outside [0, hist_len) are skipped), pos[row] += 1 and
 * kv_len[row] += 1 (device int32 arrays: a graph-replayed decode step
 * recording its token and advancing its own position and key count).
 * history needs pos.  dtype F32, BF16, F16 (converted exactly to
 * fp32 first).  No reference counterpart: it fuses the _softmax launch
 * (kuiops/softmax/wrapper_softmax.cu.j2:14-16), aten.topk(k = 1) and the
 * position updates of one greedy step.                                       */
KUIOPS_API int kuiops_softmax_top1(int64_t m, int64_t n, int dtype, const void *X, float *prob,
                        int64_t *index, int32_t *pos, int32_t *kv_len, int64_t *history,
                        int64_t hist_len, void *stream);

/* out[x] = inp[x with axis `dim` replaced by idx[x]]  (torch.gather).
 * Contiguous row-major tensors of rank 1..8; idx int64 with idx_shape
 * pointwise <= inp_shape except along `dim`; elem_bytes 1, 2, 4 or 8.
 * Negative or out-of-range indices write 0 and set *err_flag (device int,
 * optional) to 1.  Replaces kuiops/gather/wrapper_gather.cu.j2:26-32 and
 * the int64 -> u32 narrowing copy of the reference's include/kuiops.h:28-36
 * (indices are read as int64 directly).                                    */
KUIOPS_API int kuiops_gather(int rank, const int64_t *inp_shape, const int64_t *idx_shape,
                  int dim, int elem_bytes, const void *inp, const int64_t *idx,
                  void *out, int *err_flag, void *stream);

/* aten.scatter.src: for every x of idx's shape,
 *   out[x with axis `dim` replaced by idx[x]] = src[x],
 * out being a contiguous copy of self (the caller clones self into out
 * first).  src and idx are contiguous with idx_shape, pointwise <= out_shape
 * except along `dim`; rank 1..8; elem_bytes 1, 2, 4 or 8.  Out-of-range
 * indices write nothing and set *err_flag.  Where indices repeat along `dim`
 * the value that lands is unspecified (as in aten).  Replaces the reference's
 * scatter launcher (ScatterImpl kuipy/kuiops.py:757-807,
 * kuiops/scatter/wrapper_scatter.cu.j2), which returns the updated clone.   */
KUIOPS_API int kuiops_scatter(int rank, const int64_t *out_shape, const int64_t *idx_shape, int dim,
                   int elem_bytes, const void *src, const int64_t *idx, void *out,
                   int *err_flag, void *stream);

/* Row sort of X[m, n] along the last dim (aten.sort, stable): values and
 * int64 indices [m, n]; ascending or descending; NaN counts as the largest
 * value, -0 equals +0, equal values keep index order.  dtype F32, BF16, F16;
 * n < 2^32.  Workspace: kuiops_query_workspace(KUIOPS_OP_SORT, m, n, 0)
 * bytes (0 for n <= 2048).  No reference kernel (KERNELS.md row
 * aten.sort.default): aten.sort is the reference's result.                 */
KUIOPS_API int kuiops_sort_lastdim(int64_t m, int64_t n, int dtype, const void *X, void *values,
                        int64_t *indices, int descending, void *workspace,
                        size_t workspace_bytes, void *stream);

/* The masking step of transformers' TopPLogitsWarper on fp32 scores[m, n],
 * given their ascending stable sort (sorted_vals, sorted_idx [m, n], as
 * kuiops_sort_lastdim returns them) and the fp32 cumulative softmax cum[m, n]
 * of the sorted scores: out = scores with filter_value at sorted_idx[j] for
 * every j < n - min_keep whose cum[j] <= (float)(1 - top_p) (min_keep == 0
 * removes nothing, as the Python slice [-0:] does).  Written as a scatter of
 * the sorted values, so out must not alias the inputs; indices outside
 * [0, n) are skipped (out is then incomplete).  No reference kernel:
 * it replaces the aten le.Scalar / setitem / scatter / masked_fill sequence
 * the reference app runs after the sort (KERNELS.md rows aten.le.Scalar,
 * aten.scatter.src; transformers' TopPLogitsWarper).                       */
KUIOPS_API int kuiops_top_p_mask(int64_t m, int64_t n, const float *sorted_vals, const int64_t *sorted_idx,
                                 const float *cum, double top_p, int64_t min_keep, double filter_value, float *out,
                                 void *stream);

/* Inclusive prefix sum of X[m, n] along the last dim into Y (aten.cumsum):
 * dtype F32 (fp32 accumulate), F64, I64 (exact).  No reference kernel
 * (KERNELS.md rows aten.cumsum.default).                                   */
KUIOPS_API int kuiops_cumsum_lastdim(int64_t m, int64_t n, int dtype, const void *X, void *Y, void *stream);

/* Multinomial sampling with replacement from non-negative weights P[m, n]
 * (rows need not sum to 1): out[r, s] = the first index i whose running
 * weight sum (fp64) exceeds uniforms[r, s] * row total (inverse CDF), so a
 * zero weight is never drawn.  uniforms: device fp32 [m, num_samples] in
 * [0, 1), the caller's random numbers (the draws are a deterministic
 * function of them).  A row with a negative, NaN or infinite weight or a
 * zero total draws index 0 and sets *err_flag (aten raises).  dtype F32,
 * F64, BF16, F16.  No reference kernel (KERNELS.md row
 * aten.multinomial.default).                                               */
KUIOPS_API int kuiops_multinomial(int64_t m, int64_t n, int dtype, const void *probs, int64_t num_samples,
                       const float *uniforms, int64_t *out, int *err_flag, void *stream);

/* aten.index.Tensor with one int64 index tensor at axis `dim` (every other
 * axis sliced whole): out shape = inp[:dim] + idx_shape + inp[dim+1:], all
 * contiguous.  Negative indices count from the end as in aten; indices out
 * of range write 0 and set *err_flag.  inp is given as (outer, size, inner)
 * = (prod inp[:dim], inp[dim], prod inp[dim+1:]).  No reference kernel
 * exists (kuiops/index/.gitkeep).                                          */
KUIOPS_API int kuiops_index(int64_t outer, int64_t size, int64_t inner, int64_t n_idx,
                 int elem_bytes, const void *inp, const int64_t *idx,
                 void *out, int *err_flag, void *stream);

/* aten.index.Tensor with k (1..8) int64 index tensors on adjacent axes --
 * the reference app's mask[T(4,int64), T(4,int64)] (KERNELS.md:67) among
 * them: inp is viewed as (outer, sizes[0], .., sizes[k-1], inner), contiguous;
 * idx[d] points to n_pos int64 indices (the index tensors broadcast to one
 * shape, contiguous); out[o, j, i] = inp[o, idx[0][j], .., idx[k-1][j], i],
 * contiguous (outer, n_pos, inner).  Negative indices wrap; out-of-range
 * ones write 0 and set *err_flag.  Any element type (a byte copy of
 * elem_bytes 1, 2, 4 or 8).  No reference kernel (kuiops/index/.gitkeep).  */
KUIOPS_API int kuiops_index_multi(int64_t outer, int k, const int64_t *sizes, int64_t inner, int64_t n_pos,
                       const int64_t *const *idx, int elem_bytes, const void *inp, void *out,
                       int *err_flag, void *stream);

/* ---- decoder-layer glue (the elementwise / norm / cat work around the hot
 * path; bf16 or f16, rows 16-byte aligned, n % 8 == 0) ------------------- */

/* RMSNorm with an optional fused residual add, per row of [m, n]:
 *   h = x (+ residual)      res_out = h (if non-null; may equal residual)
 *   y = weight * round(h * rsqrt(mean(h^2) + eps)),  n <= 8192.
 * Replaces the reference's elementwise chain pow / mean.dim / add / rsqrt /
 * mul (ElementwiseImpl kuipy/kuiops.py:150-320, MeanImpl :860-921), one
 * launch per aten op there.                                                */
KUIOPS_API int kuiops_rmsnorm(int64_t m, int64_t n, int dtype, const void *x, int64_t ldx,
                   const void *residual, int64_t ldr, void *res_out, int64_t ldro,
                   const void *weight, float eps, void *y, int64_t ldy, void *stream);

/* SwiGLU: out[m, n] = silu(gate) * up, where row i of gate_up is
 * [gate (n) | up (n)] (one fused gate/up projection).  Replaces the
 * reference's silu + mul elementwise launches (kuipy/kuiops.py:158,166). */
KUIOPS_API int kuiops_silu_mul(int64_t m, int64_t n, int dtype, const void *gate_up, int64_t ldg,
                    void *out, int64_t ldo, void *stream);

/* Rotary embedding fused with the KV-cache append for t new tokens of n
 * sequences.  Token (b, i)'s row of qkv (at qkv + b*ld_batch + i*ld_tok
 * elements) is [q heads (hq*hd) | k heads (hkv*hd) | v heads (hkv*hd)];
 * its position is pos0[b] + i (pos0: device int32[n], or null for 0).
 * q is rotated into q_out[b, h, i, :] (strides sq = batch, head, token);
 * rotated k and plain v are stored at cache position pos (strides
 * sk / sv = batch, head, position) when pos < cache_cap.  inv_freq is a
 * device fp32 array of hd/2 rotary frequencies.  Replaces the reference's
 * rotary mul / neg / cat / add launches and the KV-cache cat
 * (CatImpl kuipy/kuiops.py:810-857).                                      */
KUIOPS_API int kuiops_rope_kv_append(int64_t n, int64_t t, int64_t hq, int64_t hkv, int64_t hd,
                          int dtype, const void *qkv, int64_t ld_tok, int64_t ld_batch,
                          const float *inv_freq, const int32_t *pos0,
                          void *q_out, const int64_t sq[3],
                          void *k_cache, const int64_t sk[3],
                          void *v_cache, const int64_t sv[3], int64_t cache_cap,
                          void *stream);

/* Batch-1 decode projection with its input stage fused in (one launch):
 * each work-group computes x[K] from `in`, then out[n] = dot(W[n, :], x)
 * (+ bias[n]) for n < N, W stored [N, K] (an nn.Linear weight, K
 * contiguous, row stride ldw).  No split-K: each output is one wave's dot
 * product, written in dtype.
 *   KUIOPS_X_PLAIN    x = in[K]
 *   KUIOPS_X_RMSNORM  h = round(in + in_add) (in_add optional),
 *                     x = norm_w * round(h * rsqrt(mean(h^2) + eps)); h is
 *                     stored to h_out if non-null (h_out must not alias in)
 *   KUIOPS_X_SWIGLU   x = round(silu(in[k])) * in[K + k]   (in = [gate | up])
 * K <= 8192, K % 8 == 0.  Replaces, for a batch-1 decode step, the
 * reference's mm / addmm launcher (kuiops/mm/wrapper_mm.cu.j2:15-19) plus the
 * elementwise / mean launches of the RMSNorm or SwiGLU feeding it
 * (kuipy/kuiops.py:150-320,860-921).                                      */
KUIOPS_API int kuiops_decode_linear(int64_t N, int64_t K, int dtype, int x_kind, const void *in,
                         const void *in_add, const void *norm_w, float eps, void *h_out,
                         const void *W, int64_t ldw, const void *bias, void *out, void *stream);

/* Batch-1 decode gate/up projection with SwiGLU fused into its epilogue:
 * W = [gate; up] stored [2*ffn, K] (rows ffn apart), x from the input stage
 * as in kuiops_decode_linear (x_kind), and
 *   out[i] = round(round(silu(g_i)) * u_i),  g_i, u_i = round(dot(W row, x))
 * for i < ffn, the rounding of the stock gate_proj / silu / up_proj / mul
 * chain.  No reference counterpart: it fuses the decoder glue around the
 * mm launcher (kuiops/mm/wrapper_mm.cu.j2:15-19) with the silu and mul
 * elementwise launches (kuipy/kuiops.py:158,166).  K <= 4096.              */
KUIOPS_API int kuiops_decode_gate_up(int64_t ffn, int64_t K, int dtype, int x_kind, const void *in,
                          const void *in_add, const void *norm_w, float eps, void *h_out,
                          const void *W, int64_t ldw, void *out, void *stream);

/* Batch-1 decode qkv projection with rotary embedding and the KV-cache
 * append fused into its epilogue.  W is the fused [q; k; v] weight
 * [(hq + 2*hkv)*hd, K]; x comes from the input stage of x_kind, reading
 * `in` at row in_row[0] (device int64, clamped to [0, in_rows)) of stride
 * ld_in when in_row is non-null (an embedding lookup), else `in` itself.
 * At position p = pos[0] (device int32): q heads are rotated into
 * q_out[hq*hd]; rotated k and plain v heads are stored at
 * k_cache + kvh*sk_head + p*sk_pos (and v likewise) when p < cache_cap.
 * Rotation and rounding as kuiops_rope_kv_append applied to the rounded
 * projections.  No reference counterpart: it fuses the mm launcher with the
 * rotary and KV-cache cat launches (CatImpl kuipy/kuiops.py:810-857) for a
 * batch-1 decode step.  K <= 4096, hd even.                                 */
KUIOPS_API int kuiops_decode_qkv_rope(int64_t hq, int64_t hkv, int64_t hd, int64_t K, int dtype, int x_kind,
                           const void *in, const int64_t *in_row, int64_t ld_in, int64_t in_rows,
                           const void *in_add, const void *norm_w, float eps, void *h_out,
                           const void *W, int64_t ldw, const float *inv_freq, const int32_t *pos,
                           void *q_out, void *k_cache, int64_t sk_head, int64_t sk_pos,
                           void *v_cache, int64_t sv_head, int64_t sv_pos, int64_t cache_cap,
                           void *stream);

/* ---- whole batch-1 decode step in one launch ---------------------------- */

/* Weights and KV cache of one decoder layer (device pointers, dtype of the
 * step): wqkv [(hq+2*hkv)*hd, d], wo [d, hq*hd], wgu [2*ffn, d] (gate rows
 * then up rows), wd [d, ffn] (nn.Linear layout, K contiguous), the two
 * RMSNorm weights [d], and the layer's K / V caches (kv head kvh, position
 * p at k_cache + kvh*sk_head + p*sk_pos, V likewise).                       */
typedef struct kuiops_step_layer {
    const void *wqkv, *wo, *wgu, *wd, *ln1, *ln2;
    void *k_cache, *v_cache;
} kuiops_step_layer;

/* n_steps (1 .. 32) greedy decode steps of a Llama-style decoder for one
 * sequence, in one launch.  `layers` points to a DEVICE array of n_layers
 * kuiops_step_layer.  The token id is read from tok[0] (device int64, an
 * index into embed [vocab, d]), the position from pos[0] and the key count
 * from kv_len[0] (device int32).  Each step: logits [vocab] (device, dtype,
 * 16-byte aligned); its token = arg-max of softmax(logits) (lowest index on
 * ties), recorded at history[pos] when history is non-null and pos <
 * hist_len; pos and kv_len advance by one and the token feeds the next step.
 * After the call tok[0], pos[0] and kv_len[0] hold the state after the last
 * step, prob[0] (optional) the last token's probability and logits the last
 * step's.  The arithmetic, rounding points and summation orders are those of
 * the per-op sequence kuiops_decode_qkv_rope -> kuiops_sdpa_decode ->
 * kuiops_decode_linear (o) -> kuiops_decode_gate_up -> kuiops_decode_linear
 * (down) per layer, then kuiops_decode_linear (LM head, RMSNorm input) and
 * kuiops_softmax_top1, so its results are bitwise those of that sequence run
 * n_steps times.  One persistent launch: work-groups take the projection row
 * blocks, attention rows and sampling rows of every step in order (the next
 * step's weights stream while a step's LM head and sampling run); the
 * vectors they hand each other live in `scratch`
 * (kuiops_decode_step_scratch_bytes(n_layers, n_steps, d, ffn, hq, hkv, hd)
 * bytes, 16-byte aligned, zero before the first call) as epoch-tagged words,
 * and `sync` (kuiops_decode_step_sync_bytes(n_layers) bytes, zero before the
 * first call) holds the LM head's completion counters, an error word, the
 * step counter and the token hand-over word.  Keep both buffers for the life
 * of the decoder (the step counter keeps old scratch contents from
 * matching).  A work-group issues its weight loads before it waits for its
 * input, so weight streaming overlaps the phase boundaries.  If a wait
 * exceeds its bound (work-groups not co-resident) the step stops waiting,
 * its results are undefined and the error word is set:
 * kuiops_decode_step_error reads and clears it.  Calls must not overlap on
 * one `sync` / `scratch` pair.  Attention runs one work-group per query row
 * over every key (the one-pass row-wide form of kuiops_sdpa_decode), so
 * cache_cap must be at most 8 * (512 / hd) * 12 keys (768 at hd 64, 384 at
 * hd 128).  Shapes: bf16 / f16, hd 64 or 128, d = hq*hd <= 4096, ffn
 * <= 8192, ffn % 8 == 0, vocab <= 32768; otherwise KUIOPS_E_UNSUPPORTED, as
 * when the step's work-group does not fit a CU (occupancy query).  No
 * reference counterpart: it replaces the whole per-token launch sequence of a
 * batch-1 greedy decode (the reference runs each aten op of generate() as its
 * own launch, infer.py:14-31, KERNELS.md).                                 */
KUIOPS_API size_t kuiops_decode_step_sync_bytes(int64_t n_layers);
KUIOPS_API size_t kuiops_decode_step_scratch_bytes(int64_t n_layers, int64_t n_steps, int64_t d, int64_t ffn,
                                                   int64_t hq, int64_t hkv, int64_t hd);
KUIOPS_API int kuiops_decode_step(int64_t n_layers, int64_t d, int64_t ffn, int64_t hq, int64_t hkv, int64_t hd,
                       int64_t vocab, int64_t cache_cap, int dtype, float eps,
                       const kuiops_step_layer *layers, int64_t sk_head, int64_t sk_pos, int64_t sv_head,
                       int64_t sv_pos, const void *embed, const void *final_norm, const void *lm_head,
                       const float *inv_freq, int64_t *tok, int32_t *pos, int32_t *kv_len,
                       int64_t *history, int64_t hist_len, float *prob, void *logits, int64_t n_steps,
                       void *scratch, size_t scratch_bytes, void *sync, size_t sync_bytes, void *stream);
/* 1 when a previous kuiops_decode_step on `sync` hit its wait bound (then
 * clears the flag), else 0; <0 on a HIP error.  Synchronises the stream.
 * The flag latches: while it is set, kuiops_decode_step launches do no work
 * (the decode state they would read is void).                              */
KUIOPS_API int kuiops_decode_step_error(void *sync, int64_t n_layers, void *stream);
/* KUIOPS_OK when kuiops_decode_step serves this shape on the current device,
 * else KUIOPS_E_UNSUPPORTED / KUIOPS_E_INVALID: the host shape gate of
 * kuiops_decode_step (including cache_cap <= 8 * (512 / hd) * 12 keys, the
 * one-pass attention's range: 768 at hd 64, 384 at hd 128) and an occupancy
 * query that one 512-thread step work-group fits a CU, which the step's
 * cross-work-group waits need (one work-group per CU, all resident).  No
 * reference counterpart: the caller's choice between the persistent step
 * and the per-op launch sequence.                                          */
KUIOPS_API int kuiops_decode_step_supported(int64_t n_layers, int64_t d, int64_t ffn, int64_t hq, int64_t hkv,
                                            int64_t hd, int64_t vocab, int64_t cache_cap, int dtype);

/* ----------------------------------------------- elementwise / mean / cat --
 * The reference's generic glue families: ElementwiseImpl
 * (kuipy/kuiops.py:150-320, its 21 aten overloads registered at
 * kuipy/registry.py:33-53), MeanImpl (kuipy/kuiops.py:860-921) and CatImpl
 * (kuipy/kuiops.py:810-857); each replaces the per-instantiation launcher of
 * kuiops/{elementwise,mean,cat}/wrapper_*.cu.j2.                            */

/* Elementwise op codes.  Values are part of the ABI. */
typedef enum kuiops_ew_op {
    KUIOPS_EW_ADD = 0,          /* a + s0 * b           (aten.add, alpha = s0)   */
    KUIOPS_EW_SUB = 1,          /* a - s0 * b           (aten.sub, alpha = s0)   */
    KUIOPS_EW_MUL = 2,
    KUIOPS_EW_DIV = 3,          /* true division                                 */
    KUIOPS_EW_NEG = 4,
    KUIOPS_EW_SILU = 5,         /* a / (1 + exp(-a))                             */
    KUIOPS_EW_RSQRT = 6,
    KUIOPS_EW_COS = 7,
    KUIOPS_EW_SIN = 8,
    KUIOPS_EW_EXP = 9,
    KUIOPS_EW_SQRT = 10,
    KUIOPS_EW_POW_SCALAR = 11,  /* a ^ s0 (aten.pow.Tensor_Scalar)               */
    KUIOPS_EW_EQ = 12,          /* comparisons: bool output                      */
    KUIOPS_EW_NE = 13,
    KUIOPS_EW_LE = 14,
    KUIOPS_EW_LT = 15,
    KUIOPS_EW_GE = 16,
    KUIOPS_EW_GT = 17,
    KUIOPS_EW_WHERE = 18,       /* a ? b : c (aten.where.self)                   */
    KUIOPS_EW_BITWISE_NOT = 19, /* integer / bool operands                       */
    KUIOPS_EW_BITWISE_AND = 20,
    KUIOPS_EW_BITWISE_OR = 21
} kuiops_ew_op;

/* out = op(in[0], in[1], in[2]) over `shape` (rank <= 8), with
 * broadcasting: operand k's element at index (i0..) is at
 * in_ptrs[k] + sum_d i_d * in_strides[k * rank + d] elements (stride 0 =
 * broadcast).  `out` is contiguous of `shape`.  n_in = the op's arity, or 1
 * for a binary op whose second operand is the scalar s1.  s0 is add / sub's
 * alpha or pow's exponent.  compute_dtype is F32 (for 16/32-bit float
 * results, aten's opmath), F64 or I64 (integers, bool, bitwise ops); every
 * operand is converted to it, and the result is rounded once to out_dtype.  */
KUIOPS_API int kuiops_elementwise(int op, int rank, const int64_t *shape, int n_in, const int *in_dtypes,
                       const void *const *in_ptrs, const int64_t *in_strides, double s0, double s1,
                       int compute_dtype, int out_dtype, void *out, void *stream);

/* out[r] = mean(x[r, 0:n]) for r < m; rows at stride ldx (elements), unit
 * stride within a row; out has x's dtype (F32, BF16, F16, F64); fp32 (fp64)
 * accumulation, the sum scaled by m / (m*n) as aten's mean.dim scales it.  */
KUIOPS_API int kuiops_mean_lastdim(int64_t m, int64_t n, int dtype, const void *x, int64_t ldx, void *out,
                        void *stream);

/* Concatenation viewed as `outer` rows: input i contributes widths[i]
 * elements to every output row, read from inputs[i] + o * outer_strides[i];
 * output rows are contiguous of sum(widths) elements, inputs in order.
 * n_inputs <= 32; elem_bytes 1, 2, 4 or 8 (a byte copy: any dtype).         */
KUIOPS_API int kuiops_cat(int n_inputs, const void *const *inputs, const int64_t *widths,
               const int64_t *outer_strides, int64_t outer, int elem_bytes, void *out, void *stream);

/* Batched decode projection for 1 <= M <= 64 sequences: the fused input
 * stage and epilogue of kuiops_decode_linear / kuiops_decode_gate_up /
 * kuiops_decode_qkv_rope, per row, over one nn.Linear weight W [N, K]
 * (K contiguous, row stride ldw).  Row m of x comes from `in` at row
 * in_row[m] (device int64, clamped to [0, in_rows)) when in_row is
 * non-null (an embedding lookup), else at row m, rows ld_in apart; x_kind:
 *   KUIOPS_X_PLAIN    x = in
 *   KUIOPS_X_RMSNORM  h = round(in + in_add[m]); x = round(w * round(h *
 *                     rsqrt(mean(h^2) + eps))); h stored to h_out[m] if set
 *   KUIOPS_X_SWIGLU   x = round(round(silu(in[:K])) * in[K:2K])
 * out_kind 0 (plain): out[m, r] = round(x_m . W[r]);
 * out_kind 1 (SwiGLU pair): rows p and p + pair_off of W -> out[m, p];
 * out_kind 2 (rotary + KV append): W = [q; k; v] heads of hd = 2 * pair_off,
 *   rows i and i + hd/2 of a head rotated at position pos[m]; q -> out[m],
 *   k / v -> caches at (m, head, pos[m]) with strides sk / sv {batch, head,
 *   position} when pos[m] < cache_cap.
 * Rounding points as the batch-1 entry points (h bit-identical; the dot
 * products differ from them only in fp32 summation order).
 * Input stages (RMSNorm, SwiGLU) and embedding rows need M <= 16 and
 * M * K * 2 <= 140 KiB (x staged in LDS); plain x takes any M <= 64.
 * With x staged (M <= 16), W must span less than 2 GiB.
 * Otherwise KUIOPS_E_UNSUPPORTED.  The unstaged (wide) form splits K over
 * work-groups when given the workspace of
 * kuiops_query_workspace(KUIOPS_OP_DECODE_ROWS_BATCHED, M, N, K) (fp32
 * partial sums, summed in split order by a second launch; no
 * initialisation needed); with none, or less, it runs unsplit.  No reference
 * counterpart: it fuses the mm launcher with the RMSNorm / SwiGLU / rotary /
 * KV-cache cat launches of a batched decode step (infer.py:57-89 generates
 * in batches).                                                              */
KUIOPS_API int kuiops_decode_rows_batched(int64_t M, int64_t N, int64_t K, int dtype, int x_kind, int out_kind,
                               const void *in, int64_t ld_in, const int64_t *in_row, int64_t in_rows,
                               const void *in_add, int64_t ld_add, const void *norm_w, float eps,
                               void *h_out, int64_t ld_h, const void *W, int64_t ldw, void *out, int64_t ld_out,
                               int64_t pair_off, int64_t hq, int64_t hkv, int64_t hd, const float *inv_freq,
                               const int32_t *pos, void *k_cache, const int64_t sk[3], void *v_cache,
                               const int64_t sv[3], int64_t cache_cap, void *workspace,
                               size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KUIOPS_H_ */
