/*
 * circatt.h -- C ABI of libcircatt, the MI355X (gfx950) circulant attention
 * library.  Drop-in compute layer for CirculantAttention.jl's hot path: the
 * reference reaches these operations through @cuda kernels, NNlib and
 * CUSPARSE.bmm!; a host binding (Julia ccall, Python ctypes) calls these
 * entry points instead.  Citations are file:line in the reference repository.
 *
 * Conventions
 *  - All array pointers are device pointers owned by the caller.  Nothing in
 *    an entry point allocates device memory; the fused backward takes a
 *    caller-provided workspace (size from circatt_fused_bwd_workspace_bytes).
 *  - Arrays use the reference's Julia column-major layout.  A signal of Julia
 *    size (N1[,N2], C, nb) holds (pixel r, channel c, batch b) at
 *    r + P*(c + C*b), P = N1*N2, r = i1 + N1*i2.  dtype CIRCATT_C32 signals
 *    are ComplexF32, interleaved (re, im).
 *  - A Circulant of size (P, P, nb) is CSR with K = ws^nsp slots per row:
 *    rowPtr (P+1, nb) and colVal (P*K, nb) Int32 1-based, nzVal (P*K, nb)
 *    Float32 (src/circulant.jl:64-106, src/array.jl:1-18).  Entry points that
 *    take nzVal use the circulant pattern implied by (nsp, n1, n2, ws).
 *  - nsp is 1 or 2; for nsp == 1, n2 is ignored.  ws must be odd
 *    (src/circulant.jl:65,87).
 *  - stream is a hipStream_t (NULL = default stream).  Launches are
 *    asynchronous; arguments are validated on the host before any launch.
 *  - Return value: CIRCATT_OK or a negative error code; circatt_last_error()
 *    returns a message for the calling thread's last failure.
 */
#ifndef CIRCATT_H
#define CIRCATT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CIRCATT_OK 0
#define CIRCATT_ERR_INVALID (-1)     /* bad argument (the reference's @assert) */
#define CIRCATT_ERR_UNSUPPORTED (-2) /* valid but not implemented here */
#define CIRCATT_ERR_HIP (-3)         /* HIP runtime error */

/* Similarity kinds: DotSimilarity / DistanceSimilarity (src/similarity.jl:1-29). */
#define CIRCATT_DOT 0
#define CIRCATT_DISTANCE 1

/* Element types of signals: Float32, ComplexF32. */
#define CIRCATT_F32 0
#define CIRCATT_C32 1

/*
 * Layout flag, OR-ed into dtype of the fused entry points (circatt_fused_*):
 * q, k, v, y, dy and the gradients are channels-last, Julia size
 * (C, N1[,N2], B): (channel c, pixel r, batch b) at c + C*(r + P*b)
 * (ComplexF32: interleaved (re, im) elements in that order).  The kernels
 * read and write this layout directly, so a model that keeps its features
 * channels-last (the layout convolutions favour) needs no transposes around
 * the attention.  lse and the workspace keep their layout.  No counterpart in
 * the reference (which is planar only); other entry points reject the flag.
 */
#define CIRCATT_CHANNELS_LAST 16

/* Library version (major*10000 + minor*100 + patch). */
int circatt_version(void);

/*
 * Arithmetic of the fused kernels' matrix products.  The reference computes
 * in Float32 throughout; it has no counterpart of this switch.
 *   CIRCATT_MATH_SPLIT_F16 (default): each Float32 operand is split into two
 *     f16 halves and a product is taken as hi*hi + lo*hi + hi*lo on the f16
 *     matrix cores with Float32 accumulation (relative error near 2^-21 per
 *     operand, the order of Float32 rounding).  Operands are scaled by powers
 *     of two per work item (a 16x16 tile of one head, 8x16 for heads of 32
 *     real components) before the split, so
 *     the halves keep Float32's range: inputs of any magnitude (1e-7 and 1e4
 *     are tested) give Float32-class results.  Where q.k scores are so large
 *     that the halves could overflow, a slower exact-scale walk takes over.
 *   CIRCATT_MATH_F32: Float32 matrix products.
 * Like any attention backward that recomputes the probabilities from the
 * stored log-sum-exp, the fused backward loses precision once scores reach
 * ~1e3 (Float32 rounding of the score itself); the reference's own Float32
 * computation misses the gradient tolerance there as well.
 * Process-wide; takes effect for launches after the call.
 */
#define CIRCATT_MATH_SPLIT_F16 0
#define CIRCATT_MATH_F32 1
int circatt_set_math(int mode);
int circatt_get_math(void);

/* Message describing the calling thread's last error ("" if none). */
const char *circatt_last_error(void);

/*
 * Circulant sparsity pattern, replicated over nb batches.
 * Replaces cucirculant(M,N) / cucirculant(M,N1,N2) + its kernel
 * (src/circulant.jl:46-106) and the batch repeat in Circulant{T}(M, dims)
 * (src/array.jl:6-11).  rowptr: (P+1, nb), colval: (P*K, nb), Int32 1-based,
 * bit-identical to the reference, also for ws > N.
 */
int circatt_pattern(int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t nb, int32_t *rowptr,
                    int32_t *colval, void *stream);

/*
 * nzval[:, b] = scale * similarity(x[..., b], y[..., b]) on the pattern.
 * Replaces circulant_similarity! and its Dot / Distance kernels
 * (src/similarity.jl:31-103, :138-142).  x is the row (query) argument, y the
 * column (key) argument; Dot: Re(sum_c x*conj(y)), Distance:
 * -sum_c |x-y|^2 / 2.  x, y: (P, C, nb) of dtype; nzval: (P*K, nb) Float32.
 * circulant_attention (src/attention.jl:19-23) uses scale = 1/sqrt(C).
 */
int circatt_similarity(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                       int64_t C, int64_t nb, float scale, const void *x, const void *y,
                       float *nzval, void *stream);

/*
 * Row softmax over the K slots of each of `rows` rows (rows = P*nb); in == out
 * allowed.  Replaces circulant_softmax! / NNlib.softmax(::Circulant)
 * (src/similarity.jl:105-126).
 */
int circatt_softmax(int64_t K, int64_t rows, const float *in, float *out, void *stream);

/*
 * dS = A .* (dA .- sum(A .* dA, dims=slots)).  Replaces the softmax pullback
 * (src/rrules.jl:42-56, NNlib.∇softmax_data).  dS may alias dA.
 */
int circatt_softmax_bwd(int64_t K, int64_t rows, const float *A, const float *dA, float *dS,
                        void *stream);

/*
 * y = A ⊗ x (trans = 0) or y = Aᵀ ⊗ x (trans = 1) with A = nzval on the
 * pattern; x, y: (P, C, nb) of dtype (real A times complex x is the promotion
 * of src/batchedmul.jl:72-75).  Replaces circulant_attention!(y, A, x) /
 * circulant_transposed_attention! (src/attention.jl:53-80) and their
 * CUSPARSE.bmm! calls (src/batchedmul.jl:82-110).  Multi-head ⨷
 * (src/attention.jl:89-103) is the same call with C = channels/nheads and
 * nb = nheads*B.
 */
int circatt_apply(int trans, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t C,
                  int64_t nb, const float *nzval, const void *x, void *y, void *stream);

/*
 * Pullback of nzval = scale * similarity(x, y):
 *   Dot:      dx = scale * dS ⊠ y,            dy = scale * dSᵀ ⊠ x
 *   Distance: dx = scale * (dS ⊠ y - rowsum(dS) .* x),
 *             dy = scale * (dSᵀ ⊠ x - colsum(dS) .* y)
 * Replaces the similarity rrules (src/rrules.jl:1-32) including their
 * sum(ΔS; dims=1/2) (src/array.jl:119-130).  dx or dy may be NULL.
 */
int circatt_similarity_bwd(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                           int64_t C, int64_t nb, float scale, const float *dS, const void *x,
                           const void *y, void *dx, void *dy, void *stream);

/*
 * sum(A; dims=2) (out: (P, nb)) and sum(A; dims=1) (out: (P, nb)) of a
 * Circulant's nzval (src/array.jl:119-130, :156-177).
 */
int circatt_rowsum(int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t nb, const float *nzval,
                   float *out, void *stream);
int circatt_colsum(int nsp, int64_t n1, int64_t n2, int32_t ws, int64_t nb, const float *nzval,
                   float *out, void *stream);

/*
 * Z[:, b] = alpha_b * X[:, b] + beta_b * Y[:, b] over nzval slices of nnz
 * entries, alpha_b = alpha ? alpha[b] : alpha0 (same for beta; Y may be NULL).
 * Covers X + Y, X - Y, c*X, -X (src/array.jl:66-81) and scale(c, A) with c of
 * size (1,1,nh,B) (src/array.jl:179-189); Z may alias X or Y.
 */
int circatt_axpby(int64_t nnz, int64_t nb, const float *alpha, float alpha0, const float *X,
                  const float *beta, float beta0, const float *Y, float *Z, void *stream);

/*
 * out[b] = sum_i X[i, b] * Y[i, b] over nnz entries per batch (Y == NULL:
 * sum_i X[i, b]); accumulated in double in a fixed order, so results are
 * reproducible.  Covers dot(X, Y) (src/array.jl:83-85, nb = 1 over all
 * batches), sum(A) and sum(A; dims=(1,2)) (src/array.jl:132-177) and the ∂c
 * of the scale rrule (src/rrules.jl:101-104).  workspace: at least
 * circatt_batch_dot_workspace_bytes(nnz, nb) bytes of device memory.
 */
int64_t circatt_batch_dot_workspace_bytes(int64_t nnz, int64_t nb);
int circatt_batch_dot(int64_t nnz, int64_t nb, const float *X, const float *Y, float *out,
                      void *workspace, int64_t workspace_bytes, void *stream);

/*
 * Fused forward of circulant (multi-head) attention without materialising A:
 * for head g of batch b (channels g*dh .. g*dh+dh-1, dh = C/nheads),
 *   y = softmax_rows(scale * sim(q, k)) ⊗ v,   scale = 1/sqrt(dh),
 * and lse[r, g + nheads*b] = log(sum_c exp(scale * sim(q_r, k_c))).
 * Equals circulant_attention (src/attention.jl:19-26, nheads = 1) and
 * circulant_mh_attention (src/attention.jl:38-42) for the returned y.
 * q, k, v, y: (P, C, B) of dtype; lse: (P, nheads*B) Float32.
 * Any number of channels per head (the reference's similarity loops over
 * any C, src/similarity.jl:97-99): heads of up to 64 real components run on
 * kernels that hold a pixel's components at once, wider heads on kernels
 * that sum the score products over 32-component chunks and form the outputs
 * in 64-component passes.  Windows whose 2D block columns exceed the LDS
 * budget (ws beyond 63) return CIRCATT_ERR_UNSUPPORTED.
 */
int circatt_fused_fwd(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                      int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                      const void *v, void *y, float *lse, void *stream);

/* Bytes of workspace circatt_fused_bwd needs (per-row D = <dy, y>). */
int64_t circatt_fused_bwd_workspace_bytes(int nsp, int64_t n1, int64_t n2, int64_t nheads,
                                          int64_t B);

/*
 * Fused backward matching the composition of the rrules of similarity,
 * softmax and ⊗ (src/rrules.jl:1-72) and the q, k scaling of
 * src/attention.jl:21: given dy, returns dq, dk, dv.  lse from
 * circatt_fused_fwd.  No atomics: a query-centric pass writes dq, a
 * key-centric pass writes dk and dv.
 */
int circatt_fused_bwd(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                      int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                      const void *v, const void *y, const void *dy, const float *lse, void *dq,
                      void *dk, void *dv, void *workspace, int64_t workspace_bytes,
                      void *stream);

/*
 * The two passes of circatt_fused_bwd, for callers that time or schedule them
 * separately.  circatt_fused_bwd_dq writes dq and the per-row D = <dy, y>
 * into workspace; circatt_fused_bwd_dkdv reads that D and writes dk, dv, so
 * it must follow circatt_fused_bwd_dq on the same stream with the same
 * workspace.
 */
int circatt_fused_bwd_dq(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                         int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                         const void *v, const void *y, const void *dy, const float *lse,
                         void *dq, void *workspace, int64_t workspace_bytes, void *stream);
int circatt_fused_bwd_dkdv(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                           int64_t C, int64_t nheads, int64_t B, const void *q, const void *k,
                           const void *v, const void *dy, const float *lse, void *dk, void *dv,
                           const void *workspace, int64_t workspace_bytes, void *stream);

/*
 * circatt_fused_bwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * per-row D = <dy, y> lives in a fixed device array inside the library, one
 * per GPU, held until the process ends: 16 MiB, i.e. at most
 * circatt_fused_bwd_noalloc_max_rows() = 4194304 rows (P * nheads * B);
 * larger problems fail with CIRCATT_ERR_INVALID.  The entry point calls no
 * allocating routine.  Every call on one GPU shares that array: calls that
 * overlap on one GPU (different streams, or different host threads) race
 * and must be serialised by the caller.  Nothing in the array needs to start
 * at zero (the dq pass writes every row's D before the dk/dv pass reads it).
 */
int64_t circatt_fused_bwd_noalloc_max_rows(void);
int circatt_fused_bwd_noalloc(int kind, int dtype, int nsp, int64_t n1, int64_t n2, int32_t ws,
                              int64_t C, int64_t nheads, int64_t B, const void *q,
                              const void *k, const void *v, const void *y, const void *dy,
                              const float *lse, void *dq, void *dk, void *dv, void *stream);

/*
 * Batch-dimension operations on a Circulant's CSR arrays (and other device
 * arrays), so that a host binding needs no array-library kernels of its own:
 *
 * circatt_fill: dst[i] = value for i < n.  The nzVal = 1 of a new pattern
 * (CUDA.ones at src/circulant.jl:68,90), a constant cotangent made dense.
 *
 * circatt_copy_blocks: for o < nouter, i < ninner, copies block_bytes bytes
 * from src + o*src_stride_outer + i*src_stride_inner to
 * dst + o*dst_stride_outer + i*dst_stride_inner (all in bytes; a stride of 0
 * replicates).  repeat over batch dims (src/array.jl:9,49-52), cat along a
 * batch dim (src/array.jl:62-64), the broadcast of a scale factor over heads
 * or batches (src/array.jl:179-186).  Destination blocks must not overlap each
 * other or the source; works on any element type (16, 8, 4 or 1-byte units,
 * the widest that divides every address, size and stride).
 *
 * circatt_sum_middle: dst[i + inner*o] = sum_s src[i + inner*(s + nsum*o)]
 * for a column-major (inner, nsum, outer) Float32 array, summed in double in
 * order of s.  sum(A; dims=d) over a batch dim d (src/array.jl:132-154), the
 * ∂c of the scale rrule over c's size-1 dims (src/rrules.jl:98-104), and the
 * pullback of repeat.
 *
 * circatt_count_unequal: *count (one device int64, overwritten) = the number
 * of i < n with a[i] != b[i], comparing 32-bit words (kind 0: Int32 rowPtr,
 * colVal) or Float32 values as floats (kind 1: -0 == 0, NaN != NaN).  == of
 * Circulants (src/array.jl:87-117) reads the count back.
 */
int circatt_fill(float *dst, int64_t n, float value, void *stream);
int circatt_copy_blocks(void *dst, const void *src, int64_t block_bytes, int64_t ninner,
                        int64_t dst_stride_inner, int64_t src_stride_inner, int64_t nouter,
                        int64_t dst_stride_outer, int64_t src_stride_outer, void *stream);
int circatt_sum_middle(const float *src, float *dst, int64_t inner, int64_t nsum, int64_t outer,
                       void *stream);
int circatt_count_unequal(int kind, int64_t n, const void *a, const void *b, int64_t *count,
                          void *stream);

/*
 * Device memory helpers for hosts without a GPU array package (the reference
 * gets these from CUDA.jl).  kind: 0 host->device, 1 device->host,
 * 2 device->device.
 */
int circatt_malloc(void **ptr, int64_t bytes);
int circatt_free(void *ptr);
int circatt_memcpy(void *dst, const void *src, int64_t bytes, int kind);
int circatt_stream_synchronize(void *stream);

#ifdef __cplusplus
}
#endif

#endif /* CIRCATT_H */
