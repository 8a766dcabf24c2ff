/*
 * sfgemm.h — C ABI of the MI355X (gfx950) matmul hot path.
 *
 * Plain C: only <stdint.h>/<stddef.h>, no HIP or CUDA headers, so the
 * Cython seam (scaffolding_amd/_cuda_ops.pyx) and any other FFI (ctypes,
 * cffi) bind it with a C compiler.  Streams and events are opaque
 * pointers; NULL means the device's default stream.
 *
 * Every function returns an int status: 0 on success, a negative SF_ERR_*
 * code otherwise.  Nothing here prints.  sf_status_string() maps a code to
 * text and sf_last_error() returns the detail of the most recent failure on
 * the calling thread.
 *
 * All matrices are row-major.  Problem sizes and leading dimensions count
 * ELEMENTS, never bytes.
 *
 * Reference interface this replaces (all /root/reference paths):
 *   _cuda_ops_decl.h:107-117   cuda_sgemm / cuda_sgemm_batched (cuBLAS)
 *   _cuda_ops_decl.h:136-137   cuda_bias_add_row_f32
 *   _cuda_ops_decl.h:69, :74   cuda_silu_f32 / cuda_gelu_f32
 *   _cuda_ops_decl.h:63        cuda_muls_f32
 *   _cuda_ops_decl.h:83-84     cuda_softmax_f32
 *   _cuda_ops.pyx:33-142       CUDA runtime calls the Cython module binds
 *                              directly (malloc/free/memcpy/device/stream/event)
 *   _cuda_ops.pyx:357-475      caching allocator (here native, in C++)
 */
#ifndef SFGEMM_H
#define SFGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* Types and status codes                                              */
/* ------------------------------------------------------------------ */

/* The two sentinels of each enum give it the value range of int, so any
 * int a caller passes (ctypes, FFI) is a valid value of the type in C++ and
 * reaches the library's validation, which rejects it (SF_ERR_INVALID_ARG). */
typedef enum {
    SF_DTYPE_INVALID = -1,
    SF_F32 = 0,   /* IEEE binary32                                  */
    SF_F16 = 1,   /* IEEE binary16                                  */
    SF_BF16 = 2,  /* bfloat16 (upper half of binary32), stored u16  */
    SF_DTYPE_RANGE_ = 0x7fffffff
} sf_dtype;

/* Epilogue applied to v = alpha * (op(A) . op(B)) in fp32 registers before
 * the single rounding to the output dtype:
 *   NONE            y = v
 *   BIAS            y = v + bias[n]
 *   BIAS_SILU       y = silu(v + bias[n])       silu(t) = t / (1 + e^-t)
 *   BIAS_GELU_TANH  y = gelu_tanh(v + bias[n])
 *   SILU            y = silu(v)
 *   GELU_TANH       y = gelu_tanh(v)
 * gelu_tanh(t) = 0.5 t (1 + tanh(0.7978845608 (t + 0.044715 t^3))). */
typedef enum {
    SF_EPI_NONE = 0,
    SF_EPI_BIAS = 1,
    SF_EPI_BIAS_SILU = 2,
    SF_EPI_BIAS_GELU_TANH = 3,
    SF_EPI_SILU = 4,
    SF_EPI_GELU_TANH = 5,
    SF_EPI_INVALID = -1,
    SF_EPI_RANGE_ = 0x7fffffff
} sf_epilogue;

#define SF_OK 0
#define SF_ERR_HIP (-1)          /* a HIP runtime call failed              */
#define SF_ERR_INVALID_ARG (-2)  /* bad size, stride, pointer or enum      */
#define SF_ERR_UNSUPPORTED (-3)  /* valid request this library does not do */
#define SF_ERR_NO_DEVICE (-4)    /* no usable GPU                          */
#define SF_ERR_OOM (-5)          /* device allocation failed               */

const char* sf_status_string(int status);
/* Detail text of the last failing call on this thread ("" if none). */
const char* sf_last_error(void);
/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int sf_version(void);

/* Test hooks: force plans the planner would not pick; none of them may
 * change a result.  No counterpart in the reference; for the library's own
 * tests only (the library never reads them from the environment).
 *   xcd_shift   0..7: each part of a persistent split tile expects the XCD
 *               this many places from its own (0: off), so every part
 *               takes the agent-scope fallback hand-off;
 *   split_spins 0..256 caps how long a split part waits for the others
 *               (0: the last part sums every slice); -1: the built-in bound;
 *   attn_parts  0, or 2..16: split every fused-attention work item into
 *               this many key ranges (at most 1 GiB of partials).
 * Process-wide; SF_ERR_INVALID_ARG outside those ranges. */
int sf_set_test_hooks(int xcd_shift, int split_spins, int attn_parts);

/* ------------------------------------------------------------------ */
/* GEMM family                                                         */
/* ------------------------------------------------------------------ */

/* C[b] = epi(alpha * op(A[b]) . op(B[b]) (+ bias)) for b in [0, batch).
 *
 * Replaces cuda_sgemm (_cuda_kernels.cu:1175-1220, decl
 * _cuda_ops_decl.h:107-111), cuda_sgemm_batched (_cuda_kernels.cu:1223-1243,
 * decl _cuda_ops_decl.h:112-117) and the separate passes
 * cuda_bias_add_row_f32 (_cuda_kernels.cu:1490-1527), cuda_silu_f32 /
 * cuda_gelu_f32 (_cuda_kernels.cu:384,428) and cuda_muls_f32
 * (_cuda_kernels.cu:237-277), which it fuses into the epilogue.
 *
 *   op(A) is M x K: A is stored M x K (lda >= K) when transA == 0, or
 *                   K x M (lda >= M) when transA != 0 ("TN", dW = dY^T X,
 *                   the four transpose cases of cuda_sgemm
 *                   _cuda_kernels.cu:1184-1217).
 *   op(B) is K x N: B is stored K x N (ldb >= N) when transB == 0, or
 *                   N x K (ldb >= K) when transB != 0 ("NT", x . W^T).
 *   C is M x N, ldc >= N.
 *   strideA/B/C: element offset between consecutive batch entries;
 *   strideA or strideB 0 broadcasts that operand over the batch (this is
 *   np.matmul's rule for a 2-D operand); when batch > 1 the entries of C
 *   must not overlap: strideC >= (M-1)*ldc + N (whole matrices apart), or
 *   strideC >= N with (batch-1)*strideC + N <= ldc (side by side within
 *   each row, e.g. attention heads written into [S, heads * D]).
 *
 * Dtypes: ab_dtype in {F32, F16, BF16} for both A and B.  c_dtype is
 * ab_dtype or F32.  bias (length N, NULL unless the epilogue has BIAS) has
 * dtype ab_dtype.  F32 inputs run on fp32 MFMA (v_mfma_f32_16x16x4_f32);
 * F16/BF16 inputs on 16-bit MFMA with fp32 accumulation.
 *
 * M, N or batch == 0 is a no-op; K == 0 writes epi(0 (+ bias)).
 * The call is asynchronous on `stream`. */
int sf_gemm(int transA, int transB,
            int64_t M, int64_t N, int64_t K, int64_t batch,
            const void* A, int64_t lda, int64_t strideA,
            const void* B, int64_t ldb, int64_t strideB,
            void* C, int64_t ldc, int64_t strideC,
            sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
            const void* bias, sf_epilogue epi, void* stream);

/* sf_gemm with a residual added after the epilogue, before the single
 * rounding to c_dtype:
 *   C[b] = epi(alpha * op(A[b]) . op(B[b]) (+ bias)) + R[b]
 * R[b] is M x N of dtype c_dtype, row stride ldr >= N, batch stride
 * strideR (0 broadcasts).  R may be C itself (R == C with ldr == ldc and
 * strideR == strideC: an in-place residual accumulate); any other overlap
 * of R and C is undefined.  Replaces the residual adds of the reference's
 * DiT block, x + self_out(attn) and x + ff(h) (diffusion/models.py:560-564,
 * :586-589), which run as separate host-side passes there.  Every other
 * argument, rule and error as sf_gemm; R == NULL is SF_ERR_INVALID_ARG. */
int sf_gemm_add(int transA, int transB,
                int64_t M, int64_t N, int64_t K, int64_t batch,
                const void* A, int64_t lda, int64_t strideA,
                const void* B, int64_t ldb, int64_t strideB,
                void* C, int64_t ldc, int64_t strideC,
                sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                const void* bias, sf_epilogue epi,
                const void* R, int64_t ldr, int64_t strideR, void* stream);

/* sf_gemm for callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  No
 * counterpart in the reference (cuBLAS keeps its workspace internally).
 *
 * Same arguments, rules, kernels and results (bit for bit) as sf_gemm.  Where
 * sf_gemm's plan splits tiles along k (it then allocates a per-device
 * workspace on first use), this entry point takes the fp32 partials and the
 * arrival counters from a fixed per-device scratch array of
 * SF_NOALLOC_SCRATCH_BYTES inside the library, which each GPU the library
 * runs on holds until the process ends; it calls no hipMalloc, hipFree or
 * other allocating routine.  A plan whose workspace exceeds the scratch
 * returns SF_ERR_UNSUPPORTED (no plan does on devices of up to 256 CUs,
 * which covers every gfx950 part; on more CUs, tail splits of up to 256
 * parts fit and larger ones are refused).  The first call on a device looks
 * the scratch address up (hipGetSymbolAddress): under HIP graph capture,
 * make one uncaptured call on that device first; the call itself launches
 * kernels only (counters are cleared by a fill kernel, no memset node).
 * Every call on one device shares that device's scratch: calls that overlap
 * on one device (different streams, or host threads without ordering) race;
 * calls on one stream are ordered by it.  Asynchronous on `stream`. */
#define SF_NOALLOC_SCRATCH_BYTES ((size_t)64 * 1024 * 1024 + 4096)
int sf_gemm_noalloc(int transA, int transB,
                    int64_t M, int64_t N, int64_t K, int64_t batch,
                    const void* A, int64_t lda, int64_t strideA,
                    const void* B, int64_t ldb, int64_t strideB,
                    void* C, int64_t ldc, int64_t strideC,
                    sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                    const void* bias, sf_epilogue epi, void* stream);

/* Diagnostic twin of sf_gemm: validates the same arguments and writes the
 * name of the kernel sf_gemm would launch (e.g. "gemm tile 256x256",
 * "gemm skinny") into buf[len] without launching anything.  Host-only, no
 * reference counterpart (cuBLAS chooses its kernels internally). */
int sf_gemm_plan(int transA, int transB,
                 int64_t M, int64_t N, int64_t K, int64_t batch,
                 const void* A, int64_t lda, int64_t strideA,
                 const void* B, int64_t ldb, int64_t strideB,
                 void* C, int64_t ldc, int64_t strideC,
                 sf_dtype ab_dtype, sf_dtype c_dtype, float alpha,
                 const void* bias, sf_epilogue epi, char* buf, int len);

/* Sum over one axis: x viewed as [outer, dim_size, inner] (C-contiguous),
 *   out[o * inner + i] = sum_{d < dim_size} x[(o * dim_size + d) * inner + i].
 * Replaces cuda_sum_dim_f32 (_cuda_kernels.cu:858-883, decl
 * _cuda_ops_decl.h:95-96); the bias gradient of a linear layer is the
 * column sum outer = 1, dim_size = rows, inner = out_features (reference
 * autograd.py:819).  in_dtype in {F32, F16, BF16}; out_dtype is in_dtype or
 * F32; fp32 accumulation in an order fixed by the shape (results do not
 * vary between calls).  dim_size == 0 writes zeros.  Column sums over many
 * rows use the library's per-device workspace.  Asynchronous on `stream`. */
int sf_sum_dim(const void* x, void* out, int64_t outer, int64_t dim_size, int64_t inner,
               sf_dtype in_dtype, sf_dtype out_dtype, void* stream);

/* Fused attention forward, head size D in {8, 16, ..., 64}:
 *   O[b] = softmax(scale * Q[b] K[b]^T) V[b],   b in [0, batch),
 * Q[b] Sq x D, K[b] and V[b] Sk x D, O[b] Sq x D, row strides ld*,
 * batch strides stride* (elements), 16-bit dtype (F16 or BF16), fp32
 * accumulation and softmax.  One launch; the Sq x Sk scores never reach
 * memory.  With scale * log2(e) <= 1 (the usual 1/sqrt(D)) Q is
 * multiplied by scale * log2(e) in registers, one more rounding of each Q
 * element into the dtype, so the score products come out as exponents;
 * otherwise the scale is applied to the fp32 scores.  Replaces the three-launch GPU path of
 * scaled_dot_product_attention (nn/functional.py:310-321: dev_batched_matmul_nt,
 * dev_muls, dev_softmax, dev_batched_matmul) when there is no mask and no
 * dropout.  Requires D a multiple of 8 up to 64 (other head sizes return
 * SF_ERR_UNSUPPORTED), 0 < scale < inf, 16-byte aligned rows and
 * strides (SF_ERR_UNSUPPORTED otherwise: callers fall back to sf_gemm +
 * sf_softmax_rows).  Any Sk >= 1.  When the last round of work items
 * (256 query rows of one batch entry) would leave most of the GPU idle,
 * those items are split over key ranges whose fp32 partials pass through
 * the library's per-device workspace (as sf_sum_dim's do) and are merged
 * by a second launch. */
int sf_attention(const void* Q, int64_t ldq, int64_t strideQ,
                 const void* K, int64_t ldk, int64_t strideK,
                 const void* V, int64_t ldv, int64_t strideV,
                 void* O, int64_t ldo, int64_t strideO,
                 int64_t batch, int64_t Sq, int64_t Sk, int64_t D,
                 float scale, sf_dtype dtype, void* stream);

/* sf_attention over batch x heads (b, h) pairs, each operand addressed as
 *   Q + b * strideQ + h * headQ  (rows of ldq), likewise K, V and O.
 * With a packed projection qkv [batch, S, 3 * heads * 64] this reads Q, K
 * and V in place (ld = 3 * heads * 64, head stride 64, K and V at column
 * offsets heads * 64 and 2 * heads * 64) and writes O straight into
 * [batch, S, heads * 64] (ldo = heads * 64, head stride 64): the head split
 * qkv[..., i*C:(i+1)*C].reshape(B, N, H, D).transpose(0, 2, 1, 3) and the
 * merge .transpose(0, 2, 1, 3).reshape(B, N, C) of the reference's DiT
 * block (diffusion/models.py:551-559, :573-577) cost no copies.  The
 * output's (b, h) entries must not overlap (heads side by side within a
 * row, or whole matrices apart).  Rules and errors as sf_attention. */
int sf_attention_heads(const void* Q, int64_t ldq, int64_t strideQ, int64_t headQ,
                       const void* K, int64_t ldk, int64_t strideK, int64_t headK,
                       const void* V, int64_t ldv, int64_t strideV, int64_t headV,
                       void* O, int64_t ldo, int64_t strideO, int64_t headO,
                       int64_t batch, int64_t heads, int64_t Sq, int64_t Sk, int64_t D,
                       float scale, sf_dtype dtype, void* stream);

/* Layer normalisation of `rows` contiguous rows of `cols` elements, with an
 * optional per-group affine modulation (adaptive layer norm):
 *   mu = mean(x[r,:]),  var = mean((x[r,:] - mu)^2)  (population variance)
 *   h  = (x[r,c] - mu) / sqrt(var + eps) * gamma[c] + beta[c]
 *   y[r,c] = h * (1 + mod_scale[g, c]) + mod_shift[g, c],  g = r / group_rows
 * gamma / beta: length cols, dtype `dt`, NULL for 1 / 0.  mod_scale /
 * mod_shift: NULL for none, else rows of `cols` elements of dtype `dt`,
 * `mod_ld` elements apart (both may point into one [groups, 2 * cols]
 * projection, shift = scale + cols).  mean_out / rstd_out: NULL, or fp32
 * arrays of `rows` receiving mu and 1 / sqrt(var + eps).  x, y of dtype
 * `dt` (F32, F16, BF16); fp32 arithmetic, one rounding per output; x == y
 * is allowed.
 * Replaces cuda_layer_norm_f32 (_cuda_kernels.cu:1013-1093, decl
 * _cuda_ops_decl.h:99-101, the GPU path of
 * nn.LayerNorm, nn/layers.py:470-493; CPU path :512-521) and, with the
 * modulation, AdaLayerNorm.forward (diffusion/models.py:479-486: LayerNorm,
 * then h * (scale + 1) + shift on the host).  Asynchronous on `stream`. */
int sf_layer_norm(const void* x, void* y, int64_t rows, int64_t cols,
                  const void* gamma, const void* beta, float eps,
                  const void* mod_scale, const void* mod_shift, int64_t mod_ld, int64_t group_rows,
                  float* mean_out, float* rstd_out, sf_dtype dt, void* stream);

/* RMS normalisation: y[r,c] = x[r,c] / sqrt(mean(x[r,:]^2) + eps) * gamma[c]
 * (gamma NULL for 1), fp32 arithmetic, dtype `dt` in and out, x == y
 * allowed.  Replaces cuda_rms_norm_f32 (_cuda_kernels.cu:1102-1160, decl
 * _cuda_ops_decl.h:102; CPU path nn/layers.py:576-581). */
int sf_rms_norm(const void* x, void* y, int64_t rows, int64_t cols,
                const void* gamma, float eps, sf_dtype dt, void* stream);

/* y = a + b over n contiguous elements of dtype `dt` (fp32 add, one
 * rounding); y may equal a or b.  Replaces cuda_add_f32 (decl
 * _cuda_ops_decl.h:56, dev_add _cuda_ops.pyx:965-966): the residual add where it is not fused into a
 * GEMM (sf_gemm_add). */
int sf_add(const void* a, const void* b, void* y, int64_t n, sf_dtype dt, void* stream);

/* Row softmax: y[r,:] = softmax(scale * x[r,:]) for r in [0, rows).
 * Contiguous rows of `cols` elements.  Replaces cuda_softmax_f32
 * (_cuda_kernels.cu:473-640, decl _cuda_ops_decl.h:83-84) with the
 * dev_muls pre-scale of scaled_dot_product_attention
 * (nn/functional.py:315-316) folded in.  in/out dtypes independently
 * F32/F16/BF16; arithmetic is fp32. */
int sf_softmax_rows(const void* x, void* y, int64_t rows, int64_t cols,
                    sf_dtype in_dtype, sf_dtype out_dtype, float scale,
                    void* stream);

/* Row softmax with an additive mask, the attn_mask of
 * scaled_dot_product_attention (reference nn/functional.py:339-341:
 * scores *= scale; scores += mask, NumPy broadcasting):
 *   y[r, j] = softmax_j(scale * x[r, j] + mask[off(r) + j * stride_col]),
 * r = b * rows_per_batch + i,
 * off(r) = (b / inner_batches) * stride_outer + (b % inner_batches) * stride_inner
 *          + i * stride_row.
 * A zero stride broadcasts the mask over that axis; the batch index b of
 * the scores' leading dims, flattened, splits into outer and inner groups
 * (e.g. [B, H] scores with a [B, 1, Sq, Sk] mask: inner_batches = H,
 * stride_inner = 0, stride_outer = Sq * Sk).  x and y are `dtype` (y == x
 * allowed); the mask is `dtype` or F32, stride_col 0 or 1.  A row whose
 * mask is -inf everywhere gives NaN, as the reference's NumPy does.  No
 * counterpart in the reference's CUDA kernels (its masked SDPA runs on the
 * host); asynchronous on `stream`. */
int sf_softmax_rows_masked(const void* x, void* y, int64_t rows, int64_t cols,
                           sf_dtype dtype, float scale,
                           const void* mask, sf_dtype mask_dtype,
                           int64_t rows_per_batch, int64_t inner_batches,
                           int64_t stride_outer, int64_t stride_inner,
                           int64_t stride_row, int64_t stride_col, void* stream);

/* Standalone elementwise ops over n contiguous elements of dtype `dt`
 * (arithmetic in fp32, one rounding on store).  x == y is allowed.
 *   sf_silu  replaces cuda_silu_f32 (_cuda_kernels.cu:384)
 *   sf_gelu  replaces cuda_gelu_f32 (_cuda_kernels.cu:428), tanh form
 *   sf_muls  replaces cuda_muls_f32 (_cuda_kernels.cu:237-277)          */
int sf_silu(const void* x, void* y, int64_t n, sf_dtype dt, void* stream);
int sf_gelu(const void* x, void* y, int64_t n, sf_dtype dt, void* stream);
int sf_muls(const void* x, float s, void* y, int64_t n, sf_dtype dt,
            void* stream);

/* Dropout over n contiguous elements: mask[i] = 1 / (1 - p) if u_i >= p
 * else 0, y[i] = x[i] * mask[i] (fp32 arithmetic, one rounding on store;
 * x == y allowed; mask may be NULL).  u_i in [0, 1) comes from the
 * counter-based Philox4x32-10 stream (seed, offset): the same arguments
 * give the same mask on any device and launch.  0 <= p < 1.
 * Replaces cuda_dropout_f32 (_cuda_kernels.cu:1431-1480, bound at
 * _cuda_ops.pyx:1243-1255): the same keep rule and scale; the random
 * stream is this library's own, not cuRAND's. */
int sf_dropout(const void* x, void* y, void* mask, int64_t n, sf_dtype dt,
               float p, uint64_t seed, uint64_t offset, void* stream);

/* C[i,j] += bias[j] in place on a contiguous M x N matrix.
 * Replaces cuda_bias_add_row_f32 (_cuda_kernels.cu:1490-1527,
 * decl _cuda_ops_decl.h:136-137). */
int sf_bias_add_rows(void* C, const void* bias, int64_t M, int64_t N,
                     sf_dtype dt, void* stream);

/* Dtype conversion of n contiguous elements (RNE; NaN stays NaN, +-Inf
 * and signed zero are preserved).  Has no reference counterpart: the
 * reference stores bfloat16 as float32 (dtype.py:31); this library keeps
 * real 16-bit storage and converts on the device. */
int sf_cast(const void* x, sf_dtype in_dtype, void* y, sf_dtype out_dtype,
            int64_t n, void* stream);

/* ------------------------------------------------------------------ */
/* Runtime: devices, memory, streams, events                           */
/* (the CUDA runtime calls _cuda_ops.pyx:33-142 binds directly)        */
/* ------------------------------------------------------------------ */

int sf_get_device_count(int* count);
int sf_set_device(int device);
int sf_get_device(int* device);
int sf_device_synchronize(void);
/* name: NUL-terminated into buf[len]; arch: e.g. "gfx950". */
int sf_get_device_name(int device, char* buf, int len);
int sf_get_device_arch(int device, char* buf, int len);
int sf_get_device_props(int device, int* cu_count, int64_t* total_mem,
                        int* clock_khz, int* l2_bytes);
int sf_mem_get_info(size_t* free_bytes, size_t* total_bytes);

/* Raw allocation (hipMalloc / hipFree) on the current device. */
int sf_malloc(void** ptr, size_t nbytes);
int sf_free(void* ptr);

/* Caching allocator (replaces _cuda_ops.pyx:357-475): per-device pools
 * keyed by exact size rounded up to 256 bytes, capped per device (bytes
 * beyond the cap go back to hipFree).  sf_cache_alloc switches to
 * `device` for the allocation and restores the caller's device. */
int sf_cache_alloc(int device, size_t nbytes, void** ptr, size_t* got_bytes);
int sf_cache_free(int device, void* ptr, size_t nbytes);
int sf_cache_empty(int device);          /* device < 0: every device */
int sf_cache_stats(int device, size_t* pooled_bytes, size_t* live_bytes);
int sf_cache_set_limit(size_t bytes_per_device);
/* Bytes of the per-device workspace that split plans (sf_gemm, sf_sum_dim,
 * sf_attention) allocate on first use, on `device` (< 0: every device); 0
 * before any such call.  Diagnostic, no reference counterpart. */
int sf_workspace_bytes(int device, size_t* bytes);

/* Copies; synchronous w.r.t. the host when stream is NULL. */
int sf_memcpy_h2d(void* dst, const void* src, size_t nbytes, void* stream);
int sf_memcpy_d2h(void* dst, const void* src, size_t nbytes, void* stream);
int sf_memcpy_d2d(void* dst, const void* src, size_t nbytes, void* stream);
/* Fill nbytes with zero using a kernel (never a memset node). */
int sf_zero(void* dst, size_t nbytes, void* stream);

int sf_stream_create(void** stream);     /* default priority, non-blocking */
int sf_stream_destroy(void* stream);
int sf_stream_synchronize(void* stream);

int sf_event_create(void** event);
int sf_event_destroy(void* event);
int sf_event_record(void* event, void* stream);
int sf_event_synchronize(void* event);
int sf_stream_wait_event(void* stream, void* event);
int sf_event_elapsed_ms(float* ms, void* start, void* end);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* SFGEMM_H */
