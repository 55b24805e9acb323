/*
 * popcorn_amd C ABI: hand-written gfx950 (MI355X) kernels for Popcorn's
 * transformer-block ops, reached from Python through ctypes.
 *
 * Conventions shared by every entry point:
 *   - every pointer is a device pointer owned by the caller (torch);
 *   - sizes and strides are int64, strides count elements, the last dimension
 *     is always contiguous;
 *   - `stream` is a hipStream_t of the current HIP device (NULL: that device's
 *     null stream), and the pointers are memory of that device; work is
 *     enqueued there and nothing synchronises;
 *   - the return value is a PK_* status; on anything but PK_OK the reason is in
 *     pk_last_error() (a per-thread string). No entry point falls back to
 *     another implementation: an unsupported call is an error.
 *
 * Popcorn has no C ABI of its own (its implementations are Python callables
 * registered with `op.register(name, source=...)`, core/dispatcher.py:324-345).
 * Each entry point below names the Popcorn reference whose arithmetic it
 * replaces and the first-party implementation it stands beside.
 */
#ifndef POPCORN_AMD_H
#define POPCORN_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_ABI_VERSION 5

/* status codes */
#define PK_OK 0
#define PK_ERR_INVALID 1     /* bad argument: null pointer, negative size, misalignment */
#define PK_ERR_UNSUPPORTED 2 /* valid call outside what the kernels implement */
#define PK_ERR_HIP 3         /* the HIP runtime refused a launch */

/* element types */
#define PK_F32 0
#define PK_BF16 1
#define PK_F16 2

/* ABI version of the loaded library (PK_ABI_VERSION at build time). */
int pk_version(void);

/* Message of the last failing call on this thread ("" after a success). */
const char* pk_last_error(void);

/*
 * SwiGLU forward, y = silu(a) * b over n elements, all of dtype `dtype`.
 * Rounding follows torch eager: silu is rounded to `dtype`, then the product.
 * Replaces: reference `swiglu` (kernels/swiglu.py:9-18, `F.silu(a) * b`);
 * stands beside the CUDA `fwd` host function (impls/swiglu.cu:77-101).
 */
int pk_swiglu_fwd(const void* a, const void* b, void* y, int64_t n, int dtype, void* stream);

/*
 * SwiGLU backward: s = sigmoid(a); da = dy*b*s*(1 + a*(1-s)); db = dy*a*s,
 * computed in fp32 and rounded once. Replaces torch autograd of the reference
 * (kernels/swiglu.py:18); stands beside `bwd` (impls/swiglu.cu:103-130).
 */
int pk_swiglu_bwd(const void* dy, const void* a, const void* b, void* da, void* db, int64_t n, int dtype,
                  void* stream);

/*
 * RMSNorm forward over `rows` contiguous rows of `cols` elements:
 *   r = 1/sqrt(mean(x^2) + eps); n = round_x(x*r); y = n * w [+ bias],
 * each product and sum rounded to w_dtype. x has `dtype`; w, bias and y have
 * `w_dtype`, which is `dtype`, or PK_F32 with a 16-bit x (torch promotes a
 * 16-bit normalised row times an fp32 weight to fp32). bias may be NULL;
 * rstd (fp32 [rows]) may be NULL and otherwise receives r for the backward.
 * Replaces: reference `rms_norm` (kernels/rms_norm.py:16-30) with `rms`
 * (kernels/_utils.py:14-16).
 */
int pk_rmsnorm_fwd(const void* x, const void* w, const void* bias, void* y, float* rstd, int64_t rows, int64_t cols,
                   float eps, int dtype, int w_dtype, void* stream);

/* Bytes of device workspace pk_rmsnorm_bwd and pk_add_rmsnorm_bwd need for rows of
   x dtype `dtype` (any weight dtype). */
int64_t pk_rmsnorm_bwd_workspace(int64_t rows, int64_t cols, int dtype);

/*
 * RMSNorm backward. With n = x*r and u = dy*w:
 *   dx = r*(u - n*mean(u*n)), dw = sum_rows dy*n, dbias = sum_rows dy.
 * Accumulation is fp32 and deterministic (per-block partial rows in
 * `workspace`, then one column reduction). x and dx have `dtype`; w, dy, dw
 * and dbias have `w_dtype` (as pk_rmsnorm_fwd); dw and dbias are rounded once.
 * dbias may be NULL. rstd is the forward's output.
 * Replaces torch autograd of the reference (kernels/rms_norm.py:29-30).
 */
int pk_rmsnorm_bwd(const void* x, const void* w, const float* rstd, const void* dy, void* dx, void* dw, void* dbias,
                   void* workspace, int64_t workspace_bytes, int64_t rows, int64_t cols, int dtype, int w_dtype,
                   void* stream);

/*
 * pk_rmsnorm_bwd without a workspace argument and without any allocation:
 * the dw / dbias partial rows and the column-sum stage live in a fixed
 * file-scope device array of 96 MiB (100,663,296 bytes), which every GPU the
 * library runs on holds until the process ends. The kernels, grid and
 * summation order are pk_rmsnorm_bwd's, so the results are identical bit for
 * bit. A shape whose partial rows and stage do not fit the array (their size
 * is at most pk_rmsnorm_bwd_workspace) is refused with PK_ERR_UNSUPPORTED
 * before any launch, and before the pointers are checked, so the limit can be
 * probed with null pointers: measured on MI355X, 65,536 rows of 8192 columns fit
 * (69 MB), and with dbias rows of 4096 columns. Calls that overlap on one GPU
 * (other streams or threads) share the array and race; serialise them.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).
 */
int pk_rmsnorm_bwd_noalloc(const void* x, const void* w, const float* rstd, const void* dy, void* dx, void* dw,
                           void* dbias, int64_t rows, int64_t cols, int dtype, int w_dtype, void* stream);

/*
 * Residual add fused with RMSNorm, over `rows` contiguous rows of `cols`:
 *   s = round(x + residual); r = 1/sqrt(mean(s^2) + eps);
 *   y = round(round(s*r) * round(w + offset)).
 * Writes y and s (the new residual stream); rstd (fp32 [rows]) may be NULL.
 * x, residual and s have `dtype`; w and y have `w_dtype`: `dtype`, or fp32
 * with a 16-bit `dtype` (torch's promotion: w + offset stays fp32 and the
 * product with the rounded 16-bit row is an fp32 y). Replaces: reference
 * `add_rms_norm` (kernels/add_rms_norm.py:8-26,
 * `s = x + residual; rms(s, eps) * (weight + offset)`).
 */
int pk_add_rmsnorm_fwd(const void* x, const void* residual, const void* w, void* y, void* s, float* rstd,
                       int64_t rows, int64_t cols, float eps, float offset, int dtype, int w_dtype, void* stream);

/*
 * Backward of pk_add_rmsnorm_fwd. With n = s*r, u = dy*(w + offset):
 *   ds_total = r*(u - n*mean(u*n)) + ds,  dw = sum_rows dy*n,
 * where ds is the gradient reaching s through the second output (may be
 * NULL). ds_total is the gradient of both x and residual (dx). s, ds and dx
 * have `dtype`; w, dy and dw have `w_dtype` (as pk_add_rmsnorm_fwd). The
 * workspace is sized by pk_rmsnorm_bwd_workspace. Replaces torch autograd of
 * the reference (kernels/add_rms_norm.py:25-26).
 */
int pk_add_rmsnorm_bwd(const void* s, const void* w, const float* rstd, const void* dy, const void* ds, void* dx,
                       void* dw, void* workspace, int64_t workspace_bytes, int64_t rows, int64_t cols, float offset,
                       int dtype, int w_dtype, void* stream);

/*
 * Rotary embedding of x [batch, seq, heads, head_dim] with tables
 * cos, sin [seq, half] (contiguous), in fp32 arithmetic, rounded once to x's
 * dtype. NeoX halves (interleaved = 0): pairs (j, j + half); GPT-J
 * (interleaved = 1): pairs (2j, 2j + 1). Channels from 2*half on are copied.
 * conjugate = 1 negates sin (the backward rotation). y may equal x (in place).
 * strides[6] = x (batch, seq, head) strides then y's, in elements.
 * Replaces: reference `rotary_embedding` (kernels/rotary_embedding.py:12-40);
 * stands beside the Triton `_rotary_kernel` (impls/rotary_embedding_tl.py:17-67).
 */
int pk_rotary(const void* x, const void* cos, const void* sin, void* y, const int64_t* strides, int64_t batch,
              int64_t seq, int64_t heads, int64_t head_dim, int64_t half, int x_dtype, int cs_dtype, int interleaved,
              int conjugate, void* stream);

/*
 * Paired rotary embedding of q [batch, q_heads, seq, head_dim] and
 * k [batch, kv_heads, seq, head_dim] with full-width tables
 * cos, sin [cos_batch, seq, head_dim] (contiguous; cos_batch 1 or batch):
 *   y[j] = x[j] cos[j] - x[j+h] sin[j],  y[j+h] = x[j+h] cos[j+h] + x[j] sin[j+h]
 * (h = head_dim/2), i.e. x*cos + rotate_half(x)*sin, fp32 arithmetic rounded
 * once to y_dtype. transpose = 1 applies the adjoint map (the backward):
 *   dx[j] = g[j] cos[j] + g[j+h] sin[j+h],  dx[j+h] = g[j+h] cos[j+h] - g[j] sin[j].
 * x_dtype is what is read (q, k, or the cotangents), y_dtype what is written:
 * one dtype, or a 16-bit one with PK_F32 either way (16-bit q/k times fp32
 * tables promote to fp32 outputs; their backward reads fp32 cotangents and
 * writes 16-bit gradients). strides[12] = q, k, yq, yk (batch, head, seq)
 * strides in elements; the last dimension is contiguous. A side with zero
 * heads may pass NULL.
 * Replaces: reference `rope` (kernels/rope.py:19-36).
 */
int pk_rope(const void* q, const void* k, const void* cos, const void* sin, void* yq, void* yk,
            const int64_t* strides, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
            int64_t cos_batch, int x_dtype, int y_dtype, int cs_dtype, int transpose, void* stream);

/*
 * Per-head RMSNorm of q and k followed by pk_rope's rotation, in one pass
 * (the kernel-writing notebook's fused op):
 *   r = 1/sqrt(mean(x^2) + eps) over head_dim,  n = x*r*w,
 *   y = n*cos + rotate_half(n)*sin,
 * with w = q_weight [head_dim] for q rows and k_weight for k rows. fp32
 * arithmetic, one rounding per output, to y_dtype: x_dtype, or PK_F32 with
 * 16-bit inputs (fp32 tables or fp32 weights promote the reference's
 * rotation to fp32; with fp32 weights y_dtype must be PK_F32).
 * rstd_q [batch, q_heads, seq] and
 * rstd_k [batch, kv_heads, seq] (fp32) receive r for the backward.
 * strides[12] = q, k, yq, yk (batch, head, seq) strides in elements, all
 * multiples of the 16-byte pack (8 bf16/fp16, 4 fp32); the last dimension is
 * contiguous and every pointer 16-byte aligned. head_dim / 2 must be a pack
 * count times a power of two up to 64 (bf16: head_dim 16..1024). Weights have
 * w_dtype: x's, or PK_F32 with 16-bit inputs (autocast's fp32 parameters);
 * cos/sin [cos_batch, seq, head_dim] as in pk_rope.
 * Replaces: the reference `qk_norm_rope` of examples/03_write_a_kernel.ipynb
 * (cell 3), `rms` (kernels/_utils.py:14-16) then `rope` (kernels/rope.py:23-36);
 * stands beside that notebook's Triton `_fwd` (cell 7).
 */
int pk_qk_norm_rope_fwd(const void* q, const void* k, const void* q_weight, const void* k_weight, const void* cos,
                        const void* sin, void* yq, void* yk, float* rstd_q, float* rstd_k, const int64_t* strides,
                        int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
                        int64_t cos_batch, float eps, int x_dtype, int y_dtype, int cs_dtype, int w_dtype,
                        void* stream);

/* Bytes of device workspace pk_qk_norm_rope_bwd needs for this shape (-1 if unsupported). */
int64_t pk_qk_norm_rope_bwd_workspace(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq,
                                      int64_t head_dim, int x_dtype);

/*
 * Backward of pk_qk_norm_rope_fwd from the inputs and the saved r:
 *   g = rotation^T(dy),  u = g*w,  dx = r*(u - x*r^2*<u, x>/head_dim),
 *   dw = sum over rows of g*x*r.
 * dw is [2, head_dim] in w_dtype: row 0 the q_weight gradient, row 1 the
 * k_weight gradient, summed deterministically through the workspace. The
 * cotangents dyq, dyk have dy_dtype (the forward's y_dtype); dq, dk x's.
 * strides[18] = q, k, dyq, dyk, dq, dk (batch, head, seq) strides.
 * Replaces: torch autograd of the notebook's reference; stands beside its
 * Triton `_bwd` (cell 9).
 */
int pk_qk_norm_rope_bwd(const void* q, const void* k, const void* q_weight, const void* k_weight, const void* cos,
                        const void* sin, const float* rstd_q, const float* rstd_k, const void* dyq, const void* dyk,
                        void* dq, void* dk, void* dw, void* workspace, int64_t workspace_bytes,
                        const int64_t* strides, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq,
                        int64_t head_dim, int64_t cos_batch, int x_dtype, int dy_dtype, int cs_dtype, int w_dtype,
                        void* stream);

/*
 * Attention forward, o = softmax(q k^T * scale + M) v, grouped-query:
 * q [batch, seq, q_heads, head_dim], k, v [batch, seq, kv_heads, head_dim],
 * o like q; q head h reads kv head h / (q_heads / kv_heads). causal = 1 masks
 * key j > query i (top-left aligned). lse (fp32 [batch, q_heads, seq],
 * natural log) may be NULL. strides[12] = q, k, v, o (batch, seq, head)
 * strides in elements. head_dim a multiple of 8 up to 256 (rows laid out at
 * 64, 128 or 256 dims, zeros past head_dim); dtype PK_BF16, PK_F16, or PK_F32
 * (the fp32 matrix-core kernel, exact online softmax; strides multiples of 4
 * elements).
 * Replaces: reference `attn` (kernels/attn.py:10-37,
 * F.scaled_dot_product_attention with enable_gqa=True).
 */
int pk_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, const int64_t* strides,
                int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float softmax_scale,
                int causal, int dtype, void* stream);

/*
 * Attention forward over packed variable-length sequences: sequence i is
 * tokens [cu_seqlens[i], cu_seqlens[i+1]) of q [total, q_heads, head_dim] and
 * k, v [total, kv_heads, head_dim], attended independently (causal masks are
 * top-left aligned within each sequence); o is like q. cu_seqlens is an int32
 * device array of num_seqs + 1 non-decreasing offsets from 0 to total, and
 * max_seqlen is at least its largest difference (values are clamped to
 * [0, total] on the device). lse (fp32 [q_heads, total], natural log) may be
 * NULL. strides[8] = q, k, v, o (token, head) strides in elements. Same dtypes
 * and head_dim as pk_attn_fwd.
 * Replaces: reference `attn_varlen` (kernels/attn_varlen.py:15-54, SDPA per
 * cu_seqlens segment).
 */
int pk_attn_varlen_fwd(const void* q, const void* k, const void* v, void* o, float* lse, const int* cu_seqlens,
                       const int64_t* strides, int64_t num_seqs, int64_t total, int64_t max_seqlen, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, float softmax_scale, int causal, int dtype, void* stream);

/*
 * Bytes of device workspace pk_attn_bwd needs for this shape on the current
 * device, or -1 for an invalid shape. It holds D = rowsum(dout * o) and
 * lse * log2(e) (twice lse's size in fp32), and, when the dk/dv grid would
 * leave CUs idle (small batches or short sequences), fp32 dk/dv partials of
 * the q-head splits [splits, 2, batch * seq, kv_heads, head_dim].
 * No counterpart in the reference (its backward is torch autograd).
 */
int64_t pk_attn_bwd_workspace(int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim);

/*
 * Attention backward for pk_attn_fwd: given o, the upstream gradient dout
 * (like o) and the forward's lse, writes dq (like q), dk and dv (like k, v).
 * workspace: 16-byte aligned device memory of at least
 * pk_attn_bwd_workspace() bytes (workspace_bytes says how many were given).
 * Arithmetic: P is recomputed from q, k and lse; dS = P (dP - D);
 * dq = scale dS k, dk = scale dS^T q (summed over the q heads of each kv
 * head), dv = P^T dout; fp32 accumulation, one rounding per output, no atomics
 * (partials of q-head splits are added in a fixed order, so the result is
 * deterministic). strides[24] = q, k, v, o, dout, dq, dk, dv (batch, token,
 * head) strides in elements, multiples of 8 (bf16, fp16) or 4 (fp32).
 * head_dim a multiple of 8 up to 256. dtype PK_BF16, PK_F16 or PK_F32 (the
 * fp32 matrix-core kernels, v_mfma_f32_32x32x2_f32).
 * Replaces torch autograd of the reference `attn` (kernels/attn.py:30-37).
 */
int pk_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                void* workspace, int64_t workspace_bytes, void* dq, void* dk, void* dv, const int64_t* strides,
                int64_t batch, int64_t seq, int64_t q_heads, int64_t kv_heads, int64_t head_dim, float softmax_scale,
                int causal, int dtype, void* stream);

/*
 * Workspace bytes of pk_attn_varlen_bwd (as pk_attn_bwd_workspace, with
 * total packed tokens in place of batch * seq), or -1 for an invalid shape.
 * No counterpart in the reference.
 */
int64_t pk_attn_varlen_bwd_workspace(int64_t num_seqs, int64_t total, int64_t max_seqlen, int64_t q_heads,
                                     int64_t kv_heads, int64_t head_dim);

/*
 * Backward of pk_attn_varlen_fwd (packed sequences). lse is fp32
 * [q_heads, total]; workspace as for pk_attn_bwd, sized by
 * pk_attn_varlen_bwd_workspace(); strides[16] = q, k, v, o, dout, dq, dk, dv
 * (token, head). Replaces torch autograd of the reference `attn_varlen`
 * (kernels/attn_varlen.py:41-54).
 */
int pk_attn_varlen_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout, const float* lse,
                       void* workspace, int64_t workspace_bytes, void* dq, void* dk, void* dv, const int* cu_seqlens,
                       const int64_t* strides, int64_t num_seqs, int64_t total, int64_t max_seqlen, int64_t q_heads,
                       int64_t kv_heads, int64_t head_dim, float softmax_scale, int causal, int dtype, void* stream);

/*
 * Matrix-core rate probe, a measurement aid with no counterpart in the
 * reference: `blocks` blocks of four waves (one per SIMD; pass the CU count to
 * fill the device) each run iters x 8 back-to-back bf16 32x32x16 products on
 * random operands, with (softmax != 0) or without the attention forward's
 * per-score vector work beside each product. out (device, uint64
 * [2 * 4 * blocks]) receives per wave the shader-clock cycles and the 100 MHz
 * real-time ticks of its loop. Reads no memory.
 */
int pk_probe_mfma(int softmax, int iters, int blocks, uint64_t* out, void* stream);

/*
 * Streaming probe, the HBM counterpart of pk_probe_mfma (no counterpart in the
 * reference): y = a (reads == 1) or y = a ^ b (reads == 2) over `bytes` bytes
 * (a multiple of 16, 16-byte aligned pointers), one 16-byte non-temporal
 * vector per thread in 64-thread blocks: the ceiling of a streaming kernel
 * with that pattern of reads and writes at that size.
 */
int pk_probe_stream(const void* a, const void* b, void* y, int64_t bytes, int reads, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* POPCORN_AMD_H */
