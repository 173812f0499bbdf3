/*
 * mi355x_kernels.h — C ABI of the gfx950 kernel library behind the eager
 * `mojo` PyTorch device.
 *
 * The reference crosses into native code once per op with `ext.call(*args)`
 * on a per-variant CPython extension (torch_mojo_backend/eager_kernels/
 * call_queue.py:283-288, eager_kernels/__init__.py:786-802), passing raw
 * device pointers as ints, shapes/strides as int tuples, floats for
 * scale/eps/lr and a device-context handle.  This header is the replacement
 * for that boundary: one shared library, plain pointers and sizes, no torch
 * types.  Each declaration cites the reference entry it replaces.
 *
 * Conventions (every function):
 *   - returns MI355X_OK (0) on success, a nonzero MI355X_E* code otherwise;
 *     mi355x_last_error() then returns a thread-local message;
 *   - never throws, never synchronises the host with the device;
 *   - never allocates device memory: outputs and workspaces are passed in
 *     (size them with the matching *_workspace_bytes query);
 *   - the last argument is the HIP stream the work is ordered on;
 *   - strides are in ELEMENTS (int64), dtypes are MI355X_* codes.
 */
#ifndef MI355X_KERNELS_H
#define MI355X_KERNELS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* mi355x_stream_t; /* == hipStream_t */

/* ---- status codes ---------------------------------------------------- */
#define MI355X_OK 0
#define MI355X_EINVAL 1      /* bad argument (shape, stride, dtype, size) */
#define MI355X_ELAUNCH 2     /* a kernel launch reported an error */
#define MI355X_EUNSUPPORTED 3
#define MI355X_EWORKSPACE 4  /* caller workspace too small */

/* ---- dtype codes ----------------------------------------------------- */
#define MI355X_F32 0
#define MI355X_BF16 1
#define MI355X_F16 2
#define MI355X_F64 3
#define MI355X_I64 4
#define MI355X_I32 5
#define MI355X_I16 6
#define MI355X_I8 7
#define MI355X_U8 8
#define MI355X_BOOL 9

#define MI355X_MAX_RANK 8

/* ---- library -------------------------------------------------------- */
/* ABI version; bumped on any signature change. */
int mi355x_abi_version(void);
/* Thread-local message describing the last nonzero status on this thread. */
const char* mi355x_last_error(void);
/* Offload target the code object was built for ("gfx950"). */
const char* mi355x_target(void);
/* Digest of the sources and flags the library was built from (no
 * counterpart in the reference, whose kernels are JIT-built per variant:
 * the loader compares it with the sources beside the package and refuses a
 * stale prebuilt library). */
const char* mi355x_source_hash(void);

/* ---- data movement (tensor_holder.mojo:144-657 CopyStrided / cast
 *      _CastSpecExtension aten_fast.py:1232, PermuteCopy
 *      torch_mojo_tensor.py:615-654) ---------------------------------- */
/* dst[i] = (dst_dtype) src[i] over an ndim-rank index space `shape`;
 * a zero src stride broadcasts.  Rank <= MI355X_MAX_RANK. */
int mi355x_copy(void* dst, int dst_dtype, const int64_t* dst_strides,
                const void* src, int src_dtype, const int64_t* src_strides,
                const int64_t* shape, int ndim, mi355x_stream_t stream);
/* dst[i] = value (factories ones/zeros/full, fill_.Scalar, zero_). */
int mi355x_fill(void* dst, int dtype, const int64_t* strides,
                const int64_t* shape, int ndim, double value,
                mi355x_stream_t stream);
/* dst[i] = start + i*step for a contiguous dst (aten::arange). */
int mi355x_arange(void* dst, int dtype, int64_t n, double start, double step,
                  mi355x_stream_t stream);

/* ---- elementwise map (logic_ops.mojo:170,381,435,513 binary_flat_vec /
 *      binary_rowvec; elementwise_ops unary family) ------------------- */
/* Map opcodes. s0/s1 are scalar operands (alpha, exponents, clamp bounds). */
enum {
  /* binary: out = f(a, b) */
  MI355X_OP_ADD = 0,      /* a + s0*b */
  MI355X_OP_SUB = 1,      /* a - s0*b */
  MI355X_OP_MUL = 2,
  MI355X_OP_DIV = 3,
  MI355X_OP_MAXIMUM = 4,
  MI355X_OP_MINIMUM = 5,
  MI355X_OP_POW = 6,
  MI355X_OP_EQ = 7,
  MI355X_OP_NE = 8,
  MI355X_OP_LT = 9,
  MI355X_OP_LE = 10,
  MI355X_OP_GT = 11,
  MI355X_OP_GE = 12,
  MI355X_OP_LOGICAL_AND = 13,
  MI355X_OP_LOGICAL_OR = 14,
  MI355X_OP_LOGICAL_XOR = 15,
  MI355X_OP_BITWISE_AND = 16,
  MI355X_OP_BITWISE_OR = 17,
  MI355X_OP_BITWISE_XOR = 18,
  MI355X_OP_REMAINDER = 19,
  MI355X_OP_FLOOR_DIVIDE = 20,
  MI355X_OP_DIV_TRUNC = 21,
  MI355X_OP_DIV_FLOOR = 22,
  /* ternary: out = f(a, b, c) */
  MI355X_OP_WHERE = 40,   /* a ? b : c */
  MI355X_OP_ADDCMUL = 41, /* a + s0*b*c */
  MI355X_OP_ADDCDIV = 42, /* a + s0*b/c */
  MI355X_OP_LERP = 43,    /* a + s0*(b-a) */
  /* unary: out = f(a) */
  MI355X_OP_IDENTITY = 60,
  MI355X_OP_NEG = 61,
  MI355X_OP_ABS = 62,
  MI355X_OP_EXP = 63,
  MI355X_OP_LOG = 64,
  MI355X_OP_SQRT = 65,
  MI355X_OP_RSQRT = 66,
  MI355X_OP_RECIPROCAL = 67,
  MI355X_OP_SIN = 68,
  MI355X_OP_COS = 69,
  MI355X_OP_TANH = 70,
  MI355X_OP_SIGMOID = 71,
  MI355X_OP_ERF = 72,
  MI355X_OP_RELU = 73,
  MI355X_OP_SILU = 74,
  MI355X_OP_LOG1P = 75,
  MI355X_OP_EXPM1 = 76,
  MI355X_OP_FLOOR = 77,
  MI355X_OP_CEIL = 78,
  MI355X_OP_ROUND = 79,
  MI355X_OP_TRUNC = 80,
  MI355X_OP_SIGN = 81,
  MI355X_OP_POW_SCALAR = 82,   /* a ** s0 */
  MI355X_OP_CLAMP = 83,        /* min(max(a, s0), s1) */
  MI355X_OP_LOGICAL_NOT = 84,
  MI355X_OP_BITWISE_NOT = 85,
  MI355X_OP_ISNAN = 86,
  MI355X_OP_ISINF = 87,
  MI355X_OP_ISFINITE = 88,
  MI355X_OP_TAN = 89,
  MI355X_OP_ATAN = 90,
  MI355X_OP_ASIN = 91,
  MI355X_OP_ACOS = 92,
  MI355X_OP_SINH = 93,
  MI355X_OP_COSH = 94,
  MI355X_OP_ASINH = 95,
  MI355X_OP_ACOSH = 96,
  MI355X_OP_ATANH = 97,
  MI355X_OP_LOG2 = 98,
  MI355X_OP_EXP2 = 99,
  MI355X_OP_LOG10 = 100,
  MI355X_OP_SQUARE = 101,
  MI355X_OP_CLAMP_MIN = 102,   /* max(a, s0) */
  MI355X_OP_CLAMP_MAX = 103,   /* min(a, s0) */
  MI355X_OP_RSUB = 104,        /* s0 - a*s1 */
};
/* out = a + r (f32 sum, as mi355x_map's add) and low = out rounded to
 * low_dtype (bf16/f16), in one pass over n contiguous elements (n % 4 == 0,
 * 16-byte aligned f32 vectors).  The gradient sum the autograd engine forms
 * on a residual stream and the autocast copy of it that the next linear's
 * backward reads: the reference runs the add (aten_fast.py:2510) and the
 * cast (_CastSpecExtension, aten_fast.py:1232) as two kernels. */
int mi355x_add_cast(float* out, void* low, int low_dtype, const float* a, const void* r, int r_dtype,
                    int64_t n, mi355x_stream_t stream);
/* out = op(in[0..nin-1]; s0, s1) over `shape`.  `strides` holds (nin+1)
 * stride vectors of `ndim` entries: out first, then each input.  A zero
 * input stride broadcasts; a NULL input pointer reads the scalar s1 instead
 * (its in_dtypes entry then gives the scalar's type).  Arithmetic is in f32 for floating outputs
 * (f64 if any operand is f64) and in int64 for integral ones.
 * Replaces fast_aten_add/mul/sub/div/... (aten_fast.py:2510 and family). */
int mi355x_map(int op, void* out, int out_dtype, int nin,
               const void* const* ins, const int* in_dtypes,
               const int64_t* strides, const int64_t* shape, int ndim,
               double s0, double s1, mi355x_stream_t stream);

/* ---- reductions (reduction_ops.mojo row sums, reduce_skeleton.mojo;
 *      fast_aten_sum aten_fast.py:5596) --------------------------------- */
enum {
  MI355X_RED_SUM = 0,
  MI355X_RED_MEAN = 1,
  MI355X_RED_MAX = 2,
  MI355X_RED_MIN = 3,
  MI355X_RED_NORM2 = 4,  /* sqrt(sum x^2) */
  MI355X_RED_SUMSQ = 5,
  MI355X_RED_AMAX = 6,   /* max |x| */
  MI355X_RED_PROD = 7,
  MI355X_RED_ANY = 8,    /* any nonzero -> 1 */
  MI355X_RED_ALL = 9,
  MI355X_RED_NORM1 = 10,
};
/* out[o, i] = reduce_r in[o, r, i], element (o,r,i) at in + o*s_o + r*s_r +
 * i*s_i; out is contiguous [outer, inner].  Accumulates in f32 (f64 for f64,
 * int64 for integral sums). */
int64_t mi355x_reduce_workspace_bytes(int64_t outer, int64_t r, int64_t inner);
int mi355x_reduce(int op, void* out, int out_dtype, const void* in,
                  int in_dtype, int64_t outer, int64_t r, int64_t inner,
                  int64_t s_o, int64_t s_r, int64_t s_i, void* workspace,
                  int64_t ws_bytes, mi355x_stream_t stream);
/* Arg-reduction along r: out_idx[o,i] = argmax/argmin (first occurrence,
 * NaN wins as torch does); optional out_val (may be NULL).  int64 output. */
int mi355x_argreduce(int is_min, int64_t* out_idx, void* out_val,
                     const void* in, int dtype, int64_t outer, int64_t r,
                     int64_t inner, int64_t s_o, int64_t s_r, int64_t s_i,
                     mi355x_stream_t stream);

/* ---- index ops ---------------------------------------------------- */
/* out[o, j, i] = in[o, idx[j], i] (index_select / embedding gather).
 * in row (o, j) lives at o*in_so + idx[j]*in_sj + i (inner contiguous).
 * Bit-exact; indices are bounds-checked on the device (an out-of-range
 * index writes nothing and sets *err_flag to 1 if err_flag != NULL). */
int mi355x_index_select(void* out, const void* in, int dtype,
                        const int64_t* idx, int64_t outer, int64_t n_idx,
                        int64_t in_rows, int64_t inner, int64_t in_so,
                        int64_t in_sj, int32_t* err_flag,
                        mi355x_stream_t stream);

/* ---- embedding (Gather0 nn_ops.mojo:1774-1796;
 *      EmbeddingDenseBackwardF32I64 embedding_backward_kernels.mojo:152-534)
 */
/* out[n, :] = weight[idx[n], :], weight rows at weight + r*w_row_stride. */
int mi355x_embedding_fwd(void* out, const void* weight, int dtype,
                         const int64_t* idx, int64_t n_idx,
                         int64_t num_weights, int64_t dim,
                         int64_t w_row_stride, int32_t* err_flag,
                         mi355x_stream_t stream);
/* grad_weight[r, :] = sum over n with idx[n]==r (ascending n) of
 * grad_out[n, :]; rows equal to padding_idx (if >= 0) are zero.
 * Deterministic: a stable sort of idx, then one ordered sum per row. */
int64_t mi355x_embedding_bwd_workspace_bytes(int64_t n_idx,
                                             int64_t num_weights);
int mi355x_embedding_bwd(void* grad_weight, const void* grad_out, int dtype,
                         const int64_t* idx, int64_t n_idx,
                         int64_t num_weights, int64_t dim,
                         int64_t padding_idx, void* workspace,
                         int64_t ws_bytes, mi355x_stream_t stream);
/* grad_weight = base + the gradient mi355x_embedding_bwd would write (each
 * row's sum rounded to dtype, then added): rows idx names get base + sum,
 * the others (and padding_idx) base's row, copied, or not touched at all
 * when base == grad_weight (in place).  Same workspace.  No counterpart in
 * the reference: it serves a tied embedding, whose gradient autograd adds
 * to the output projection's (`grad + embedding_dense_backward`), in one
 * pass without the dense sum. */
int mi355x_embedding_bwd_accumulate(void* grad_weight, const void* base, const void* grad_out, int dtype,
                                    const int64_t* idx, int64_t n_idx, int64_t num_weights,
                                    int64_t dim, int64_t padding_idx, void* workspace,
                                    int64_t ws_bytes, mi355x_stream_t stream);

/* ---- layer norm (LayerNormForward normalization_forward_ops.mojo:118;
 *      LayerNormBackwardF32 normalization_backward_dx.mojo:190-388,
 *      normalization_backward_params.mojo:41-143) ---------------------- */
/* RMSNorm forward over the last dim (rows x cols, contiguous):
 * y = x / sqrt(mean(x^2) + eps) * (weight + weight_offset), rstd[rows] f32.
 * weight (optional; without it the scale is 1) is f32 or the input dtype;
 * weight_offset = 1 gives Gemma's (1 + w) scale without a separate add.  The reference has no eager RMSNorm (its
 * Gemma-3 path runs under torch.compile, demo_scripts/gemma3.py:11); this
 * serves aten::rms_norm for the Gemma-3-shaped workload and follows
 * fast_aten_native_layer_norm's contract (aten_fast.py:5248-5371) minus the
 * mean and bias. */
int mi355x_rms_norm_fwd(void* y, float* rstd, const void* x, const void* weight, int weight_dtype,
                        double weight_offset, int64_t rows, int64_t cols, double eps, int dtype,
                        mi355x_stream_t stream);
/* RMSNorm backward (the gradient of mi355x_rms_norm_fwd, its rstd saved):
 * with s = weight + weight_offset, dx = rstd * (dy s - x rstd^2 mean(dy s x))
 * and dweight = sum over rows of dy x rstd (optional, summed in a fixed
 * order through the mi355x_layer_norm_bwd_workspace_bytes workspace).
 * weight is the input dtype; rows contiguous, cols a multiple of 4 up to
 * 2048 (others return MI355X_EUNSUPPORTED).  No reference counterpart (see
 * mi355x_rms_norm_fwd): it replaces the decomposition of the rms_norm
 * backward into device elementwise and reduction ops. */
int mi355x_rms_norm_bwd(void* dx, void* dweight, const void* dy, const void* x, const float* rstd,
                        const void* weight, double weight_offset, int64_t rows, int64_t cols, int dtype,
                        void* workspace, int64_t ws_bytes, mi355x_stream_t stream);
/* Rotary position embedding, half-split ("rotate_half") form, over
 * [batch, heads, seq, d] views (unit d stride, *_bht = the batch/head/seq
 * element strides, multiples of 4): y[i] = x[i] cos[t][i] - x[i+d/2] sin[t][i],
 * y[i+d/2] = x[i+d/2] cos[t][i+d/2] + x[i] sin[t][i+d/2]; inverse = 1 applies
 * the transposed map (the backward).  cos/sin: dense [seq][d] in dtype; d a
 * multiple of 8.  The Gemma-3-shaped workload's RoPE; the reference has no
 * eager kernel for it (its Gemma-3 demo runs under torch.compile,
 * demo_scripts/gemma3.py:11) and would run the elementwise chain through
 * its _to_copy / add / mul ops (aten_fast.py:1232, :2510). */
int mi355x_rope(void* y, const int64_t* y_bht, const void* x, const int64_t* x_bht, const void* cos_table,
                const void* sin_table, int64_t batch, int64_t heads, int64_t seq, int64_t d, int inverse,
                int dtype, mi355x_stream_t stream);
/* GeGLU: y = gelu(gate) * up over n contiguous elements, gelu exact or tanh
 * (approximate), gelu(gate) rounded to dtype before the product as the
 * aten gelu + mul pair does (fast_aten_gelu aten_fast.py:2940-2968, then
 * the elementwise mul). */
int mi355x_geglu_fwd(void* y, const void* gate, const void* up, int64_t n, int approximate, int dtype,
                     mi355x_stream_t stream);
/* GeGLU backward in one pass, bit-exact with the ATen chain it replaces:
 * d_up = grad * round(gelu(gate)), d_gate = gelu_backward(round(grad * up),
 * gate), every product rounded to dtype.  No reference counterpart (as
 * mi355x_geglu_fwd). */
int mi355x_geglu_bwd(void* dgate, void* dup, const void* grad, const void* gate, const void* up, int64_t n,
                     int approximate, int dtype, mi355x_stream_t stream);
/* y = (x - mean)*rstd*gamma + beta over rows of `cols` contiguous elements.
 * gamma/beta may be NULL.  mean/rstd: f32 [rows]. */
int mi355x_layer_norm_fwd(void* y, float* mean, float* rstd, const void* x,
                          const void* gamma, const void* beta, int64_t rows,
                          int64_t cols, double eps, int dtype,
                          mi355x_stream_t stream);
/* mi355x_layer_norm_fwd plus y_low: an optional second copy of y in a
 * 16-bit type (low_dtype bf16/f16; f32 input only), written by the same
 * kernel.  Under autocast the f32 layer_norm output is cast to the matmul
 * dtype right away (fp32 policy for layer_norm, lower precision for linear:
 * mojo_device_autocast.py:537-567); the copy saves that cast's read of y.
 * y may be NULL when y_low is given: only the copy and the statistics are
 * written, and mi355x_layer_norm_apply produces y later if it is read.
 * No counterpart in the reference, whose cast is a separate _to_copy. */
int mi355x_layer_norm_fwd_ex(void* y, void* y_low, int low_dtype, float* mean,
                             float* rstd, const void* x, const void* gamma,
                             const void* beta, int64_t rows, int64_t cols,
                             double eps, int dtype, mi355x_stream_t stream);
/* The residual add of a pre-LayerNorm block fused into the norm that reads
 * it: x_out = a + r (a f32, r f32/bf16/f16, summed in f32 exactly as a
 * separate add would), then y = LayerNorm(x_out) with y_low as in
 * mi355x_layer_norm_fwd_ex.  f32 rows only, cols a multiple of 4 up to 2048
 * with 16-byte aligned rows (else MI355X_EUNSUPPORTED: run the add and the
 * norm separately).  Serves nanoGPT's `x = x + f(ln(x))` followed by the next
 * ln(x): the reference runs the add (fast_aten_add, aten_fast.py:2510) and
 * the norm (aten_fast.py:5248-5371) as two kernels. */
int mi355x_layer_norm_fwd_add(void* y, void* y_low, int low_dtype, float* mean, float* rstd,
                              void* x_out, const void* a, const void* r, int r_dtype,
                              const void* gamma, const void* beta, int64_t rows, int64_t cols,
                              double eps, int dtype, mi355x_stream_t stream);
/* y = (x - mean)*rstd*gamma + beta from x and the statistics a forward
 * saved (mean/rstd f32 [rows]; gamma/beta may be NULL), bit-identical to the
 * y that forward (mi355x_layer_norm_fwd_ex or _fwd_add, whose x is x_out)
 * would have written.  No counterpart in the reference: it serves the
 * autocast forward that writes only the 16-bit copy and defers the f32
 * output until something reads it (the next linear takes the copy, so in
 * a training step nothing does). */
int mi355x_layer_norm_apply(void* y, const void* x, const float* mean, const float* rstd,
                            const void* gamma, const void* beta, int64_t rows, int64_t cols,
                            int dtype, mi355x_stream_t stream);
/* Any of dx/dgamma/dbeta may be NULL (output_mask, aten_fast.py:5475). */
int64_t mi355x_layer_norm_bwd_workspace_bytes(int64_t rows, int64_t cols);
int mi355x_layer_norm_bwd(void* dx, void* dgamma, void* dbeta,
                          const void* dy, const void* x, const float* mean,
                          const float* rstd, const void* gamma, int64_t rows,
                          int64_t cols, int dtype, void* workspace,
                          int64_t ws_bytes, mi355x_stream_t stream);

/* ---- GELU (GeluForwardBF16 activation_forward_kernels.mojo:115,138;
 *      gelu_backward_* activation_backward_ops.mojo:80,105,199,233) ---- */
/* approximate: 0 = exact erf form, 1 = tanh form.  Contiguous n elements. */
int mi355x_gelu_fwd(void* y, const void* x, int64_t n, int approximate,
                    int dtype, mi355x_stream_t stream);
int mi355x_gelu_bwd(void* dx, const void* dy, const void* x, int64_t n,
                    int approximate, int dtype, mi355x_stream_t stream);

/* ---- softmax / log_softmax (SoftmaxSpec nn_ops.mojo:364,449,1223;
 *      LogSoftmaxSpec reduction_ops.mojo:852,1010-1060;
 *      LogSoftmaxBackwardData softmax_backward_kernels.mojo:76,159,231) */
/* Row-wise over the contiguous last dim; computes in f32. */
int mi355x_softmax_fwd(void* y, int y_dtype, const void* x, int x_dtype,
                       int64_t rows, int64_t cols, int log,
                       mi355x_stream_t stream);
/* log: dx = dy - exp(y)*sum(dy);  softmax: dx = y*(dy - sum(dy*y)). */
int mi355x_softmax_bwd(void* dx, int dx_dtype, const void* dy, int dy_dtype,
                       const void* y, int y_dtype, int64_t rows,
                       int64_t cols, int log, mi355x_stream_t stream);

/* ---- NLL loss (NllLossForwardF32 loss_ops.mojo:73-207;
 *      NllLossBackwardF32 loss_ops.mojo:254,306) --------------------- */
/* reduction: 0 none, 1 mean, 2 sum.  out: [N] for none, scalar otherwise.
 * total_weight: scalar (count of non-ignored targets, or sum of weights).
 * weight may be NULL.  A target outside [0, C) that is not ignore_index
 * sets *err_flag. */
int64_t mi355x_nll_workspace_bytes(int64_t n);
int mi355x_nll_fwd(void* out, void* total_weight, const void* logp,
                   int dtype, const int64_t* target, const void* weight,
                   int64_t n, int64_t c, int reduction, int64_t ignore_index,
                   int32_t* err_flag, void* workspace, int64_t ws_bytes,
                   mi355x_stream_t stream);
/* Writes every element of grad_input [N, C]. */
int mi355x_nll_bwd(void* grad_input, const void* grad_out,
                   const int64_t* target, const void* weight,
                   const void* total_weight, int64_t n, int64_t c,
                   int reduction, int64_t ignore_index, int dtype,
                   mi355x_stream_t stream);

/* ---- fused cross-entropy (the log_softmax -> nll_loss chain of the step:
 *      fast_aten__log_softmax aten_fast.py:5792-5825, nll_loss_forward/
 *      backward aten_fast.py:5974-6130, log_softmax backward :5828-5971) -- */
/* out: f32 scalar (reduction mean/sum) or f32 [n] (none); total_weight: f32
 * scalar (non-ignored rows); lse: f32 [n] natural-log row log-sum-exp, kept
 * for the backward.  logits rows at logits + i*ld. */
int64_t mi355x_cross_entropy_workspace_bytes(int64_t n);
int mi355x_cross_entropy_fwd(void* out, float* total_weight, float* lse,
                             const void* logits, int dtype, int64_t ld,
                             const int64_t* target, int64_t n, int64_t c,
                             int reduction, int64_t ignore_index,
                             int32_t* err_flag, void* workspace,
                             int64_t ws_bytes, mi355x_stream_t stream);
/* dx[i, :] = g_i * (softmax(x_i) - onehot(t_i)) with rows at dx + i*ld_dx;
 * columns [c, ld_dx) are written as zero.  grad_out: f32 scalar or [n].
 * dx has the logits' dtype, a 16-byte aligned base and ld_dx a multiple of
 * 16 bytes' worth of elements (8 for bf16/f16, 4 for f32). */
int mi355x_cross_entropy_bwd(void* dx, int dx_dtype, int64_t ld_dx,
                             const void* logits, int dtype, int64_t ld,
                             const float* lse, const int64_t* target,
                             const float* grad_out, int reduction,
                             const float* total_weight, int64_t n, int64_t c,
                             int64_t ignore_index, mi355x_stream_t stream);
/* mi355x_cross_entropy_fwd and mi355x_cross_entropy_bwd in one pass over
 * the logits, for reduction mean (1) or sum (2): writes out, total_weight,
 * lse and dx with the values the two calls would write (each row's logits
 * held in registers between its log-sum-exp and its gradient).  Rows of up
 * to 8192 16-byte chunks (about 65500 bf16/f16 or 32760 f32 classes, and
 * ld_dx / (16 / element size) <= 8192); longer rows return
 * MI355X_EUNSUPPORTED, and the two calls remain.
 * Workspace: mi355x_cross_entropy_workspace_bytes(n).  No counterpart in the
 * reference: it serves a training step, where the loss is first read after
 * the backward, so the forward's read of the logits can be skipped. */
int mi355x_cross_entropy_fwd_bwd(void* out, float* total_weight, float* lse, void* dx, int64_t ld_dx,
                                 const void* logits, int dtype, int64_t ld, const int64_t* target,
                                 const float* grad_out, int64_t n, int64_t c, int reduction,
                                 int64_t ignore_index, int32_t* err_flag, void* workspace,
                                 int64_t ws_bytes, mi355x_stream_t stream);

/* ---- optimizer (enqueue_fused_adamw_f32 optimizer_kernels.mojo:339-454,
 *      AdamWDesc optimizer_contract.mojo:11-56;
 *      foreach_l2_norm_f32_* foreach_clip_kernels.mojo:64,101;
 *      foreach_*_desc_* foreach_batched_kernels.mojo:345) ------------- */
typedef struct mi355x_adamw_tensor {
  float* param;
  const float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  float* max_exp_avg_sq; /* amsgrad only, else NULL */
  const float* step;     /* device scalar, already incremented */
  int64_t numel;
} mi355x_adamw_tensor;
#define MI355X_ADAMW_AMSGRAD 1
#define MI355X_ADAMW_MAXIMIZE 2
/* torch.optim AdamW (decoupled weight decay) over n tensors.  lr_ptr (if
 * not NULL) overrides lr; grad_scale divides grads; a nonzero *found_inf
 * skips the update.  Any n (batched 160 tensors per launch). */
int mi355x_fused_adamw(const mi355x_adamw_tensor* tensors, int n, double lr,
                       const float* lr_ptr, double beta1, double beta2,
                       double weight_decay, double eps, int flags,
                       const float* grad_scale, const float* found_inf,
                       mi355x_stream_t stream);
/* mi355x_fused_adamw plus param_low: n pointers (NULL entries allowed, or
 * param_low itself NULL) to 16-bit copies (low_dtype bf16/f16) that the
 * kernel fills with each updated parameter, for the autocast forward that
 * follows (mojo_device_autocast.py:537-567 casts every f32 weight to the
 * matmul dtype); and grad_mul (NULL, or a device f32 scalar) multiplying
 * every gradient as it is read (before maximize and grad_scale), which
 * applies a pending in-place gradient scale (clip_grad_norm_'s
 * _foreach_mul_) without a pass over the gradients: the same product the
 * separate multiply stores.  No counterpart in the reference. */
int mi355x_fused_adamw_ex(const mi355x_adamw_tensor* tensors, void* const* param_low,
                          int low_dtype, int n, double lr, const float* lr_ptr,
                          double beta1, double beta2, double weight_decay, double eps,
                          int flags, const float* grad_scale, const float* found_inf,
                          const float* grad_mul, mi355x_stream_t stream);

/* Per-tensor p-norm (ord 2 or 1, or inf when ord_inf) of n f32/bf16 tensors
 * into outs[i] (a device scalar of out_dtype). */
int64_t mi355x_foreach_norm_workspace_bytes(const int64_t* numels, int n);
int mi355x_foreach_norm(void* const* outs, int out_dtype,
                        const void* const* ins, int in_dtype,
                        const int64_t* numels, int n, double ord,
                        void* workspace, int64_t ws_bytes,
                        mi355x_stream_t stream);
/* In-place foreach update over n contiguous tensors of one dtype:
 *   op MI355X_OP_ADD:      a[i] += s0 * b[i]        (b NULL: a += s0)
 *   op MI355X_OP_MUL:      a[i] *= (scalars? scalars[i] : b? b[i] : s0)
 *   op MI355X_OP_DIV:      a[i] /= (scalars? scalars[i] : b? b[i] : s0)
 *   op MI355X_OP_LERP:     a[i] += s0 * (b[i] - a[i])
 *   op MI355X_OP_ADDCMUL:  a[i] += (scalars? scalars[i] : s0) * b[i]*c[i]
 *   op MI355X_OP_ADDCDIV:  a[i] += (scalars? scalars[i] : s0) * b[i]/c[i]
 *   op MI355X_OP_SQRT:     a[i] = sqrt(a[i])
 * tensor_scalar: optional device f32 scalar multiplying (MUL) or dividing
 * (DIV) every tensor (_foreach_mul_.Tensor).  b/c/scalars may be NULL. */
int mi355x_foreach_apply(int op, void* const* a, const void* const* b,
                         const void* const* c, const double* scalars,
                         const int64_t* numels, int n, int dtype, double s0,
                         const float* tensor_scalar, mi355x_stream_t stream);

/* ---- GEMM (fast_aten_mm/addmm/bmm/linear aten_fast.py:8713-8935 ->
 *      _matmul_spec_into_go / _matmul_bias_spec_into_go / _bmm_spec_into_go
 *      matmul_ops.mojo:7009,7040,7095) ---------------------------------- */
/* C[b, m, n] = sum_k A[b, m, k] * B[b, k, n] (+ bias[n]).
 * A element at a + b*a_bs + m*a_rs + k*a_cs (a_rs == 1 or a_cs == 1),
 * B element at b + b*b_bs + k*b_rs + n*b_cs (b_rs == 1 or b_cs == 1),
 * C element at c + b*c_bs + m*c_rs + n (rows contiguous).
 * ab_dtype: F32, BF16 or F16 (A and B share it); c_dtype and bias_dtype:
 * F32/BF16/F16.  Accumulates in f32; bf16/f16 use MFMA.  beta == 1 adds the
 * existing C (accumulate), beta == 0 overwrites. */
/* Workspace for the call with these operands (split-K partials, and packed
 * copies of operands that cannot be read in place). */
int64_t mi355x_gemm_workspace_bytes(const void* a, int64_t a_rs, int64_t a_cs,
                                    int64_t a_bs, const void* b, int64_t b_rs,
                                    int64_t b_cs, int64_t b_bs, int ab_dtype,
                                    int64_t batch, int64_t m, int64_t n,
                                    int64_t k);
int mi355x_gemm(void* c, int c_dtype, int64_t c_rs, int64_t c_bs,
                const void* a, int64_t a_rs, int64_t a_cs, int64_t a_bs,
                const void* b, int64_t b_rs, int64_t b_cs, int64_t b_bs,
                int ab_dtype, const void* bias, int bias_dtype, int beta,
                int64_t batch, int64_t m, int64_t n, int64_t k,
                void* workspace, int64_t ws_bytes, mi355x_stream_t stream);
/* mi355x_gemm with options (the linear backward of the autocast path,
 * fast_aten_linear_backward aten_fast.py:8815-8907: dW = dY^T X and
 * db = sum(dY, 0) from one pass over dY):
 *   flags MI355X_GEMM_BETA   add the existing C (as beta == 1 above);
 *         MI355X_GEMM_ROUND  round C (and the row sums) to ab_dtype before
 *                            storing them in a wider c_dtype, the value a
 *                            16-bit result widened afterwards would have;
 *   a_rowsum (optional, [batch][m] of a_rowsum_dtype): sum over k of each
 *                            row of A, accumulated in f32.
 * Same workspace query as mi355x_gemm. */
#define MI355X_GEMM_BETA 1
#define MI355X_GEMM_ROUND 2
int mi355x_gemm_ex(void* c, int c_dtype, int64_t c_rs, int64_t c_bs,
                   const void* a, int64_t a_rs, int64_t a_cs, int64_t a_bs,
                   const void* b, int64_t b_rs, int64_t b_cs, int64_t b_bs,
                   int ab_dtype, const void* bias, int bias_dtype, int flags,
                   void* a_rowsum, int a_rowsum_dtype,
                   int64_t batch, int64_t m, int64_t n, int64_t k,
                   void* workspace, int64_t ws_bytes, mi355x_stream_t stream);

/* ---- causal flash attention (fast_fused_flash_attention_forward
 *      aten_fast.py:7533-7587 -> flash_attention_ops.mojo:48-112 ->
 *      enqueue_flash_attention_fwd flash_attention_fwd_kernels.mojo:885-963;
 *      backward aten_fast.py:7590-7664 -> flash_attention_ops.mojo:115-220
 *      -> enqueue_flash_attention_bwd flash_attention_bwd_kernels.mojo:
 *      1354-1456) -------------------------------------------------------- */
/* O = softmax(scale*Q K^T [+ causal mask, top-left aligned]) V,
 * LSE[b,h,i] = natural-log row log-sum-exp (f32, contiguous [B,H,Sq]).
 * Each *_bhs gives the (batch, head, seq) element strides; head_dim stride
 * is 1.  dtype: BF16 or F16 (MFMA) or F32. */
int mi355x_attn_fwd(void* o, const int64_t* o_bhs, float* lse, const void* q,
                    const int64_t* q_bhs, const void* k,
                    const int64_t* k_bhs, const void* v,
                    const int64_t* v_bhs, int64_t batch, int64_t heads,
                    int64_t sq, int64_t skv, int64_t d, double scale,
                    int causal, int dtype, mi355x_stream_t stream);
/* The same forward with grouped-query K/V heads (heads % kv_heads == 0,
 * query head h reads K/V head h / (heads / kv_heads); k_bhs/v_bhs index the
 * kv_heads heads), a causal sliding window (window > 0: query i sees keys
 * i-window+1 .. i) and head_dim 256 (forward only).  It serves the
 * Gemma-3-shaped prefill, which the reference runs through its masked-math
 * SDPA decomposition instead (aten_fast.py:9112-9123, :6869) and
 * fast_fused_flash_attention_forward's contract otherwise
 * (aten_fast.py:7533-7587).  mi355x_attn_fwd is this call with
 * kv_heads = heads and window = 0. */
int mi355x_attn_fwd_ex(void* o, const int64_t* o_bhs, float* lse, const void* q,
                       const int64_t* q_bhs, const void* k, const int64_t* k_bhs,
                       const void* v, const int64_t* v_bhs, int64_t batch, int64_t heads,
                       int64_t kv_heads, int64_t sq, int64_t skv, int64_t d, double scale,
                       int causal, int64_t window, int dtype, mi355x_stream_t stream);
/* dQ, dK, dV (written, never accumulated).  workspace holds two f32 row
 * terms per query: D_i = sum(dO*O) and LSE_i * log2(e). */
int64_t mi355x_attn_bwd_workspace_bytes(int64_t batch, int64_t heads,
                                        int64_t sq, int64_t skv, int64_t d);
int mi355x_attn_bwd(void* dq, const int64_t* dq_bhs, void* dk,
                    const int64_t* dk_bhs, void* dv, const int64_t* dv_bhs,
                    const void* dout, const int64_t* do_bhs, const void* q,
                    const int64_t* q_bhs, const void* k, const int64_t* k_bhs,
                    const void* v, const int64_t* v_bhs, const void* o,
                    const int64_t* o_bhs, const float* lse, int64_t batch,
                    int64_t heads, int64_t sq, int64_t skv, int64_t d,
                    double scale, int causal, int dtype, void* workspace,
                    int64_t ws_bytes, mi355x_stream_t stream);
/* ---- attention for the inputs the MFMA kernels do not take (the rest of
 *      _fused_fa_inputs' gate, aten_fast.py:7462-7530: f32 and any head_dim
 *      up to 256; the reference runs these through its scalar kernels,
 *      flash_attention_bwd_kernels.mojo:215-310) ----------------------
 * f32 math; q/k/v/o/dout/grads need only a unit head_dim stride.  Grouped
 * K/V heads and the causal sliding window as in mi355x_attn_fwd_ex; the
 * backward's dK/dV of a K/V head sum over its query heads (the backward of
 * grouped or windowed attention, which the reference leaves to its
 * masked-math decomposition, aten_fast.py:9112-9123). */
int mi355x_attn_fwd_gen(void* o, const int64_t* o_bhs, float* lse, const void* q,
                        const int64_t* q_bhs, const void* k, const int64_t* k_bhs,
                        const void* v, const int64_t* v_bhs, int64_t batch, int64_t heads,
                        int64_t kv_heads, int64_t sq, int64_t skv, int64_t d, double scale,
                        int causal, int64_t window, int dtype, mi355x_stream_t stream);
/* Workspace of mi355x_attn_bwd_gen: 2 floats per query row, plus (grouped
 * heads) 2 * batch * heads * skv * d floats of per-query-head dK/dV
 * partials that the bf16/f16 MFMA backward sums in head order. */
int64_t mi355x_attn_bwd_gen_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads,
                                            int64_t sq, int64_t skv, int64_t d);
int mi355x_attn_bwd_gen(void* dq, const int64_t* dq_bhs, void* dk, const int64_t* dk_bhs,
                        void* dv, const int64_t* dv_bhs, const void* dout,
                        const int64_t* do_bhs, const void* q, const int64_t* q_bhs,
                        const void* k, const int64_t* k_bhs, const void* v,
                        const int64_t* v_bhs, const void* o, const int64_t* o_bhs,
                        const float* lse, int64_t batch, int64_t heads, int64_t kv_heads,
                        int64_t sq, int64_t skv, int64_t d, double scale, int causal,
                        int64_t window, int dtype, void* workspace, int64_t ws_bytes,
                        mi355x_stream_t stream);
/* mi355x_attn_bwd without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The row terms live in a fixed 32 MiB device array per GPU,
 * which limits batch * heads * sq to 4,194,272 query rows (larger shapes
 * return MI355X_EINVAL).  Every call on one GPU shares that array: calls
 * that overlap on one GPU (different streams or threads) race.  The array
 * used is the one on the device that owns `stream` (the current device for
 * the null stream). */
int mi355x_attn_bwd_noalloc(void* dq, const int64_t* dq_bhs, void* dk,
                            const int64_t* dk_bhs, void* dv, const int64_t* dv_bhs,
                            const void* dout, const int64_t* do_bhs, const void* q,
                            const int64_t* q_bhs, const void* k, const int64_t* k_bhs,
                            const void* v, const int64_t* v_bhs, const void* o,
                            const int64_t* o_bhs, const float* lse, int64_t batch,
                            int64_t heads, int64_t sq, int64_t skv, int64_t d,
                            double scale, int causal, int dtype, mi355x_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MI355X_KERNELS_H */
