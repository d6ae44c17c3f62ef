/*
 * ember_amd.h -- C ABI of libember_amd.so, the MI355X (gfx950) backend for
 * Ember's native core.
 *
 * The library is a drop-in for the reference's GPU backend: it exports the
 * same symbols with the same signatures that the reference's CPython binding
 * (src/tensor/tensor_api.c, src/random/random_api.c) links against, so that
 * binding can be linked against this library unchanged.  All pointers named
 * a/b/out/q/k/v/... are device pointers obtained from alloc_memory() (or any
 * other hipMalloc'd memory); sizes are in float elements unless noted.
 * Work is enqueued on the HIP null stream, exactly like the reference's
 * default-stream launches; results are visible after sync_device() or a
 * copy_from_device(), which synchronises.
 *
 * Threads.  Like the reference (single-threaded, every call made under the
 * Python GIL), the library expects one host thread in it at a time per
 * device: operators that use library scratch (attention_bwd's row
 * statistics, split-K and reduction partials) share one buffer per device
 * and operator, and two threads' launches may interleave on the null
 * stream.  The allocator and the error slots are thread-safe.
 *
 * Error behaviour.  The reference prints and calls exit() on any device
 * error (src/core/utils_gpu.cuh:13-19).  Here the void entry points keep
 * their signatures but record the first error in a sticky per-thread slot
 * (ember_get_last_error) and print it to stderr; the process is not killed.
 * The attention entry points, which are new, return that status directly.
 * Argument errors never launch a kernel.
 */
#ifndef EMBER_AMD_H
#define EMBER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
enum {
    EMBER_OK = 0,
    EMBER_ERR_INVALID_ARGUMENT = 1, /* bad sizes, strides or alignment */
    EMBER_ERR_UNSUPPORTED = 2,      /* e.g. head_dim outside {32, 64, 128} */
    EMBER_ERR_OUT_OF_MEMORY = 3,
    EMBER_ERR_DEVICE = 4            /* a HIP runtime error; see stderr */
};

/* Returns the first status recorded on this thread since the last call, and
 * clears it (hipGetLastError-style).  No reference counterpart: the reference
 * exits instead (src/core/utils_gpu.cuh:17). */
int ember_get_last_error(void);
const char *ember_error_string(int status);

/* ---- device memory: replaces src/core/memory.h:10-14 (memory_gpu.cu:10-43) ---- */
void *alloc_memory(size_t bytes);  /* NULL on failure, like memory_gpu.cu:15-19 */
void free_memory(void *ptr);
void copy_to_device(void *dst_device, const void *src_host, size_t bytes);
void copy_from_device(void *dst_host, const void *src_device, size_t bytes);
void sync_device(void);
/* alloc_memory/free_memory cache freed blocks per device instead of calling
 * hipFree (which synchronises the device) on every free; reuse is ordered by
 * the null stream all library work runs on.  EMBER_AMD_NO_CACHE=1 turns the
 * cache off.  No reference counterpart (memory_gpu.cu:10-28 calls
 * cudaMalloc/cudaFree each time); these two report and release the cache.
 * ember_empty_cache synchronises the current device and hipFrees every
 * cached block and the library's own scratch buffers (attention_bwd's row
 * statistics and dq partials, reduction partials), which are otherwise kept
 * for reuse; call it when no other thread is inside the library (a call in
 * flight may hold a scratch buffer it has not launched on yet).
 * ember_memory_stats gives the current device's bytes handed out, bytes
 * cached and peak bytes handed out (rounded block sizes). */
void ember_empty_cache(void);
void ember_memory_stats(size_t *in_use, size_t *cached, size_t *peak);

/* Bitwise-reproducible results (no reference counterpart: the reference
 * has no operator whose result depends on timing).  Off by default.  The
 * only such operator here is attention_bwd's dq at S > 128 (S > 64 at
 * D = 32); with the switch on its atomic adds are made in a fixed order
 * instead (per-tile counters; see attention_bwd).  Every other operator of this library
 * is reproducible either way.  The switch is process-wide; set it between
 * calls, not while another thread is inside the library. */
void ember_set_deterministic(int enabled);
int ember_get_deterministic(void);
/* Deterministic mode's waits for a dq tile's turn that gave up, on the
 * current device since the library was loaded (0 on success; -1 and a
 * recorded error if the device cannot be read).  A wait gives up only after
 * about 2 s; the sum is then still complete, but its order is the arrival
 * order, so 0 means every deterministic dq was added in its fixed order.
 * Synchronises the device.  No reference counterpart. */
int ember_deterministic_timeouts(void);

/* Launch log, for tests and profiling scripts that must know which kernel
 * a call ran (the attention entry points pick one of several kernels by
 * sequence length, head dimension and launch size).  No reference
 * counterpart.  ember_launch_log returns the names of the kernels the
 * calling thread has launched through this library since its last
 * ember_launch_log_reset, comma-separated in launch order (at most about
 * 1 KiB; a log that would grow past that ends in "...").  The string
 * belongs to the library and stays valid until the thread's next library
 * call. */
void ember_launch_log_reset(void);
const char *ember_launch_log(void);

/* ---- random tensors: replaces src/random/distributions.h:8-9 ----
 * (distributions_gpu.cu:11-32; called by src/random/random_api.c:70,88.)
 * uniform fills out[0..size) with low + (rand()/RAND_MAX)*(high - low) in
 * fp32, drawn on the host from the C library's rand() -- the generator the
 * reference binding's _seed() seeds with srand() -- and copied to the
 * device.  constant sets out[0..size) to value (a fill kernel on the null
 * stream).  size <= 0 does nothing; errors are recorded as above. */
void uniform(float low, float high, float *out, int size);
void constant(float value, float *out, int size);

/* ---- element-wise operators: replaces src/tensor/operators.h:10-18 ----
 * One declaration per row of ember_amd/csrc/operators.def, which lists the
 * same 37 operators as the reference's src/tensor/operators.def:39-82. */
#define EMBER_BINARY_OP(name, expr) \
    void name##_tensor(const float *a, const float *b, float *out, int size);
#define EMBER_SCALAR_OP(name, expr) \
    void name##_scalar(const float *a, float b, float *out, int size);
#define EMBER_BROADCAST_OP(name, expr)                                                    \
    void name##_broadcasted(const float *a, const float *b, float *out, const int *shape, \
                            const int *strides_a, const int *strides_b, int ndim);
#define EMBER_UNARY_OP(name, expr) void name##_tensor(const float *a, float *out, int size);
#include "../ember_amd/csrc/operators.def"

/* ---- non-element-wise operators: replaces src/tensor/operators.h:20-27 ---- */

/* out(n x m) = a(n x k) @ b(k x m), row-major fp32, fp32 MFMA with fp32
 * accumulation.  Replaces operators_gpu.cu:114-124 (cublasSgemm). */
void matmul(const float *a, const float *b, float *out, int n, int m, int k);
/* `batch` independent products with strides n*k, k*m, n*m.
 * Replaces operators_gpu.cu:126-136 (cublasSgemmStridedBatched). */
void matmul_batched(const float *a, const float *b, float *out, int batch, int n, int m, int k);
/* out(m x n) = a(n x m)^T.  Replaces operators_gpu.cu:138-151. */
void transpose(const float *a, float *out, int n, int m);
/* Sum of all elements; replaces operators_gpu.cu:153-166 (the device
 * reduction is summed in a fixed tree order, not sequentially). */
float sum(const float *a, int size);

/* Ember's MSELoss in one pass (ember/loss/losses.py:19-26): grad[i] =
 * (pred[i] - target[i]) * scale and *loss = sum over i of (pred - target)^2,
 * computed exactly as sum(diff * diff) above (same partition and order), so
 * with scale = fp32(2/n) both are bit-identical to the composed operators.
 * No reference counterpart as one symbol: it fuses sub_tensor, mul_tensor,
 * sum and mul_scalar.  Synchronises (the loss is read back). */
int mse_loss(const float *pred, const float *target, float *grad, int size, float scale, float *loss);
/* Product of shape[start:end]; replaces operators_gpu.cu:168-173. */
int sum_axis_product(const int *shape, int start, int end);
/* Reduce the middle axis of (outer, axis_dim, inner); sequential fp32 sum /
 * max in index order per output, as operators_gpu.cu:175-219. */
void sum_axis(const float *a, float *out, int outer_stride, int inner_stride, int axis_dim);
void max_axis(const float *a, float *out, int outer_stride, int inner_stride, int axis_dim);
/* out = exp(a - max) / sum(exp(a - max)) along the middle axis of
 * (outer, axis_dim, inner), in one launch: Ember's softmax
 * (ember/tensor/tensor.py:430-437, five operators in the reference) with the
 * same per-element fp32 operations; along the last axis (inner == 1) the sum
 * is taken in a fixed tree order instead of index order.  Returns a status. */
int softmax_axis(const float *a, float *out, int outer, int inner, int axis_dim);

/* ---- fused attention (new; no reference counterpart exists) ----
 *
 * Shapes: batch B, heads H, sequence S (queries == keys), head_dim D in
 * {32, 64, 128}.  Element (b, h, s, d) of q, k, v (and dq, dk, dv) lives at
 *     b*in_sb + h*in_sh + s*in_ss + d
 * and of o (and d_o) at b*out_sb + h*out_sh + s*out_ss + d, so packed
 * (B, S, 3, H, D) projections are read and (B, S, H, D) outputs written
 * without copies.  d must be contiguous, every stride a multiple of 4, the
 * row strides (in_ss, out_ss) below 2^24, B*H*S*D at most 2^33, every
 * pointer 16-byte aligned and scale finite and >= 0.  lse is dense
 * (B, H, S), natural log.
 *
 * Semantics (the CPU restatement in oracle/ember_oracle.c is the checker):
 *   s[i][j] = scale * <q_i, k_j>;  key j visible to query i iff j <= i when
 *   causal (top-left aligned), always otherwise;
 *   o_i = softmax_j(s[i][.]) v;  lse_i = ln sum_j exp(s[i][j]).
 * Slots the reference would fill: src/tensor/operators.h:20-27 (new rows
 * beside matmul), called from new _attention_fwd / _attention_bwd wrappers
 * beside _matmul in src/tensor/tensor_api.c:305-354. */
int attention_fwd(const float *q, const float *k, const float *v, float *o, float *lse,
                  int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                  int64_t in_sb, int64_t in_sh, int64_t in_ss,
                  int64_t out_sb, int64_t out_sh, int64_t out_ss);

/* Backward of attention_fwd: given q, k, v, the forward's o and lse, and the
 * upstream gradient d_o, writes dq, dk, dv (same layout as q, k, v).  P is
 * recomputed from lse; the S x S matrix is never stored.  Needs
 * 2*B*H*S_pad*4 bytes of device scratch (S_pad = S rounded up to 32; none at
 * S <= 64, nor at S <= 128 with D = 64 or 128), which the library keeps
 * cached between calls.
 * Determinism: dk and dv are bitwise reproducible.  For S > 128 (S > 64 at
 * D = 32), dq is accumulated in HBM with fp32 atomic adds from every key
 * block (128 keys; 64 at D = 64) that sees a query row, so its last bits
 * vary from run to run (each run within the stated tolerance).  At S <= 64,
 * and at S <= 128 with D = 64 or 128 (one workgroup per head, which forms
 * each element of dq whole), dq is stored once and reproducible too.
 * Because of the atomics dq must be device memory (not host or managed
 * memory), and dq must not overlap q, k, v, o, lse, d_o, dk or dv.
 * With ember_set_deterministic(1), the atomic cases add each dq tile's
 * key-block contributions in a fixed order (highest key block first), each
 * key block waiting on a per-tile counter for its turn: dq is then bitwise
 * reproducible, and dk, dv are the same bits as without the switch.  Extra
 * scratch: B*H*S_pad/16 ints. */
int attention_bwd(const float *q, const float *k, const float *v, const float *o,
                  const float *lse, const float *d_o, float *dq, float *dk, float *dv,
                  int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                  int64_t in_sb, int64_t in_sh, int64_t in_ss,
                  int64_t out_sb, int64_t out_sh, int64_t out_ss);

/* attention_bwd without any device allocation.  No counterpart in the
 * reference.  It is for callers that cannot allocate device memory during the
 * call: tight serving loops and harnesses that forbid hipMalloc.  Same
 * arguments, kernels, results and errors as attention_bwd, also in
 * deterministic mode, except where the row statistics and deterministic
 * mode's tile counters live: a fixed device array of 16.5 MiB inside the
 * library, one per GPU, held until the process ends, instead of
 * library-allocated scratch.  Limit: B*H*S_pad <= 2^21 rows (S_pad = S
 * rounded up to 32); a larger call returns EMBER_ERR_INVALID_ARGUMENT and
 * launches nothing (S <= 64, and S <= 128 at D = 64 or 128, need no
 * statistics and so no array space).  Like every entry point here it
 * enqueues on the null stream, which cannot be captured into a HIP graph.
 * Every call on one GPU shares that GPU's array.  Calls are ordered because
 * all library work runs on the null stream; launches of this entry point
 * that overlap on one GPU would race on the array.  Each call writes every
 * statistic and counter it reads before reading it, so nothing carries over
 * between calls. */
int attention_bwd_noalloc(const float *q, const float *k, const float *v, const float *o,
                          const float *lse, const float *d_o, float *dq, float *dk, float *dv,
                          int64_t B, int64_t H, int64_t S, int64_t D, float scale, int causal,
                          int64_t in_sb, int64_t in_sh, int64_t in_ss,
                          int64_t out_sb, int64_t out_sh, int64_t out_ss);

/* ---- fused Adam: replaces ember/optim/adam.py:24-45 (Adam.apply) ----
 *
 * One Adam step over `ntensors` parameter tensors in as few launches as
 * possible (48 tensors per launch).  params[i], grads[i], exp_avg[i] (m),
 * exp_avg_sq[i] (v) are device pointers to sizes[i] floats each; the
 * pointer and size tables themselves are host memory.  p, m, v are updated
 * in place.  The arithmetic is Ember's, operation by operation:
 *   m = m*b1 + g*(1-b1);  v = v*b2 + (g*g)*(1-b2);
 *   p = p - ((m/(1-b1^t))*lr) / (sqrt(v/(1-b2^t)) + eps)
 * each step an fp32 operation rounded on its own (no fused multiply-add),
 * with every scalar formed in double and rounded to fp32 once, so the result
 * is bit-identical to the reference's composed element-wise operators.
 * `step` (t) starts at 1.  Returns a status; argument errors launch nothing. */
int adam_step(float *const *params, const float *const *grads, float *const *exp_avg,
              float *const *exp_avg_sq, const int64_t *sizes, int ntensors, double lr,
              double beta1, double beta2, double eps, int64_t step);

/* ---- fused AdamW: replaces ember/optim/adamw.py:33-56 (AdamW.apply) ----
 * adam_step's m, v, m_hat, v_hat, then the decoupled decay and the Adam
 * step, each an fp32 operation in Ember's order:
 *   p = p - p*(lr*wd);  p = p - ((m/(1-b1^t))*lr) / (sqrt(v/(1-b2^t)) + eps)
 * with lr*wd one double product rounded to fp32 (Python forms it before the
 * tensor multiply), so the result is bit-identical to the reference's
 * composed operators.  Same arguments and errors as adam_step plus
 * weight_decay. */
int adamw_step(float *const *params, const float *const *grads, float *const *exp_avg,
               float *const *exp_avg_sq, const int64_t *sizes, int ntensors, double lr,
               double beta1, double beta2, double eps, double weight_decay, int64_t step);

/* ---- fused SGD: replaces ember/optim/sgd.py:25-35 (SGD.apply) ----
 * v = v*momentum;  v = v + g;  p = p - v*lr  (fp32, Ember's order; v is the
 * velocity, updated in place), over `ntensors` tensors as adam_step. */
int sgd_step(float *const *params, const float *const *grads, float *const *velocity,
             const int64_t *sizes, int ntensors, double lr, double momentum);

/* ---- transformer-block pieces (config 5's pre-LN decoder block) ----
 * None has a counterpart in the reference; each replaces a composition of
 * its element-wise operators.  All return a status and launch nothing on an
 * argument error.  Row-major fp32, device pointers, 16-byte alignment where
 * noted. */

/* out(n x m) = act(a @ b + bias) + residual, with pre = a @ b + bias stored
 * before the activation when pre is not NULL (what the activation's backward
 * needs).  bias (m), residual (n x m) and pre may each be NULL; act 0 = none,
 * 1 = Ember's GELU 0.5*x*(1 + tanh(0.8x)) (ember/nn/activations.py:58).
 * Replaces Linear.forward's `b + x @ w` (ember/nn/layers.py:45-48) plus the
 * activation and the residual add as separate operators. */
int linear_fwd(const float *a, const float *b, const float *bias, const float *residual,
               float *out, float *pre, int n, int m, int k, int act);

/* out = act(op(a) @ op(b) + bias) + residual for `batch` products (strides
 * n*k, k*m, n*m), where op(a) is a (n x k) or, with trans_a, the transpose of
 * a stored (k x n), and op(b) is b (k x m) or, with trans_b, the transpose of
 * b stored (m x k); pre as in linear_fwd.  Replaces Linear.backward's
 * `em.T(x) @ grad_y` and `grad_y @ em.T(w)` (ember/nn/layers.py:50-56),
 * which materialise the transposes, and generalises matmul /
 * matmul_batched (operators_gpu.cu:114-136).  Products with fewer output
 * tiles than CUs split k and add the parts in a fixed order (library
 * scratch of splits * batch * n * m floats). */
int gemm_ex(const float *a, const float *b, float *out, int batch, int n, int m, int k,
            int trans_a, int trans_b, const float *bias, const float *residual, float *pre, int act);

/* dx = dy * ((1 + tanh(0.8u)) * (0.5 + 0.8(u - y))): the backward of Ember's
 * GELU (ember/nn/activations.py:61-66) with u its input and y its output.
 * y may be NULL: it is then recomputed from u as (0.5u)(1 + tanh(0.8u)),
 * the forward's own fp32 operations, so dx is bit-identical to passing the
 * stored output (and one array less is read). */
int gelu_bwd(const float *dy, const float *u, const float *y, float *dx, int64_t n);

/* out[c] = sum over rows of x[r][c] (x is rows x cols): a Linear layer's bias
 * gradient, em.sum(grad_y, axis=0) in ember/nn/layers.py:53.  Deterministic
 * (fixed summation order); uses library scratch. */
int col_sum(const float *x, float *out, int64_t rows, int64_t cols);

/* dx = gelu_bwd(dy, u) (output recomputed) and dbias = col_sum(dx) in one
 * pass: the same bits as the two calls in turn, without re-reading dx.
 * Replaces GELU.backward followed by em.sum(grad_y, axis=0) in a Linear
 * layer with a GELU activation (ember/nn/activations.py:61-66,
 * ember/nn/layers.py:54).  Uses library scratch. */
int gelu_bwd_col_sum(const float *dy, const float *u, float *dx, float *dbias, int64_t rows, int64_t cols);

/* LayerNorm over the last dimension d (d % 4 == 0, d <= 4096; all pointers
 * 16-byte aligned and non-NULL):
 *   mean = sum(x)/d, var = sum((x-mean)^2)/d, rstd = 1/sqrt(var + eps),
 *   y = (x - mean)*rstd*gamma + beta;  mean and rstd (rows) are kept for
 * the backward, which gives dx (plus dres when dres is not NULL: the gradient
 * that reaches x through a residual connection, added in the same pass) and
 * the parameter gradients
 *   dgamma = sum_rows(dy*xhat), dbeta = sum_rows(dy)   (xhat = (x-mean)*rstd)
 * deterministically (fixed-order reduction over library scratch). */
int layernorm_fwd(const float *x, const float *gamma, const float *beta, float *y, float *mean,
                  float *rstd, int64_t rows, int64_t d, float eps);
int layernorm_bwd(const float *x, const float *gamma, const float *mean, const float *rstd,
                  const float *dy, const float *dres, float *dx, float *dgamma, float *dbeta,
                  int64_t rows, int64_t d);

#undef EMBER_BINARY_OP
#undef EMBER_SCALAR_OP
#undef EMBER_BROADCAST_OP
#undef EMBER_UNARY_OP

#ifdef __cplusplus
}
#endif

#endif /* EMBER_AMD_H */
