/*
 * rtensor_hip.h -- C ABI of the MI355X (gfx950) training backend for rtensor.
 *
 * The backend replaces rtensor's wgpu module (crates/rtensor/src/gpu/mod.rs)
 * for the MLP training step.  Each entry point below names the rtensor::gpu
 * call it stands in for (file:line in the rtensor crate).  A Rust FFI crate
 * binds these symbols one-for-one.
 *
 * Conventions
 *   - Every function returns an int status (rt_status); 0 is success.  The
 *     reference panics on misuse (mod.rs:1342-1343, 1487-1491, 799); here the
 *     same conditions return RT_ERR_SHAPE / RT_ERR_INVALID / RT_ERR_LABEL and
 *     leave a message in rt_last_error(ctx).
 *   - Host memory is caller-owned: the library never keeps a host pointer
 *     past the call and never calls back.
 *   - One HIP stream per rt_ctx.  Kernel entry points only enqueue work, like
 *     Gpu::record + Gpu::submit (mod.rs:609, 1231-1237); rt_download,
 *     rt_sync and the rt_mlp_* readers block, like Gpu::download
 *     (mod.rs:530-544).  An rt_ctx is not thread-safe, as Gpu is not Send.
 *   - Freed buffers return to a per-context cache and are reused by later
 *     allocations of the same size class; device memory is given back by
 *     rt_close (or when an allocation would otherwise fail).  Reuse is safe
 *     because all work of a context runs in order on its one stream.
 *   - Tensors are dense row-major.  Weights are [in, out], biases [1, out],
 *     parameters travel in the order [W1, b1, W2, b2, ...] (nn.rs:190-192).
 *     Labels are u32 (mod.rs:1672-1675).
 */
#ifndef RTENSOR_HIP_H
#define RTENSOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct rt_ctx rt_ctx; /* ~ rtensor::gpu::Gpu        (mod.rs:224-255)   */
typedef struct rt_buf rt_buf; /* ~ rtensor::gpu::GpuTensor  (mod.rs:190-208)   */
typedef struct rt_mlp rt_mlp; /* ~ rtensor::gpu::GpuMlp     (mod.rs:1322-1336) */

typedef enum {
  RT_OK = 0,
  RT_ERR_NO_DEVICE = 1,   /* Gpu::new() -> Err (mod.rs:263-277)             */
  RT_ERR_INVALID = 2,     /* null handle, bad enum, bad size                 */
  RT_ERR_SHAPE = 3,       /* the reference's shape assert! (mod.rs:1487-1491) */
  RT_ERR_DTYPE = 4,       /* operand dtype not supported by the entry point  */
  RT_ERR_OOM = 5,         /* device allocation failed                        */
  RT_ERR_LABEL = 6,       /* a label >= number of classes (undefined in the
                             reference's xent kernel, kernels.rs:158-159)    */
  RT_ERR_HIP = 7,         /* a HIP runtime call failed                       */
  RT_ERR_OVERFLOW = 8     /* non-finite gradient under loss scaling          */
} rt_status;

typedef enum { RT_F32 = 0, RT_BF16 = 1, RT_F16 = 2, RT_U32 = 3 } rt_dtype;

/* C = A·B, Aᵀ·B (A stored [K, M]) or A·Bᵀ (B stored [N, K]). */
typedef enum { RT_NN = 0, RT_TN = 1, RT_NT = 2 } rt_layout;

typedef enum {
  RT_EPI_NONE = 0,      /* C = acc                                           */
  RT_EPI_BIAS = 1,      /* C = acc + 1ₙb               (mm_bias, gemm.rs:452) */
  RT_EPI_BIAS_RELU = 2, /* C = max(acc + 1ₙb, 0)       (flag_relu, gemm.rs:389) */
  RT_EPI_RELU_MASK = 3  /* C = acc ⊙ 1[aux > 0]        (relu_bwd, kernels.rs:119) */
} rt_epilogue;

/* ------------------------------------------------------------- device */

/* Gpu::new / Gpu::with_preference (mod.rs:263-277).  device = HIP ordinal. */
int rt_open(int device, rt_ctx** out);
int rt_close(rt_ctx* ctx);
/* Message for the last failed call on ctx (or, when ctx is NULL, of the
 * calling thread's last failed rt_open). */
const char* rt_last_error(const rt_ctx* ctx);
/* Gpu::info (mod.rs:412): device name and arch, NUL-terminated into buf. */
int rt_info(rt_ctx* ctx, char* buf, size_t len);
/* Gpu::sync (mod.rs:564-566): wait for all enqueued work.  Returns
 * RT_ERR_LABEL (once) if a softmax-xent launch saw a label >= classes. */
int rt_sync(rt_ctx* ctx);

/* ------------------------------------------------------------- buffers */

/* Gpu::zeros (mod.rs:501-506). rank <= 4. */
int rt_zeros(rt_ctx* ctx, rt_dtype dtype, const size_t* shape, int rank, rt_buf** out);
/* Gpu::upload (mod.rs:509-517); host holds prod(shape) elements of dtype. */
int rt_upload(rt_ctx* ctx, rt_dtype dtype, const size_t* shape, int rank, const void* host, rt_buf** out);
/* Gpu::download (mod.rs:530-544): blocking copy of the whole tensor;
 * bytes must equal the tensor's size in bytes. */
int rt_download(rt_ctx* ctx, const rt_buf* buf, void* host, size_t bytes);
/* Asynchronous host->device overwrite of an existing buffer (the plan's
 * per-step writes, mod.rs:1486-1495). */
int rt_write(rt_ctx* ctx, rt_buf* buf, const void* host, size_t bytes);
int rt_free(rt_ctx* ctx, rt_buf* buf);
/* GpuTensor::shape / len (mod.rs:197-208).  shape needs room for 4. */
int rt_buf_info(const rt_buf* buf, rt_dtype* dtype, size_t* shape, int* rank);
/* upload_labels (mod.rs:1672-1675): usize labels -> u32 device buffer. */
int rt_upload_labels(rt_ctx* ctx, const uint64_t* labels, size_t n, rt_buf** out);
/* f32 -> bf16/f16 with round-to-nearest-even, or half -> f32 (same shape):
 * upload_f16 / op_empacota_f16 (mod.rs:1151-1185, EMPACOTA mista.rs:326-341). */
int rt_convert(rt_ctx* ctx, const rt_buf* src, rt_buf* dst);

/* ------------------------------------------------------------- ops */

/* GEMM with f32 accumulate.  op_matmul / op_matmul_at_b / op_matmul_a_bt
 * (mod.rs:685-700), op_matmul_bias (mod.rs:722-749) and op_matmul_f16
 * (mod.rs:1191-1229).  A and B are both f32, both bf16 or both f16; C is
 * f32, or bf16 for half inputs.  aux is the bias [1, N] for RT_EPI_BIAS*,
 * or the mask source [M, N] for RT_EPI_RELU_MASK, else NULL.  colsum, if not
 * NULL, receives f32 column sums of B over K (= 1ᵀ·B, the bias gradient when
 * B is δ): supported for RT_TN. */
int rt_gemm(rt_ctx* ctx, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* c,
            rt_epilogue epi, const rt_buf* aux, rt_buf* colsum);

/* The backward of a Linear layer Z = X·W + 1ₙb (nn.rs:82-98 adjoints; the
 * op_matmul_at_b + op_matmul_a_bt + ops_colsum of GpuMlp's backward,
 * mod.rs:1432-1467): dW = Xᵀ·δ [K, N], db = 1ᵀ·δ [N] (NULL to skip) and
 * dX = δ·Wᵀ [M, K] (NULL to skip), with X [M, K], δ [M, N], W [K, N].  f32
 * shapes the paired kernel takes run as ONE launch; anything else is the two
 * rt_gemm calls. */
int rt_linear_backward(rt_ctx* ctx, const rt_buf* x, const rt_buf* delta, const rt_buf* w, rt_buf* dx, rt_buf* dw,
                       rt_buf* db);

/* ops_split_k (mod.rs:1095-1146): C = A·B (RT_NN) or Aᵀ·B (RT_TN) with K cut
 * into `slices`; slice s writes partials[s] and a fixed-order reduction sums
 * them (deterministic, no atomics).  partials is f32 with >= slices*M*N
 * elements.  colsum as in rt_gemm (RT_TN only). */
int rt_gemm_splitk(rt_ctx* ctx, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* c,
                   rt_buf* partials, size_t slices, rt_buf* colsum);
/* rt_gemm_splitk for callers that cannot allocate device memory (code under
 * HIP graph capture, serving or training loops, harnesses that forbid
 * hipMalloc); no counterpart in the reference.  The same kernels and results,
 * bit for bit, but the partial planes (and the half GEMM's column-sum shares)
 * live in a static 64 MiB device array of the library: each GPU it runs on
 * holds its own copy until the process ends.  The call allocates nothing; it
 * returns RT_ERR_SHAPE when slices·M·N + slices·N (+ the shares) floats
 * exceed 64 MiB.  Calls that overlap on one GPU (other contexts, other
 * threads) share the array and race; calls on one context are ordered. */
int rt_gemm_splitk_static(rt_ctx* ctx, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* c,
                          size_t slices, rt_buf* colsum);
/* fatias_sugeridas (mod.rs:1079-1088), re-derived for 256 CUs. */
size_t rt_splitk_slices(size_t m, size_t n, size_t k);

/* Row and column counts of rt_colsum, rt_bias_add, rt_softmax_xent,
 * rt_argmax_rows and rt_accuracy, and M, N, K of the GEMM entry points, are
 * at most 2^30 each (RT_ERR_SHAPE otherwise). */
/* ops_colsum (mod.rs:838-855): dst[1, C] (f32) = 1ᵀ·src[R, C] (f32/bf16/f16). */
int rt_colsum(rt_ctx* ctx, const rt_buf* src, rt_buf* dst);
/* op_bias_add (mod.rs:752-762): Z += 1ₙb in place. */
int rt_bias_add(rt_ctx* ctx, rt_buf* z, const rt_buf* b);
/* op_relu (mod.rs:765-775): Y = max(X, 0). */
int rt_relu(rt_ctx* ctx, const rt_buf* x, rt_buf* y);
/* op_relu_bwd (mod.rs:778-788): δ ← δ ⊙ 1[A > 0] in place. */
int rt_relu_bwd(rt_ctx* ctx, const rt_buf* a, rt_buf* delta);
/* op_softmax_xent (mod.rs:791-808): per row loss -ln(max(p_y, 1e-12)) into
 * loss_rows[B] and δ = (softmax(z) - onehot(y)) * (scale / B).  Labels >= C
 * are reported by the next blocking call as RT_ERR_LABEL. */
int rt_softmax_xent(rt_ctx* ctx, const rt_buf* logits, const rt_buf* labels, rt_buf* delta,
                    rt_buf* loss_rows, float scale);
/* op_adam + atualizar_adam (mod.rs:859-907) with Adam::step's arithmetic
 * (optim.rs:162-198): t is the 1-based step that sets c1 = 1-β1^t, c2 = 1-β2^t. */
int rt_adam(rt_ctx* ctx, rt_buf* theta, rt_buf* m, rt_buf* v, const rt_buf* g, float lr, float beta1,
            float beta2, float eps, int t);
/* Sgd::step (optim.rs:80-114); velocity may be NULL when momentum == 0. */
int rt_sgd(rt_ctx* ctx, rt_buf* theta, rt_buf* velocity, const rt_buf* g, float lr, float momentum);
/* Adam::step / Sgd::step over a whole parameter list (optim.rs:80-114,
 * 162-198: the loop over params), as one launch per 24 tensors instead of
 * one per tensor.  Arrays of n buffers; for SGD without momentum velocity
 * may be NULL.  Arithmetic identical to rt_adam / rt_sgd.  A tensor listed
 * again is updated again, after its earlier listing (the repeat starts a new
 * launch), as the loop over the list would. */
int rt_adam_many(rt_ctx* ctx, int n, rt_buf* const* theta, rt_buf* const* m, rt_buf* const* v,
                 const rt_buf* const* g, float lr, float beta1, float beta2, float eps, int t);
int rt_sgd_many(rt_ctx* ctx, int n, rt_buf* const* theta, rt_buf* const* velocity, const rt_buf* const* g,
                float lr, float momentum);

/* ------------------------------------------------------------- model */

typedef enum { RT_OPT_ADAM = 0, RT_OPT_SGD = 1 } rt_optimizer;
typedef enum { RT_PREC_F32 = 0, RT_PREC_BF16 = 1 } rt_precision;

typedef struct {
  int optimizer;    /* rt_optimizer                                      */
  float lr;         /* GpuMlp::from_params lr (mod.rs:1341)              */
  float beta1;      /* 0.9   (mod.rs:1462)                               */
  float beta2;      /* 0.999                                            */
  float eps;        /* 1e-8  (mod.rs:873)                                */
  float momentum;   /* Sgd momentum (optim.rs:96-100)                    */
  int precision;    /* rt_precision: bf16 weights/activations with f32
                       master weights when RT_PREC_BF16                 */
  float loss_scale; /* static loss scale (RT_PREC_BF16), 1 = none       */
} rt_mlp_config;

/* GpuMlp::from_params (mod.rs:1341-1482).  n_layers Dense layers with
 * dims[0..n_layers]; weights[l] is host [dims[l], dims[l+1]], biases[l] is
 * host [1, dims[l+1]].  Hidden layers are ReLU and the output is linear, as
 * in the reference plan (mod.rs:1418-1424).  batch fixes the plan's shapes.
 * 1 <= n_layers <= 1024. */
int rt_mlp_create(rt_ctx* ctx, int n_layers, const size_t* dims, const float* const* weights,
                  const float* const* biases, size_t batch, const rt_mlp_config* cfg, rt_mlp** out);
int rt_mlp_destroy(rt_mlp* mlp);
/* GpuMlp::step (mod.rs:1499-1511): forward, softmax cross-entropy, backward
 * and optimizer update, enqueued without waiting.  x is [batch, dims[0]]
 * (f32, or bf16 for RT_PREC_BF16), labels u32 [batch].  A label >= the
 * number of classes (undefined behaviour in the reference's XENT,
 * kernels.rs:158-159) raises the plan's own label flag: that update and every
 * later one are skipped (weights, moments and t unchanged) until the next
 * blocking call on the plan (last_loss, logits, weights, grads, overflow,
 * set_weights, get/set_optimizer_state) reports RT_ERR_LABEL once and clears
 * the flag. */
int rt_mlp_step(rt_mlp* mlp, const rt_buf* x, const rt_buf* labels);
/* GpuMlp::forward_only (mod.rs:1514-1521). */
int rt_mlp_forward(rt_mlp* mlp, const rt_buf* x);
/* GpuMlp::logits (mod.rs:1524-1526): blocking, n = batch*classes floats. */
int rt_mlp_logits(rt_mlp* mlp, float* host, size_t n);
/* GpuMlp::last_loss (mod.rs:1529-1531): blocking; mean of the per-row
 * losses summed in row order.  Returns RT_ERR_LABEL if a label was >= C
 * (see rt_mlp_step). */
int rt_mlp_last_loss(rt_mlp* mlp, float* out);
/* GpuMlp::weights / grads (mod.rs:1534-1551): blocking; host[i] receives
 * parameter i of [W1, b1, W2, b2, ...] (f32; the master copy for bf16;
 * gradients are reported unscaled when a loss scale is set). */
int rt_mlp_weights(rt_mlp* mlp, float* const* host, int n);
int rt_mlp_grads(rt_mlp* mlp, float* const* host, int n);
/* The plan's stored intermediates of the last step (or forward), blocking,
 * as n = batch x dims[layer+1] f32 values.  rt_mlp_activation: layer < n-1
 * gives the hidden activation A = ReLU(Z) the plan keeps for the next layer
 * and the ReLU mask (bf16 values widened exactly under RT_PREC_BF16), the
 * last layer the logits (= GpuMlp::logits, mod.rs:1524-1526).  rt_mlp_delta:
 * δ = ∂L/∂Z of that layer as the backward GEMMs read it (bf16 under
 * RT_PREC_BF16, and then multiplied by the loss scale).  No counterpart in
 * the reference beyond logits: they let a caller check each GEMM of the step
 * on its own inputs. */
int rt_mlp_activation(rt_mlp* mlp, int layer, float* host, size_t n);
int rt_mlp_delta(rt_mlp* mlp, int layer, float* host, size_t n);
/* GpuMlp::dispatches_por_passo (mod.rs:1559-1561): kernel launches per step. */
int rt_mlp_dispatches(rt_mlp* mlp, int* out);
/* Whether the last completed step was skipped for a non-finite gradient
 * under loss scaling (blocking). */
int rt_mlp_overflow(rt_mlp* mlp, int* out);

/* ------------------------------------------------- checkpoint and resume */

/* Param::set (tape.rs:119-121) for every parameter of the plan: n = 2 x layers
 * host arrays in parameter order [W1, b1, ...] (W [in, out], b [1, out]).
 * Refreshes the bf16 weight copy under mixed precision.  Blocking. */
int rt_mlp_set_weights(rt_mlp* mlp, const float* const* host, int n);

/* Optimizer state, which rtensor's GpuMlp keeps private (mod.rs:1291-1314,
 * 1334): the first and second moments (Adam m, v; SGD keeps its velocity in
 * m) per parameter, in the order of rt_mlp_weights, and t, the number of
 * updates applied so far (under loss scaling, skipped steps do not count).
 * A null m or v array list skips that part.  get blocks; set takes effect for
 * the next step. */
int rt_mlp_get_optimizer_state(rt_mlp* mlp, float* const* m, float* const* v, int n, int* t);
int rt_mlp_set_optimizer_state(rt_mlp* mlp, const float* const* m, const float* const* v, int n, int t);

/* ------------------------------------------------------------- tensor ops
 * Device versions of the Tensor operations rtensor's autodiff tape records
 * (tensor.rs, ops.rs, losses.rs), so a Tape/Sequential model of any shape
 * trains on the device; matmul and its VJPs are rt_gemm (RT_NN, RT_NT, RT_TN
 * = tensor.rs:318 and ops.rs:125-129).  All f32, rank <= 4, enqueue only.
 * Elementwise results round exactly like the reference except where a
 * transcendental (exp, ln, tanh, sqrt is exact) differs in its last bits;
 * rt_reduce_to is exact; rt_sum_all and rt_loss add in a fixed tree order
 * instead of the reference's left-to-right loop. */

typedef enum {
  RT_U_SCALE = 0,      /* v * k                 ops.rs:132-135 */
  RT_U_OFFSET = 1,     /* v + k                 ops.rs:139-142 */
  RT_U_NEG = 2,        /* v * -1                ops.rs:145-147 */
  RT_U_SQUARE = 3,     /* v * v                 ops.rs:150-154 */
  RT_U_SQRT = 4,       /* sqrt(v)               ops.rs:158-162 */
  RT_U_EXP = 5,        /* exp(v)                ops.rs:166-170 */
  RT_U_LN = 6,         /* ln(max(v, 1e-12))     ops.rs:176-180 */
  RT_U_RELU = 7,       /* max(v, 0)             ops.rs:190-194 */
  RT_U_LEAKY_RELU = 8, /* v > 0 ? v : k v       ops.rs:197-203 */
  RT_U_SIGMOID = 9,    /* 1 / (1 + exp(-v))     ops.rs:212-216 */
  RT_U_TANH = 10       /* tanh(v)               ops.rs:223-227 */
} rt_unary_op;

typedef enum { RT_B_ADD = 0, RT_B_SUB = 1, RT_B_MUL = 2, RT_B_DIV = 3 } rt_binary_op;

typedef enum {
  RT_LOSS_MAE = 1,                 /* losses.rs:46-53, on d = pred - target        */
  RT_LOSS_SOFTMAX_XENT = 2,        /* losses.rs:99-115, on p = softmax_rows(z)     */
  RT_LOSS_BCE = 3,                 /* losses.rs:143-162, on probabilities          */
  RT_LOSS_SOFTMAX_XENT_LOGITS = 4, /* losses.rs:99-115 on the logits z: softmax,
                                      loss and dir in one pass per row            */
  RT_LOSS_SOFTMAX_XENT_LOGITS_MEAN = 5 /* the same with dir = (P − Y)·(1/batch):
                                      the VJP for ḡ = 1, as rt_fill_scaled(1,
                                      batch, P − Y) gives it, bit for bit         */
} rt_loss_kind;                    /* mse (losses.rs:31-34) is sub, square, mean    */

/* Tensor::map (tensor.rs:160-181) with the forward closure of op:
 * y = f(x), same element count. */
int rt_map(rt_ctx* ctx, rt_unary_op op, float k, const rt_buf* x, rt_buf* y);
/* The VJP closure of op (ops.rs:132-227): dx from the upstream g, the op's
 * input x and its output y.  x is needed by SQUARE, LN, RELU, LEAKY_RELU;
 * y by SQRT, EXP, SIGMOID, TANH; either may be NULL when unused. */
int rt_map_vjp(rt_ctx* ctx, rt_unary_op op, float k, const rt_buf* g, const rt_buf* x, const rt_buf* y,
               rt_buf* dx);
/* Tensor::zip (tensor.rs:183-246) with numpy broadcasting
 * (broadcast_shapes, tensor.rs:575-592): out must have the broadcast shape.
 * out may alias a or b only when it has that operand's shape. */
int rt_zip(rt_ctx* ctx, rt_binary_op op, const rt_buf* a, const rt_buf* b, rt_buf* out);
/* Tensor::reduce_to (tensor.rs:399-438): out's shape is the target, right-
 * aligned against g's, each axis equal to g's or 1.  Every output element
 * sums its sources in increasing index order, as the reference does (exact),
 * except a one-element target, which is rt_sum_all. */
int rt_reduce_to(rt_ctx* ctx, const rt_buf* g, rt_buf* out);
/* sum_all / mean_all (tensor.rs:279-286): out[0] = (sum of x) / div, out has
 * one element.  div = 1 for sum, len(x) for mean. */
int rt_sum_all(rt_ctx* ctx, const rt_buf* x, float div, rt_buf* out);
/* The scalar-scaled VJPs (ops.rs:239-255, losses.rs:53, 114, 160):
 * out[i] = x[i] * (s[0] / div), or s[0] / div everywhere (Tensor::full) when
 * x is NULL.  s has one element; x, if given, has out's element count. */
int rt_fill_scaled(rt_ctx* ctx, const rt_buf* s, float div, const rt_buf* x, rt_buf* out);
/* Tensor::softmax_rows (tensor.rs:455-472) of z [R, C] into y [R, C]. */
int rt_softmax_rows(rt_ctx* ctx, const rt_buf* z, rt_buf* y);
/* softmax's VJP (ops.rs:291-309): dx = s ⊙ (g − rowsum(g ⊙ s)), s the
 * forward output. */
int rt_softmax_rows_vjp(rt_ctx* ctx, const rt_buf* s, const rt_buf* g, rt_buf* dx);
/* Loss value and unscaled gradient direction (losses.rs): value[0] = total /
 * batch (batch = rows of p for softmax-xent, len(p) otherwise); dir (NULL to
 * skip) = sign(d), p − y, or (c − y)/(c(1 − c)) with c = clamp(p, 1e-7,
 * 1 − 1e-7).  The loss node's VJP is rt_fill_scaled(g, batch, dir).  y is
 * NULL for RT_LOSS_MAE (p is already pred − target).  RT_LOSS_SOFTMAX_XENT_LOGITS
 * takes the logits as p and needs dir; its row sums are added before the
 * tree, so its value may differ from RT_LOSS_SOFTMAX_XENT's in the last bits. */
int rt_loss(rt_ctx* ctx, rt_loss_kind kind, const rt_buf* p, const rt_buf* y, rt_buf* value, rt_buf* dir);

/* Gpu::zeros without the zero fill (contents undefined), for op outputs
 * that are written whole.  No counterpart in rtensor (wgpu buffers start
 * zeroed). */
int rt_empty(rt_ctx* ctx, rt_dtype dtype, const size_t* shape, int rank, rt_buf** out);

/* GpuMlp::carregar (mod.rs:1486-1495), overlapped: rt_mlp_load copies a host
 * batch (x in the plan's input dtype: f32, or bf16 bits under RT_PREC_BF16;
 * n = batch labels) into pinned staging and starts its host-to-device copy
 * on a copy stream, into one of two device slots that alternate.  The call
 * first waits (on the host) for the last step that read the same slot, two
 * steps back, so the copy runs while the step on the other slot computes.
 * The host buffers may be reused on return.  A label >= the number of
 * classes is rejected here (RT_ERR_LABEL, nothing is loaded).
 * rt_mlp_step_loaded runs rt_mlp_step on the most recently loaded batch after
 * its copy; it may be called again on the same batch. */
int rt_mlp_load(rt_mlp* mlp, const void* x, size_t x_bytes, const uint64_t* labels, size_t n);
int rt_mlp_step_loaded(rt_mlp* mlp);

/* ------------------------------------------------------------- inference */

/* Tensor::argmax_rows (tensor.rs:476-493) on the device: out[r] is the first
 * index of the maximum of row r of logits f32 [B, C].  As in the reference, a
 * NaN in column 0 wins its row and later NaNs never do.  out: u32 [B]. */
int rt_argmax_rows(rt_ctx* ctx, const rt_buf* logits, rt_buf* out);

/* losses::accuracy (losses.rs:181-185): the fraction of rows whose argmax
 * equals the label, hits / B in f32 (NaN for B = 0, as 0/0; 0 for zero
 * columns, which give no predictions).  labels: u32 [B].
 * Blocking. */
int rt_accuracy(rt_ctx* ctx, const rt_buf* logits, const rt_buf* labels, float* out);

/* ------------------------------------------------------------- profiling */

/* Gpu::perfilar (mod.rs:1245-1286): while enabled, every launch on ctx is
 * bracketed by HIP events on the ctx stream.  rt_profile_report blocks and
 * fills, per distinct kernel label, its name (up to name_len bytes), launch
 * count and summed device milliseconds; returns the number of labels in
 * *n_out (at most cap). */
int rt_profile_enable(rt_ctx* ctx, int on);
int rt_profile_reset(rt_ctx* ctx);
int rt_profile_report(rt_ctx* ctx, char* names, size_t name_len, int* counts, double* ms, int cap,
                      int* n_out);

/* Region timer, a measurement helper with no counterpart in rtensor: HIP
 * events recorded on the ctx stream around everything enqueued between the
 * two calls (no per-launch events inside the region).  rt_timer_end blocks
 * and returns the elapsed device milliseconds; RT_ERR_INVALID without a
 * preceding rt_timer_begin. */
int rt_timer_begin(rt_ctx* ctx);
int rt_timer_end(rt_ctx* ctx, float* ms);

#ifdef __cplusplus
}
#endif
#endif /* RTENSOR_HIP_H */
