//! Raw bindings of include/rtensor_hip.h, one line per entry point, in the
//! header's order.  C enums are passed as `c_int`; handles are opaque.
//! tests/test_rust_binding.py checks this file against the header: the same
//! symbols, parameter types, return types, enum values and config fields.
#![allow(non_camel_case_types, dead_code)]

use std::os::raw::{c_char, c_int, c_void};

#[repr(C)]
pub struct RtCtx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct RtBuf {
    _p: [u8; 0],
}
#[repr(C)]
pub struct RtMlp {
    _p: [u8; 0],
}

// rt_status
pub const RT_OK: c_int = 0;
pub const RT_ERR_NO_DEVICE: c_int = 1;
pub const RT_ERR_INVALID: c_int = 2;
pub const RT_ERR_SHAPE: c_int = 3;
pub const RT_ERR_DTYPE: c_int = 4;
pub const RT_ERR_OOM: c_int = 5;
pub const RT_ERR_LABEL: c_int = 6;
pub const RT_ERR_HIP: c_int = 7;
pub const RT_ERR_OVERFLOW: c_int = 8;

// rt_dtype
pub const RT_F32: c_int = 0;
pub const RT_BF16: c_int = 1;
pub const RT_F16: c_int = 2;
pub const RT_U32: c_int = 3;

// rt_layout
pub const RT_NN: c_int = 0;
pub const RT_TN: c_int = 1;
pub const RT_NT: c_int = 2;

// rt_epilogue
pub const RT_EPI_NONE: c_int = 0;
pub const RT_EPI_BIAS: c_int = 1;
pub const RT_EPI_BIAS_RELU: c_int = 2;
pub const RT_EPI_RELU_MASK: c_int = 3;

// rt_optimizer, rt_precision
pub const RT_OPT_ADAM: c_int = 0;
pub const RT_OPT_SGD: c_int = 1;
pub const RT_PREC_F32: c_int = 0;
pub const RT_PREC_BF16: c_int = 1;

// rt_unary_op (ops.rs)
pub const RT_U_SCALE: c_int = 0;
pub const RT_U_OFFSET: c_int = 1;
pub const RT_U_NEG: c_int = 2;
pub const RT_U_SQUARE: c_int = 3;
pub const RT_U_SQRT: c_int = 4;
pub const RT_U_EXP: c_int = 5;
pub const RT_U_LN: c_int = 6;
pub const RT_U_RELU: c_int = 7;
pub const RT_U_LEAKY_RELU: c_int = 8;
pub const RT_U_SIGMOID: c_int = 9;
pub const RT_U_TANH: c_int = 10;

// rt_binary_op
pub const RT_B_ADD: c_int = 0;
pub const RT_B_SUB: c_int = 1;
pub const RT_B_MUL: c_int = 2;
pub const RT_B_DIV: c_int = 3;

// rt_loss_kind (losses.rs)
pub const RT_LOSS_MAE: c_int = 1;
pub const RT_LOSS_SOFTMAX_XENT: c_int = 2;
pub const RT_LOSS_BCE: c_int = 3;
pub const RT_LOSS_SOFTMAX_XENT_LOGITS: c_int = 4;
pub const RT_LOSS_SOFTMAX_XENT_LOGITS_MEAN: c_int = 5;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct RtMlpConfig {
    pub optimizer: c_int,
    pub lr: f32,
    pub beta1: f32,
    pub beta2: f32,
    pub eps: f32,
    pub momentum: f32,
    pub precision: c_int,
    pub loss_scale: f32,
}

extern "C" {
    // Device (Gpu::new, info, sync).
    pub fn rt_open(device: c_int, out: *mut *mut RtCtx) -> c_int;
    pub fn rt_close(ctx: *mut RtCtx) -> c_int;
    pub fn rt_last_error(ctx: *const RtCtx) -> *const c_char;
    pub fn rt_info(ctx: *mut RtCtx, buf: *mut c_char, len: usize) -> c_int;
    pub fn rt_sync(ctx: *mut RtCtx) -> c_int;

    // Buffers (zeros, upload, download, upload_labels).
    pub fn rt_zeros(ctx: *mut RtCtx, dtype: c_int, shape: *const usize, rank: c_int, out: *mut *mut RtBuf) -> c_int;
    pub fn rt_upload(ctx: *mut RtCtx, dtype: c_int, shape: *const usize, rank: c_int, host: *const c_void,
                     out: *mut *mut RtBuf) -> c_int;
    pub fn rt_download(ctx: *mut RtCtx, buf: *const RtBuf, host: *mut c_void, bytes: usize) -> c_int;
    pub fn rt_write(ctx: *mut RtCtx, buf: *mut RtBuf, host: *const c_void, bytes: usize) -> c_int;
    pub fn rt_free(ctx: *mut RtCtx, buf: *mut RtBuf) -> c_int;
    pub fn rt_buf_info(buf: *const RtBuf, dtype: *mut c_int, shape: *mut usize, rank: *mut c_int) -> c_int;
    pub fn rt_upload_labels(ctx: *mut RtCtx, labels: *const u64, n: usize, out: *mut *mut RtBuf) -> c_int;
    pub fn rt_convert(ctx: *mut RtCtx, src: *const RtBuf, dst: *mut RtBuf) -> c_int;

    // Kernels (op_matmul*, ops_split_k, ops_colsum, op_softmax_xent, op_adam).
    pub fn rt_gemm(ctx: *mut RtCtx, layout: c_int, a: *const RtBuf, b: *const RtBuf, c: *mut RtBuf, epi: c_int,
                   aux: *const RtBuf, colsum: *mut RtBuf) -> c_int;
    pub fn rt_linear_backward(ctx: *mut RtCtx, x: *const RtBuf, delta: *const RtBuf, w: *const RtBuf,
                              dx: *mut RtBuf, dw: *mut RtBuf, db: *mut RtBuf) -> c_int;
    pub fn rt_gemm_splitk(ctx: *mut RtCtx, layout: c_int, a: *const RtBuf, b: *const RtBuf, c: *mut RtBuf,
                          partials: *mut RtBuf, slices: usize, colsum: *mut RtBuf) -> c_int;
    pub fn rt_gemm_splitk_static(ctx: *mut RtCtx, layout: c_int, a: *const RtBuf, b: *const RtBuf, c: *mut RtBuf,
                                 slices: usize, colsum: *mut RtBuf) -> c_int;
    pub fn rt_splitk_slices(m: usize, n: usize, k: usize) -> usize;
    pub fn rt_colsum(ctx: *mut RtCtx, src: *const RtBuf, dst: *mut RtBuf) -> c_int;
    pub fn rt_bias_add(ctx: *mut RtCtx, z: *mut RtBuf, b: *const RtBuf) -> c_int;
    pub fn rt_relu(ctx: *mut RtCtx, x: *const RtBuf, y: *mut RtBuf) -> c_int;
    pub fn rt_relu_bwd(ctx: *mut RtCtx, a: *const RtBuf, delta: *mut RtBuf) -> c_int;
    pub fn rt_softmax_xent(ctx: *mut RtCtx, logits: *const RtBuf, labels: *const RtBuf, delta: *mut RtBuf,
                           loss_rows: *mut RtBuf, scale: f32) -> c_int;
    pub fn rt_adam(ctx: *mut RtCtx, theta: *mut RtBuf, m: *mut RtBuf, v: *mut RtBuf, g: *const RtBuf, lr: f32,
                   beta1: f32, beta2: f32, eps: f32, t: c_int) -> c_int;
    pub fn rt_sgd(ctx: *mut RtCtx, theta: *mut RtBuf, velocity: *mut RtBuf, g: *const RtBuf, lr: f32,
                  momentum: f32) -> c_int;
    pub fn rt_adam_many(ctx: *mut RtCtx, n: c_int, theta: *const *mut RtBuf, m: *const *mut RtBuf,
                        v: *const *mut RtBuf, g: *const *const RtBuf, lr: f32, beta1: f32, beta2: f32, eps: f32,
                        t: c_int) -> c_int;
    pub fn rt_sgd_many(ctx: *mut RtCtx, n: c_int, theta: *const *mut RtBuf, velocity: *const *mut RtBuf,
                       g: *const *const RtBuf, lr: f32, momentum: f32) -> c_int;

    // The fixed MLP plan (GpuMlp).
    pub fn rt_mlp_create(ctx: *mut RtCtx, n_layers: c_int, dims: *const usize, weights: *const *const f32,
                         biases: *const *const f32, batch: usize, cfg: *const RtMlpConfig,
                         out: *mut *mut RtMlp) -> c_int;
    pub fn rt_mlp_destroy(mlp: *mut RtMlp) -> c_int;
    pub fn rt_mlp_step(mlp: *mut RtMlp, x: *const RtBuf, labels: *const RtBuf) -> c_int;
    pub fn rt_mlp_forward(mlp: *mut RtMlp, x: *const RtBuf) -> c_int;
    pub fn rt_mlp_logits(mlp: *mut RtMlp, host: *mut f32, n: usize) -> c_int;
    pub fn rt_mlp_last_loss(mlp: *mut RtMlp, out: *mut f32) -> c_int;
    pub fn rt_mlp_weights(mlp: *mut RtMlp, host: *const *mut f32, n: c_int) -> c_int;
    pub fn rt_mlp_grads(mlp: *mut RtMlp, host: *const *mut f32, n: c_int) -> c_int;
    pub fn rt_mlp_activation(mlp: *mut RtMlp, layer: c_int, host: *mut f32, n: usize) -> c_int;
    pub fn rt_mlp_delta(mlp: *mut RtMlp, layer: c_int, host: *mut f32, n: usize) -> c_int;
    pub fn rt_mlp_dispatches(mlp: *mut RtMlp, out: *mut c_int) -> c_int;
    pub fn rt_mlp_overflow(mlp: *mut RtMlp, out: *mut c_int) -> c_int;

    // Checkpoint / resume (Param::set for every parameter; Adam m, v, t).
    pub fn rt_mlp_set_weights(mlp: *mut RtMlp, host: *const *const f32, n: c_int) -> c_int;
    pub fn rt_mlp_get_optimizer_state(mlp: *mut RtMlp, m: *const *mut f32, v: *const *mut f32, n: c_int,
                                      t: *mut c_int) -> c_int;
    pub fn rt_mlp_set_optimizer_state(mlp: *mut RtMlp, m: *const *const f32, v: *const *const f32, n: c_int,
                                      t: c_int) -> c_int;

    // Op-level backend for the autodiff tape (tensor.rs, ops.rs, losses.rs).
    pub fn rt_map(ctx: *mut RtCtx, op: c_int, k: f32, x: *const RtBuf, y: *mut RtBuf) -> c_int;
    pub fn rt_map_vjp(ctx: *mut RtCtx, op: c_int, k: f32, g: *const RtBuf, x: *const RtBuf, y: *const RtBuf,
                      dx: *mut RtBuf) -> c_int;
    pub fn rt_zip(ctx: *mut RtCtx, op: c_int, a: *const RtBuf, b: *const RtBuf, out: *mut RtBuf) -> c_int;
    pub fn rt_reduce_to(ctx: *mut RtCtx, g: *const RtBuf, out: *mut RtBuf) -> c_int;
    pub fn rt_sum_all(ctx: *mut RtCtx, x: *const RtBuf, div: f32, out: *mut RtBuf) -> c_int;
    pub fn rt_fill_scaled(ctx: *mut RtCtx, s: *const RtBuf, div: f32, x: *const RtBuf, out: *mut RtBuf) -> c_int;
    pub fn rt_softmax_rows(ctx: *mut RtCtx, z: *const RtBuf, y: *mut RtBuf) -> c_int;
    pub fn rt_softmax_rows_vjp(ctx: *mut RtCtx, s: *const RtBuf, g: *const RtBuf, dx: *mut RtBuf) -> c_int;
    pub fn rt_loss(ctx: *mut RtCtx, kind: c_int, p: *const RtBuf, y: *const RtBuf, value: *mut RtBuf,
                   dir: *mut RtBuf) -> c_int;
    pub fn rt_empty(ctx: *mut RtCtx, dtype: c_int, shape: *const usize, rank: c_int, out: *mut *mut RtBuf) -> c_int;

    // Data path (carregar) and inference (argmax_rows, accuracy).
    pub fn rt_mlp_load(mlp: *mut RtMlp, x: *const c_void, x_bytes: usize, labels: *const u64, n: usize) -> c_int;
    pub fn rt_mlp_step_loaded(mlp: *mut RtMlp) -> c_int;
    pub fn rt_argmax_rows(ctx: *mut RtCtx, logits: *const RtBuf, out: *mut RtBuf) -> c_int;
    pub fn rt_accuracy(ctx: *mut RtCtx, logits: *const RtBuf, labels: *const RtBuf, out: *mut f32) -> c_int;

    // Profiling (Gpu::perfilar) and a region timer (no rtensor counterpart).
    pub fn rt_profile_enable(ctx: *mut RtCtx, on: c_int) -> c_int;
    pub fn rt_profile_reset(ctx: *mut RtCtx) -> c_int;
    pub fn rt_profile_report(ctx: *mut RtCtx, names: *mut c_char, name_len: usize, counts: *mut c_int,
                             ms: *mut f64, cap: c_int, n_out: *mut c_int) -> c_int;
    pub fn rt_timer_begin(ctx: *mut RtCtx) -> c_int;
    pub fn rt_timer_end(ctx: *mut RtCtx, ms: *mut f32) -> c_int;
}
