//! rtensor's training backend for AMD MI355X, with the method shapes of
//! `rtensor::gpu` (crates/rtensor/src/gpu/mod.rs:224-1562), so that code
//! written against the wgpu backend switches by changing its `use` line.
//!
//! Every entry point is a call into librtensor_hip.so (hand-written HIP for
//! gfx950).  As in `rtensor::gpu`:
//! * errors other than opening the device panic (mod.rs:1342-1343, 1487-1491);
//! * work is enqueued on one stream and the sync points are `download`,
//!   `logits`, `last_loss`, `weights`, `grads` and `sync`;
//! * the types are not `Send`/`Sync` (the context is shared through `Rc`).
//!
//! Handles keep the context alive, so a tensor or plan dropped after its
//! `Gpu` still frees cleanly.

mod ffi;

pub use ffi::RtMlpConfig;

use rtensor::prelude::*;
use std::ffi::CStr;
use std::os::raw::c_int;
use std::rc::Rc;

struct Ctx(*mut ffi::RtCtx);

impl Drop for Ctx {
    fn drop(&mut self) {
        unsafe {
            ffi::rt_close(self.0);
        }
    }
}

fn last_error(ctx: *const ffi::RtCtx) -> String {
    unsafe { CStr::from_ptr(ffi::rt_last_error(ctx)).to_string_lossy().into_owned() }
}

fn check(ctx: *const ffi::RtCtx, rc: c_int) {
    if rc != ffi::RT_OK {
        panic!("rtensor-hip: {} (status {rc})", last_error(ctx));
    }
}

/// `rtensor::gpu::Gpu` (mod.rs:224-255).
pub struct Gpu {
    ctx: Rc<Ctx>,
    info: String,
}

/// `rtensor::gpu::GpuTensor` (mod.rs:190-208): owns its device buffer.
pub struct GpuTensor {
    ctx: Rc<Ctx>,
    buf: *mut ffi::RtBuf,
    shape: Vec<usize>,
}

/// The label buffer `upload_labels` returns (u32 on the device, mod.rs:1672-1675).
pub struct GpuLabels {
    ctx: Rc<Ctx>,
    buf: *mut ffi::RtBuf,
    len: usize,
}

/// `rtensor::gpu::GpuMlp` (mod.rs:1291-1562): the fixed training plan.
pub struct GpuMlp {
    ctx: Rc<Ctx>,
    mlp: *mut ffi::RtMlp,
    shapes: Vec<Vec<usize>>,
    classes: usize,
    batch: usize,
}

impl Gpu {
    /// `Gpu::new` (mod.rs:263): `Err` when there is no gfx950 device.
    pub fn new() -> Result<Gpu, String> {
        Gpu::with_device(0)
    }

    pub fn with_device(device: i32) -> Result<Gpu, String> {
        let mut ctx = std::ptr::null_mut();
        let rc = unsafe { ffi::rt_open(device, &mut ctx) };
        if rc != ffi::RT_OK {
            return Err(last_error(std::ptr::null()));
        }
        let mut text = vec![0u8; 256];
        unsafe { ffi::rt_info(ctx, text.as_mut_ptr().cast(), text.len()) };
        let end = text.iter().position(|&c| c == 0).unwrap_or(text.len());
        Ok(Gpu { ctx: Rc::new(Ctx(ctx)), info: String::from_utf8_lossy(&text[..end]).into_owned() })
    }

    fn raw(&self) -> *mut ffi::RtCtx {
        self.ctx.0
    }

    fn check(&self, rc: c_int) {
        check(self.raw(), rc)
    }

    /// `Gpu::info` (mod.rs:412).
    pub fn info(&self) -> &str {
        &self.info
    }

    /// `Gpu::zeros` (mod.rs:501).
    pub fn zeros(&self, shape: &[usize]) -> GpuTensor {
        let mut buf = std::ptr::null_mut();
        self.check(unsafe { ffi::rt_zeros(self.raw(), ffi::RT_F32, shape.as_ptr(), shape.len() as c_int, &mut buf) });
        GpuTensor { ctx: self.ctx.clone(), buf, shape: shape.to_vec() }
    }

    /// `Gpu::upload` (mod.rs:509).
    pub fn upload(&self, t: &Tensor) -> GpuTensor {
        let mut buf = std::ptr::null_mut();
        self.check(unsafe {
            ffi::rt_upload(self.raw(), ffi::RT_F32, t.shape().as_ptr(), t.shape().len() as c_int,
                           t.data().as_ptr().cast(), &mut buf)
        });
        GpuTensor { ctx: self.ctx.clone(), buf, shape: t.shape().to_vec() }
    }

    /// `Gpu::download` (mod.rs:530): blocks until the stream has drained.
    pub fn download(&self, g: &GpuTensor) -> Tensor {
        let n: usize = g.shape.iter().product();
        let mut data = vec![0f32; n];
        self.check(unsafe { ffi::rt_download(self.raw(), g.buf, data.as_mut_ptr().cast(), n * 4) });
        Tensor::new(&g.shape, data)
    }

    /// `Gpu::sync` (mod.rs:564).
    pub fn sync(&self) {
        self.check(unsafe { ffi::rt_sync(self.raw()) })
    }

    /// `op_matmul` / `op_matmul_at_b` / `op_matmul_a_bt` / `op_matmul_bias`
    /// (mod.rs:685-749), enqueued at once: C = op(A)·op(B) with an epilogue.
    pub fn matmul(&self, layout: i32, a: &GpuTensor, b: &GpuTensor, c: &mut GpuTensor, epilogue: i32,
                  aux: Option<&GpuTensor>) {
        let aux = aux.map_or(std::ptr::null(), |t| t.buf as *const _);
        self.check(unsafe {
            ffi::rt_gemm(self.raw(), layout, a.buf, b.buf, c.buf, epilogue, aux, std::ptr::null_mut())
        })
    }

    /// `ops_colsum` (mod.rs:838-855).
    pub fn colsum(&self, src: &GpuTensor, dst: &mut GpuTensor) {
        self.check(unsafe { ffi::rt_colsum(self.raw(), src.buf, dst.buf) })
    }
}

impl GpuTensor {
    pub fn shape(&self) -> &[usize] {
        &self.shape
    }
}

impl Drop for GpuTensor {
    fn drop(&mut self) {
        unsafe {
            ffi::rt_free(self.ctx.0, self.buf);
        }
    }
}

impl GpuLabels {
    pub fn len(&self) -> usize {
        self.len
    }
    pub fn is_empty(&self) -> bool {
        self.len == 0
    }
}

impl Drop for GpuLabels {
    fn drop(&mut self) {
        unsafe {
            ffi::rt_free(self.ctx.0, self.buf);
        }
    }
}

/// `upload_labels` (mod.rs:1672): usize labels become u32 on the device; a
/// label that does not fit u32 is an error, not a silent truncation.
pub fn upload_labels(gpu: &Gpu, labels: &[usize]) -> GpuLabels {
    let v: Vec<u64> = labels.iter().map(|&l| l as u64).collect();
    let mut buf = std::ptr::null_mut();
    gpu.check(unsafe { ffi::rt_upload_labels(gpu.raw(), v.as_ptr(), v.len(), &mut buf) });
    GpuLabels { ctx: gpu.ctx.clone(), buf, len: labels.len() }
}

impl GpuMlp {
    /// `GpuMlp::from_params` (mod.rs:1341): params `[W1, b1, W2, b2, ...]`,
    /// weights `[in, out]`, biases `[1, out]`; hidden layers ReLU, output
    /// linear; Adam(lr, 0.9, 0.999, 1e-8) as in the reference.
    pub fn from_params(gpu: &Gpu, params: &[Param], lote: usize, lr: f32) -> GpuMlp {
        let cfg = RtMlpConfig { optimizer: ffi::RT_OPT_ADAM, lr, beta1: 0.9, beta2: 0.999, eps: 1e-8,
                                momentum: 0.0, precision: ffi::RT_PREC_F32, loss_scale: 1.0 };
        GpuMlp::with_config(gpu, params, lote, &cfg)
    }

    /// The same plan with another optimizer (SGD) or bf16 storage with f32
    /// master weights (`precision: RT_PREC_BF16`, `loss_scale`).
    pub fn with_config(gpu: &Gpu, params: &[Param], lote: usize, cfg: &RtMlpConfig) -> GpuMlp {
        assert!(params.len() >= 2 && params.len() % 2 == 0, "GpuMlp expects (W, b) pairs");
        let values: Vec<Tensor> = params.iter().map(|p| p.value().clone()).collect();
        let mut dims = vec![values[0].shape()[0]];
        for w in values.iter().step_by(2) {
            assert_eq!(w.shape().len(), 2, "weights are [in, out]");
            dims.push(w.shape()[1]);
        }
        let wp: Vec<*const f32> = values.iter().step_by(2).map(|w| w.data().as_ptr()).collect();
        let bp: Vec<*const f32> = values.iter().skip(1).step_by(2).map(|b| b.data().as_ptr()).collect();
        let mut mlp = std::ptr::null_mut();
        gpu.check(unsafe {
            ffi::rt_mlp_create(gpu.raw(), wp.len() as c_int, dims.as_ptr(), wp.as_ptr(), bp.as_ptr(), lote, cfg,
                               &mut mlp)
        });
        GpuMlp {
            ctx: gpu.ctx.clone(),
            mlp,
            shapes: values.iter().map(|t| t.shape().to_vec()).collect(),
            classes: *dims.last().unwrap(),
            batch: lote,
        }
    }

    fn check(&self, rc: c_int) {
        check(self.ctx.0, rc)
    }

    /// `step` (mod.rs:1499): forward, backward and update, enqueued.
    pub fn step(&mut self, _gpu: &Gpu, x: &GpuTensor, labels: &GpuLabels) {
        self.check(unsafe { ffi::rt_mlp_step(self.mlp, x.buf, labels.buf) })
    }

    /// `carregar` (mod.rs:1486-1495) followed by a step: the batch is copied
    /// from host memory while the previous step runs.
    pub fn step_host(&mut self, x: &[f32], labels: &[usize]) {
        let lab: Vec<u64> = labels.iter().map(|&l| l as u64).collect();
        self.check(unsafe {
            ffi::rt_mlp_load(self.mlp, x.as_ptr().cast(), x.len() * 4, lab.as_ptr(), lab.len())
        });
        self.check(unsafe { ffi::rt_mlp_step_loaded(self.mlp) })
    }

    /// `forward_only` (mod.rs:1514).
    pub fn forward_only(&self, _gpu: &Gpu, x: &GpuTensor) {
        self.check(unsafe { ffi::rt_mlp_forward(self.mlp, x.buf) })
    }

    /// `logits` (mod.rs:1524): [batch, classes], syncs.
    pub fn logits(&self, _gpu: &Gpu) -> Tensor {
        let mut data = vec![0f32; self.batch * self.classes];
        self.check(unsafe { ffi::rt_mlp_logits(self.mlp, data.as_mut_ptr(), data.len()) });
        Tensor::new(&[self.batch, self.classes], data)
    }

    /// `last_loss` (mod.rs:1529): mean loss of the last step, syncs.
    pub fn last_loss(&self, _gpu: &Gpu) -> f32 {
        let mut l = 0f32;
        self.check(unsafe { ffi::rt_mlp_last_loss(self.mlp, &mut l) });
        l
    }

    fn get_all(&self, f: unsafe extern "C" fn(*mut ffi::RtMlp, *const *mut f32, c_int) -> c_int) -> Vec<Tensor> {
        let mut out: Vec<Vec<f32>> = self.shapes.iter().map(|s| vec![0f32; s.iter().product()]).collect();
        let ptrs: Vec<*mut f32> = out.iter_mut().map(|v| v.as_mut_ptr()).collect();
        self.check(unsafe { f(self.mlp, ptrs.as_ptr(), ptrs.len() as c_int) });
        out.into_iter().zip(&self.shapes).map(|(d, s)| Tensor::new(s, d)).collect()
    }

    /// `weights` (mod.rs:1534): `[W1, b1, ...]`, syncs.
    pub fn weights(&self, _gpu: &Gpu) -> Vec<Tensor> {
        self.get_all(ffi::rt_mlp_weights)
    }

    /// `grads` (mod.rs:1544): `[dW1, db1, ...]` of the last step, syncs.
    pub fn grads(&self, _gpu: &Gpu) -> Vec<Tensor> {
        self.get_all(ffi::rt_mlp_grads)
    }

    /// `Param::set` for every parameter (tape.rs:119-121), for resume.
    pub fn set_weights(&mut self, values: &[Tensor]) {
        assert_eq!(values.len(), self.shapes.len(), "one tensor per parameter");
        let ptrs: Vec<*const f32> = values.iter().map(|t| t.data().as_ptr()).collect();
        self.check(unsafe { ffi::rt_mlp_set_weights(self.mlp, ptrs.as_ptr(), ptrs.len() as c_int) })
    }

    /// Adam's first and second moments and step count, which the
    /// reference's plan keeps on the device only (mod.rs:1291-1314).
    pub fn optimizer_state(&self) -> (Vec<Tensor>, Vec<Tensor>, i32) {
        let mut m: Vec<Vec<f32>> = self.shapes.iter().map(|s| vec![0f32; s.iter().product()]).collect();
        let mut v = m.clone();
        let mp: Vec<*mut f32> = m.iter_mut().map(|x| x.as_mut_ptr()).collect();
        let vp: Vec<*mut f32> = v.iter_mut().map(|x| x.as_mut_ptr()).collect();
        let mut t: c_int = 0;
        self.check(unsafe {
            ffi::rt_mlp_get_optimizer_state(self.mlp, mp.as_ptr(), vp.as_ptr(), mp.len() as c_int, &mut t)
        });
        let wrap = |xs: Vec<Vec<f32>>| xs.into_iter().zip(&self.shapes).map(|(d, s)| Tensor::new(s, d)).collect();
        (wrap(m), wrap(v), t)
    }

    pub fn set_optimizer_state(&mut self, m: &[Tensor], v: &[Tensor], t: i32) {
        assert!(m.len() == self.shapes.len() && v.len() == self.shapes.len(), "one tensor per parameter");
        let mp: Vec<*const f32> = m.iter().map(|x| x.data().as_ptr()).collect();
        let vp: Vec<*const f32> = v.iter().map(|x| x.data().as_ptr()).collect();
        self.check(unsafe {
            ffi::rt_mlp_set_optimizer_state(self.mlp, mp.as_ptr(), vp.as_ptr(), mp.len() as c_int, t)
        })
    }

    /// `batch_size` (mod.rs:1553).
    pub fn batch_size(&self) -> usize {
        self.batch
    }

    /// `dispatches_por_passo` (mod.rs:1559): kernel launches per step.
    pub fn dispatches_por_passo(&self) -> usize {
        let mut n: c_int = 0;
        self.check(unsafe { ffi::rt_mlp_dispatches(self.mlp, &mut n) });
        n as usize
    }
}

impl Drop for GpuMlp {
    fn drop(&mut self) {
        unsafe {
            ffi::rt_mlp_destroy(self.mlp);
        }
    }
}
