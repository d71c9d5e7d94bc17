// The MLP training plan: rtensor's GpuMlp (crates/rtensor/src/gpu/mod.rs:1291-1562)
// rebuilt around one HIP stream and one device arena.
//
// Memory layout (one hipMalloc, every region 256-byte aligned):
//   theta | grad | m | v     flat f32 vectors in parameter order
//                            [W1, b1, W2, b2, ...], each segment padded to a
//                            multiple of 64 floats, so the whole optimizer is
//                            one contiguous sweep (padding stays zero)
//   theta_bf16               bf16 copy of theta written by the optimizer
//                            (mixed precision only)
//   act[l], delta[l]         [batch, dims[l+1]] per layer: post-ReLU
//                            activation of hidden layers (the ReLU mask comes
//                            from it, as mod.rs:1453-1455 notes), logits for
//                            the last layer; δ = ∂L/∂Z
//   partials                 split-K planes (largest user), reused by every
//                            split GEMM of the step
//   cs_shares[l]             column-sum shares of layer l's half dW GEMM
//                            (mixed), kept until the split reduction or the
//                            non-finite check launch adds them
//   loss_rows [batch]
//
// Step (mod.rs:1399-1467 order): forward GEMMs with bias(+ReLU) epilogues;
// softmax-xent → δ_L; per layer, last to first: dW = A_{l-1}ᵀ·δ_l with the
// bias gradient summed from the same δ tiles, then (l > 0)
// δ_{l-1} = (δ_l·W_lᵀ) ⊙ 1[A_{l-1} > 0]; then one fused optimizer launch.
// Narrow layers (the 10-class head, its dW) use split-K with a fixed-order
// reduction, chosen by rt_splitk_slices.

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "rt_internal.h"

namespace rt {
hipError_t gemm_launch(hipStream_t s, const GemmDesc& d);
}
using namespace rt;

namespace {

struct Layer {
  size_t din = 0, dout = 0;
  size_t w_off = 0, b_off = 0;  // offsets (floats) into the flat parameter vectors
  void* act = nullptr;          // [batch, dout], f32 (or bf16 for mixed-precision hidden layers)
  float* delta = nullptr;       // [batch, dout] f32
  void* delta_h = nullptr;      // [batch, ldh] bf16 (mixed precision)
  // Row stride of delta_h: dout, except for an output layer whose width is
  // not a multiple of 64, padded so that its dX GEMM (K = its width) runs on
  // whole 64-k stages; the padding columns stay zero.
  size_t ldh = 0;
  int splits_dw = 1;
  int splits_fwd = 1;
  int splits_dx = 1;  // dX = δ·Wᵀ of this layer (l > 0)
  bool pair_bwd = false;  // dW and dX of this layer in one launch
  // dW / db split-K planes of this layer summed by the optimizer (f32 plans):
  // [splits_dw][din*dout] then [splits_dw][dout], owned by this layer.
  float* dw_parts = nullptr;
  // Mixed plans: the column-sum shares of this layer's dW launch (its own
  // region; the split reduction or the non-finite check launch adds them).
  float* cs_shares = nullptr;
  size_t cs_share_elems = 0;
  // Mixed plans, hidden layers: the ReLU predicate of act as one bit per
  // element (GemmDesc::relu_bits_out), written by the forward GEMM when its
  // launch can (bits_fresh) and read by the next layer's dX GEMM in place of
  // act's 16-bit values.
  unsigned* relu_bits = nullptr;
  bool bits_fresh = false;
  std::string lbl_fwd, lbl_fwd_red, lbl_dw, lbl_dw_red, lbl_dx, lbl_dx_red, lbl_bwd;
};

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// K slices for a bf16 GEMM whose 256x256 tiles alone leave CUs idle: up to
// 256 workgroups, at least 8 stages of 64 k per slice, and every slice whole
// stages (so the direct-to-LDS kernel takes it).
int half_slices(size_t m, size_t n, size_t k) {
  const size_t tiles = ((m + 255) / 256) * ((n + 255) / 256);
  if (tiles >= 256 || k % 64 != 0) return 1;
  int s = (int)std::min<size_t>(256 / tiles, k / 512);
  while (s > 1 && k % (64 * (size_t)s) != 0) --s;
  return std::max(s, 1);
}

}  // namespace

struct rt_mlp {
  rt_ctx* ctx = nullptr;
  size_t batch = 0;
  int n_layers = 0;
  rt_mlp_config cfg{};
  std::vector<Layer> L;
  size_t n_params = 0;  // padded flat length
  char* arena = nullptr;
  float* theta = nullptr;
  float* grad = nullptr;
  float* m = nullptr;
  float* v = nullptr;
  void* theta_h = nullptr;  // bf16 copy
  float* partials = nullptr;
  size_t partial_elems = 0;
  float* loss_rows = nullptr;
  // Double-buffered batch slots for rt_mlp_load / rt_mlp_step_loaded: pinned
  // host staging, device copies, and per slot the event of its last
  // host-to-device copy (copy stream) and of the last step that read it.
  struct Slot {
    void* x_host = nullptr;
    uint32_t* y_host = nullptr;
    rt_buf x, y;
    hipEvent_t copied = nullptr, used = nullptr;
    bool copy_pending = false, use_pending = false;
  } slot[2];
  bool slots_ready = false;
  int next_slot = 0, loaded = -1;
  // Device state words: [0] applied Adam updates, [1] overflow flag of the
  // last step, [2] a step was issued (mixed precision, see step_begin_launch);
  // [3] label flag: a loss of this plan saw a label >= the classes (sticky
  // until reported; every update is skipped while it is set); [4] updates
  // skipped while it was set (f32 plans, whose t lives on the host).
  int* state = nullptr;
  int t = 0;
  int dispatches = 0;
  bool mixed = false;
  bool head_fused = false;  // output layer GEMM + softmax-xent in one launch
};

static bool valid_cfg(const rt_mlp_config* c) {
  if (c->optimizer != RT_OPT_ADAM && c->optimizer != RT_OPT_SGD) return false;
  if (c->precision != RT_PREC_F32 && c->precision != RT_PREC_BF16) return false;
  if (!(c->loss_scale > 0.0f) || !std::isfinite(c->loss_scale)) return false;
  return true;
}

// One GEMM of the plan as a descriptor.  With splits > 1 it writes partial
// planes into the plan's partials buffer, summed by finish_split.
static GemmDesc plan_desc(rt_mlp* p, int layout, int in_dtype, const void* A, const void* B, void* C, int out_dtype,
                          int M, int N, int K, int lda, int ldb, int epi, const float* bias, const void* mask,
                          int mask_dtype, float* colsum, int splits, float* parts = nullptr) {
  GemmDesc d;
  d.overread_ok = true;  // every arena region is followed by >= 1 KiB of slack; x is never a B operand
  d.layout = layout;
  d.in_dtype = in_dtype;
  d.out_dtype = out_dtype;
  d.A = A;
  d.B = B;
  d.M = M;
  d.N = N;
  d.K = K;
  d.lda = lda;
  d.ldb = ldb;
  d.ldc = N;
  if (splits <= 1) {
    d.C = C;
    d.epi = epi;
    d.bias = bias;
    d.mask = mask;
    d.mask_dtype = mask_dtype;
    d.colsum = colsum;
    return d;
  }
  if (parts == nullptr) parts = p->partials;
  d.C = parts;
  d.out_dtype = RT_F32;
  d.splits = splits;
  d.split_stride = (long long)M * N;
  d.colsum_partials = colsum ? parts + (size_t)splits * M * N : nullptr;
  d.cs_shares_to_caller = true;  // finish_split adds the column-sum shares
  // Where the reduction puts the result and what it applies.
  d.epi = RT_EPI_NONE;
  return d;
}

// A mixed plan's dW launch writes its db shares into the layer's own region
// and leaves them there: a split launch's reduction adds them (finish_split),
// the non-finite check launch adds a whole launch's (share jobs).
static void layer_shares(const Layer& Ly, GemmDesc& d) {
  if (Ly.cs_shares == nullptr) return;
  d.cs_scratch = Ly.cs_shares;
  d.cs_scratch_elems = Ly.cs_share_elems;
  d.cs_shares_to_caller = true;
}

static int finish_split(rt_mlp* p, const GemmDesc& d, const char* lbl_red, void* C, int out_dtype, int epi,
                        const float* bias, const void* mask, int mask_dtype, float* colsum) {
  if (d.splits <= 1) return RT_OK;
  rt_ctx* c = p->ctx;
  const int cs_rows = gemm_cs_share_rows(d);
  Launch Lz(c, lbl_red);
  hipError_t e = splitk_reduce_launch(c->stream, p->partials, d.splits, d.split_stride, d.M, d.N, C, out_dtype, d.N,
                                      epi, bias, mask, mask_dtype, cs_rows ? d.cs_scratch : d.colsum_partials,
                                      colsum, cs_rows);
  if (e != hipSuccess) return hip_fail(c, e, lbl_red);
  return RT_OK;
}

// Run one GEMM of the plan, with optional split-K.
static int plan_gemm(rt_mlp* p, const char* lbl, const char* lbl_red, int layout, int in_dtype, const void* A,
                     const void* B, void* C, int out_dtype, int M, int N, int K, int lda, int ldb, int epi,
                     const float* bias, const void* mask, int mask_dtype, float* colsum, int splits,
                     unsigned* relu_bits_out = nullptr, bool* bits_written = nullptr) {
  rt_ctx* c = p->ctx;
  GemmDesc d = plan_desc(p, layout, in_dtype, A, B, C, out_dtype, M, N, K, lda, ldb, epi, bias, mask, mask_dtype,
                         colsum, splits);
  if (relu_bits_out != nullptr) {
    d.relu_bits_out = relu_bits_out;
    if (!gemm_relu_bits_ok(d)) d.relu_bits_out = nullptr;
    *bits_written = d.relu_bits_out != nullptr;
  }
  {
    Launch Lz(c, lbl);
    hipError_t e = gemm_launch(c->stream, d);
    if (e != hipSuccess) return hip_fail(c, e, lbl);
  }
  return finish_split(p, d, lbl_red, C, out_dtype, epi, bias, mask, mask_dtype, colsum);
}

// Forward pass; with labels, also the loss and δ of the output layer (scaled
// by `scale`).  A narrow f32 output layer runs as one fused GEMM + softmax
// cross-entropy launch; otherwise its GEMM (split-K when narrow) is followed
// by the softmax cross-entropy launch.
static int run_forward(rt_mlp* p, const rt_buf* x, const rt_buf* labels, float scale) {
  rt_ctx* c = p->ctx;
  const int nl = p->n_layers;
  const int B = (int)p->batch;
  const int in_dtype = p->mixed ? RT_BF16 : RT_F32;
  for (int l = 0; l < nl; ++l) {
    Layer& Ly = p->L[l];
    const void* in = l == 0 ? x->ptr : p->L[l - 1].act;
    const bool last = l == nl - 1;
    const float* bias = p->theta + Ly.b_off;
    if (last && p->head_fused) {
      Launch Lz(c, "head_xent");
      hipError_t e = head_xent_launch(c->stream, (const float*)in, (int)Ly.din, p->theta + Ly.w_off, bias,
                                      labels ? (const uint32_t*)labels->ptr : nullptr, (float*)Ly.act, Ly.delta,
                                      p->loss_rows, B, (int)Ly.dout, scale / (float)B, p->state + 3);
      if (e != hipSuccess) return hip_fail(c, e, "head_xent");
      return RT_OK;
    }
    const void* W = p->mixed ? (const void*)((unsigned short*)p->theta_h + Ly.w_off) : (const void*)(p->theta + Ly.w_off);
    const int out_dtype = (p->mixed && !last) ? RT_BF16 : RT_F32;
    Ly.bits_fresh = false;
    int rc = plan_gemm(p, Ly.lbl_fwd.c_str(), Ly.lbl_fwd_red.c_str(), RT_NN, in_dtype, in, W, Ly.act, out_dtype, B,
                       (int)Ly.dout, (int)Ly.din, (int)Ly.din, (int)Ly.dout, last ? RT_EPI_BIAS : RT_EPI_BIAS_RELU,
                       bias, nullptr, RT_F32, nullptr, Ly.splits_fwd, Ly.relu_bits, &Ly.bits_fresh);
    if (rc) return rc;
  }
  if (labels != nullptr) {
    Layer& top = p->L[nl - 1];
    Launch Lz(c, "softmax_xent");
    hipError_t e = xent_launch(c->stream, (const float*)top.act, (const uint32_t*)labels->ptr, top.delta, top.delta_h,
                               p->loss_rows, B, (int)top.dout, scale / (float)B, p->state + 3, (int)top.ldh);
    if (e != hipSuccess) return hip_fail(c, e, "softmax_xent");
  }
  return RT_OK;
}

// The optimizer's tensor list over the flat vectors of layers [l0, l1):
// plain runs of segments as one tensor each, and the W / b segments of
// layers whose dW planes are still split as tensors that sum their planes
// first.
static std::vector<OptTensor> opt_tensors(const rt_mlp* p, int l0, int l1) {
  std::vector<OptTensor> ts;
  auto seg = [&](size_t off, size_t n) {
    OptTensor T{p->theta + off, p->grad + off, p->m + off, p->v + off,
                p->theta_h ? (void*)((unsigned short*)p->theta_h + off) : nullptr, n};
    return T;
  };
  size_t run0 = p->L[l0].w_off;
  const size_t end = l1 < p->n_layers ? p->L[l1].w_off : p->n_params;
  for (int l = l0; l < l1; ++l) {
    const Layer& Ly = p->L[l];
    if (Ly.dw_parts == nullptr) continue;
    if (Ly.w_off > run0) ts.push_back(seg(run0, Ly.w_off - run0));
    const size_t nw = Ly.din * Ly.dout;
    OptTensor Tw = seg(Ly.w_off, nw);
    Tw.parts = Ly.dw_parts;
    Tw.n_parts = Ly.splits_dw;
    Tw.part_stride = (long long)nw;
    Tw.grad_store = p->grad + Ly.w_off;
    ts.push_back(Tw);
    OptTensor Tb = seg(Ly.b_off, Ly.dout);
    Tb.parts = Ly.dw_parts + (size_t)Ly.splits_dw * nw;
    Tb.n_parts = Ly.splits_dw;
    Tb.part_stride = (long long)Ly.dout;
    Tb.grad_store = p->grad + Ly.b_off;
    ts.push_back(Tb);
    run0 = Ly.b_off + Ly.dout;  // the b segment's padding stays untouched (zero)
  }
  if (run0 < end) ts.push_back(seg(run0, end - run0));
  return ts;
}

// The update's method and hyper-parameters (the step's t and flags are set
// by the step itself).
static OptParams plan_params(const rt_mlp* p) {
  OptParams P;
  P.kind = p->cfg.optimizer == RT_OPT_ADAM ? 0 : 1;
  P.lr = p->cfg.lr;
  P.beta1 = p->cfg.beta1;
  P.beta2 = p->cfg.beta2;
  P.eps = p->cfg.eps;
  P.momentum = p->cfg.momentum;
  return P;
}

static std::vector<OptTensor> plan_tensors(const rt_mlp* p, int l0, int l1, const OptParams& P) {
  std::vector<OptTensor> ts = opt_tensors(p, l0, l1);
  if (P.kind == 1 && P.momentum == 0.0f)
    for (auto& T : ts) T.m = nullptr;
  return ts;
}

// f32 plans: the update of layers 1.. (its gradients are final once layer
// 1's backward has run) goes into layer 0's dW launch, its HBM-bound blocks
// next to the GEMM's tiles; layer 0's own update follows.  Not under mixed
// precision, whose update waits for the non-finite check of every gradient.
static bool fuse_update(const rt_mlp* p) {
  if (p->mixed || p->n_layers < 2) return false;
  const OptParams P = plan_params(p);
  const std::vector<OptTensor> ts = plan_tensors(p, 1, p->n_layers, P);
  return optimizer_fits_cache(ts.data(), (int)ts.size(), P);
}

// Layer 0's W and b as the targets of an update done by its own dW tiles.
static std::array<OptTensor, 2> layer_update(const rt_mlp* p, int l, const OptParams& P) {
  const Layer& Ly = p->L[l];
  auto seg = [&](size_t off, size_t n) {
    OptTensor T{p->theta + off, p->grad + off, p->m + off, p->v + off, nullptr, n};
    if (P.kind == 1 && P.momentum == 0.0f) T.m = nullptr;
    return T;
  };
  return {seg(Ly.w_off, Ly.din * Ly.dout), seg(Ly.b_off, Ly.dout)};
}

// Layer 0's dW of an f32 plan as one unsplit launch of DMA tiles: with the
// update of layers 1.. in the same launch (fuse_update), its tiles also
// update layer 0 itself (gemm_opt_update_ok), and the step has no optimizer
// launch of its own.
static bool update_in_tiles(const rt_mlp* p, const GemmDesc& dw) {
  if (!fuse_update(p) || p->L[0].dw_parts != nullptr || p->L[0].splits_dw > 1) return false;
  const OptParams P = plan_params(p);
  return gemm_opt_update_ok(dw, layer_update(p, 0, P).data(), P);
}
// Layer l's f32 dW launch as the step builds it; in = the layer's input (for
// layer 0 the batch: any 16-byte aligned pointer, nullptr included, gives
// the step's tile decisions).
static GemmDesc f32_dw(rt_mlp* p, int l, const void* in) {
  const Layer& Ly = p->L[l];
  return plan_desc(p, RT_TN, RT_F32, in, Ly.delta, p->grad + Ly.w_off, RT_F32, (int)Ly.din, (int)Ly.dout,
                   (int)p->batch, (int)Ly.din, (int)Ly.ldh, RT_EPI_NONE, nullptr, nullptr, RT_F32,
                   p->grad + Ly.b_off, Ly.splits_dw, Ly.dw_parts);
}
static GemmDesc layer0_dw(rt_mlp* p, const void* x) { return f32_dw(p, 0, x); }

// Layer 1's dW joins layer 0's launch as well (f32 plans of 3+ layers whose
// layer 0 is updated by its dW tiles, and whose layer 1 runs its dW alone,
// unsplit, on the same tiles): those tiles update layer 1, the launch's
// optimizer blocks take layers 2.., and the step has one launch fewer.
// Layer 1's dW reads only δ₁ and the layer's input, which its dX launch
// before it does not change.
static bool fold_l1(rt_mlp* p, const void* x) {
  if (p->mixed || p->n_layers < 3) return false;
  const Layer& L1 = p->L[1];
  if (L1.pair_bwd || L1.splits_dw > 1 || L1.dw_parts != nullptr || !update_in_tiles(p, layer0_dw(p, x)))
    return false;
  const OptParams P = plan_params(p);
  const std::vector<OptTensor> rest = plan_tensors(p, 2, p->n_layers, P);
  return !rest.empty() && (int)rest.size() <= kMaxOptTensors &&
         optimizer_fits_cache(rest.data(), (int)rest.size(), P) &&
         gemm_opt_update_ok(f32_dw(p, 1, p->L[0].act), layer_update(p, 1, P).data(), P);
}

// Optimizer launches after the backward: none when layer 0's dW tiles do
// its update, layer 0's update alone when the rest is fused into its dW
// launch, else the whole model's.
static int opt_launches(rt_mlp* p) {
  if (!p->mixed && update_in_tiles(p, layer0_dw(p, nullptr))) return 0;
  const int n = (int)opt_tensors(p, 0, fuse_update(p) ? 1 : p->n_layers).size();
  return (n + kMaxOptTensors - 1) / kMaxOptTensors;
}

namespace rt {
void mlp_release(rt_mlp* p) {
  hipStreamSynchronize(p->ctx->stream);
  if (p->ctx->copy_stream) hipStreamSynchronize(p->ctx->copy_stream);
  for (auto& s : p->slot) {
    if (s.x_host) hipHostFree(s.x_host);
    if (s.y_host) hipHostFree(s.y_host);
    if (s.x.ptr) hipFree(s.x.ptr);
    if (s.y.ptr) hipFree(s.y.ptr);
    if (s.copied) hipEventDestroy(s.copied);
    if (s.used) hipEventDestroy(s.used);
  }
  hipFree(p->arena);
  delete p;
}

// Allocates the two batch slots on first use.
static int ensure_slots(rt_mlp* p) {
  if (p->slots_ready) return RT_OK;
  rt_ctx* c = p->ctx;
  hipError_t e = hipSuccess;
  if (!c->copy_stream) e = hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking);
  const rt_dtype xd = p->mixed ? RT_BF16 : RT_F32;
  const size_t xn = p->batch * p->L[0].din, xb = xn * dtype_size(xd), yb = p->batch * 4;
  for (auto& s : p->slot) {
    if (e == hipSuccess) e = hipHostMalloc(&s.x_host, xb, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc((void**)&s.y_host, yb, hipHostMallocDefault);
    if (e == hipSuccess) e = hipMalloc(&s.x.ptr, (xb + 255) / 256 * 256);
    if (e == hipSuccess) e = hipMalloc(&s.y.ptr, (yb + 255) / 256 * 256);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.copied, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&s.used, hipEventDisableTiming);
    s.x.dtype = xd;
    s.x.rank = 2;
    s.x.shape[0] = p->batch;
    s.x.shape[1] = p->L[0].din;
    s.x.n = xn;
    s.x.bytes = xb;
    s.y.dtype = RT_U32;
    s.y.rank = 1;
    s.y.shape[0] = p->batch;
    s.y.n = p->batch;
    s.y.bytes = yb;
  }
  if (e != hipSuccess) {  // undo the partial allocation; a later call may retry
    for (auto& sl : p->slot) {
      if (sl.x_host) hipHostFree(sl.x_host);
      if (sl.y_host) hipHostFree(sl.y_host);
      if (sl.x.ptr) hipFree(sl.x.ptr);
      if (sl.y.ptr) hipFree(sl.y.ptr);
      if (sl.copied) hipEventDestroy(sl.copied);
      if (sl.used) hipEventDestroy(sl.used);
      sl = rt_mlp::Slot();
    }
    return hip_fail(c, e, "batch slots");
  }
  p->slots_ready = true;
  return RT_OK;
}
}  // namespace rt

extern "C" {

int rt_mlp_create(rt_ctx* c, int n_layers, const size_t* dims, const float* const* weights, const float* const* biases,
                  size_t batch, const rt_mlp_config* cfg, rt_mlp** out) {
  CHECK_CTX(c);
  if (out == nullptr || dims == nullptr || weights == nullptr || biases == nullptr || cfg == nullptr)
    return fail(c, RT_ERR_INVALID, "null argument");
  *out = nullptr;
  if (n_layers < 1 || n_layers > 1024) return fail(c, RT_ERR_INVALID, "n_layers must be in [1, 1024]");
  if (batch < 1 || batch > (1u << 30)) return fail(c, RT_ERR_INVALID, "batch must be >= 1");
  if (!valid_cfg(cfg)) return fail(c, RT_ERR_INVALID, "bad rt_mlp_config");
  for (int l = 0; l <= n_layers; ++l)
    if (dims[l] < 1 || dims[l] > (1u << 24)) return fail(c, RT_ERR_SHAPE, "layer width %d out of range", l);
  for (int l = 0; l < n_layers; ++l)
    if (!weights[l] || !biases[l]) return fail(c, RT_ERR_INVALID, "null parameter %d", l);

  auto* p = new rt_mlp();
  p->ctx = c;
  p->batch = batch;
  p->n_layers = n_layers;
  p->cfg = *cfg;
  p->mixed = cfg->precision == RT_PREC_BF16;
  p->L.resize(n_layers);

  size_t off = 0;
  for (int l = 0; l < n_layers; ++l) {
    Layer& Ly = p->L[l];
    Ly.din = dims[l];
    Ly.dout = dims[l + 1];
    Ly.w_off = off;
    off += round_up(Ly.din * Ly.dout, 64);
    Ly.b_off = off;
    off += round_up(Ly.dout, 64);
    const bool last = l == n_layers - 1;
    // Split-K where the output tiles alone cannot fill the chip: the
    // output layer's forward (as mod.rs:1360-1367 does) and, at small
    // batches, the hidden layers' forward and dX too, whose bias+ReLU or
    // ReLU-mask epilogue then runs in the reduction (f32 plans; the bf16
    // plan's hidden outputs are bf16, which the reduction does not write).
    // Forward and dX products of at most 64 rows go whole to the skinny f32
    // kernel instead (one launch, its own epilogue).  The bf16 plan counts
    // its 256x256 tiles (half_slices): a 1000-class head at batch 4096 has
    // 64 of them.
    if (p->mixed) {
      Ly.splits_fwd = last ? half_slices(batch, Ly.dout, Ly.din) : 1;
      Ly.splits_dw = half_slices(Ly.din, Ly.dout, batch);
    } else {
      auto slices = [](size_t m, size_t n, size_t k) {
        return gemm_f32_skinny_shape((int)m, (int)n, (int)k) ? 1 : (int)rt_splitk_slices(m, n, k);
      };
      Ly.splits_fwd = slices(batch, Ly.dout, Ly.din);
      Ly.splits_dx = l > 0 ? slices(batch, Ly.din, Ly.dout) : 1;
      Ly.splits_dw = (int)rt_splitk_slices(Ly.din, Ly.dout, batch);
    }
    Ly.ldh = (p->mixed && last) ? round_up(Ly.dout, 64) : Ly.dout;
    Ly.lbl_fwd = "fwd_l" + std::to_string(l);
    Ly.lbl_fwd_red = "fwd_reduce_l" + std::to_string(l);
    Ly.lbl_dw = "dw_l" + std::to_string(l);
    Ly.lbl_dw_red = "dw_reduce_l" + std::to_string(l);
    Ly.lbl_dx = "dx_l" + std::to_string(l);
    Ly.lbl_dx_red = "dx_reduce_l" + std::to_string(l);
    Ly.lbl_bwd = "dwdx_l" + std::to_string(l);
  }
  p->n_params = off;

  // Split-K planes: f32 plans keep each layer's dW planes until the optimizer
  // sums them; everything else shares one buffer consumed right away.
  size_t part = 0;
  std::vector<size_t> dw_part_elems(n_layers, 0);
  for (int l = 0; l < n_layers; ++l) {
    const Layer& Ly = p->L[l];
    if (Ly.splits_fwd > 1) part = std::max(part, (size_t)Ly.splits_fwd * batch * Ly.dout);
    if (Ly.splits_dx > 1) part = std::max(part, (size_t)Ly.splits_dx * batch * Ly.din);
    if (Ly.splits_dw > 1) {
      const size_t e = (size_t)Ly.splits_dw * (Ly.din * Ly.dout + Ly.dout);
      if (p->mixed) part = std::max(part, e);
      else dw_part_elems[l] = e;
    }
  }
  p->partial_elems = part;
  // Column-sum shares of the half dW GEMMs (mixed precision only), one
  // region per layer.
  std::vector<size_t> cs_elems(n_layers, 0);
  if (p->mixed)
    for (int l = 0; l < n_layers; ++l)
      cs_elems[l] = colsum_scratch_need((int)p->L[l].din, (int)p->L[l].dout, p->L[l].splits_dw);

  // Arena layout.
  const size_t A = 256;
  size_t bytes = 0;
  // Each region is followed by 1 KiB of slack, so a GEMM may over-read the
  // last row of a B operand whose width is not a multiple of its tile.
  auto reserve = [&](size_t nbytes) {
    size_t o = bytes;
    bytes += round_up(std::max<size_t>(nbytes, 1), A) + 1024;
    return o;
  };
  size_t o_theta = reserve(p->n_params * 4), o_grad = reserve(p->n_params * 4), o_m = reserve(p->n_params * 4),
         o_v = reserve(p->n_params * 4);
  size_t o_theta_h = p->mixed ? reserve(p->n_params * 2) : 0;
  std::vector<size_t> o_act(n_layers), o_delta(n_layers), o_delta_h(n_layers), o_bits(n_layers, 0);
  std::vector<char> has_bits(n_layers, 0);
  for (int l = 0; l < n_layers; ++l) {
    const bool last = l == n_layers - 1;
    size_t elems = batch * p->L[l].dout;
    o_act[l] = reserve(elems * ((p->mixed && !last) ? 2 : 4));
    o_delta[l] = reserve(elems * 4);
    o_delta_h[l] = p->mixed ? reserve(batch * p->L[l].ldh * 2) : 0;
    has_bits[l] = p->mixed && !last && batch % 16 == 0 && p->L[l].dout % 64 == 0;
    if (has_bits[l]) o_bits[l] = reserve(elems / 8);
  }
  size_t o_part = reserve(part * 4);
  std::vector<size_t> o_dw_part(n_layers, 0);
  for (int l = 0; l < n_layers; ++l)
    if (dw_part_elems[l]) o_dw_part[l] = reserve(dw_part_elems[l] * 4);
  std::vector<size_t> o_cs(n_layers, 0);
  for (int l = 0; l < n_layers; ++l)
    if (cs_elems[l]) o_cs[l] = reserve(cs_elems[l] * 4);
  size_t o_loss = reserve(batch * 4);
  size_t o_state = reserve(16 * 4);

  hipError_t e = hipSetDevice(c->device);
  if (e == hipSuccess) e = hipMalloc(&p->arena, bytes);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(c, e, "mlp arena");
  }
  p->theta = (float*)(p->arena + o_theta);
  p->grad = (float*)(p->arena + o_grad);
  p->m = (float*)(p->arena + o_m);
  p->v = (float*)(p->arena + o_v);
  p->theta_h = p->mixed ? (void*)(p->arena + o_theta_h) : nullptr;
  for (int l = 0; l < n_layers; ++l) {
    p->L[l].act = p->arena + o_act[l];
    p->L[l].delta = (float*)(p->arena + o_delta[l]);
    p->L[l].delta_h = p->mixed ? (void*)(p->arena + o_delta_h[l]) : nullptr;
    p->L[l].relu_bits = has_bits[l] ? (unsigned*)(p->arena + o_bits[l]) : nullptr;
  }
  p->partials = part ? (float*)(p->arena + o_part) : nullptr;
  for (int l = 0; l < n_layers; ++l) p->L[l].dw_parts = dw_part_elems[l] ? (float*)(p->arena + o_dw_part[l]) : nullptr;
  p->loss_rows = (float*)(p->arena + o_loss);
  for (int l = 0; l < n_layers; ++l) {
    p->L[l].cs_shares = cs_elems[l] ? (float*)(p->arena + o_cs[l]) : nullptr;
    p->L[l].cs_share_elems = cs_elems[l];
  }
  p->state = (int*)(p->arena + o_state);

  // Zero everything (padding and moments must start at 0), then upload θ.
  e = fill_i32_launch(c->stream, (int*)p->arena, 0, bytes / 4);
  std::vector<float> host(p->n_params, 0.0f);
  for (int l = 0; l < n_layers && e == hipSuccess; ++l) {
    const Layer& Ly = p->L[l];
    std::memcpy(&host[Ly.w_off], weights[l], Ly.din * Ly.dout * 4);
    std::memcpy(&host[Ly.b_off], biases[l], Ly.dout * 4);
  }
  if (e == hipSuccess) e = hipMemcpyAsync(p->theta, host.data(), p->n_params * 4, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess && p->mixed) e = convert_launch(c->stream, p->theta, RT_F32, p->theta_h, RT_BF16, p->n_params);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    hipFree(p->arena);
    delete p;
    return hip_fail(c, e, "mlp init");
  }

  // Hidden layers whose dW and dX fit the fused pair launch.
  for (int l = 1; l < n_layers; ++l) {
    Layer& Ly = p->L[l];
    const int dt = p->mixed ? RT_BF16 : RT_F32;
    const GemmDesc dw = plan_desc(p, RT_TN, dt, p->L[l - 1].act, Ly.delta, p->grad + Ly.w_off, RT_F32, (int)Ly.din,
                                  (int)Ly.dout, (int)batch, (int)Ly.din, (int)Ly.dout, RT_EPI_NONE, nullptr, nullptr,
                                  RT_F32, p->grad + Ly.b_off, Ly.splits_dw);
    const GemmDesc dx = plan_desc(p, RT_NT, dt, Ly.delta, p->theta + Ly.w_off, p->L[l - 1].delta, RT_F32, (int)batch,
                                  (int)Ly.din, (int)Ly.dout, (int)Ly.dout, (int)Ly.dout, RT_EPI_RELU_MASK, nullptr,
                                  p->L[l - 1].act, RT_F32, nullptr, 1);
    // Not when the dX product runs on the skinny kernel: in the pair its
    // tiles would walk the whole K alone (batch 32: 41 µs against ~14).
    const bool skinny_dx = !p->mixed && gemm_f32_skinny_shape((int)batch, (int)Ly.din, (int)Ly.dout);
    Ly.pair_bwd = Ly.splits_dx == 1 && !skinny_dx && gemm_pair_supported(dw, dx);
  }

  const Layer& top = p->L[n_layers - 1];
  p->head_fused = !p->mixed && head_xent_supported((int)top.din, (int)top.dout);

  // Launch count of one step.
  const bool fold = fold_l1(p, nullptr);
  int n = 0;
  for (int l = 0; l < n_layers; ++l) {
    const bool fused = l == n_layers - 1 && p->head_fused;
    n += fused ? 1 : (p->L[l].splits_fwd > 1 ? 2 : 1);
    if (!(fold && l == 1)) n += (p->L[l].splits_dw > 1 && !p->L[l].dw_parts) ? 2 : 1;
    if (p->mixed) {  // the dW GEMM's shares are added elsewhere: one launch
      const Layer& Ly = p->L[l];
      const void* a_in = l == 0 ? nullptr : p->L[l - 1].act;
      GemmDesc dw = plan_desc(p, RT_TN, RT_BF16, a_in, Ly.delta_h, p->grad + Ly.w_off, RT_F32, (int)Ly.din,
                              (int)Ly.dout, (int)batch, (int)Ly.din, (int)Ly.ldh, RT_EPI_NONE, nullptr, nullptr, RT_F32,
                              p->grad + Ly.b_off, Ly.splits_dw);
      layer_shares(Ly, dw);
      n += gemm_launch_count(dw) - 1;
    }
    if (l > 0 && !p->L[l].pair_bwd) n += p->L[l].splits_dx > 1 ? 2 : 1;
  }
  if (!p->head_fused) n += 1;  // softmax-xent
  n += opt_launches(p);  // optimizer
  if (p->mixed) {
    n += 1;  // step prologue
    int unchecked = 0;  // layers whose dW GEMM cannot flag non-finite values itself
    int jobs = 0;       // whole dW launches whose db shares the check launch adds
    for (int l = 0; l < n_layers; ++l) {
      const Layer& Ly = p->L[l];
      GemmDesc dw = plan_desc(p, RT_TN, RT_BF16, l == 0 ? nullptr : p->L[l - 1].act, Ly.delta_h, p->grad + Ly.w_off,
                              RT_F32, (int)Ly.din, (int)Ly.dout, (int)batch, (int)Ly.din, (int)Ly.ldh, RT_EPI_NONE,
                              nullptr, nullptr, RT_F32, p->grad + Ly.b_off, Ly.splits_dw);
      layer_shares(Ly, dw);
      dw.nf_flag = p->state + 1;
      unchecked += !gemm_checks_nonfinite(dw);
      jobs += Ly.splits_dw <= 1 && gemm_cs_share_rows(dw) > 0;
    }
    // Separate checks, 24 tensors and 32 share jobs per launch.
    n += std::max((jobs + kMaxShareJobs - 1) / kMaxShareJobs, (2 * unchecked + kMaxOptTensors - 1) / kMaxOptTensors);
  }
  p->dispatches = n;
  c->mlps.push_back(p);
  *out = p;
  return RT_OK;
}

int rt_mlp_destroy(rt_mlp* p) {
  if (p == nullptr) return RT_OK;
  bind_device(p->ctx);
  auto& v = p->ctx->mlps;
  v.erase(std::remove(v.begin(), v.end(), p), v.end());
  mlp_release(p);
  return RT_OK;
}

static int check_inputs(rt_mlp* p, const rt_buf* x) {
  rt_ctx* c = p->ctx;
  if (x == nullptr) return fail(c, RT_ERR_INVALID, "null batch");
  const rt_dtype want = p->mixed ? RT_BF16 : RT_F32;
  if (x->dtype != want) return fail(c, RT_ERR_DTYPE, "batch must be %s", p->mixed ? "bf16" : "f32");
  if (x->n != p->batch * p->L[0].din)
    return fail(c, RT_ERR_SHAPE, "batch with %zu elements, plan built for %zu", x->n, p->batch * p->L[0].din);
  return RT_OK;
}

int rt_mlp_step(rt_mlp* p, const rt_buf* x, const rt_buf* labels) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  int rc = check_inputs(p, x);
  if (rc) return rc;
  if (labels == nullptr || labels->dtype != RT_U32 || labels->n != p->batch)
    return fail(c, RT_ERR_SHAPE, "labels must be u32 [%zu]", p->batch);
  const int nl = p->n_layers;
  const int B = (int)p->batch;
  const float scale = p->mixed ? p->cfg.loss_scale : 1.0f;
  int* overflow = p->state + 1;

  if (p->mixed) {
    Launch Lz(c, "step_begin");
    hipError_t e = step_begin_launch(c->stream, p->state);
    if (e != hipSuccess) return hip_fail(c, e, "step prologue");
  }
  if ((rc = run_forward(p, x, labels, scale))) return rc;

  // This step's update (t + 1), set up before the backward so that layer 0's
  // dW launch can carry the update of layers 1.. (fuse_update).
  OptParams P = plan_params(p);
  if (P.kind == 0) {
    const float c1 = 1.0f - powi_f32(P.beta1, p->t + 1), c2 = 1.0f - powi_f32(P.beta2, p->t + 1);
    P.inv_c1 = 1.0f / c1;
    P.inv_c2 = 1.0f / c2;
  }
  if (p->mixed) {
    // Unscale exactly (the loss scale is a power of two in practice) and skip
    // the whole update on a non-finite gradient; a skipped step does not
    // advance Adam's t (the count lives on the device).
    P.grad_scale = 1.0f / p->cfg.loss_scale;
    P.skip_flag = overflow;
    P.device_t = p->state;
  }
  // A label >= the classes skips the update (weights and moments stay as
  // they were); an f32 plan counts the skipped step (in its first update
  // launch) so that the report can take it back out of t.
  P.skip_flag2 = p->state + 3;
  const bool fuse = fuse_update(p);
  bool fused = false;  // layers 1..'s update ran in layer 0's dW launch
  bool upd0 = false;   // and layer 0's in that launch's tiles
  const bool fold = fold_l1(p, x->ptr);  // layer 1's dW (and update) in that launch too

  const int in_dtype = p->mixed ? RT_BF16 : RT_F32;
  std::vector<char> unchecked(nl, 1);
  std::vector<ShareJob> jobs;
  for (int l = nl - 1; l >= 0; --l) {
    Layer& Ly = p->L[l];
    const void* in = l == 0 ? x->ptr : p->L[l - 1].act;
    const void* dl = p->mixed ? Ly.delta_h : (const void*)Ly.delta;
    const int ld_dl = (int)Ly.ldh;  // == dout for f32 plans and hidden layers
    // dW_l = A_{l-1}ᵀ·δ_l  (TN; A stored [batch, din]), db_l = 1ᵀ·δ_l fused.
    GemmDesc dw = plan_desc(p, RT_TN, in_dtype, in, dl, p->grad + Ly.w_off, RT_F32, (int)Ly.din, (int)Ly.dout, B,
                            (int)Ly.din, ld_dl, RT_EPI_NONE, nullptr, nullptr, RT_F32, p->grad + Ly.b_off,
                            Ly.splits_dw, Ly.dw_parts);
    if (p->mixed) {
      // The overflow flag is set by the GEMM's own epilogue where it can;
      // the other layers' dW/db go to the separate check below, which also
      // adds a whole launch's db shares into db.
      layer_shares(Ly, dw);
      dw.nf_flag = overflow;
      unchecked[l] = !gemm_checks_nonfinite(dw);
      if (unchecked[l]) dw.nf_flag = nullptr;
      const int rows = dw.splits <= 1 ? gemm_cs_share_rows(dw) : 0;
      if (rows > 0) jobs.push_back(ShareJob{Ly.cs_shares, p->grad + Ly.b_off, rows, (int)Ly.dout});
    }
    if (l == 0) {
      const std::vector<OptTensor> rest = fuse ? plan_tensors(p, fold ? 2 : 1, nl, P) : std::vector<OptTensor>();
      if (fuse && gemm_opt_supported(dw, rest.data(), (int)rest.size(), P)) {
        OptParams Pr = P;
        Pr.skip_count = p->state + 4;
        upd0 = update_in_tiles(p, dw);
        const std::array<OptTensor, 2> wb = layer_update(p, 0, P);
        Launch Lz(c, Ly.lbl_dw.c_str());
        hipError_t e;
        if (fold) {
          const std::array<OptTensor, 2> wb1 = layer_update(p, 1, P);
          e = gemm_opt_update2_launch(c->stream, dw, wb.data(), f32_dw(p, 1, Ly.act), wb1.data(), rest.data(),
                                      (int)rest.size(), Pr);
        } else {
          e = gemm_opt_launch(c->stream, dw, rest.data(), (int)rest.size(), Pr, upd0 ? wb.data() : nullptr);
        }
        if (e != hipSuccess) return hip_fail(c, e, Ly.lbl_dw.c_str());
        fused = true;
      } else {
        Launch Lz(c, Ly.lbl_dw.c_str());
        hipError_t e = gemm_launch(c->stream, dw);
        if (e != hipSuccess) return hip_fail(c, e, Ly.lbl_dw.c_str());
      }
    } else {
      Layer& Lp = p->L[l - 1];
      const void* W = p->mixed ? (const void*)((unsigned short*)p->theta_h + Ly.w_off) : (const void*)(p->theta + Ly.w_off);
      // δ_{l-1} = (δ_l·W_lᵀ) ⊙ 1[A_{l-1} > 0]  (NT; W stored [din, dout] = [N, K]).
      // With a padded δ_l (ld_dl > dout) K runs over the zero padding too:
      // those k read W's next row (finite weights) times zero.
      void* dst = p->mixed ? Lp.delta_h : (void*)Lp.delta;
      GemmDesc dx = plan_desc(p, RT_NT, in_dtype, dl, W, dst, p->mixed ? RT_BF16 : RT_F32, B, (int)Ly.din, ld_dl,
                              ld_dl, (int)Ly.dout, RT_EPI_RELU_MASK, nullptr, Lp.act, p->mixed ? RT_BF16 : RT_F32,
                              nullptr, Ly.splits_dx);
      if (Lp.bits_fresh) {  // the same predicate, 1/16 of the bytes
        dx.relu_bits = Lp.relu_bits;
        if (!gemm_relu_bits_ok(dx)) dx.relu_bits = nullptr;
      }
      if (Ly.pair_bwd) {
        // Both read δ_l and neither feeds the other: one launch.
        Launch Lz(c, Ly.lbl_bwd.c_str());
        hipError_t e = gemm_pair_launch(c->stream, dw, dx);
        if (e != hipSuccess) return hip_fail(c, e, Ly.lbl_bwd.c_str());
      } else {
        if (!(fold && l == 1)) {  // under fold_l1 it runs in layer 0's dW launch
          Launch Lz(c, Ly.lbl_dw.c_str());
          hipError_t e = gemm_launch(c->stream, dw);
          if (e != hipSuccess) return hip_fail(c, e, Ly.lbl_dw.c_str());
        }
        {
          Launch Lz(c, Ly.lbl_dx.c_str());
          hipError_t e = gemm_launch(c->stream, dx);
          if (e != hipSuccess) return hip_fail(c, e, Ly.lbl_dx.c_str());
        }
        // Split dX (small batches): the reduction applies the ReLU mask.
        rc = finish_split(p, dx, Ly.lbl_dx_red.c_str(), dst, RT_F32, RT_EPI_RELU_MASK, nullptr, Lp.act, RT_F32,
                          nullptr);
        if (rc) return rc;
      }
    }
    if (Ly.dw_parts == nullptr) {  // otherwise the optimizer sums the planes
      rc = finish_split(p, dw, Ly.lbl_dw_red.c_str(), p->grad + Ly.w_off, RT_F32, RT_EPI_NONE, nullptr, nullptr,
                        RT_F32, p->grad + Ly.b_off);
      if (rc) return rc;
    }
  }

  if (p->mixed) {
    std::vector<const float*> ptrs;
    std::vector<size_t> ns;
    for (int l = 0; l < nl; ++l) {
      if (!unchecked[l]) continue;
      ptrs.push_back(p->grad + p->L[l].w_off);
      ns.push_back(p->L[l].din * p->L[l].dout);
      ptrs.push_back(p->grad + p->L[l].b_off);
      ns.push_back(p->L[l].dout);
    }
    // Launch i checks tensors [24 i, 24 i + 24) and adds jobs [32 i, 32 i + 32).
    for (size_t i = 0; i * kMaxOptTensors < ptrs.size() || i * kMaxShareJobs < jobs.size(); ++i) {
      const size_t t0 = std::min(ptrs.size(), i * kMaxOptTensors), j0 = std::min(jobs.size(), i * kMaxShareJobs);
      const int k = (int)std::min<size_t>(kMaxOptTensors, ptrs.size() - t0);
      const int nj = (int)std::min<size_t>(kMaxShareJobs, jobs.size() - j0);
      Launch Lz(c, "nonfinite_check");
      hipError_t e = nonfinite_check_launch(c->stream, ptrs.data() + t0, ns.data() + t0, k, overflow,
                                            jobs.data() + j0, nj);
      if (e != hipSuccess) return hip_fail(c, e, "non-finite check");
    }
  }

  p->t += 1;
  if (upd0) return RT_OK;
  const std::vector<OptTensor> ts = plan_tensors(p, 0, fused ? 1 : nl, P);
  for (size_t i0 = 0; i0 < ts.size(); i0 += kMaxOptTensors) {
    const int nt = (int)std::min<size_t>(kMaxOptTensors, ts.size() - i0);
    P.skip_count = (!p->mixed && !fused && i0 == 0) ? p->state + 4 : nullptr;
    Launch Lz(c, "optimizer");
    hipError_t e = optimizer_launch(c->stream, ts.data() + i0, nt, P);
    if (e != hipSuccess) return hip_fail(c, e, "optimizer");
  }
  return RT_OK;
}

int rt_mlp_load(rt_mlp* p, const void* x, size_t x_bytes, const uint64_t* labels, size_t n) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  if (x == nullptr || labels == nullptr) return fail(c, RT_ERR_INVALID, "null batch");
  int rc = ensure_slots(p);
  if (rc) return rc;
  const int k = p->next_slot;
  auto& s = p->slot[k];
  if (x_bytes != s.x.bytes) return fail(c, RT_ERR_SHAPE, "batch of %zu bytes, plan takes %zu", x_bytes, s.x.bytes);
  if (n != p->batch) return fail(c, RT_ERR_SHAPE, "%zu labels, plan takes %zu", n, p->batch);
  const size_t classes = p->L[p->n_layers - 1].dout;
  for (size_t i = 0; i < n; ++i)
    if (labels[i] >= classes) return fail(c, RT_ERR_LABEL, "label %zu is %llu, >= the %zu classes", i,
                                          (unsigned long long)labels[i], classes);
  // The staging buffers are free once this slot's previous copy has run.
  if (s.copy_pending) HIP_TRY(c, hipEventSynchronize(s.copied), "staging wait");
  std::memcpy(s.x_host, x, x_bytes);
  for (size_t i = 0; i < n; ++i) s.y_host[i] = (uint32_t)labels[i];
  // The device slot is free once the last step that read it has run (two
  // steps back); the step on the other slot runs meanwhile (the overlap).
  // The wait is on the host: a copy-engine queue made to wait on the compute
  // queue starts late (measured: 0.33 vs 0.21 ms per batch-2048 step).
  if (s.use_pending) HIP_TRY(c, hipEventSynchronize(s.used), "slot wait");
  HIP_TRY(c, hipMemcpyAsync(s.x.ptr, s.x_host, s.x.bytes, hipMemcpyHostToDevice, c->copy_stream), "batch copy");
  HIP_TRY(c, hipMemcpyAsync(s.y.ptr, s.y_host, s.y.bytes, hipMemcpyHostToDevice, c->copy_stream), "label copy");
  HIP_TRY(c, hipEventRecord(s.copied, c->copy_stream), "copy event");
  s.copy_pending = true;
  p->loaded = k;
  p->next_slot = k ^ 1;
  return RT_OK;
}

int rt_mlp_step_loaded(rt_mlp* p) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  if (p->loaded < 0) return fail(c, RT_ERR_INVALID, "no batch loaded");
  auto& s = p->slot[p->loaded];
  HIP_TRY(c, hipStreamWaitEvent(c->stream, s.copied, 0), "copy wait");
  int rc = rt_mlp_step(p, &s.x, &s.y);
  if (rc) return rc;
  HIP_TRY(c, hipEventRecord(s.used, c->stream), "use event");
  s.use_pending = true;
  return RT_OK;
}

// The label flag of the plan, read on the host (blocking).  If a loss saw a
// label >= the classes, the updates skipped since are taken back out of an
// f32 plan's t (a mixed plan's device count never included them), the flag
// is cleared, and RT_ERR_LABEL is returned: every blocking call on the plan
// reports it once.
static int report_label(rt_mlp* p) {
  rt_ctx* c = p->ctx;
  int st[5] = {0, 0, 0, 0, 0};
  HIP_TRY(c, hipMemcpyAsync(st, p->state, sizeof st, hipMemcpyDeviceToHost, c->stream), "label flag");
  HIP_TRY(c, hipStreamSynchronize(c->stream), "label flag");
  if (st[3] == 0) return RT_OK;
  if (!p->mixed) p->t -= st[4];
  // Mixed: the pending step (state[2]) was skipped, so it must not be counted.
  HIP_TRY(c, fill_i32_launch(c->stream, p->state + 2, 0, 3), "label flag reset");
  HIP_TRY(c, hipStreamSynchronize(c->stream), "label flag reset");
  return fail(c, RT_ERR_LABEL, "a label was >= the number of classes (%zu); the update was skipped",
              p->L[p->n_layers - 1].dout);
}

int rt_mlp_forward(rt_mlp* p, const rt_buf* x) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  int rc = check_inputs(p, x);
  if (rc) return rc;
  return run_forward(p, x, nullptr, 1.0f);
}

int rt_mlp_logits(rt_mlp* p, float* host, size_t n) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  const Layer& top = p->L[p->n_layers - 1];
  if (host == nullptr || n != p->batch * top.dout) return fail(c, RT_ERR_SHAPE, "logits need %zu floats", p->batch * top.dout);
  int rc = report_label(p);
  if (rc) return rc;
  hipError_t e = hipMemcpyAsync(host, top.act, n * 4, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "logits");
  return RT_OK;
}

// Copies one stored [batch, width] intermediate to host f32: bf16 values are
// widened exactly; a padded row stride (the bf16 output layer's δ) is dropped.
static int copy_rows_f32(rt_mlp* p, const void* src, bool half, size_t ld, size_t width, float* host) {
  rt_ctx* c = p->ctx;
  const size_t rows = p->batch;
  if (!half) {
    HIP_TRY(c, hipMemcpy2DAsync(host, width * 4, src, ld * 4, width * 4, rows, hipMemcpyDeviceToHost, c->stream),
            "intermediate");
    HIP_TRY(c, hipStreamSynchronize(c->stream), "intermediate");
    return RT_OK;
  }
  std::vector<uint16_t> tmp(rows * width);
  HIP_TRY(c, hipMemcpy2DAsync(tmp.data(), width * 2, src, ld * 2, width * 2, rows, hipMemcpyDeviceToHost, c->stream),
          "intermediate");
  HIP_TRY(c, hipStreamSynchronize(c->stream), "intermediate");
  for (size_t i = 0; i < tmp.size(); ++i) {
    const uint32_t u = (uint32_t)tmp[i] << 16;
    std::memcpy(host + i, &u, 4);
  }
  return RT_OK;
}

int rt_mlp_activation(rt_mlp* p, int layer, float* host, size_t n) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  if (layer < 0 || layer >= p->n_layers) return fail(c, RT_ERR_INVALID, "layer %d out of range", layer);
  const Layer& Ly = p->L[layer];
  if (host == nullptr || n != p->batch * Ly.dout) return fail(c, RT_ERR_SHAPE, "need %zu floats", p->batch * Ly.dout);
  int rc = report_label(p);
  if (rc) return rc;
  const bool half = p->mixed && layer < p->n_layers - 1;
  return copy_rows_f32(p, Ly.act, half, Ly.dout, Ly.dout, host);
}

int rt_mlp_delta(rt_mlp* p, int layer, float* host, size_t n) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  if (layer < 0 || layer >= p->n_layers) return fail(c, RT_ERR_INVALID, "layer %d out of range", layer);
  const Layer& Ly = p->L[layer];
  if (host == nullptr || n != p->batch * Ly.dout) return fail(c, RT_ERR_SHAPE, "need %zu floats", p->batch * Ly.dout);
  int rc = report_label(p);
  if (rc) return rc;
  if (p->mixed) return copy_rows_f32(p, Ly.delta_h, true, Ly.ldh, Ly.dout, host);
  return copy_rows_f32(p, Ly.delta, false, Ly.dout, Ly.dout, host);
}

int rt_mlp_last_loss(rt_mlp* p, float* out) {
  if (p == nullptr || out == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  int rc = report_label(p);
  if (rc) return rc;
  std::vector<float> rows(p->batch);
  hipError_t e = hipMemcpyAsync(rows.data(), p->loss_rows, p->batch * 4, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "last_loss");
  // Tensor::mean_all (tensor.rs:284-286): sequential f32 sum, then divide.
  float s = 0.0f;
  for (float r : rows) s += r;
  *out = s / (float)p->batch;
  return RT_OK;
}

static int fetch(rt_mlp* p, const float* base, float* const* host, int n) {
  rt_ctx* c = p->ctx;
  if (host == nullptr || n != 2 * p->n_layers) return fail(c, RT_ERR_SHAPE, "need %d host arrays", 2 * p->n_layers);
  for (int i = 0; i < n; ++i)
    if (host[i] == nullptr) return fail(c, RT_ERR_INVALID, "null host array %d", i);
  hipError_t e = hipSuccess;
  for (int l = 0; l < p->n_layers && e == hipSuccess; ++l) {
    const Layer& Ly = p->L[l];
    e = hipMemcpyAsync(host[2 * l], base + Ly.w_off, Ly.din * Ly.dout * 4, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(host[2 * l + 1], base + Ly.b_off, Ly.dout * 4, hipMemcpyDeviceToHost, c->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "download parameters");
  return RT_OK;
}

static int put(rt_mlp* p, float* base, const float* const* host, int n) {
  rt_ctx* c = p->ctx;
  if (host == nullptr || n != 2 * p->n_layers) return fail(c, RT_ERR_SHAPE, "need %d host arrays", 2 * p->n_layers);
  for (int i = 0; i < n; ++i)
    if (host[i] == nullptr) return fail(c, RT_ERR_INVALID, "null host array %d", i);
  hipError_t e = hipSuccess;
  for (int l = 0; l < p->n_layers && e == hipSuccess; ++l) {
    const Layer& Ly = p->L[l];
    e = hipMemcpyAsync(base + Ly.w_off, host[2 * l], Ly.din * Ly.dout * 4, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(base + Ly.b_off, host[2 * l + 1], Ly.dout * 4, hipMemcpyHostToDevice, c->stream);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "upload parameters");
  return RT_OK;
}

int rt_mlp_set_weights(rt_mlp* p, const float* const* host, int n) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  int rc = report_label(p);
  if (rc) return rc;
  rc = put(p, p->theta, host, n);
  if (rc || !p->mixed) return rc;
  rt_ctx* c = p->ctx;
  hipError_t e = convert_launch(c->stream, p->theta, RT_F32, p->theta_h, RT_BF16, p->n_params);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "bf16 weight copy");
  return RT_OK;
}

int rt_mlp_get_optimizer_state(rt_mlp* p, float* const* m, float* const* v, int n, int* t) {
  if (p == nullptr || t == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  int rc = report_label(p);
  if (rc) return rc;
  if (m != nullptr && (rc = fetch(p, p->m, m, n))) return rc;
  if (v != nullptr && (rc = fetch(p, p->v, v, n))) return rc;
  if (!p->mixed) {
    *t = p->t;
    return RT_OK;
  }
  // Device count of applied updates, plus the last step if it was issued and
  // did not overflow (step_begin_launch folds that in at the next step).
  int st[3] = {0, 0, 0};
  hipError_t e = hipMemcpyAsync(st, p->state, sizeof st, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "optimizer state");
  *t = st[0] + ((st[2] != 0 && st[1] == 0) ? 1 : 0);
  return RT_OK;
}

int rt_mlp_set_optimizer_state(rt_mlp* p, const float* const* m, const float* const* v, int n, int t) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  if (t < 0) return fail(c, RT_ERR_INVALID, "t must be >= 0");
  int rc = report_label(p);
  if (rc) return rc;
  if (m != nullptr && (rc = put(p, p->m, m, n))) return rc;
  if (v != nullptr && (rc = put(p, p->v, v, n))) return rc;
  p->t = t;
  if (p->mixed) {
    const int st[3] = {t, 0, 0};  // t applied updates, no overflow, no step pending
    hipError_t e = hipMemcpyAsync(p->state, st, sizeof st, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "optimizer state");
  }
  return RT_OK;
}

int rt_mlp_weights(rt_mlp* p, float* const* host, int n) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  int rc = report_label(p);
  if (rc) return rc;
  return fetch(p, p->theta, host, n);
}

int rt_mlp_grads(rt_mlp* p, float* const* host, int n) {
  if (p == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  int rc = report_label(p);
  if (rc) return rc;
  rc = fetch(p, p->grad, host, n);
  if (rc || !p->mixed || p->cfg.loss_scale == 1.0f) return rc;
  // Gradients are held scaled by the loss scale; report dL/dθ.
  const float inv = 1.0f / p->cfg.loss_scale;
  for (int l = 0; l < p->n_layers; ++l) {
    const Layer& Ly = p->L[l];
    for (size_t i = 0; i < Ly.din * Ly.dout; ++i) host[2 * l][i] *= inv;
    for (size_t i = 0; i < Ly.dout; ++i) host[2 * l + 1][i] *= inv;
  }
  return RT_OK;
}

int rt_mlp_dispatches(rt_mlp* p, int* out) {
  if (p == nullptr || out == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  *out = p->dispatches;
  return RT_OK;
}

int rt_mlp_overflow(rt_mlp* p, int* out) {
  if (p == nullptr || out == nullptr) return RT_ERR_INVALID;
  bind_device(p->ctx);
  rt_ctx* c = p->ctx;
  int rc = report_label(p);
  if (rc) return rc;
  int flag = 0;
  hipError_t e = hipMemcpyAsync(&flag, p->state + 1, sizeof(int), hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "overflow flag");
  *out = flag;
  return RT_OK;
}

}  // extern "C"
