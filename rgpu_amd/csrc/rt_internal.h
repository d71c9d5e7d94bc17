// Internal declarations shared by the host runtime and the kernel sources.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "rtensor_hip.h"

struct rt_buf {
  void* ptr = nullptr;
  rt_dtype dtype = RT_F32;
  size_t shape[4] = {0, 0, 0, 0};
  int rank = 0;
  size_t n = 0;      // elements
  size_t bytes = 0;  // n * element size
  size_t cap = 0;    // bytes of the device allocation (its cache size class)
};

struct rt_prof_rec {
  std::string label;
  hipEvent_t e0, e1;
};

struct rt_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  std::string arch;
  std::string name;
  int num_cus = 0;
  // Device flags written by kernels: [0] label out of range, [1] non-finite
  // gradient.  Zeroed by a fill kernel, read back by the blocking readers.
  int* d_flags = nullptr;
  // Grow-only device scratch for ops that need temporaries (colsum stage 1,
  // sum partials, loss terms, argmax predictions); see ensure_scratch.
  float* scratch = nullptr;
  size_t scratch_elems = 0;
  // Freed buffer allocations by size class, reused in stream order.
  std::unordered_map<size_t, std::vector<void*>> pool;
  size_t pool_bytes = 0;
  bool profiling = false;
  // Children freed by rt_close if the caller has not freed them.
  std::unordered_set<rt_buf*> bufs;
  std::vector<rt_mlp*> mlps;
  std::vector<rt_prof_rec> prof;
  std::vector<hipEvent_t> event_pool;
  // Region timer (rt_timer_begin / rt_timer_end).
  hipEvent_t timer0 = nullptr, timer1 = nullptr;
  bool timer_running = false;
  // Host-to-device copies of staged batches (rt_mlp_load), created on first
  // use; default priority like the main stream.
  hipStream_t copy_stream = nullptr;
  // This device's copy of rt_gemm_splitk_static's static scratch array.
  float* static_scratch = nullptr;
};

namespace rt {

void mlp_release(rt_mlp* p);  // frees the plan's device memory and the struct
size_t dtype_size(rt_dtype d);
int fail(rt_ctx* c, int code, const char* fmt, ...);
int hip_fail(rt_ctx* c, hipError_t e, const char* what);
// Makes c->scratch hold at least elems floats (grow-only; waits for queued
// work before replacing a smaller one).
int ensure_scratch(rt_ctx* c, size_t elems);

// The split-K GEMM behind rt_gemm_splitk and rt_gemm_splitk_static: argument
// checks, then the launches with the partial planes at part (slices·M·N, then
// slices·N column-sum rows) and, for a half TN product with column sums, the
// column-sum shares at cs_scratch (cs_elems floats; 0 for none).
int splitk_check(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, const rt_buf* out, size_t slices,
                 const rt_buf* colsum, size_t* M, size_t* N, size_t* K);
int splitk_run(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* out, size_t slices,
               rt_buf* colsum, size_t M, size_t N, size_t K, float* part, float* cs_scratch, size_t cs_elems);
// noalloc.hip: the device address of the static scratch array on the current
// device, and its size in floats.
hipError_t static_scratch_address(float** out);
size_t static_scratch_floats();

// HIP's current device is per thread: every entry point makes the context's
// device current first, so a context works from any thread and next to a
// context on another device.
inline void bind_device(const rt_ctx* c) {
  int d = -1;
  if (hipGetDevice(&d) != hipSuccess || d != c->device) (void)hipSetDevice(c->device);
}

#define CHECK_CTX(c)                           \
  do {                                         \
    if ((c) == nullptr) return RT_ERR_INVALID; \
    ::rt::bind_device(c);                      \
  } while (0)

#define HIP_TRY(c, expr, what)                                  \
  do {                                                          \
    hipError_t _e = (expr);                                     \
    if (_e != hipSuccess) return ::rt::hip_fail((c), _e, what); \
  } while (0)

// The events the kernel launches of the current profiled Launch scope carry
// (per thread; null when not profiling): the first kernel takes `start`, every
// kernel takes `stop`, so the pair spans the scope's kernels.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
  bool used = false;
};
extern thread_local LaunchEvents* g_launch_events;

// Every kernel of the library is launched through here.  While a profiled
// Launch scope is open the kernel's own dispatch carries its events
// (hipExtLaunchKernel timestamps the dispatch packet, the clock rocprofv3's
// kernel trace reads), so profiling adds no marker packets between kernels.
template <typename F, typename... Args>
inline void launch(F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t s, Args... args) {
  if (LaunchEvents* ev = g_launch_events) {
    hipExtLaunchKernelGGL(kernel, grid, block, shm, s, ev->used ? nullptr : ev->start, ev->stop, 0u, args...);
    ev->used = true;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shm, s, args...);
  }
}

// Labels the kernels launched in its scope for rt_profile_report when
// profiling is on.
class Launch {
 public:
  Launch(rt_ctx* c, const char* label);
  ~Launch();
  Launch(const Launch&) = delete;
  Launch& operator=(const Launch&) = delete;

 private:
  rt_ctx* c_;
  const char* label_;
  LaunchEvents ev_;
  LaunchEvents* prev_ = nullptr;
  bool on_ = false;
};

// ---------------------------------------------------------------- GEMM
struct GemmDesc {
  int layout = RT_NN;        // rt_layout
  int in_dtype = RT_F32;     // dtype of A and B
  int out_dtype = RT_F32;    // dtype of C (f32, or bf16 for half inputs)
  const void* A = nullptr;
  const void* B = nullptr;
  void* C = nullptr;
  int M = 0, N = 0, K = 0;
  int lda = 0, ldb = 0, ldc = 0;  // leading dimensions in elements
  int epi = RT_EPI_NONE;
  const float* bias = nullptr;    // [N] f32
  const void* mask = nullptr;     // [M, N], ld = ldc, dtype = mask_dtype
  int mask_dtype = RT_F32;
  float* colsum = nullptr;        // [N] f32 = 1ᵀ·B over this launch's K range
  int splits = 1;                 // K slices (blockIdx.z); >1 writes f32 partial planes
  long long split_stride = 0;     // elements between partial planes of C
  float* colsum_partials = nullptr;  // [splits, N] when splits > 1
  // Optional f32 scratch for the half GEMM's column sums: with room for
  // colsum_scratch_need(M, N, splits) floats, every M tile of the direct-to-LDS
  // kernel sums a share of the K stages and a second small launch adds the
  // shares in a fixed order (otherwise the first M tile sums all of K alone).
  float* cs_scratch = nullptr;
  size_t cs_scratch_elems = 0;
  // Launches whose column sums go through those shares: leave the shares,
  // [splits, gemm_cs_share_rows(d), N], in cs_scratch for the caller to add
  // (splitk_reduce_launch for a split launch, nonfinite_check_launch's share
  // jobs for a whole one) instead of a second launch that adds them into
  // colsum (colsum_partials when split).
  bool cs_shares_to_caller = false;
  // The caller guarantees that A and B may be read up to 1 KiB past their
  // last element (memory inside the same allocation): lets the half GEMM's
  // direct-to-LDS kernel take an N that is not a multiple of its tile.
  bool overread_ok = false;
  // Optional: set *nf_flag = 1 if any f32 result is not finite.  Honoured
  // only where gemm_checks_nonfinite(d) is true.
  int* nf_flag = nullptr;
  // Optional ReLU predicate bits, one per element of C: a bf16 bias+ReLU
  // launch writes them (relu_bits_out: bit set where the stored value is
  // > 0), a ReLU-mask launch reads them instead of `mask` (relu_bits), 1/16
  // of a bf16 mask's bytes.  Layout, in the direct epilogue's lane order:
  // rows 16R.. and columns 64G.. of C are the 32 dwords from 32·(R·N/64 +
  // G); byte b of dword j covers the 16x16 block of columns 64G + 16b, and
  // its low / high nibble lane 2j / 2j + 1, where lane L stands for row
  // 16R + L%16 and columns 4·(L/16) + q, q = 0..3 the nibble's bits.  A
  // launch that sets either pointer must satisfy gemm_relu_bits_ok(d)
  // (whole tiles, M % 16 == 0, N % 64 == 0); otherwise it fails rather than
  // ignore them.
  unsigned* relu_bits_out = nullptr;
  const unsigned* relu_bits = nullptr;
};
bool gemm_checks_nonfinite(const GemmDesc& d);
bool gemm_relu_bits_ok(const GemmDesc& d);
// Narrow f32 NN products (<= 16 columns) go to the output-layer kernel, in
// rt_gemm and in a one-slice split-K alike.
bool narrow_nn(const GemmDesc& d);
hipError_t narrow_nn_launch(hipStream_t s, const GemmDesc& d);
size_t colsum_scratch_need(int M, int N, int splits);
// Rows of column-sum shares per K slice that a cs_shares_to_caller launch of
// d leaves in cs_scratch (0: it writes colsum_partials itself).
int gemm_cs_share_rows(const GemmDesc& d);
// Kernel launches gemm_launch issues for d (1, or 2 with shared column sums).
int gemm_launch_count(const GemmDesc& d);

// Enqueues C (or its partial planes) on stream.  Shapes and pointers are
// validated by the caller.
hipError_t gemm_launch(hipStream_t s, const GemmDesc& d);
// The shapes an unsplit f32 NN / NT product of at most 64 rows runs on the
// skinny kernel (whole K per block, no partial planes) when its operands are
// float4-aligned: 16-column and 16-k blocks, K >= 128.
bool gemm_f32_skinny_shape(int M, int N, int K);
// Two independent GEMMs in one launch: d0 TN (any K slices) and d1 NT
// (whole K), f32, where both would run on 64x64 tiles.  gemm_pair_supported
// says whether gemm_pair_launch accepts the pair.
bool gemm_pair_supported(const GemmDesc& d0, const GemmDesc& d1);
hipError_t gemm_pair_launch(hipStream_t s, const GemmDesc& d0, const GemmDesc& d1);
// Sums `splits` f32 partial planes of [M, N] in slice order into C and applies
// the epilogue; also sums colsum partials [splits, N] into colsum if given.
// With cs_rows > 0 colsum_partials holds a split half GEMM's column-sum
// shares [splits, cs_rows, N] instead: each slice's rows are added in order
// from zero, then the slices in order (the bits of the GEMM's own shares
// launch followed by the plain reduction).
hipError_t splitk_reduce_launch(hipStream_t s, const float* partials, int splits, long long stride, int M,
                                int N, void* C, int out_dtype, int ldc, int epi, const float* bias,
                                const void* mask, int mask_dtype, const float* colsum_partials, float* colsum,
                                int cs_rows = 0);

// ---------------------------------------------------------------- row / column kernels
hipError_t colsum_launch(hipStream_t s, const void* src, int dtype, int rows, int cols, float* dst,
                         float* scratch, size_t scratch_elems);
size_t colsum_scratch_elems(int rows, int cols, int dtype);
hipError_t bias_add_launch(hipStream_t s, float* z, const float* b, int rows, int cols);
hipError_t relu_launch(hipStream_t s, const float* x, float* y, size_t n);
hipError_t relu_bwd_launch(hipStream_t s, const void* a, int a_dtype, float* delta, size_t n);
// delta_half (optional bf16 copy of δ) has row stride ld_half (0: cols).
hipError_t xent_launch(hipStream_t s, const float* logits, const uint32_t* labels, float* delta, void* delta_half,
                       float* loss_rows, int rows, int cols, float scale, int* err_flag, int ld_half = 0);
// Output layer z = A·W + b (f32, cols <= 16 classes, K a multiple of 128, A
// 16-byte aligned) fused with
// the softmax cross-entropy of xent_launch; labels == nullptr writes only z.
bool head_xent_supported(int K, int cols);
hipError_t head_xent_launch(hipStream_t s, const float* A, int K, const float* W, const float* bias,
                            const uint32_t* labels, float* logits, float* delta, float* loss_rows, int rows, int cols,
                            float scale, int* err_flag);
// out[r] = Tensor::argmax_rows of row r of z [rows, cols] (first max; a NaN in
// column 0 wins the row, later NaNs never do).
hipError_t argmax_launch(hipStream_t s, const float* z, uint32_t* out, int rows, int cols);
hipError_t convert_launch(hipStream_t s, const void* src, int src_dtype, void* dst, int dst_dtype, size_t n);
hipError_t fill_i32_launch(hipStream_t s, int* p, int v, size_t n);

// ---------------------------------------------------------------- optimizer
struct OptTensor {
  float* theta;       // f32 parameter (master copy under mixed precision)
  const float* grad;  // f32 gradient
  float* m;           // Adam first moment / SGD velocity (nullable for plain SGD)
  float* v;           // Adam second moment
  void* half_copy;    // optional bf16 copy of theta written after the update
  size_t n;
  // Deferred split-K reduction: when parts is set the gradient is the sum of
  // the n_parts planes parts[s * part_stride + i] in slice order (exactly what
  // splitk_reduce computes) and is also stored to grad_store[i].
  const float* parts = nullptr;
  int n_parts = 0;
  long long part_stride = 0;
  float* grad_store = nullptr;
  bool vec = false;  // set by optimizer_launch: float4 streams are aligned
};
struct OptParams {
  int kind = 0;  // 0 Adam, 1 SGD
  float lr = 0, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f, momentum = 0;
  float inv_c1 = 1, inv_c2 = 1;  // Adam bias corrections, 1/(1-β^t) in f32
  float grad_scale = 1;          // multiplies g first (1/loss_scale), exact for powers of two
  // If either flag is non-null and set, the update is skipped; the first
  // launch of a step may then count the skipped step in *skip_count (one
  // thread of block 0 adds 1).
  const int* skip_flag = nullptr;
  const int* skip_flag2 = nullptr;
  int* skip_count = nullptr;
  // If non-null, Adam's bias corrections come from the device step count
  // (*device_t + 1 = this update's t) instead of inv_c1 / inv_c2.
  const int* device_t = nullptr;
};
// Mixed-precision step prologue on state[0] = applied updates t, state[1] =
// overflow flag, state[2] = a step was issued, state[3] = label flag:
// t += (issued && !overflow && !label); issued = 1; overflow = 0.  One thread.
hipError_t step_begin_launch(hipStream_t s, int* state);
constexpr int kMaxOptTensors = 24;
hipError_t optimizer_launch(hipStream_t s, const OptTensor* ts, int nt, const OptParams& p);
// The update of ts fits one launch and moves no more than the last-level
// cache holds (so it takes the cached, not the streaming, path).
bool optimizer_fits_cache(const OptTensor* ts, int nt, const OptParams& p);
// An f32 TN GEMM (a weight gradient) and an optimizer update of other
// tensors in one launch: the GEMM gives the bits of its own launch, the
// update those of optimizer_launch.  For updates that fit the cache.
// With upd = {W, b} (gemm_opt_update_ok) the GEMM's tiles also update W and
// b from the dW (d.C) and db (d.colsum) they compute, as optimizer_launch
// would on those gradients.
bool gemm_opt_supported(const GemmDesc& d, const OptTensor* ts, int nt, const OptParams& p);
bool gemm_opt_update_ok(const GemmDesc& d, const OptTensor* wb, const OptParams& p);
hipError_t gemm_opt_launch(hipStream_t s, const GemmDesc& d, const OptTensor* ts, int nt, const OptParams& p,
                           const OptTensor* upd = nullptr);
// Two unsplit TN dW products, each with its {W, b} update done by its tiles
// (both gemm_opt_update_ok), and the update of ts, in one launch.
hipError_t gemm_opt_update2_launch(hipStream_t s, const GemmDesc& d0, const OptTensor* upd0, const GemmDesc& d1,
                                   const OptTensor* upd1, const OptTensor* ts, int nt, const OptParams& p);
// Column sums of a whole (unsplit) half GEMM left as shares: dst[j] = the
// rows src[t * n + j], t = 0 .. rows-1, added in order from zero (what the
// GEMM's own shares launch computes).
struct ShareJob {
  const float* src;
  float* dst;
  int rows, n;
};
constexpr int kMaxShareJobs = 32;
// Sets *flag = 1 if any of the n floats of any tensor is not finite; in the
// same launch, adds the column-sum shares of each job into its dst and flags
// a non-finite sum the same way.
hipError_t nonfinite_check_launch(hipStream_t s, const float* const* ptrs, const size_t* ns, int nt, int* flag,
                                  const ShareJob* jobs = nullptr, int njobs = 0);

// ---------------------------------------------------------------- tensor ops (tensor_ops.hip)
hipError_t unary_launch(hipStream_t s, int op, float k, const float* x, float* y, long long n);
hipError_t unary_vjp_launch(hipStream_t s, int op, float k, const float* g, const float* x, const float* y, float* dx,
                            long long n);
// out[l] = a[ia] op b[ib] over the output shape (rank 1..4); sa / sb are the
// operands' strides in the output index space (0 on broadcast axes).
hipError_t binary_launch(hipStream_t s, int op, const float* a, const long long* sa, const float* b,
                         const long long* sb, float* out, const long long* shape, int rank);
// tshape: same rank as gshape, each axis equal to g's or 1.
hipError_t reduce_to_launch(hipStream_t s, const float* g, const long long* gshape, int grank, float* out,
                            const long long* tshape);
size_t sum_scratch_elems(long long n);
hipError_t sum_all_launch(hipStream_t s, const float* x, long long n, float div, float* out, float* scratch);
hipError_t scalar_fill_launch(hipStream_t s, const float* scalar, float div, const float* x, float* out, long long n);
hipError_t softmax_rows_launch(hipStream_t s, const float* z, float* y, long long rows, long long cols);
hipError_t softmax_rows_vjp_launch(hipStream_t s, const float* sm, const float* g, float* dx, long long rows,
                                   long long cols);
// dir = (P − Y)·dir_scale (1: the plain direction).
hipError_t xent_logits_launch(hipStream_t s, const float* z, const float* y, float* dir, long long rows,
                              long long cols, float div, float* out, float* scratch, size_t scratch_elems,
                              float dir_scale);
hipError_t loss_terms_launch(hipStream_t s, int kind, const float* p, const float* y, float* term, float* dir,
                             long long n);

// f32 powi as rtensor's Adam computes β^t (square-and-multiply).
float powi_f32(float a, int b);

}  // namespace rt
