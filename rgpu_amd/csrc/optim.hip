// Fused optimizer: every parameter tensor of the model updated by ONE launch.
// A tensor whose gradient is still split into K-slice partial planes is
// reduced here (fixed slice order) instead of by a separate launch.
//
// rtensor's GPU plan issues one ADAM dispatch per tensor (mod.rs:1460-1467,
// kernels.rs:205-224) and has no GPU SGD; here Adam and SGD share a single
// multi-tensor kernel whose workgroups are assigned to tensors by a prefix
// table carried in the kernel arguments.  It is HBM-bound: Adam moves 28
// bytes per parameter (read θ, g, m, v; write θ, m, v).
//
// Arithmetic follows the CPU Adam::step / Sgd::step expression by expression
// (optim.rs:88-95, 187-195), compiled with -ffp-contract=off and correctly
// rounded division and square root, so identical inputs give identical bits:
//   m = m·β1 + g·(1−β1);  v = v·β2 + (g·g)·(1−β2);
//   θ = θ − ((m·(1/c1)) / (√(v·(1/c2)) + ε))·lr
// Under loss scaling the gradient is first multiplied by 1/scale (a power of
// two, exact) and the whole update is skipped when the overflow flag is set;
// a training plan also skips it when its loss saw a label >= the classes.

#include <algorithm>

#include "optim_dev.h"
#include "rt_internal.h"

namespace {

using rt_opt::kPerBlock;
using rt_opt::kThreads;
using rt_opt::OptBatch;
// MI355X's last-level (Infinity) cache: 256 MB.
constexpr double kLastLevelCacheBytes = 256.0 * 1024 * 1024;

// STREAM: the launch moves more than the last-level cache holds, so its
// float4 streams are read and written non-temporally (measured: the 138
// M-parameter Adam launch ~50 us faster; a launch that fits is slower that
// way, its state no longer cached for the next step).
template <bool STREAM>
__global__ __launch_bounds__(kThreads) void optimizer_kernel(OptBatch b) {
  rt_opt::optimizer_block<STREAM>(b, blockIdx.x);
}

struct NonFiniteArgs {
  const float* p[rt::kMaxOptTensors];
  long long n[rt::kMaxOptTensors];
  int nt;
  int* flag;
  rt::ShareJob job[rt::kMaxShareJobs];
  int job_start[rt::kMaxShareJobs + 1];  // first block of each job, after the check blocks
  int njobs;
  int check_blocks;
};

// Blocks [0, check_blocks) grid-stride over every tensor; any lane that sees
// a NaN/Inf stores 1.  The blocks after them take 256 columns of a share job
// each: the job's rows added in order from zero, 8 loads in flight.
__global__ __launch_bounds__(256) void nonfinite_kernel(NonFiniteArgs a) {
  bool bad = false;
  if ((int)blockIdx.x >= a.check_blocks) {
    const int b = blockIdx.x - a.check_blocks;
    int j = 0;
    while (j + 1 < a.njobs && a.job_start[j + 1] <= b) ++j;
    const rt::ShareJob& J = a.job[j];
    const int col = (b - a.job_start[j]) * 256 + threadIdx.x;
    if (col >= J.n) return;
    const float* q = J.src + col;
    float v = 0.0f;
    int t = 0;
    for (; t + 8 <= J.rows; t += 8) {
      float w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = q[(long long)(t + u) * J.n];
#pragma unroll
      for (int u = 0; u < 8; ++u) v += w[u];
    }
    for (; t < J.rows; ++t) v += q[(long long)t * J.n];
    J.dst[col] = v;
    if (!(fabsf(v) <= 3.402823466e38f)) *a.flag = 1;
    return;
  }
  for (int t = 0; t < a.nt; ++t) {
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < a.n[t]; i += (long long)a.check_blocks * 256) {
      const float v = a.p[t][i];
      bad |= !(fabsf(v) <= 3.402823466e38f);
    }
  }
  if (bad) *a.flag = 1;
}

__global__ void step_begin_kernel(int* state) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    if (state[2] != 0 && state[1] == 0 && state[3] == 0) state[0] += 1;
    state[2] = 1;
    state[1] = 0;
  }
}

}  // namespace

namespace rt_opt {

hipError_t make_batch(const rt::OptTensor* ts, int nt, const rt::OptParams& p, OptBatch& b, long long* blocks,
                      double* bytes) {
  if (nt < 0 || nt > rt::kMaxOptTensors) return hipErrorInvalidValue;
  b.nt = nt;
  b.p = p;
  long long nb = 0;
  double by = 0.0;
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  for (int i = 0; i < nt; ++i) {
    b.t[i] = ts[i];
    const rt::OptTensor& T = ts[i];
    // float4 streams: every base 16-byte aligned (the bf16 copy 8-byte) and
    // the partial planes 4-float strided.
    b.t[i].vec = al16(T.theta) && al16(T.grad) && (T.m == nullptr || al16(T.m)) && (T.v == nullptr || al16(T.v)) &&
                 (T.half_copy == nullptr || (reinterpret_cast<uintptr_t>(T.half_copy) & 7) == 0) &&
                 (T.parts == nullptr || (al16(T.parts) && al16(T.grad_store) && T.part_stride % 4 == 0));
    b.block_start[i] = (int)nb;
    nb += (long long)((ts[i].n + kPerBlock - 1) / kPerBlock);
    const int streams = 2 + (T.m ? 2 : 0) + (p.kind == 0 ? 2 : 0) + (T.parts ? T.n_parts + 1 : 1);
    by += (double)T.n * (4.0 * streams + (T.half_copy ? 2.0 : 0.0));
  }
  b.block_start[nt] = (int)nb;
  if (nb > 0x7fffffffLL) return hipErrorInvalidValue;
  *blocks = nb;
  *bytes = by;
  return hipSuccess;
}

}  // namespace rt_opt

namespace rt {

hipError_t step_begin_launch(hipStream_t s, int* state) {
  rt::launch(step_begin_kernel, dim3(1), dim3(64), 0, s, state);
  return hipGetLastError();
}

float powi_f32(float a, int b) {
  // Square-and-multiply from the least significant exponent bit, as f32::powi
  // evaluates β^t for Adam's bias correction (optim.rs:165-166).
  bool recip = b < 0;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

hipError_t optimizer_launch(hipStream_t s, const OptTensor* ts, int nt, const OptParams& p) {
  if (nt <= 0) return hipSuccess;
  OptBatch b{};
  long long blocks = 0;
  double bytes = 0.0;
  hipError_t e = rt_opt::make_batch(ts, nt, p, b, &blocks, &bytes);
  if (e != hipSuccess || blocks == 0) return e;
  if (bytes > kLastLevelCacheBytes)
    rt::launch(optimizer_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s, b);
  else
    rt::launch(optimizer_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s, b);
  return hipGetLastError();
}

bool optimizer_fits_cache(const OptTensor* ts, int nt, const OptParams& p) {
  OptBatch b{};
  long long blocks = 0;
  double bytes = 0.0;
  return nt <= kMaxOptTensors && rt_opt::make_batch(ts, nt, p, b, &blocks, &bytes) == hipSuccess &&
         bytes <= kLastLevelCacheBytes;
}

hipError_t nonfinite_check_launch(hipStream_t s, const float* const* ptrs, const size_t* ns, int nt, int* flag,
                                  const ShareJob* jobs, int njobs) {
  if (nt <= 0 && njobs <= 0) return hipSuccess;
  if (nt > kMaxOptTensors || njobs > kMaxShareJobs) return hipErrorInvalidValue;
  NonFiniteArgs a{};
  long long total = 0;
  for (int i = 0; i < nt; ++i) {
    a.p[i] = ptrs[i];
    a.n[i] = (long long)ns[i];
    total += a.n[i];
  }
  a.nt = nt < 0 ? 0 : nt;
  a.flag = flag;
  a.check_blocks = total > 0 ? (int)std::min<long long>((total + 255) / 256, 2048) : 0;
  int blocks = a.check_blocks;
  a.njobs = njobs < 0 ? 0 : njobs;
  for (int j = 0; j < a.njobs; ++j) {
    a.job[j] = jobs[j];
    a.job_start[j] = blocks - a.check_blocks;
    blocks += (jobs[j].n + 255) / 256;
  }
  a.job_start[a.njobs] = blocks - a.check_blocks;
  if (blocks == 0) return hipSuccess;
  rt::launch(nonfinite_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace rt
