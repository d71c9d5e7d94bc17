// Fused optimizer: every parameter tensor of the model updated by ONE launch.
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
// two, exact) and the whole update is skipped when the overflow flag is set.

#include <algorithm>

#include "rt_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;
constexpr int kPerBlock = kThreads * kPerThread;

struct OptBatch {
  rt::OptTensor t[rt::kMaxOptTensors];
  int block_start[rt::kMaxOptTensors + 1];
  int nt;
  rt::OptParams p;
};

__device__ inline unsigned short f32_to_bf16_rne(float x) {
  unsigned int u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

__device__ inline float powi_dev(float a, int b) {
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return r;
}

__global__ __launch_bounds__(kThreads) void optimizer_kernel(OptBatch b) {
  if (b.p.skip_flag != nullptr && *b.p.skip_flag != 0) return;
  float inv_c1 = b.p.inv_c1, inv_c2 = b.p.inv_c2;
  if (b.p.device_t != nullptr) {
    const int t = *b.p.device_t + 1;
    inv_c1 = 1.0f / (1.0f - powi_dev(b.p.beta1, t));
    inv_c2 = 1.0f / (1.0f - powi_dev(b.p.beta2, t));
  }
  const int blk = blockIdx.x;
  int ti = 0;
  while (ti + 1 < b.nt && b.block_start[ti + 1] <= blk) ++ti;
  const rt::OptTensor& T = b.t[ti];
  const long long base = (long long)(blk - b.block_start[ti]) * kPerBlock + threadIdx.x;
  const rt::OptParams& P = b.p;
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const long long i = base + (long long)e * kThreads;
    if (i >= (long long)T.n) break;
    const float g = T.grad[i] * P.grad_scale;
    float th = T.theta[i];
    if (P.kind == 0) {
      const float mi = T.m[i] * P.beta1 + g * (1.0f - P.beta1);
      const float vi = T.v[i] * P.beta2 + (g * g) * (1.0f - P.beta2);
      T.m[i] = mi;
      T.v[i] = vi;
      const float m_hat = mi * inv_c1;
      const float v_hat = vi * inv_c2;
      th = th - (m_hat / (sqrtf(v_hat) + P.eps)) * P.lr;
    } else if (P.momentum == 0.0f) {
      th = th - g * P.lr;
    } else {
      const float vel = T.m[i] * P.momentum + g * P.lr;
      T.m[i] = vel;
      th = th - vel;
    }
    T.theta[i] = th;
    if (T.half_copy != nullptr) static_cast<unsigned short*>(T.half_copy)[i] = f32_to_bf16_rne(th);
  }
}

struct NonFiniteArgs {
  const float* p[rt::kMaxOptTensors];
  long long n[rt::kMaxOptTensors];
  int nt;
  int* flag;
};

// Grid-stride over every tensor; any lane that sees a NaN/Inf stores 1.
__global__ __launch_bounds__(256) void nonfinite_kernel(NonFiniteArgs a) {
  bool bad = false;
  for (int t = 0; t < a.nt; ++t) {
    for (long long i = blockIdx.x * 256LL + threadIdx.x; i < a.n[t]; i += (long long)gridDim.x * 256) {
      const float v = a.p[t][i];
      bad |= !(fabsf(v) <= 3.402823466e38f);
    }
  }
  if (bad) *a.flag = 1;
}

__global__ void step_begin_kernel(int* state) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    if (state[2] != 0 && state[1] == 0) state[0] += 1;
    state[2] = 1;
    state[1] = 0;
  }
}

}  // namespace

namespace rt {

hipError_t step_begin_launch(hipStream_t s, int* state) {
  hipLaunchKernelGGL(step_begin_kernel, dim3(1), dim3(64), 0, s, state);
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
  if (nt > kMaxOptTensors) return hipErrorInvalidValue;
  OptBatch b{};
  b.nt = nt;
  b.p = p;
  long long blocks = 0;
  for (int i = 0; i < nt; ++i) {
    b.t[i] = ts[i];
    b.block_start[i] = (int)blocks;
    blocks += (long long)((ts[i].n + kPerBlock - 1) / kPerBlock);
  }
  b.block_start[nt] = (int)blocks;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(optimizer_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, s, b);
  return hipGetLastError();
}

hipError_t nonfinite_check_launch(hipStream_t s, const float* const* ptrs, const size_t* ns, int nt, int* flag) {
  if (nt <= 0) return hipSuccess;
  if (nt > kMaxOptTensors) return hipErrorInvalidValue;
  NonFiniteArgs a{};
  long long total = 0;
  for (int i = 0; i < nt; ++i) {
    a.p[i] = ptrs[i];
    a.n[i] = (long long)ns[i];
    total += a.n[i];
  }
  a.nt = nt;
  a.flag = flag;
  int blocks = (int)std::max<long long>(1, std::min<long long>((total + 255) / 256, 2048));
  hipLaunchKernelGGL(nonfinite_kernel, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace rt
