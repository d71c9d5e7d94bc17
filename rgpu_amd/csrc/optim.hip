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

#include "rt_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;
constexpr int kPerBlock = kThreads * kPerThread;
// MI355X's last-level (Infinity) cache: 256 MB.
constexpr double kLastLevelCacheBytes = 256.0 * 1024 * 1024;

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

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));

struct Coef {
  float inv_c1, inv_c2;
};

// One element's update, the CPU expression order (optim.rs:88-95, 187-195).
// m / v are read only where the method uses them.
__device__ inline void update(const rt::OptParams& P, Coef c, float graw, float& th, float* m, float* v) {
  const float g = graw * P.grad_scale;
  if (P.kind == 0) {
    const float mi = *m * P.beta1 + g * (1.0f - P.beta1);
    const float vi = *v * P.beta2 + (g * g) * (1.0f - P.beta2);
    *m = mi;
    *v = vi;
    const float m_hat = mi * c.inv_c1;
    const float v_hat = vi * c.inv_c2;
    th = th - (m_hat / (sqrtf(v_hat) + P.eps)) * P.lr;
  } else if (P.momentum == 0.0f) {
    th = th - g * P.lr;
  } else {
    const float vel = *m * P.momentum + g * P.lr;
    *m = vel;
    th = th - vel;
  }
}

// Each thread owns 4 consecutive elements: one float4 of every stream when
// the tensor allows it (T.vec), else four scalars.  STREAM: the launch moves
// more than the last-level cache holds, so its float4 streams are read and
// written non-temporally (measured: the 138 M-parameter Adam launch ~50 us
// faster; a launch that fits is slower that way, its state no longer cached
// for the next step).
template <bool STREAM>
__global__ __launch_bounds__(kThreads) void optimizer_kernel(OptBatch b) {
  if ((b.p.skip_flag != nullptr && *b.p.skip_flag != 0) || (b.p.skip_flag2 != nullptr && *b.p.skip_flag2 != 0)) {
    if (b.p.skip_count != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *b.p.skip_count += 1;
    return;
  }
  Coef c{b.p.inv_c1, b.p.inv_c2};
  if (b.p.device_t != nullptr) {
    const int t = *b.p.device_t + 1;
    c.inv_c1 = 1.0f / (1.0f - powi_dev(b.p.beta1, t));
    c.inv_c2 = 1.0f / (1.0f - powi_dev(b.p.beta2, t));
  }
  const int blk = blockIdx.x;
  int ti = 0;
  while (ti + 1 < b.nt && b.block_start[ti + 1] <= blk) ++ti;
  const rt::OptTensor& T = b.t[ti];
  const rt::OptParams& P = b.p;
  const long long i0 = (long long)(blk - b.block_start[ti]) * kPerBlock + (long long)kPerThread * threadIdx.x;
  if (i0 >= (long long)T.n) return;
  const bool adam = P.kind == 0, has_m = T.m != nullptr;

  if (T.vec && i0 + 4 <= (long long)T.n) {
    auto ld = [](const float* q) {
      if constexpr (STREAM) return __builtin_nontemporal_load(reinterpret_cast<const f4*>(q));
      else return *reinterpret_cast<const f4*>(q);
    };
    auto st = [](float* q, f4 x) {
      if constexpr (STREAM) __builtin_nontemporal_store(x, reinterpret_cast<f4*>(q));
      else *reinterpret_cast<f4*>(q) = x;
    };
    f4 g;
    if (T.parts != nullptr) {
      g = ld(T.parts + i0);
#pragma unroll 4
      for (int s = 1; s < T.n_parts; ++s) g = g + ld(T.parts + (long long)s * T.part_stride + i0);
      st(T.grad_store + i0, g);
    } else {
      g = ld(T.grad + i0);
    }
    f4 th = ld(T.theta + i0);
    f4 m = has_m ? ld(T.m + i0) : f4{0, 0, 0, 0};
    f4 v = adam ? ld(T.v + i0) : f4{0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float te = th[e], me = m[e], ve = v[e];
      update(P, c, g[e], te, &me, &ve);
      th[e] = te;
      m[e] = me;
      v[e] = ve;
    }
    st(T.theta + i0, th);
    if (has_m) st(T.m + i0, m);
    if (adam) st(T.v + i0, v);
    if (T.half_copy != nullptr) {  // 8-byte aligned (T.vec)
      u2 w;
      w[0] = (unsigned)f32_to_bf16_rne(th[0]) | ((unsigned)f32_to_bf16_rne(th[1]) << 16);
      w[1] = (unsigned)f32_to_bf16_rne(th[2]) | ((unsigned)f32_to_bf16_rne(th[3]) << 16);
      u2* h = reinterpret_cast<u2*>(static_cast<unsigned short*>(T.half_copy) + i0);
      if constexpr (STREAM) __builtin_nontemporal_store(w, h);
      else *h = w;
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < kPerThread; ++e) {
    const long long i = i0 + e;
    if (i >= (long long)T.n) break;
    float graw;
    if (T.parts != nullptr) {
      graw = T.parts[i];
      for (int s = 1; s < T.n_parts; ++s) graw = graw + T.parts[(long long)s * T.part_stride + i];
      T.grad_store[i] = graw;
    } else {
      graw = T.grad[i];
    }
    float th = T.theta[i];
    float mi = has_m ? T.m[i] : 0.0f, vi = adam ? T.v[i] : 0.0f;
    update(P, c, graw, th, &mi, &vi);
    if (has_m) T.m[i] = mi;
    if (adam) T.v[i] = vi;
    T.theta[i] = th;
    if (T.half_copy != nullptr) static_cast<unsigned short*>(T.half_copy)[i] = f32_to_bf16_rne(th);
  }
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
  if (nt > kMaxOptTensors) return hipErrorInvalidValue;
  OptBatch b{};
  b.nt = nt;
  b.p = p;
  long long blocks = 0;
  double bytes = 0.0;  // HBM bytes the launch moves
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  for (int i = 0; i < nt; ++i) {
    b.t[i] = ts[i];
    const OptTensor& T = ts[i];
    // float4 streams: every base 16-byte aligned (the bf16 copy 8-byte) and
    // the partial planes 4-float strided.
    b.t[i].vec = al16(T.theta) && al16(T.grad) && (T.m == nullptr || al16(T.m)) && (T.v == nullptr || al16(T.v)) &&
                 (T.half_copy == nullptr || (reinterpret_cast<uintptr_t>(T.half_copy) & 7) == 0) &&
                 (T.parts == nullptr || (al16(T.parts) && al16(T.grad_store) && T.part_stride % 4 == 0));
    b.block_start[i] = (int)blocks;
    blocks += (long long)((ts[i].n + kPerBlock - 1) / kPerBlock);
    const int streams = 2 + (T.m ? 2 : 0) + (p.kind == 0 ? 2 : 0) + (T.parts ? T.n_parts + 1 : 1);
    bytes += (double)T.n * (4.0 * streams + (T.half_copy ? 2.0 : 0.0));
  }
  b.block_start[nt] = (int)blocks;
  if (blocks == 0) return hipSuccess;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  if (bytes > kLastLevelCacheBytes)
    rt::launch(optimizer_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s, b);
  else
    rt::launch(optimizer_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s, b);
  return hipGetLastError();
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
