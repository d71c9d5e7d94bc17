// Device side of the multi-tensor optimizer: the batch one launch carries
// and the per-block update.  optimizer_kernel runs it alone; a GEMM launch
// can run optimizer blocks next to its tiles (gemm_f32.hip).  The arithmetic
// follows the CPU expression order and is never contracted into FMAs, in
// whatever file it is compiled.
#pragma once

#include <hip/hip_runtime.h>

#include "rt_internal.h"

namespace rt_opt {

constexpr int kThreads = 256;
constexpr int kPerThread = 4;
constexpr int kPerBlock = kThreads * kPerThread;

struct OptBatch {
  rt::OptTensor t[rt::kMaxOptTensors];
  int block_start[rt::kMaxOptTensors + 1];
  int nt;
  rt::OptParams p;
};

// Fills b for the tensors ts[0, nt) (float4 streams where aligned); *blocks
// = the launch's workgroups, *bytes = the HBM bytes the update moves.
hipError_t make_batch(const rt::OptTensor* ts, int nt, const rt::OptParams& p, OptBatch& b, long long* blocks,
                      double* bytes);

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));

__device__ inline unsigned short f32_to_bf16_rne(float x) {
  unsigned int u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

__device__ inline float powi_dev(float a, int b) {
#pragma clang fp contract(off)
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return r;
}

struct Coef {
  float inv_c1, inv_c2;
};

// Whether this step's update is skipped (a non-finite gradient or a label
// past the classes).
__device__ inline bool skipped(const rt::OptParams& P) {
  return (P.skip_flag != nullptr && *P.skip_flag != 0) || (P.skip_flag2 != nullptr && *P.skip_flag2 != 0);
}

// Adam's bias corrections of this update: from the host, or from the device
// step count (*device_t + 1 = this update's t).
__device__ inline Coef coef(const rt::OptParams& P) {
#pragma clang fp contract(off)
  Coef c{P.inv_c1, P.inv_c2};
  if (P.device_t != nullptr) {
    const int t = *P.device_t + 1;
    c.inv_c1 = 1.0f / (1.0f - powi_dev(P.beta1, t));
    c.inv_c2 = 1.0f / (1.0f - powi_dev(P.beta2, t));
  }
  return c;
}

// One element's update, the CPU expression order (optim.rs:88-95, 187-195).
// m / v are read only where the method uses them.
__device__ inline void update(const rt::OptParams& P, Coef c, float graw, float& th, float* m, float* v) {
#pragma clang fp contract(off)
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
__device__ inline void optimizer_block(const OptBatch& b, int blk) {
#pragma clang fp contract(off)
  if (skipped(b.p)) {
    if (b.p.skip_count != nullptr && blk == 0 && threadIdx.x == 0) *b.p.skip_count += 1;
    return;
  }
  const Coef c = coef(b.p);
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

}  // namespace rt_opt
