// Device versions of the Tensor operations rtensor's tape calls (ops.rs,
// tensor.rs, losses.rs), so that any Sequential model -- not only the fixed
// ReLU MLP plan -- can train on the GPU.  All HBM- or latency-bound.
// Built with -ffp-contract=off and every expression in the reference's
// order, so results differ from the CPU path only where a transcendental
// (exp, log, tanh) differs in its last bits, or where a scalar reduction
// (sum_all, losses) adds in a different order.
//   unary ops and their VJPs      ops.rs:132-227
//   broadcast binary ops          tensor.rs:183-246
//   reduce_to                     tensor.rs:399-438 (per output element, source order: exact)
//   sum / mean of all elements    tensor.rs:279-286 (fixed-order two-stage tree)
//   softmax_rows and its VJP      tensor.rs:455-472, ops.rs:291-309 (one thread per row, sequential)
//   mae / softmax-xent / bce      losses.rs:46-53, 99-115, 143-162

#include <algorithm>

#include "rt_internal.h"

namespace {

constexpr int kMaxRank = 4;

struct Shape4 {
  long long n[kMaxRank];   // output shape, right-aligned, leading 1s
  long long sa[kMaxRank];  // strides of operand a in the output index space (0 on broadcast axes)
  long long sb[kMaxRank];
};

__device__ inline float unary_fwd(int op, float k, float v) {
  switch (op) {
    case RT_U_SCALE: return v * k;
    case RT_U_OFFSET: return v + k;
    case RT_U_NEG: return v * -1.0f;
    case RT_U_SQUARE: return v * v;
    case RT_U_SQRT: return sqrtf(v);
    case RT_U_EXP: return expf(v);
    case RT_U_LN: return logf(fmaxf(v, 1e-12f));
    case RT_U_RELU: return fmaxf(v, 0.0f);
    case RT_U_LEAKY_RELU: return v > 0.0f ? v : k * v;
    case RT_U_SIGMOID: return 1.0f / (1.0f + expf(-v));
    case RT_U_TANH: return tanhf(v);
  }
  return __uint_as_float(0x7fc00000u);
}

// dx from the upstream gradient g, the input x and the output y (ops.rs VJPs).
__device__ inline float unary_vjp(int op, float k, float g, float x, float y) {
  switch (op) {
    case RT_U_SCALE: return g * k;
    case RT_U_OFFSET: return g;
    case RT_U_NEG: return g * -1.0f;
    case RT_U_SQUARE: return (g * x) * 2.0f;
    case RT_U_SQRT: return g / (y * 2.0f);
    case RT_U_EXP: return g * y;
    case RT_U_LN: return g / x;
    case RT_U_RELU: return g * (x > 0.0f ? 1.0f : 0.0f);
    case RT_U_LEAKY_RELU: return g * (x > 0.0f ? 1.0f : k);
    case RT_U_SIGMOID: return g * (y * (1.0f - y));
    case RT_U_TANH: return g * (1.0f - y * y);
  }
  return __uint_as_float(0x7fc00000u);
}

__global__ __launch_bounds__(256) void unary_kernel(int op, float k, const float* __restrict__ x, float* __restrict__ y,
                                                    long long n) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    y[i] = unary_fwd(op, k, x[i]);
}

__global__ __launch_bounds__(256) void unary_vjp_kernel(int op, float k, const float* __restrict__ g,
                                                        const float* __restrict__ x, const float* __restrict__ y,
                                                        float* __restrict__ dx, long long n) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    dx[i] = unary_vjp(op, k, g[i], x ? x[i] : 0.0f, y ? y[i] : 0.0f);
}

__device__ inline float binary_op(int op, float a, float b) {
  switch (op) {
    case RT_B_ADD: return a + b;
    case RT_B_SUB: return a - b;
    case RT_B_MUL: return a * b;
    case RT_B_DIV: return a / b;
  }
  return __uint_as_float(0x7fc00000u);
}

// R = rank after the host merged contiguous axes; I = index type (32-bit
// when the output has fewer than 2^31 elements).  R == 1 with unit strides
// is the same-shape case.
template <int R, typename I>
__global__ __launch_bounds__(256) void binary_kernel(int op, const float* __restrict__ a, const float* __restrict__ b,
                                                     float* __restrict__ out, Shape4 s, I n) {
  I nn[R], sa[R], sb[R];
#pragma unroll
  for (int ax = 0; ax < R; ++ax) {
    nn[ax] = (I)s.n[kMaxRank - R + ax];
    sa[ax] = (I)s.sa[kMaxRank - R + ax];
    sb[ax] = (I)s.sb[kMaxRank - R + ax];
  }
  for (I l = (I)blockIdx.x * 256 + (I)threadIdx.x; l < n; l += (I)gridDim.x * 256) {
    I rem = l, ia = 0, ib = 0;
#pragma unroll
    for (int ax = R - 1; ax > 0; --ax) {
      const I idx = rem % nn[ax];
      rem /= nn[ax];
      ia += idx * sa[ax];
      ib += idx * sb[ax];
    }
    ia += rem * sa[0];
    ib += rem * sb[0];
    out[l] = binary_op(op, a[ia], b[ib]);
  }
}

// reduce_to: out[t] = sum of g over the source elements that map to t, added
// in increasing source index (what every reference path does).  One thread
// per output element; the kept axes give the source base, the reduced axes
// (padded to four with extent 1) are walked by nested loops in row-major
// order.
struct ReduceArgs {
  long long keep_n[kMaxRank], keep_s[kMaxRank];  // output index -> source base
  long long red_n[kMaxRank], red_s[kMaxRank];    // reduced axes, outermost first
  int n_keep;
  long long n_out;
};

__global__ __launch_bounds__(256) void reduce_to_kernel(const float* __restrict__ g, float* __restrict__ out,
                                                        ReduceArgs r) {
  for (long long t = blockIdx.x * 256LL + threadIdx.x; t < r.n_out; t += (long long)gridDim.x * 256) {
    long long rem = t, base = 0;
    for (int ax = r.n_keep - 1; ax >= 0; --ax) {
      base += (rem % r.keep_n[ax]) * r.keep_s[ax];
      rem /= r.keep_n[ax];
    }
    // The adds form one dependent chain.  Loads go out in batches of kBatch,
    // the next batch issued before the current one is added, so the chain
    // rarely waits on memory.
    constexpr int kBatch = 32;
    const long long n3 = r.red_n[3], s3 = r.red_s[3];
    float acc = 0.0f;
    for (long long i0 = 0; i0 < r.red_n[0]; ++i0)
      for (long long i1 = 0; i1 < r.red_n[1]; ++i1)
        for (long long i2 = 0; i2 < r.red_n[2]; ++i2) {
          const float* p = g + base + i0 * r.red_s[0] + i1 * r.red_s[1] + i2 * r.red_s[2];
          long long i3 = 0;
          if (n3 >= kBatch) {
            float cur[kBatch], nxt[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) cur[u] = p[u * s3];
            for (i3 = kBatch; i3 + kBatch <= n3; i3 += kBatch) {
#pragma unroll
              for (int u = 0; u < kBatch; ++u) nxt[u] = p[(i3 + u) * s3];
#pragma unroll
              for (int u = 0; u < kBatch; ++u) acc += cur[u];
#pragma unroll
              for (int u = 0; u < kBatch; ++u) cur[u] = nxt[u];
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) acc += cur[u];
          }
          for (; i3 < n3; ++i3) acc += p[i3 * s3];
        }
    out[t] = acc;
  }
}

// Fixed-order two-stage sum of n floats: block b adds its 256 x chunk
// elements (each thread strided, then a shared-memory tree); stage 2 adds
// the block sums in order and divides by `div`.
// With a single block (n <= 65536) stage 1 also finishes the sum: out[0] =
// (0 + block sum) / div, the value stage 2 would produce from one part.
__global__ __launch_bounds__(256) void sum_stage1(const float* __restrict__ x, long long n, long long chunk,
                                                  float* __restrict__ part, float div, float* __restrict__ out) {
  __shared__ float sh[256];
  const long long b0 = blockIdx.x * chunk, b1 = min(n, b0 + chunk);
  float acc = 0.0f;
  for (long long i = b0 + threadIdx.x; i < b1; i += 256) acc += x[i];
  sh[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (gridDim.x == 1) out[0] = (0.0f + sh[0]) / div;
    else part[blockIdx.x] = sh[0];
  }
}

__global__ void sum_stage2(const float* __restrict__ part, int parts, float div, float* __restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  float acc = 0.0f;
  for (int i = 0; i < parts; ++i) acc += part[i];
  out[0] = acc / div;
}

// out[i] = (s[0] / div) * (x ? x[i] : 1): the VJPs of sum / mean (Tensor::full)
// and the "scale by g / n" of the losses.
__global__ __launch_bounds__(256) void scalar_fill_kernel(const float* __restrict__ s, float div,
                                                          const float* __restrict__ x, float* __restrict__ out,
                                                          long long n) {
  const float v = s[0] / div;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    out[i] = x ? x[i] * v : v;
}

// tensor.rs:455-472: max, exp and a sequential sum, then divide; one thread per row.
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ z, float* __restrict__ y,
                                                           long long rows, long long cols) {
  const long long i = blockIdx.x * 256LL + threadIdx.x;
  if (i >= rows) return;
  const float* row = z + i * cols;
  float* dst = y + i * cols;
  float mx = -INFINITY;
  for (long long j = 0; j < cols; ++j) mx = fmaxf(mx, row[j]);
  float sum = 0.0f;
  for (long long j = 0; j < cols; ++j) {
    const float e = expf(row[j] - mx);
    dst[j] = e;
    sum += e;
  }
  for (long long j = 0; j < cols; ++j) dst[j] = dst[j] / sum;
}

// ops.rs:291-309: dx = s ⊙ (g − Σ_j g_j s_j), per row, sequential dot.
__global__ __launch_bounds__(256) void softmax_rows_vjp_kernel(const float* __restrict__ s, const float* __restrict__ g,
                                                               float* __restrict__ dx, long long rows, long long cols) {
  const long long i = blockIdx.x * 256LL + threadIdx.x;
  if (i >= rows) return;
  const float* sr = s + i * cols;
  const float* gr = g + i * cols;
  float dot = 0.0f;
  for (long long j = 0; j < cols; ++j) dot += gr[j] * sr[j];
  for (long long j = 0; j < cols; ++j) dx[i * cols + j] = sr[j] * (gr[j] - dot);
}

// Per-element loss terms (summed by the two-stage sum) and the unscaled
// gradient directions (scaled by g / n with scalar_fill_kernel).
__global__ __launch_bounds__(256) void loss_terms_kernel(int kind, const float* __restrict__ p,
                                                         const float* __restrict__ y, float* __restrict__ term,
                                                         float* __restrict__ dir, long long n) {
  const float lo = 1e-7f, hi = 1.0f - 1e-7f;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    const float pi = p[i], yi = y[i];
    switch (kind) {
      case RT_LOSS_MAE: {  // losses.rs:46-53 (p = pred - target already)
        term[i] = fabsf(pi);
        if (dir) dir[i] = pi >= 0.0f ? 1.0f : -1.0f;
        break;
      }
      case RT_LOSS_SOFTMAX_XENT: {  // losses.rs:99-115 (p = softmax(pred))
        term[i] = yi != 0.0f ? -(yi * logf(fmaxf(pi, 1e-12f))) : 0.0f;
        if (dir) dir[i] = pi - yi;
        break;
      }
      case RT_LOSS_BCE: {  // losses.rs:143-162
        const float c = pi < lo ? lo : (pi > hi ? hi : pi);  // f32::clamp: NaN stays NaN
        term[i] = -(yi * logf(c) + (1.0f - yi) * logf(1.0f - c));
        if (dir) dir[i] = (c - yi) / (c * (1.0f - c));
        break;
      }
    }
  }
}

// losses.rs:99-115 from the logits in one pass per row (one thread per row):
// the softmax of tensor.rs:455-472 (max, exp into dir, sequential sum,
// divide), then dir = p − y and the row's loss terms −y·ln(max(p, 1e-12))
// (y ≠ 0) added in column order.  The row sums are added by a block tree;
// with one block the launch also writes value = (0 + total) / div, else each
// block writes its part for sum_stage2.
__global__ __launch_bounds__(256) void xent_logits_kernel(const float* __restrict__ z, const float* __restrict__ y,
                                                          float* __restrict__ dir, long long rows, long long cols,
                                                          float* __restrict__ part, float div,
                                                          float* __restrict__ out, float dir_scale) {
  __shared__ float sh[256];
  const long long i = blockIdx.x * 256LL + threadIdx.x;
  float row_term = 0.0f;
  if (i < rows) {
    const float* zr = z + i * cols;
    const float* yr = y + i * cols;
    float* d = dir + i * cols;
    float mx = -INFINITY;
    for (long long j = 0; j < cols; ++j) mx = fmaxf(mx, zr[j]);
    float sum = 0.0f;
    for (long long j = 0; j < cols; ++j) {
      const float e = expf(zr[j] - mx);
      d[j] = e;
      sum += e;
    }
    for (long long j = 0; j < cols; ++j) {
      const float pj = d[j] / sum, yj = yr[j];
      if (yj != 0.0f) row_term += -(yj * logf(fmaxf(pj, 1e-12f)));
      d[j] = (pj - yj) * dir_scale;  // dir_scale 1 leaves P − Y exactly as it is
    }
  }
  sh[threadIdx.x] = row_term;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (gridDim.x == 1) out[0] = (0.0f + sh[0]) / div;
    else part[blockIdx.x] = sh[0];
  }
}

unsigned grid_for(long long n) { return (unsigned)std::max<long long>(1, std::min<long long>((n + 255) / 256, 8192)); }

}  // namespace

namespace rt {

hipError_t unary_launch(hipStream_t s, int op, float k, const float* x, float* y, long long n) {
  if (n <= 0) return hipSuccess;
  rt::launch(unary_kernel, dim3(grid_for(n)), dim3(256), 0, s, op, k, x, y, n);
  return hipGetLastError();
}

hipError_t unary_vjp_launch(hipStream_t s, int op, float k, const float* g, const float* x, const float* y, float* dx,
                            long long n) {
  if (n <= 0) return hipSuccess;
  rt::launch(unary_vjp_kernel, dim3(grid_for(n)), dim3(256), 0, s, op, k, g, x, y, dx, n);
  return hipGetLastError();
}

template <int R>
hipError_t binary_launch_r(hipStream_t s, int op, const float* a, const float* b, float* out, const Shape4& sh,
                           long long n) {
  const dim3 grid(grid_for(n)), block(256);
  // 32-bit indices only where the grid-stride index cannot pass INT32_MAX
  // (its last step goes up to n - 1 + the grid's threads).
  if (n <= (1LL << 31) - 1 - (long long)grid.x * 256)
    rt::launch((binary_kernel<R, int>), grid, block, 0, s, op, a, b, out, sh, (int)n);
  else
    rt::launch((binary_kernel<R, long long>), grid, block, 0, s, op, a, b, out, sh, n);
  return hipGetLastError();
}

hipError_t binary_launch(hipStream_t s, int op, const float* a, const long long* sa, const float* b,
                         const long long* sb, float* out, const long long* shape, int rank) {
  if (rank < 1 || rank > kMaxRank) return hipErrorInvalidValue;
  // Merge axis i into i + 1 where both operands step contiguously across the
  // boundary (a broadcast axis next to a broadcast axis also merges), so a
  // same-shape zip is rank 1 and a bias broadcast rank 2.
  long long n_[kMaxRank], a_[kMaxRank], b_[kMaxRank];
  int r = 0;
  long long n = 1;
  for (int i = 0; i < rank; ++i) {
    n *= shape[i];
    if (shape[i] == 1) continue;  // extent-1 axes contribute nothing
    if (r > 0 && a_[r - 1] == sa[i] * shape[i] && b_[r - 1] == sb[i] * shape[i]) {
      n_[r - 1] *= shape[i];
      a_[r - 1] = sa[i];
      b_[r - 1] = sb[i];
    } else {
      n_[r] = shape[i];
      a_[r] = sa[i];
      b_[r] = sb[i];
      ++r;
    }
  }
  if (n <= 0) return hipSuccess;
  if (r == 0) {  // every axis has extent 1: one element
    n_[0] = 1;
    a_[0] = b_[0] = 0;
    r = 1;
  }
  Shape4 sh{};
  for (int i = 0; i < kMaxRank; ++i) {
    const int src = i - (kMaxRank - r);
    sh.n[i] = src >= 0 ? n_[src] : 1;
    sh.sa[i] = src >= 0 ? a_[src] : 0;
    sh.sb[i] = src >= 0 ? b_[src] : 0;
  }
  switch (r) {
    case 1: return binary_launch_r<1>(s, op, a, b, out, sh, n);
    case 2: return binary_launch_r<2>(s, op, a, b, out, sh, n);
    case 3: return binary_launch_r<3>(s, op, a, b, out, sh, n);
    default: return binary_launch_r<4>(s, op, a, b, out, sh, n);
  }
}

hipError_t reduce_to_launch(hipStream_t s, const float* g, const long long* gshape, int grank, float* out,
                            const long long* tshape) {
  // tshape is aligned with gshape (same rank, 1 on the reduced axes).
  if (grank < 1 || grank > kMaxRank) return hipErrorInvalidValue;
  ReduceArgs r{};
  long long gstride[kMaxRank];
  long long stride = 1;
  for (int ax = grank - 1; ax >= 0; --ax) {
    gstride[ax] = stride;
    stride *= gshape[ax];
  }
  long long red_n[kMaxRank], red_s[kMaxRank];
  int n_red = 0;
  r.n_out = 1;
  for (int ax = 0; ax < grank; ++ax) {
    if (gshape[ax] == 1) continue;
    if (tshape[ax] == gshape[ax]) {
      r.keep_n[r.n_keep] = gshape[ax];
      r.keep_s[r.n_keep] = gstride[ax];
      ++r.n_keep;
      r.n_out *= gshape[ax];
    } else {
      if (tshape[ax] != 1) return hipErrorInvalidValue;
      red_n[n_red] = gshape[ax];
      red_s[n_red] = gstride[ax];
      ++n_red;
    }
  }
  for (int i = 0; i < kMaxRank; ++i) {  // pad the reduced axes in front with extent 1
    const int src = i - (kMaxRank - n_red);
    r.red_n[i] = src >= 0 ? red_n[src] : 1;
    r.red_s[i] = src >= 0 ? red_s[src] : 0;
  }
  if (r.n_out <= 0) return hipSuccess;
  rt::launch(reduce_to_kernel, dim3(grid_for(r.n_out)), dim3(256), 0, s, g, out, r);
  return hipGetLastError();
}

size_t sum_scratch_elems(long long n) { return (size_t)std::max<long long>(1, std::min<long long>((n + 65535) / 65536, 4096)); }

hipError_t sum_all_launch(hipStream_t s, const float* x, long long n, float div, float* out, float* scratch) {
  const long long parts = (long long)sum_scratch_elems(n);
  const long long chunk = std::max<long long>(1, (n + parts - 1) / parts);
  rt::launch(sum_stage1, dim3((unsigned)parts), dim3(256), 0, s, x, n, chunk, scratch, div, out);
  if (parts > 1) rt::launch(sum_stage2, dim3(1), dim3(64), 0, s, scratch, (int)parts, div, out);
  return hipGetLastError();
}

hipError_t scalar_fill_launch(hipStream_t s, const float* scalar, float div, const float* x, float* out, long long n) {
  if (n <= 0) return hipSuccess;
  rt::launch(scalar_fill_kernel, dim3(grid_for(n)), dim3(256), 0, s, scalar, div, x, out, n);
  return hipGetLastError();
}

hipError_t softmax_rows_launch(hipStream_t s, const float* z, float* y, long long rows, long long cols) {
  if (rows <= 0) return hipSuccess;
  rt::launch(softmax_rows_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, z, y, rows, cols);
  return hipGetLastError();
}

hipError_t softmax_rows_vjp_launch(hipStream_t s, const float* sm, const float* g, float* dx, long long rows,
                                   long long cols) {
  if (rows <= 0) return hipSuccess;
  rt::launch(softmax_rows_vjp_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, sm, g, dx, rows,
                     cols);
  return hipGetLastError();
}

hipError_t xent_logits_launch(hipStream_t s, const float* z, const float* y, float* dir, long long rows,
                              long long cols, float div, float* out, float* scratch, size_t scratch_elems,
                              float dir_scale) {
  const long long blocks = std::max<long long>(1, (rows + 255) / 256);
  if (blocks > 1 && (size_t)blocks > scratch_elems) return hipErrorInvalidValue;
  rt::launch(xent_logits_kernel, dim3((unsigned)blocks), dim3(256), 0, s, z, y, dir, rows, cols, scratch, div,
                     out, dir_scale);
  if (blocks > 1) rt::launch(sum_stage2, dim3(1), dim3(64), 0, s, scratch, (int)blocks, div, out);
  return hipGetLastError();
}

hipError_t loss_terms_launch(hipStream_t s, int kind, const float* p, const float* y, float* term, float* dir,
                             long long n) {
  if (n <= 0) return hipSuccess;
  rt::launch(loss_terms_kernel, dim3(grid_for(n)), dim3(256), 0, s, kind, p, y, term, dir, n);
  return hipGetLastError();
}

}  // namespace rt

// ------------------------------------------------------------------ C ABI
using namespace rt;

namespace {

bool is_f32(const rt_buf* b) { return b && b->dtype == RT_F32; }

// Shape of b right-aligned to rank r with leading 1s.
void aligned_shape(const rt_buf* b, int r, long long* out) {
  for (int i = 0; i < r; ++i) {
    const int src = i - (r - b->rank);
    out[i] = src >= 0 ? (long long)b->shape[src] : 1;
  }
}

// Strides of b in the index space of an output of rank r and shape `shape`
// (0 on axes where b has extent 1 and the output does not).
void broadcast_strides(const rt_buf* b, int r, const long long* shape, long long* out) {
  long long bs[kMaxRank];
  aligned_shape(b, r, bs);
  long long acc = 1;
  for (int i = r - 1; i >= 0; --i) {
    out[i] = (bs[i] == shape[i]) ? acc : 0;
    acc *= bs[i];
  }
}

bool needs_x(int op) {
  return op == RT_U_SQUARE || op == RT_U_LN || op == RT_U_RELU || op == RT_U_LEAKY_RELU;
}
bool needs_y(int op) { return op == RT_U_SQRT || op == RT_U_EXP || op == RT_U_SIGMOID || op == RT_U_TANH; }

const char* kUnaryNames[] = {"map_scale", "map_offset", "map_neg",  "map_square", "map_sqrt", "map_exp",
                             "map_ln",    "map_relu",   "map_leaky", "map_sigmoid", "map_tanh"};

}  // namespace

extern "C" {

int rt_map(rt_ctx* c, rt_unary_op op, float k, const rt_buf* x, rt_buf* y) {
  CHECK_CTX(c);
  if (!x || !y) return fail(c, RT_ERR_INVALID, "null buffer");
  if (op < RT_U_SCALE || op > RT_U_TANH) return fail(c, RT_ERR_INVALID, "unknown unary op %d", (int)op);
  if (!is_f32(x) || !is_f32(y)) return fail(c, RT_ERR_DTYPE, "map takes f32");
  if (x->n != y->n) return fail(c, RT_ERR_SHAPE, "map: %zu elements into %zu", x->n, y->n);
  Launch L(c, kUnaryNames[op]);
  HIP_TRY(c, unary_launch(c->stream, op, k, static_cast<const float*>(x->ptr), static_cast<float*>(y->ptr), x->n),
          "map");
  return RT_OK;
}

int rt_map_vjp(rt_ctx* c, rt_unary_op op, float k, const rt_buf* g, const rt_buf* x, const rt_buf* y, rt_buf* dx) {
  CHECK_CTX(c);
  if (!g || !dx) return fail(c, RT_ERR_INVALID, "null buffer");
  if (op < RT_U_SCALE || op > RT_U_TANH) return fail(c, RT_ERR_INVALID, "unknown unary op %d", (int)op);
  if (needs_x(op) && !x) return fail(c, RT_ERR_INVALID, "this VJP needs the op's input");
  if (needs_y(op) && !y) return fail(c, RT_ERR_INVALID, "this VJP needs the op's output");
  if (!is_f32(g) || !is_f32(dx) || (x && !is_f32(x)) || (y && !is_f32(y))) return fail(c, RT_ERR_DTYPE, "f32 only");
  if (g->n != dx->n || (x && x->n != g->n) || (y && y->n != g->n))
    return fail(c, RT_ERR_SHAPE, "map_vjp: operands differ in size");
  Launch L(c, "map_vjp");
  HIP_TRY(c,
          unary_vjp_launch(c->stream, op, k, static_cast<const float*>(g->ptr),
                           needs_x(op) ? static_cast<const float*>(x->ptr) : nullptr,
                           needs_y(op) ? static_cast<const float*>(y->ptr) : nullptr, static_cast<float*>(dx->ptr),
                           g->n),
          "map_vjp");
  return RT_OK;
}

int rt_zip(rt_ctx* c, rt_binary_op op, const rt_buf* a, const rt_buf* b, rt_buf* out) {
  CHECK_CTX(c);
  if (!a || !b || !out) return fail(c, RT_ERR_INVALID, "null buffer");
  if (op < RT_B_ADD || op > RT_B_DIV) return fail(c, RT_ERR_INVALID, "unknown binary op %d", (int)op);
  if (!is_f32(a) || !is_f32(b) || !is_f32(out)) return fail(c, RT_ERR_DTYPE, "zip takes f32");
  const int r = std::max(std::max(a->rank, b->rank), 1);
  long long sa_shape[kMaxRank], sb_shape[kMaxRank], shape[kMaxRank];
  aligned_shape(a, r, sa_shape);
  aligned_shape(b, r, sb_shape);
  for (int i = 0; i < r; ++i) {
    if (sa_shape[i] == sb_shape[i] || sb_shape[i] == 1) shape[i] = sa_shape[i];
    else if (sa_shape[i] == 1) shape[i] = sb_shape[i];
    else return fail(c, RT_ERR_SHAPE, "shapes do not broadcast (axis %d: %lld vs %lld)", i, sa_shape[i], sb_shape[i]);
  }
  // out must have exactly the broadcast shape (leading 1s may be dropped).
  long long os[kMaxRank];
  if (out->rank > r) return fail(c, RT_ERR_SHAPE, "zip output rank too large");
  aligned_shape(out, r, os);
  for (int i = 0; i < r; ++i)
    if (os[i] != shape[i]) return fail(c, RT_ERR_SHAPE, "zip output does not have the broadcast shape");
  // Aliasing is allowed only between same-shaped tensors (elementwise in place).
  if ((out->ptr == a->ptr && a->n != out->n) || (out->ptr == b->ptr && b->n != out->n))
    return fail(c, RT_ERR_INVALID, "zip output aliases a broadcast operand");
  if (out->n == 0) return RT_OK;
  long long sa[kMaxRank], sb[kMaxRank];
  broadcast_strides(a, r, shape, sa);
  broadcast_strides(b, r, shape, sb);
  Launch L(c, "zip");
  HIP_TRY(c,
          binary_launch(c->stream, op, static_cast<const float*>(a->ptr), sa, static_cast<const float*>(b->ptr), sb,
                        static_cast<float*>(out->ptr), shape, r),
          "zip");
  return RT_OK;
}

int rt_sum_all(rt_ctx* c, const rt_buf* x, float div, rt_buf* out) {
  CHECK_CTX(c);
  if (!x || !out) return fail(c, RT_ERR_INVALID, "null buffer");
  if (!is_f32(x) || !is_f32(out)) return fail(c, RT_ERR_DTYPE, "sum_all takes f32");
  if (out->n != 1) return fail(c, RT_ERR_SHAPE, "sum_all writes one element");
  int rc = ensure_scratch(c, sum_scratch_elems((long long)x->n));
  if (rc) return rc;
  Launch L(c, "sum_all");
  HIP_TRY(c,
          sum_all_launch(c->stream, static_cast<const float*>(x->ptr), (long long)x->n, div,
                         static_cast<float*>(out->ptr), c->scratch),
          "sum_all");
  return RT_OK;
}

int rt_reduce_to(rt_ctx* c, const rt_buf* g, rt_buf* out) {
  CHECK_CTX(c);
  if (!g || !out) return fail(c, RT_ERR_INVALID, "null buffer");
  if (!is_f32(g) || !is_f32(out)) return fail(c, RT_ERR_DTYPE, "reduce_to takes f32");
  const int r = std::max(g->rank, 1);
  if (out->rank > r) return fail(c, RT_ERR_SHAPE, "reduce_to target has a larger rank than the source");
  long long gs[kMaxRank], ts[kMaxRank];
  aligned_shape(g, r, gs);
  aligned_shape(out, r, ts);
  for (int i = 0; i < r; ++i)
    if (ts[i] != gs[i] && ts[i] != 1)
      return fail(c, RT_ERR_SHAPE, "reduce_to: target axis %d is %lld, source %lld", i, ts[i], gs[i]);
  if (out->n == g->n) {
    // Same shape: the reference returns a copy (tensor.rs:400-402).
    if (out->ptr != g->ptr && g->n > 0)
      HIP_TRY(c, hipMemcpyAsync(out->ptr, g->ptr, g->bytes, hipMemcpyDeviceToDevice, c->stream), "reduce_to copy");
    return RT_OK;
  }
  if (out->n == 1) return rt_sum_all(c, g, 1.0f, out);  // tensor.rs:406-409
  Launch L(c, "reduce_to");
  HIP_TRY(c, reduce_to_launch(c->stream, static_cast<const float*>(g->ptr), gs, r, static_cast<float*>(out->ptr), ts),
          "reduce_to");
  return RT_OK;
}

int rt_fill_scaled(rt_ctx* c, const rt_buf* s, float div, const rt_buf* x, rt_buf* out) {
  CHECK_CTX(c);
  if (!s || !out) return fail(c, RT_ERR_INVALID, "null buffer");
  if (!is_f32(s) || !is_f32(out) || (x && !is_f32(x))) return fail(c, RT_ERR_DTYPE, "fill_scaled takes f32");
  if (s->n != 1) return fail(c, RT_ERR_SHAPE, "the scale must have one element");
  if (x && x->n != out->n) return fail(c, RT_ERR_SHAPE, "fill_scaled: x and out differ in size");
  Launch L(c, "fill_scaled");
  HIP_TRY(c,
          scalar_fill_launch(c->stream, static_cast<const float*>(s->ptr), div,
                             x ? static_cast<const float*>(x->ptr) : nullptr, static_cast<float*>(out->ptr),
                             (long long)out->n),
          "fill_scaled");
  return RT_OK;
}

int rt_softmax_rows(rt_ctx* c, const rt_buf* z, rt_buf* y) {
  CHECK_CTX(c);
  if (!z || !y) return fail(c, RT_ERR_INVALID, "null buffer");
  if (!is_f32(z) || !is_f32(y)) return fail(c, RT_ERR_DTYPE, "softmax_rows takes f32");
  if (z->rank != 2) return fail(c, RT_ERR_SHAPE, "softmax_rows needs rank 2");
  if (y->n != z->n) return fail(c, RT_ERR_SHAPE, "softmax_rows: output size");
  Launch L(c, "softmax_rows");
  HIP_TRY(c,
          softmax_rows_launch(c->stream, static_cast<const float*>(z->ptr), static_cast<float*>(y->ptr),
                              (long long)z->shape[0], (long long)z->shape[1]),
          "softmax_rows");
  return RT_OK;
}

int rt_softmax_rows_vjp(rt_ctx* c, const rt_buf* s, const rt_buf* g, rt_buf* dx) {
  CHECK_CTX(c);
  if (!s || !g || !dx) return fail(c, RT_ERR_INVALID, "null buffer");
  if (!is_f32(s) || !is_f32(g) || !is_f32(dx)) return fail(c, RT_ERR_DTYPE, "f32 only");
  if (s->rank != 2) return fail(c, RT_ERR_SHAPE, "softmax VJP needs rank 2");
  if (g->n != s->n || dx->n != s->n) return fail(c, RT_ERR_SHAPE, "softmax VJP: operands differ in size");
  Launch L(c, "softmax_rows_vjp");
  HIP_TRY(c,
          softmax_rows_vjp_launch(c->stream, static_cast<const float*>(s->ptr), static_cast<const float*>(g->ptr),
                                  static_cast<float*>(dx->ptr), (long long)s->shape[0], (long long)s->shape[1]),
          "softmax_rows_vjp");
  return RT_OK;
}

int rt_loss(rt_ctx* c, rt_loss_kind kind, const rt_buf* p, const rt_buf* y, rt_buf* value, rt_buf* dir) {
  CHECK_CTX(c);
  if (!p || !value) return fail(c, RT_ERR_INVALID, "null buffer");
  if (kind != RT_LOSS_MAE && kind != RT_LOSS_SOFTMAX_XENT && kind != RT_LOSS_BCE &&
      kind != RT_LOSS_SOFTMAX_XENT_LOGITS && kind != RT_LOSS_SOFTMAX_XENT_LOGITS_MEAN)
    return fail(c, RT_ERR_INVALID, "unknown loss kind %d", (int)kind);
  if (kind != RT_LOSS_MAE && !y) return fail(c, RT_ERR_INVALID, "this loss needs targets");
  if (!is_f32(p) || !is_f32(value) || (y && !is_f32(y)) || (dir && !is_f32(dir)))
    return fail(c, RT_ERR_DTYPE, "losses take f32");
  if (value->n != 1) return fail(c, RT_ERR_SHAPE, "the loss value has one element");
  if (y && y->n != p->n) return fail(c, RT_ERR_SHAPE, "predictions and targets differ in size");
  if (dir && dir->n != p->n) return fail(c, RT_ERR_SHAPE, "dir must match the predictions");
  float batch = (float)p->n;
  if (kind == RT_LOSS_SOFTMAX_XENT_LOGITS || kind == RT_LOSS_SOFTMAX_XENT_LOGITS_MEAN) {
    if (p->rank != 2 || y->rank != 2 || y->shape[0] != p->shape[0] || y->shape[1] != p->shape[1])
      return fail(c, RT_ERR_SHAPE, "logits and targets differ in shape");  // losses.rs:100
    if (!dir) return fail(c, RT_ERR_INVALID, "the logits form writes dir (it holds the softmax on the way)");
    const long long rows = (long long)p->shape[0], cols = (long long)p->shape[1];
    const size_t blocks = (size_t)std::max<long long>(1, (rows + 255) / 256);
    int rc = ensure_scratch(c, blocks);
    if (rc) return rc;
    Launch L(c, "loss");
    HIP_TRY(c,
            xent_logits_launch(c->stream, static_cast<const float*>(p->ptr), static_cast<const float*>(y->ptr),
                               static_cast<float*>(dir->ptr), rows, cols, (float)rows, static_cast<float*>(value->ptr),
                               c->scratch, c->scratch_elems,
                               kind == RT_LOSS_SOFTMAX_XENT_LOGITS_MEAN ? 1.0f / (float)rows : 1.0f),
            "softmax-xent");
    return RT_OK;
  }
  if (kind == RT_LOSS_SOFTMAX_XENT) {
    if (p->rank != 2) return fail(c, RT_ERR_SHAPE, "softmax cross-entropy takes [batch, classes]");
    if (y->rank != 2 || y->shape[0] != p->shape[0] || y->shape[1] != p->shape[1])
      return fail(c, RT_ERR_SHAPE, "logits and targets differ in shape");  // losses.rs:100
    batch = (float)p->shape[0];
  }
  const long long n = (long long)p->n;
  const size_t parts = sum_scratch_elems(n);
  int rc = ensure_scratch(c, (size_t)n + parts);
  if (rc) return rc;
  float* term = c->scratch + parts;
  Launch L(c, "loss");
  HIP_TRY(c,
          loss_terms_launch(c->stream, kind, static_cast<const float*>(p->ptr),
                            y ? static_cast<const float*>(y->ptr) : nullptr, term,
                            dir ? static_cast<float*>(dir->ptr) : nullptr, n),
          "loss terms");
  HIP_TRY(c, sum_all_launch(c->stream, term, n, batch, static_cast<float*>(value->ptr), c->scratch), "loss sum");
  return RT_OK;
}

}  // extern "C"
