// Row and column kernels of the training step (all HBM- or latency-bound):
//   softmax cross-entropy   XENT      kernels.rs:138-167  (one wave64 per row)
//   column sum              COLSUM    kernels.rs:182-199  (two fixed-order stages)
//   bias add / ReLU / ReLU backward   kernels.rs:99-131
//   f32 <-> bf16/f16 conversion       EMPACOTA mista.rs:326-341
// Built with -ffp-contract=off: every product and sum rounds on its own, in
// the order rtensor's CPU path uses (losses.rs:99-115, tensor.rs:455-472).

#include <algorithm>

#include "rt_internal.h"

namespace {

__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ inline unsigned short f32_to_bf16_rne(float x) {
  unsigned int u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

__device__ inline float bf16_to_f32(unsigned short h) { return __uint_as_float((unsigned int)h << 16); }

// One wave per row: max, Σexp, p = e/Σ, δ = (p − onehot)·scale, loss = −ln max(p_y, 1e-12).
// A label >= cols raises err_flag (plain store) and makes that row's loss NaN;
// nothing is read out of bounds.  The optional bf16 copy of δ has row stride
// ld_half (>= cols; its columns past cols are left alone).
__global__ __launch_bounds__(256) void xent_kernel(const float* __restrict__ logits, const uint32_t* __restrict__ labels,
                                                   float* __restrict__ delta, unsigned short* __restrict__ delta_bf16,
                                                   int ld_half, float* __restrict__ loss_rows, int rows, int cols,
                                                   float scale, int* err_flag) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* z = logits + (long long)row * cols;
  const uint32_t y = labels[row];
  const bool bad = y >= (uint32_t)cols;
  if (bad && lane == 0) {
    *err_flag = 1;
    loss_rows[row] = __uint_as_float(0x7fc00000u);
  }
  float* d = delta + (long long)row * cols;
  auto put = [&](int j, float pj) {
    const float yj = (!bad && (uint32_t)j == y) ? 1.0f : 0.0f;
    const float dj = (pj - yj) * scale;
    d[j] = dj;
    if (delta_bf16 != nullptr) delta_bf16[(long long)row * ld_half + j] = f32_to_bf16_rne(dj);
    if (!bad && (uint32_t)j == y) loss_rows[row] = -logf(fmaxf(pj, 1e-12f));
  };
  constexpr int R = 16;  // row values per lane held in registers (rows up to 1024)
  if (cols <= 64 * R) {
    // One read of the row; the same operations in the same order as below.
    float v[R];
#pragma unroll
    for (int q = 0; q < R; ++q) v[q] = z[min(lane + 64 * q, cols - 1)];  // all issued at once, in bounds
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < R; ++q)
      if (lane + 64 * q < cols) mx = fmaxf(mx, v[q]);
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int q = 0; q < R; ++q)
      if (lane + 64 * q < cols) {
        v[q] = expf(v[q] - mx);
        sum += v[q];
      }
    sum = wave_sum(sum);
#pragma unroll
    for (int q = 0; q < R; ++q)
      if (lane + 64 * q < cols) put(lane + 64 * q, v[q] / sum);
    return;
  }
  float mx = -INFINITY;
  for (int j = lane; j < cols; j += 64) mx = fmaxf(mx, z[j]);
  mx = wave_max(mx);
  float sum = 0.0f;
  for (int j = lane; j < cols; j += 64) sum += expf(z[j] - mx);
  sum = wave_sum(sum);
  for (int j = lane; j < cols; j += 64) put(j, expf(z[j] - mx) / sum);
}

// Narrow output layer fused with the loss: z = A·W + b for C <= 16 classes
// (rtensor runs the head GEMM with split-K and then XENT, mod.rs:1360-1367 and
// 1399-1410), then the softmax cross-entropy of xent_kernel, in one launch.
// Block = 16 rows and HW waves (8, or 16 when K is a multiple of 256); wave w
// sums k in [w K/HW, (w+1) K/HW) with v_mfma_f32_16x16x4_f32, both operands
// straight from global memory (A as float4 row segments, W as scalars, 8
// chunks of 16 k in flight per batch).
// Lane (g, r) feeds A(row r, k) and W(k, class r) with k = chunk + 4g + s at
// MFMA step s, and ends with z(rows 4g..4g+3, class r).  The HW partial
// tiles are added in LDS in wave order; then the 16 lanes of each row run
// the softmax with width-16 shuffles.  With labels == null only the logits
// are written (and bias may be null: z = A·W).  The K sum order differs from the CPU path's; the rest
// follows xent_kernel.
typedef float f4v __attribute__((ext_vector_type(4)));
constexpr int HEAD_C = 16, HEAD_ROWS = 16;

template <int HW>  // waves per block: 8, or 16 when K is a multiple of 256
__global__ __launch_bounds__(64 * HW) void head_xent_kernel(const float* __restrict__ A, int K,
                                                            const float* __restrict__ W,
                                                            const float* __restrict__ bias,
                                                            const uint32_t* __restrict__ labels,
                                                            float* __restrict__ logits, float* __restrict__ delta,
                                                            float* __restrict__ loss_rows, int rows, int cols,
                                                            float scale, int* err_flag) {
  __shared__ float red[HW][HEAD_ROWS][HEAD_C + 1];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, r = lane & 15;
  const int r0 = blockIdx.x * HEAD_ROWS;
  const int kq = K / HW;       // k per wave (K is a multiple of 16 HW)
  const int nch = kq / 16;     // chunks of 16 k per wave
  const int kw = wave * kq;
  const float* arow = A + (long long)min(r0 + r, rows - 1) * K + kw + 4 * g;  // rows past the end read the last row
  // The softmax lanes' label and bias, loaded first so that their latency
  // runs under the K loop.
  uint32_t ylab = 0;
  float bv = 0.0f;
  if (threadIdx.x < HEAD_ROWS * HEAD_C) {
    const int row = r0 + (int)(threadIdx.x >> 4), cc = threadIdx.x & 15;
    if (labels != nullptr && row < rows) ylab = labels[row];
    if (bias != nullptr && cc < cols) bv = bias[cc];
  }
  f4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < nch; c0 += 8) {
    f4v av[8];
    float wv[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (c0 + i < nch) {
        av[i] = *reinterpret_cast<const f4v*>(arow + 16 * (c0 + i));
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int k = kw + 16 * (c0 + i) + 4 * g + s;
          wv[i][s] = r < cols ? W[(long long)k * cols + r] : 0.0f;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (c0 + i < nch) {
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][s], wv[i][s], acc, 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) red[wave][4 * g + q][r] = acc[q];
  __syncthreads();

  if (threadIdx.x >= HEAD_ROWS * HEAD_C) return;  // no barrier after this point
  const int rr = threadIdx.x >> 4, cc = threadIdx.x & 15;  // one row per 16 lanes
  const int row = r0 + rr;
  float zs = red[0][rr][cc];
#pragma unroll
  for (int w = 1; w < HW; ++w) zs += red[w][rr][cc];
  const float z = cc < cols ? (bias != nullptr ? zs + bv : zs) : -INFINITY;
  if (row >= rows) return;
  if (cc < cols) logits[(long long)row * cols + cc] = z;
  if (labels == nullptr) return;
  float mx = z;
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 16));
  const float e = cc < cols ? expf(z - mx) : 0.0f;
  float sum = e;
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 16);
  const uint32_t y = ylab;
  const bool bad = y >= (uint32_t)cols;
  if (bad && cc == 0) {
    *err_flag = 1;
    loss_rows[row] = __uint_as_float(0x7fc00000u);
  }
  if (cc < cols) {
    const float pj = e / sum;
    const float yj = (!bad && (uint32_t)cc == y) ? 1.0f : 0.0f;
    delta[(long long)row * cols + cc] = (pj - yj) * scale;
    if (!bad && (uint32_t)cc == y) loss_rows[row] = -logf(fmaxf(pj, 1e-12f));
  }
}

// Row argmax with Tensor::argmax_rows' semantics (tensor.rs:476-493): the
// first index j with j == 0 or z_j > (best so far).  Hence a NaN in column 0
// wins the row, later NaNs never win, and ties go to the first index.  As a
// reduction: if z_0 is NaN the answer is 0, else the first index of the
// largest non-NaN value (column 0 is non-NaN then, so one exists).  One wave
// per row; lanes scan strided columns, then (value, index) pairs are combined
// with "larger value, or equal value and smaller index".
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ z, uint32_t* __restrict__ out, int rows,
                                                     int cols) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* zr = z + (long long)row * cols;
  float bv = -INFINITY;
  int bj = 0x7fffffff;
  for (int j = lane; j < cols; j += 64) {
    const float v = zr[j];
    if (!(v != v) && (bj == 0x7fffffff || v > bv)) {  // strided scan: keep the first max of this lane
      bv = v;
      bj = j;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oj = __shfl_xor(bj, off, 64);
    if (oj != 0x7fffffff && (bj == 0x7fffffff || ov > bv || (ov == bv && oj < bj))) {
      bv = ov;
      bj = oj;
    }
  }
  if (lane == 0) {
    const float z0 = zr[0];
    out[row] = (z0 != z0 || bj == 0x7fffffff) ? 0u : (uint32_t)bj;
  }
}

// Stage 1: block (cx, cy) sums rows [cy*chunk, (cy+1)*chunk) of 256 columns
// starting at cx*256, one column per thread, rows in increasing order.
template <typename T>
__device__ inline float load_as_f32(const T* p, long long i);
template <>
__device__ inline float load_as_f32<float>(const float* p, long long i) { return p[i]; }
template <>
__device__ inline float load_as_f32<unsigned short>(const unsigned short* p, long long i) { return bf16_to_f32(p[i]); }
template <>
__device__ inline float load_as_f32<_Float16>(const _Float16* p, long long i) { return (float)p[i]; }

// Column sums (rt_colsum, the reference's COLSUM kernels.rs:182-199), two
// stages, both reduced inside wavefronts and blocks.
//
// Stage 1: a block of 16 waves takes a band of LR*V columns over a chunk of
// rows.  Lane (ro, cg) of a wave, ro = lane / LR and cg = lane % LR, reads V
// consecutive columns (16 bytes) of row ro of each of the wave's row groups
// (RW = 64 / LR rows per group; the 16 waves take the groups in turn, four
// groups' loads issued together) and accumulates them.  The RW rows of a
// group are then added across lanes with butterfly shuffles (lanes cg, cg +
// LR, ...), the 16 waves' sums through LDS in wave order, and the chunk's
// partial row is written (the result itself for one chunk).
constexpr int kCsWaves = 16, kCsUnroll = 4;

template <typename T>
struct ColsumVec {  // 16 bytes of T
  static constexpr int V = 16 / sizeof(T);
};

template <typename T>
__device__ inline void colsum_load(const T* __restrict__ src, long long off, int c, int cols, bool vec,
                                   float (&x)[ColsumVec<T>::V]) {
  constexpr int V = ColsumVec<T>::V;
  if (vec && c + V <= cols) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v w = *reinterpret_cast<const u4v*>(src + off + c);
    const T* e = reinterpret_cast<const T*>(&w);
#pragma unroll
    for (int j = 0; j < V; ++j) x[j] = load_as_f32<T>(e, j);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) x[j] = c + j < cols ? load_as_f32<T>(src, off + c + j) : 0.0f;
  }
}

template <typename T>
__global__ __launch_bounds__(64 * kCsWaves) void colsum_stage1(const T* __restrict__ src, int rows, int cols,
                                                               int chunk, int lr, bool vec, float* __restrict__ out) {
  constexpr int V = ColsumVec<T>::V;
  __shared__ float red[kCsWaves * 64 * V];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rw = 64 / lr, ro = lane / lr, cg = lane % lr;
  const int c = blockIdx.x * lr * V + cg * V;
  const int r0 = blockIdx.y * chunk, r1 = min(rows, r0 + chunk);
  float acc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) acc[j] = 0.0f;
  // Row group q covers rows r0 + q*rw .. + rw-1; wave w takes q = w, w + 16, ...
  const int groups = (r1 - r0 + rw - 1) / rw;
  for (int q0 = wave; q0 < groups; q0 += kCsWaves * kCsUnroll) {
    float x[kCsUnroll][V];
#pragma unroll
    for (int u = 0; u < kCsUnroll; ++u) {
      const int r = r0 + (q0 + u * kCsWaves) * rw + ro;
      if (q0 + u * kCsWaves < groups && r < r1 && c < cols)
        colsum_load<T>(src, (long long)r * cols, c, cols, vec, x[u]);
      else
#pragma unroll
        for (int j = 0; j < V; ++j) x[u][j] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kCsUnroll; ++u)
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] += x[u][j];
  }
  // The wave's rw row lanes of each column group, added across lanes.
  for (int d = lr; d < 64; d <<= 1)
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] += __shfl_xor(acc[j], d);
  if (ro == 0)
#pragma unroll
    for (int j = 0; j < V; ++j) red[(wave * 64 + cg) * V + j] = acc[j];
  __syncthreads();
  // Thread t < lr*V finishes column band offset t: the waves in order.
  const int t = threadIdx.x;
  if (t < lr * V) {
    const int col = blockIdx.x * lr * V + t;
    if (col < cols) {
      const int g = t / V, j = t % V;
      float v = red[g * V + j];
      for (int w = 1; w < kCsWaves; ++w) v += red[(w * 64 + g) * V + j];
      out[(long long)blockIdx.y * cols + col] = v;
    }
  }
}

// Stage 2: dst[col] = the partial rows of the chunks added up.  A block
// takes 64 columns; wave w adds the parts w, w + 16, ... of its lane's
// column (four loads in flight), the 16 waves' sums are added in LDS in
// wave order.
__global__ __launch_bounds__(64 * kCsWaves) void colsum_stage2(const float* __restrict__ part, int parts, int cols,
                                                               float* __restrict__ dst) {
  __shared__ float red[kCsWaves * 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + lane;
  float acc = 0.0f;
  if (col < cols) {
    for (int p0 = wave; p0 < parts; p0 += kCsWaves * kCsUnroll) {
      float x[kCsUnroll];
#pragma unroll
      for (int u = 0; u < kCsUnroll; ++u) {
        const int p = p0 + u * kCsWaves;
        x[u] = p < parts ? part[(long long)p * cols + col] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kCsUnroll; ++u) acc += x[u];
    }
  }
  red[wave * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0 && col < cols) {
    float v = red[lane];
    for (int w = 1; w < kCsWaves; ++w) v += red[w * 64 + lane];
    dst[col] = v;
  }
}

__global__ __launch_bounds__(256) void bias_add_kernel(float* z, const float* b, int rows, int cols) {
  const long long total = (long long)rows * cols;
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (long long)gridDim.x * 256)
    z[i] = z[i] + b[i % cols];
}

__global__ __launch_bounds__(256) void relu_kernel(const float* x, float* y, long long n) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256) y[i] = fmaxf(x[i], 0.0f);
}

template <typename T>
__global__ __launch_bounds__(256) void relu_bwd_kernel(const T* a, float* delta, long long n) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    if (!(load_as_f32<T>(a, i) > 0.0f)) delta[i] = 0.0f;
}

__global__ __launch_bounds__(256) void convert_kernel(const void* src, int sd, void* dst, int dd, long long n) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    float v;
    if (sd == RT_F32) v = static_cast<const float*>(src)[i];
    else if (sd == RT_BF16) v = bf16_to_f32(static_cast<const unsigned short*>(src)[i]);
    else v = (float)static_cast<const _Float16*>(src)[i];
    if (dd == RT_F32) static_cast<float*>(dst)[i] = v;
    else if (dd == RT_BF16) static_cast<unsigned short*>(dst)[i] = f32_to_bf16_rne(v);
    else static_cast<_Float16*>(dst)[i] = (_Float16)v;  // v_cvt_f16_f32: round to nearest even, keeps subnormals
  }
}

__global__ void fill_i32_kernel(int* p, int v, long long n) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256) p[i] = v;
}

int grid_for(long long n) {
  long long b = (n + 255) / 256;
  return (int)std::max<long long>(1, std::min<long long>(b, 8192));
}

}  // namespace

namespace rt {

bool head_xent_supported(int K, int cols) { return cols >= 1 && cols <= HEAD_C && K >= 128 && K % 128 == 0; }

hipError_t head_xent_launch(hipStream_t s, const float* A, int K, const float* W, const float* bias,
                            const uint32_t* labels, float* logits, float* delta, float* loss_rows, int rows, int cols,
                            float scale, int* err_flag) {
  if (!head_xent_supported(K, cols) || rows < 1 || (reinterpret_cast<uintptr_t>(A) & 15) != 0)
    return hipErrorInvalidValue;
  const unsigned blocks = (unsigned)((rows + HEAD_ROWS - 1) / HEAD_ROWS);
  // 16 waves when K splits into 16 whole 16-k chunks per wave (shorter
  // dependent load chains per wave; the block count is fixed by the rows).
  if (K % 256 == 0)
    rt::launch(head_xent_kernel<16>, dim3(blocks), dim3(1024), 0, s, A, K, W, bias, labels, logits, delta,
                       loss_rows, rows, cols, scale, err_flag);
  else
    rt::launch(head_xent_kernel<8>, dim3(blocks), dim3(512), 0, s, A, K, W, bias, labels, logits, delta,
                       loss_rows, rows, cols, scale, err_flag);
  return hipGetLastError();
}

hipError_t argmax_launch(hipStream_t s, const float* z, uint32_t* out, int rows, int cols) {
  if (rows < 1 || cols < 1) return hipSuccess;
  rt::launch(argmax_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, z, out, rows, cols);
  return hipGetLastError();
}

hipError_t xent_launch(hipStream_t s, const float* logits, const uint32_t* labels, float* delta, void* delta_half,
                       float* loss_rows, int rows, int cols, float scale, int* err_flag, int ld_half) {
  if (rows <= 0) return hipSuccess;
  if (ld_half < cols) ld_half = cols;
  rt::launch(xent_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, logits, labels, delta,
                     static_cast<unsigned short*>(delta_half), ld_half, loss_rows, rows, cols, scale, err_flag);
  return hipGetLastError();
}

// Column sums: lanes per row LR (a power of two covering the columns at 16
// bytes a lane, at most 64), bands of LR*V columns, and row chunks: about 512
// blocks over the bands, at least one unrolled round of row groups each.
struct ColsumPlan {
  int lr, bands, chunk, parts;
};
static ColsumPlan colsum_plan(int rows, int cols, int esize) {
  const int V = 16 / esize;
  int lr = 1;
  while (lr < 64 && lr * V < cols) lr *= 2;
  const int bands = (cols + lr * V - 1) / (lr * V);
  const int rw = 64 / lr;
  const int min_rows = rw * kCsWaves * kCsUnroll;
  int chunks = std::max(1, 512 / bands);
  chunks = std::min(chunks, std::max(1, (rows + min_rows - 1) / min_rows));
  const int chunk = (rows + chunks - 1) / chunks;
  return ColsumPlan{lr, bands, chunk, (rows + chunk - 1) / chunk};
}

static int dtype_bytes(int dtype) { return dtype == RT_F32 ? 4 : 2; }

size_t colsum_scratch_elems(int rows, int cols, int dtype) {
  if (rows <= 0 || cols <= 0) return 0;
  const ColsumPlan cp = colsum_plan(rows, cols, dtype_bytes(dtype));
  return cp.parts > 1 ? (size_t)cp.parts * cols : 0;
}

hipError_t colsum_launch(hipStream_t s, const void* src, int dtype, int rows, int cols, float* dst, float* scratch,
                         size_t scratch_elems) {
  if (cols <= 0) return hipSuccess;
  const dim3 block(64 * kCsWaves);
  if (rows <= 0) {
    rt::launch(colsum_stage2, dim3((cols + 63) / 64), block, 0, s, (const float*)nullptr, 0, cols, dst);
    return hipGetLastError();
  }
  const int esize = dtype_bytes(dtype);
  const ColsumPlan cp = colsum_plan(rows, cols, esize);
  float* out1 = cp.parts > 1 ? scratch : dst;
  if (cp.parts > 1 && (scratch == nullptr || scratch_elems < (size_t)cp.parts * cols)) return hipErrorInvalidValue;
  // 16-byte loads when every row starts 16-byte aligned.
  const bool vec = (reinterpret_cast<uintptr_t>(src) & 15) == 0 && ((size_t)cols * esize) % 16 == 0;
  const dim3 g1(cp.bands, cp.parts);
  if (dtype == RT_F32)
    rt::launch(colsum_stage1<float>, g1, block, 0, s, static_cast<const float*>(src), rows, cols, cp.chunk, cp.lr,
               vec, out1);
  else if (dtype == RT_BF16)
    rt::launch(colsum_stage1<unsigned short>, g1, block, 0, s, static_cast<const unsigned short*>(src), rows, cols,
               cp.chunk, cp.lr, vec, out1);
  else
    rt::launch(colsum_stage1<_Float16>, g1, block, 0, s, static_cast<const _Float16*>(src), rows, cols, cp.chunk,
               cp.lr, vec, out1);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || cp.parts == 1) return e;
  rt::launch(colsum_stage2, dim3((cols + 63) / 64), block, 0, s, scratch, cp.parts, cols, dst);
  return hipGetLastError();
}

hipError_t bias_add_launch(hipStream_t s, float* z, const float* b, int rows, int cols) {
  rt::launch(bias_add_kernel, dim3(grid_for((long long)rows * cols)), dim3(256), 0, s, z, b, rows, cols);
  return hipGetLastError();
}

hipError_t relu_launch(hipStream_t s, const float* x, float* y, size_t n) {
  rt::launch(relu_kernel, dim3(grid_for((long long)n)), dim3(256), 0, s, x, y, (long long)n);
  return hipGetLastError();
}

hipError_t relu_bwd_launch(hipStream_t s, const void* a, int a_dtype, float* delta, size_t n) {
  if (a_dtype == RT_F32)
    rt::launch(relu_bwd_kernel<float>, dim3(grid_for((long long)n)), dim3(256), 0, s,
                       static_cast<const float*>(a), delta, (long long)n);
  else if (a_dtype == RT_BF16)
    rt::launch(relu_bwd_kernel<unsigned short>, dim3(grid_for((long long)n)), dim3(256), 0, s,
                       static_cast<const unsigned short*>(a), delta, (long long)n);
  else
    rt::launch(relu_bwd_kernel<_Float16>, dim3(grid_for((long long)n)), dim3(256), 0, s,
                       static_cast<const _Float16*>(a), delta, (long long)n);
  return hipGetLastError();
}

hipError_t convert_launch(hipStream_t s, const void* src, int src_dtype, void* dst, int dst_dtype, size_t n) {
  rt::launch(convert_kernel, dim3(grid_for((long long)n)), dim3(256), 0, s, src, src_dtype, dst, dst_dtype,
                     (long long)n);
  return hipGetLastError();
}

hipError_t fill_i32_launch(hipStream_t s, int* p, int v, size_t n) {
  rt::launch(fill_i32_kernel, dim3(grid_for((long long)n)), dim3(256), 0, s, p, v, (long long)n);
  return hipGetLastError();
}

}  // namespace rt
