// bf16 / f16 GEMM with f32 accumulation on CDNA4 matrix cores
// (v_mfma_f32_16x16x32_bf16 / _f16).
//
// Behavioural spec: rtensor's f16-storage GEMM MM_F16 (crates/rtensor/src/gpu/
// mista.rs:58-323) -- half operands, f32 accumulate, the three layouts of the
// backward pass -- rebuilt for gfx950 matrix cores and extended to bf16.
//
// Block = 256 threads = 4 wave64s (2x2), block tile 128x128, K staged 64 at a
// time through LDS, double-buffered with register staging.  Both operand
// tiles live in LDS k-contiguous, [row][64 + 8 pad] halves, so every MFMA
// operand is one ds_read_b128 (8 consecutive k of one row; lane 16g+r reads
// row r, k = 8g..8g+7).  The 72-half (36-dword) row stride puts the 16 rows
// read by a lane group on distinct 4-bank groups.
//
// Operands stored K-contiguous (A of NN/NT, B of NT) are copied 8 halves per
// b128.  Operands stored M/N-contiguous (A of TN, B of NN/TN) are transposed
// on the way into LDS: each thread loads a 4(k) x 8(m) block as four b128 rows
// and writes eight 4-half k-runs (ds_write_b64), one per m.  For TN with a
// colsum target, the blocks of the first M tile sum their LDS B tile rows
// over k: db = 1ᵀ·δ in f32 with no extra HBM pass.

#include <algorithm>

#include "rt_internal.h"

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));
typedef unsigned int u2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;
constexpr int BM = 128, BN = 128, BK = 64, KPAD = 8;
constexpr int ROW = BK + KPAD;  // halves per LDS row

struct HalfArgs {
  const unsigned short* A;
  const unsigned short* B;
  void* C;
  int M, N, K, lda, ldb, ldc;
  int epi;
  const float* bias;
  const void* mask;
  int mask_bf16;  // mask dtype: 1 = bf16, 0 = f32
  int out_bf16;
  float* colsum;
  int k_per_split;
  long long split_stride;
  int tiles_m, tiles_n;
  int vec_a, vec_b;
};

__device__ inline float bf16_to_f32(unsigned short h) { return __uint_as_float((unsigned int)h << 16); }

__device__ inline unsigned short f32_to_bf16_rne(float x) {
  unsigned int u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

template <bool IS_BF16>
__device__ inline float half_to_f32(unsigned short h) {
  if constexpr (IS_BF16) return bf16_to_f32(h);
  else return (float)__builtin_bit_cast(_Float16, h);
}

// 8 consecutive halves (one b128) of a row-major matrix; zero outside.
__device__ inline u4 load8(const unsigned short* base, int ld, int row, int col, int rows, int cols, int vec) {
  const unsigned short* src = base + (long long)row * ld + col;
  if (vec && row < rows && col + 7 < cols) return *reinterpret_cast<const u4*>(src);
  unsigned short h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = (row < rows && col + e < cols) ? src[e] : (unsigned short)0;
  u4 v;
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = (unsigned int)h[2 * d] | ((unsigned int)h[2 * d + 1] << 16);
  return v;
}

// Staged global data of one operand tile for one thread (4 x b128).
struct Stage {
  u4 v[4];
};

// K-contiguous operand ([rows][K]): 128 rows x 64 k = 1024 b128, 4 per thread.
__device__ inline void load_kc(Stage& st, const unsigned short* base, int ld, int r0, int k0, int rows, int ke, int vec,
                               int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + kThreads * i;
    st.v[i] = load8(base, ld, r0 + (idx >> 3), k0 + 8 * (idx & 7), rows, ke, vec);
  }
}
__device__ inline void store_kc(const Stage& st, unsigned short* lds, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + kThreads * i;
    *reinterpret_cast<u4*>(&lds[(idx >> 3) * ROW + 8 * (idx & 7)]) = st.v[i];
  }
}

// M/N-contiguous operand ([K][rows]): thread owns k rows 4kq..4kq+3 and
// columns 8mq..8mq+7 of the 64 x 128 tile.
__device__ inline void load_mc(Stage& st, const unsigned short* base, int ld, int r0, int k0, int rows, int ke, int vec,
                               int tid) {
  const int kq = tid >> 4, mq = tid & 15;
#pragma unroll
  for (int j = 0; j < 4; ++j) st.v[j] = load8(base, ld, k0 + 4 * kq + j, r0 + 8 * mq, ke, rows, vec);
}
__device__ inline void store_mc(const Stage& st, unsigned short* lds, int tid) {
  const int kq = tid >> 4, mq = tid & 15;
#pragma unroll
  for (int mi = 0; mi < 8; ++mi) {
    const int d = mi >> 1;
    const int sh = (mi & 1) * 16;
    const unsigned int h0 = (st.v[0][d] >> sh) & 0xffffu, h1 = (st.v[1][d] >> sh) & 0xffffu;
    const unsigned int h2 = (st.v[2][d] >> sh) & 0xffffu, h3 = (st.v[3][d] >> sh) & 0xffffu;
    u2 w;
    w[0] = h0 | (h1 << 16);
    w[1] = h2 | (h3 << 16);
    *reinterpret_cast<u2*>(&lds[(8 * mq + mi) * ROW + 4 * kq]) = w;
  }
}

template <bool A_KC, bool B_KC, bool IS_BF16>
__global__ __launch_bounds__(kThreads) void gemm_half_kernel(HalfArgs p) {
  __shared__ __attribute__((aligned(16))) unsigned short sA[2][BM * ROW];
  __shared__ __attribute__((aligned(16))) unsigned short sB[2][BN * ROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

  // XCD-contiguous renumbering + grouped raster (as in the f32 kernel).
  int bid = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) bid = (bid & 7) * (nb >> 3) + (bid >> 3);
  constexpr int GROUP = 8;
  const int per_group = GROUP * p.tiles_n;
  const int grp = bid / per_group;
  const int first_m = grp * GROUP;
  const int gsize = min(p.tiles_m - first_m, GROUP);
  const int in_grp = bid - grp * per_group;
  const int tile_m = first_m + in_grp % gsize;
  const int tile_n = in_grp / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int kb = blockIdx.z * p.k_per_split;
  const int ke = min(p.K, kb + p.k_per_split);
  const int nk = ke > kb ? (ke - kb + BK - 1) / BK : 0;

  Stage sa, sb;
  auto load_tiles = [&](int k0) {
    if constexpr (A_KC) load_kc(sa, p.A, p.lda, m0, k0, p.M, ke, p.vec_a, tid);
    else load_mc(sa, p.A, p.lda, m0, k0, p.M, ke, p.vec_a, tid);
    if constexpr (B_KC) load_kc(sb, p.B, p.ldb, n0, k0, p.N, ke, p.vec_b, tid);
    else load_mc(sb, p.B, p.ldb, n0, k0, p.N, ke, p.vec_b, tid);
  };
  auto store_tiles = [&](int buf) {
    if constexpr (A_KC) store_kc(sa, sA[buf], tid);
    else store_mc(sa, sA[buf], tid);
    if constexpr (B_KC) store_kc(sb, sB[buf], tid);
    else store_mc(sb, sB[buf], tid);
  };

  f4 acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[t][u] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int buf) {
    const unsigned short* as = sA[buf];
    const unsigned short* bs = sB[buf];
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      u4 af[4], bf[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) af[t] = *reinterpret_cast<const u4*>(&as[(wm + 16 * t + r) * ROW + 32 * kk + 8 * g]);
#pragma unroll
      for (int u = 0; u < 4; ++u) bf[u] = *reinterpret_cast<const u4*>(&bs[(wn + 16 * u + r) * ROW + 32 * kk + 8 * g]);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if constexpr (IS_BF16)
            acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[t]),
                                                                __builtin_bit_cast(bf16x8, bf[u]), acc[t][u], 0, 0, 0);
          else
            acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, af[t]),
                                                               __builtin_bit_cast(f16x8, bf[u]), acc[t][u], 0, 0, 0);
        }
    }
  };

  const bool do_cs = !B_KC && p.colsum != nullptr && tile_m == 0 && tid < BN;
  float cs = 0.0f;

  if (nk > 0) {
    load_tiles(kb);
    store_tiles(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tiles(kb + (kt + 1) * BK);
      compute(cur);
      if constexpr (!B_KC) {
        if (do_cs) {
          const unsigned short* row = &sB[cur][tid * ROW];
#pragma unroll 8
          for (int k = 0; k < BK; ++k) cs += half_to_f32<IS_BF16>(row[k]);
        }
      }
      if (kt + 1 < nk) store_tiles(cur ^ 1);
      __syncthreads();
    }
  }

  if (do_cs && n0 + tid < p.N) p.colsum[(long long)blockIdx.z * p.N + n0 + tid] = cs;

  // Epilogue: acc[t][u][q] is C(m0+wm+16t+4g+q, n0+wn+16u+r).
  const bool partial = gridDim.z > 1;
  const bool out_bf16 = !partial && p.out_bf16;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int col = n0 + wn + 16 * u + r;
    if (col >= p.N) continue;
    const float bv = (!partial && p.bias != nullptr) ? p.bias[col] : 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = m0 + wm + 16 * t + 4 * g + q;
        if (row >= p.M) continue;
        float v = acc[t][u][q];
        const long long off = (long long)row * p.ldc + col;
        if (!partial) {
          if (p.epi == RT_EPI_BIAS || p.epi == RT_EPI_BIAS_RELU) {
            v = v + bv;
            if (p.epi == RT_EPI_BIAS_RELU) v = fmaxf(v, 0.0f);
          } else if (p.epi == RT_EPI_RELU_MASK) {
            const float mv = p.mask_bf16 ? bf16_to_f32(static_cast<const unsigned short*>(p.mask)[off])
                                         : static_cast<const float*>(p.mask)[off];
            if (!(mv > 0.0f)) v = 0.0f;
          }
        }
        if (out_bf16) static_cast<unsigned short*>(p.C)[off] = f32_to_bf16_rne(v);
        else static_cast<float*>(p.C)[off + (long long)blockIdx.z * p.split_stride] = v;
      }
    }
  }
}

template <bool A_KC, bool B_KC>
hipError_t launch_half(hipStream_t s, HalfArgs a, int splits, bool bf16) {
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  dim3 grid(a.tiles_m * a.tiles_n, 1, splits);
  if (bf16)
    hipLaunchKernelGGL((gemm_half_kernel<A_KC, B_KC, true>), grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((gemm_half_kernel<A_KC, B_KC, false>), grid, dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

namespace rt {

hipError_t gemm_half_launch(hipStream_t s, const GemmDesc& d) {
  if (d.in_dtype != RT_BF16 && d.in_dtype != RT_F16) return hipErrorInvalidValue;
  HalfArgs a{};
  a.A = static_cast<const unsigned short*>(d.A);
  a.B = static_cast<const unsigned short*>(d.B);
  a.C = d.C;
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  a.epi = d.epi;
  a.bias = d.bias;
  a.mask = d.mask;
  a.mask_bf16 = d.mask_dtype == RT_BF16;
  const int splits = d.splits < 1 ? 1 : d.splits;
  a.out_bf16 = splits == 1 && d.out_dtype == RT_BF16;
  a.colsum = splits > 1 ? d.colsum_partials : d.colsum;
  int kps = (d.K + splits - 1) / splits;
  kps = ((kps + BK - 1) / BK) * BK;
  a.k_per_split = splits > 1 ? kps : (d.K > 0 ? d.K : 1);
  a.split_stride = splits > 1 ? d.split_stride : 0;
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  a.vec_a = (d.lda % 8 == 0) && al16(d.A);
  a.vec_b = (d.ldb % 8 == 0) && al16(d.B);
  const bool bf16 = d.in_dtype == RT_BF16;
  switch (d.layout) {
    case RT_NN: return launch_half<true, false>(s, a, splits, bf16);
    case RT_TN: return launch_half<false, false>(s, a, splits, bf16);
    case RT_NT: return launch_half<true, true>(s, a, splits, bf16);
  }
  return hipErrorInvalidValue;
}

}  // namespace rt
