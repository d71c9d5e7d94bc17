// bf16 / f16 GEMM with f32 accumulation on CDNA4 matrix cores
// (v_mfma_f32_16x16x32_bf16 / _f16).
//
// Behavioural spec: rtensor's f16-storage GEMM MM_F16 (crates/rtensor/src/gpu/
// mista.rs:58-323) -- half operands, f32 accumulate, the three layouts of the
// backward pass -- rebuilt for gfx950 matrix cores and extended to bf16.
//
// Tiling.  Block = WGM x WGN wave64s, block tile BM x BN, K staged BK = 64 at
// a time through LDS, double-buffered with register staging (one barrier per
// K step).  Each wave owns (BM/WGM) x (BN/WGN) = TM x TN MFMA 16x16 tiles.
// Large problems use 256x256 blocks of 8 waves (64x128 wave tiles): two waves
// per SIMD hide each other's LDS and barrier latency (measured faster than one
// 128x128 wave per SIMD, which holds 256 accumulators per lane in AGPRs).
//
// Operands are copied into LDS exactly as they are stored (b128 copies, no
// transposition): K-contiguous operands as swizzled [row][64], M/N-contiguous
// ones as [k][cols+16].  An MFMA 16x16x32 operand is 8 halves per lane; lane
// 16g+r takes row/col r and k = 8g .. 8g+7 of the 32-wide step:
//   * K-contiguous tile: one ds_read_b128 of [row r][8g .. 8g+7] (swizzled);
//   * M/N-contiguous tile: two ds_read_b64_tr_b16.  Within each 16-lane
//     group, destination lane d = 4a+e receives element e of the 8-byte chunks
//     read by source lanes a, a+4, a+8, a+12; so when source lane s reads
//     [k = 8g + s/4 (+4)][c0 + 4(s%4) .. +3], lane d receives four
//     consecutive k of column c0 + d.
// All of these access patterns were measured conflict-free on gfx950 (a b128
// read moves twice the bytes per LDS cycle of a b64 read, so K-contiguous
// fragments use one b128).
//
// For TN with a colsum target, the blocks of the first M tile also sum their
// LDS B tiles over k (db = 1ᵀ·δ in f32, no extra HBM pass).  Split-K slices
// write f32 partial planes reduced in slice order by splitk_reduce.

#include <algorithm>
#include <type_traits>

#include "rt_internal.h"

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));
typedef unsigned int u2 __attribute__((ext_vector_type(2)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int BK = 64;    // K per LDS stage: two 32-wide MFMA k-steps
constexpr int MPAD = 16;  // M/N-contiguous rows: cols + 16 halves (8 banks)

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

// 8 consecutive halves of a row-major matrix at (row, col); zero outside.
// One 16-byte load whenever the operand is 16-byte aligned (vec) and the whole
// chunk is inside, so edge tiles stay vectorised except for their last chunk.
__device__ inline u4 load8(const unsigned short* base, int ld, int row, int col, int rows, int cols, bool vec) {
  const unsigned short* src = base + (long long)row * ld + col;
  if (vec && row < rows && col + 8 <= cols) return *reinterpret_cast<const u4*>(src);
  if (row >= rows) return u4{0u, 0u, 0u, 0u};
  unsigned short h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = (row < rows && col + e < cols) ? src[e] : (unsigned short)0;
  u4 v;
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = (unsigned int)h[2 * d] | ((unsigned int)h[2 * d + 1] << 16);
  return v;
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).  Used
// where the body indexes the accumulator array, which must stay in registers.
template <int B, int E, class F>
__device__ inline void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

__device__ inline u2 lds_tr(const unsigned short* p) {
  s4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p));
  return __builtin_bit_cast(u2, r);
}

// One operand of the block: tile geometry and its global <-> LDS movement.
// ROWS = BM (A) or BN (B); KC = stored K-contiguous.
//
// K-contiguous tiles are [row][64 halves] with no padding; the eight 16-byte
// granules of a row are stored at granule ^ ((row >> 1) & 7), which makes the
// fragment reads (16 consecutive rows, one granule each) and the tile writes
// conflict-free.  M/N-contiguous tiles are [k][ROWS + 16].
template <int ROWS, bool KC, int THREADS>
struct Operand {
  static constexpr int STRIDE = KC ? BK : (ROWS + MPAD);  // halves per LDS row
  static constexpr int ELEMS = KC ? ROWS * STRIDE : BK * STRIDE;
  static constexpr int CHUNKS = ROWS * BK / 8;  // b128 per tile
  static constexpr int PER_THREAD = CHUNKS / THREADS;
  static_assert(CHUNKS % THREADS == 0, "tile must split evenly over threads");

  u4 v[PER_THREAD];

  __device__ static inline int swz(int row, int granule) { return (granule ^ ((row >> 1) & 7)) * 8; }

  // Global (rows r0.., k0..) -> registers.
  __device__ inline void load(const unsigned short* base, int ld, int r0, int k0, int rows, int ke, bool vec,
                              int tid) {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int idx = tid + THREADS * i;
      if constexpr (KC) {
        const int row = idx / (BK / 8), kc = idx % (BK / 8);
        v[i] = load8(base, ld, r0 + row, k0 + 8 * kc, rows, ke, vec);
      } else {
        const int kk = idx / (ROWS / 8), c = idx % (ROWS / 8);
        v[i] = load8(base, ld, k0 + kk, r0 + 8 * c, ke, rows, vec);
      }
    }
  }
  __device__ inline void store(unsigned short* lds, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
      const int idx = tid + THREADS * i;
      if constexpr (KC) {
        const int row = idx / (BK / 8), kc = idx % (BK / 8);
        *reinterpret_cast<u4*>(&lds[row * STRIDE + swz(row, kc)]) = v[i];
      } else {
        *reinterpret_cast<u4*>(&lds[(idx / (ROWS / 8)) * STRIDE + 8 * (idx % (ROWS / 8))]) = v[i];
      }
    }
  }
  // MFMA operand (8 halves) of k-step kk (k in [32kk, 32kk+32)) for the 16
  // rows [rbase, rbase+16), lane (g, r): k = 32kk + 8g .. 32kk + 8g + 7.
  __device__ inline u4 frag(const unsigned short* lds, int kk, int rbase, int g, int r) const {
    if constexpr (KC) {
      const int row = rbase + r;
      return *reinterpret_cast<const u4*>(&lds[row * STRIDE + swz(row, 4 * kk + g)]);
    } else {
      const unsigned short* p = &lds[(32 * kk + 8 * g + (r >> 2)) * STRIDE + rbase + 4 * (r & 3)];
      const u2 lo = lds_tr(p), hi = lds_tr(p + 4 * STRIDE);
      return u4{lo[0], lo[1], hi[0], hi[1]};
    }
  }
};

template <int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC, bool IS_BF16>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_half_kernel(HalfArgs p) {
  constexpr int THREADS = 64 * WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;
  using OpA = Operand<BM, A_KC, THREADS>;
  using OpB = Operand<BN, B_KC, THREADS>;
  // One LDS buffer: A tiles (2 stages), then B tiles (2 stages); the
  // epilogue reuses all of it for staging.
  __shared__ __attribute__((aligned(16))) unsigned short smem[2 * OpA::ELEMS + 2 * OpB::ELEMS];
  auto sA = [&](int buf) { return smem + buf * OpA::ELEMS; };
  auto sB = [&](int buf) { return smem + 2 * OpA::ELEMS + buf * OpB::ELEMS; };

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;

  // XCD-contiguous renumbering + grouped raster (GROUP M tiles per band).
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

  OpA oa;
  OpB ob;
  auto load_tiles = [&](int k0) {
    oa.load(p.A, p.lda, m0, k0, p.M, ke, p.vec_a, tid);
    ob.load(p.B, p.ldb, n0, k0, p.N, ke, p.vec_b, tid);
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int u = 0; u < TN; ++u) acc[t][u] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int buf) {
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
    u4 bf[TN];
#pragma unroll
    for (int u = 0; u < TN; ++u) bf[u] = ob.frag(sB(buf), kk, wn + 16 * u, g, r);
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const u4 af = oa.frag(sA(buf), kk, wm + 16 * t, g, r);
#pragma unroll
      for (int u = 0; u < TN; ++u) {
        if constexpr (IS_BF16)
          acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af),
                                                              __builtin_bit_cast(bf16x8, bf[u]), acc[t][u], 0, 0, 0);
        else
          acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, af),
                                                             __builtin_bit_cast(f16x8, bf[u]), acc[t][u], 0, 0, 0);
      }
    }
    }
  };

  // Column sums of B over k (the bias gradient when B = δ), first M tile only.
  const bool do_cs = !B_KC && p.colsum != nullptr && tile_m == 0;
  float cs[(BN + THREADS - 1) / THREADS];
#pragma unroll
  for (int i = 0; i < (BN + THREADS - 1) / THREADS; ++i) cs[i] = 0.0f;

  if (nk > 0) {
    load_tiles(kb);
    oa.store(sA(0), tid);
    ob.store(sB(0), tid);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      if (kt + 1 < nk) load_tiles(kb + (kt + 1) * BK);
      compute(cur);
      if constexpr (!B_KC) {
        if (do_cs) {
#pragma unroll
          for (int i = 0; i < (BN + THREADS - 1) / THREADS; ++i) {
            const int col = tid + THREADS * i;
            if (col < BN) {
              const unsigned short* colp = &sB(cur)[col];
#pragma unroll 8
              for (int k = 0; k < BK; ++k) cs[i] += half_to_f32<IS_BF16>(colp[k * OpB::STRIDE]);
            }
          }
        }
      }
      if (kt + 1 < nk) {
        oa.store(sA(cur ^ 1), tid);
        ob.store(sB(cur ^ 1), tid);
      }
      __syncthreads();
    }
  }

  if (do_cs) {
#pragma unroll
    for (int i = 0; i < (BN + THREADS - 1) / THREADS; ++i) {
      const int col = tid + THREADS * i;
      if (col < BN && n0 + col < p.N) p.colsum[(long long)blockIdx.z * p.N + n0 + col] = cs[i];
    }
  }

  // Epilogue through LDS, one 16-row slab of the wave tile at a time: the
  // accumulators acc[t][u][q] = C(m0+wm+16t+4g+q, n0+wn+16u+r) are parked in
  // a per-wave [16][WN+4] f32 region, then each lane reads 4 consecutive
  // columns back, applies bias / ReLU / mask and stores 16 (f32) or 8 (bf16)
  // bytes.  Bounded register use and coalesced stores.
  constexpr int SROW = WN + 4;
  static_assert(16 * SROW * 4 * WGM * WGN <= (int)sizeof(smem), "epilogue staging must fit in LDS");
  float* stage = reinterpret_cast<float*>(smem) + wave * 16 * SROW;
  const bool partial = gridDim.z > 1;
  const bool out_bf16 = !partial && p.out_bf16;
  const bool vec_c = (p.ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0);
  float* Cf = static_cast<float*>(p.C) + (partial ? (long long)blockIdx.z * p.split_stride : 0);
  unsigned short* Ch = static_cast<unsigned short*>(p.C);
  __syncthreads();  // main-loop LDS reads are finished
  static_for<0, TM>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
#pragma unroll
    for (int u = 0; u < TN; ++u)
#pragma unroll
      for (int q = 0; q < 4; ++q) stage[(4 * g + q) * SROW + 16 * u + r] = acc[t][u][q];
    __syncthreads();
    constexpr int C4 = WN / 4;  // float4 columns per slab row
#pragma unroll
    for (int j = 0; j < 16 * C4 / 64; ++j) {
      const int idx = lane + 64 * j;
      const int rr = idx / C4, c4 = idx % C4;
      const int row = m0 + wm + 16 * t + rr;
      const int col = n0 + wn + 4 * c4;
      if (row >= p.M || col >= p.N) continue;
      f4 v = *reinterpret_cast<const f4*>(&stage[rr * SROW + 4 * c4]);
      const long long off = (long long)row * p.ldc + col;
      const int nv = min(4, p.N - col);
      if (!partial) {
        if (p.epi == RT_EPI_BIAS || p.epi == RT_EPI_BIAS_RELU) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (e < nv) v[e] = v[e] + p.bias[col + e];
            if (p.epi == RT_EPI_BIAS_RELU) v[e] = fmaxf(v[e], 0.0f);
          }
        } else if (p.epi == RT_EPI_RELU_MASK) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (e < nv) {
              const float mv = p.mask_bf16 ? bf16_to_f32(static_cast<const unsigned short*>(p.mask)[off + e])
                                           : static_cast<const float*>(p.mask)[off + e];
              if (!(mv > 0.0f)) v[e] = 0.0f;
            }
          }
        }
      }
      if (out_bf16) {
        if (vec_c && nv == 4) {
          u2 w;
          w[0] = (unsigned)f32_to_bf16_rne(v[0]) | ((unsigned)f32_to_bf16_rne(v[1]) << 16);
          w[1] = (unsigned)f32_to_bf16_rne(v[2]) | ((unsigned)f32_to_bf16_rne(v[3]) << 16);
          *reinterpret_cast<u2*>(&Ch[off]) = w;
        } else {
          for (int e = 0; e < nv; ++e) Ch[off + e] = f32_to_bf16_rne(v[e]);
        }
      } else {
        if (vec_c && nv == 4) *reinterpret_cast<f4*>(&Cf[off]) = v;
        else
          for (int e = 0; e < nv; ++e) Cf[off + e] = v[e];
      }
    }
    __syncthreads();
  });
}

template <int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC>
hipError_t launch_cfg(hipStream_t s, HalfArgs a, int splits, bool bf16) {
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  dim3 grid(a.tiles_m * a.tiles_n, 1, splits);
  dim3 block(64 * WGM * WGN);
  if (bf16)
    hipLaunchKernelGGL((gemm_half_kernel<BM, BN, WGM, WGN, A_KC, B_KC, true>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((gemm_half_kernel<BM, BN, WGM, WGN, A_KC, B_KC, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

template <bool A_KC, bool B_KC>
hipError_t launch_half(hipStream_t s, HalfArgs a, int splits, bool bf16) {
  // 256x256 blocks of 8 waves (2 per SIMD, 64x128 wave tiles) when they give
  // at least one block per CU -- the fastest measured shape for all three
  // layouts at 8192x4096x4096; 128x128 (4 waves) for mid sizes; 64x64 for
  // small ones.
  const long long tbig = (long long)((a.M + 255) / 256) * ((a.N + 255) / 256) * splits;
  const long long t128 = (long long)((a.M + 127) / 128) * ((a.N + 127) / 128) * splits;
  if (tbig >= 256) return launch_cfg<256, 256, 4, 2, A_KC, B_KC>(s, a, splits, bf16);
  if (t128 >= 128) return launch_cfg<128, 128, 2, 2, A_KC, B_KC>(s, a, splits, bf16);
  return launch_cfg<64, 64, 2, 2, A_KC, B_KC>(s, a, splits, bf16);
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
