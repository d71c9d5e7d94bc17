// f32 GEMM on CDNA4 matrix cores: v_mfma_f32_16x16x4_f32, f32 accumulate.
//
// Replaces rtensor's MM_FAST / MM_EPILOGO / MM_SPLITK WGSL kernels
// (crates/rtensor/src/gpu/gemm.rs:65-494, splitk.rs:33-237) for the three
// operand layouts of the training step:
//   NN  C = A·B      A [M,K] (K contiguous),  B [K,N] (N contiguous)  forward
//   TN  C = Aᵀ·B     A [K,M] (M contiguous),  B [K,N] (N contiguous)  dW = Xᵀ·δ
//   NT  C = A·Bᵀ     A [M,K] (K contiguous),  B [N,K] (K contiguous)  dX = δ·Wᵀ
//
// Block = 256 threads = 4 wave64s in a 2x2 arrangement; block tile BM x BN,
// K staged through LDS 32 at a time, double-buffered with register staging
// (one barrier per K step).  Each wave owns a (BM/2) x (BN/2) tile made of
// TM x TN MFMA 16x16 tiles.
//
// Lane/element mapping.  A 16x16x4 MFMA takes, in lane l = 16g + r, the A
// value (row r, k g) and the B value (k g, col r), and returns D(4g+q, r) in
// accumulator register q.  Rows, columns and k inside a wave tile may be
// permuted freely as long as A and B agree on k, so:
//   * MFMA row r of row-tile t is wave row TM*r + t, MFMA col r of col-tile u
//     is wave col TN*r + u: a lane's TM (TN) rows (cols) are adjacent, so one
//     LDS vector read serves all of its tiles when the operand is M (N)
//     contiguous, and the lane finally owns 4*TM adjacent rows x TN adjacent
//     columns of C (vector stores along N);
//   * within a 16-wide k chunk, MFMA step s of lane group g uses k = 4g + s,
//     so a lane's 4 steps are adjacent k when the operand is K contiguous (one
//     LDS vector read serves all four steps).
//
// Epilogues run on the accumulators in registers: bias, bias+ReLU (forward,
// mm_bias in gemm.rs:452-493) and the ReLU mask (δ ← acc ⊙ 1[A>0], fusing
// RELU_BWD, kernels.rs:119-131).  For TN with a colsum target the blocks of
// the first M tile also sum the B tiles they stage in LDS over K: that is
// db = 1ᵀ·δ (COLSUM, kernels.rs:182-199) at no extra HBM traffic.
// With more than one K slice, each slice writes a raw f32 partial plane and
// splitk_reduce sums the planes in slice order (REDUZ, splitk.rs:240-256):
// deterministic, no float atomics.

#include "device_util.h"
#include "optim_dev.h"
#include "rt_internal.h"

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

struct F32Args {
  const float* A;
  const float* B;
  float* C;
  int M, N, K, lda, ldb, ldc;
  int epi;
  const float* bias;
  const float* mask;
  float* colsum;  // [N], or [splits, N] partial rows when splits > 1
  int k_per_split;
  long long split_stride;
  int tiles_m, tiles_n, splits;
  int vec_a, vec_b, vec_c;
};

// Consecutive workgroups go to different XCDs (round robin over 8), each
// with its own L2.  Renumber so that every XCD gets a contiguous run of
// tile indices; the grouped raster below then keeps the tiles resident on
// one XCD sharing A rows and B columns.
__device__ inline int xcd_local(int bid, int nb) { return (nb & 7) == 0 ? (bid & 7) * (nb >> 3) + (bid >> 3) : bid; }

// Loads `cnt` consecutive floats (cnt = 1, 2 or 4) from LDS as one access.
template <int CNT>
__device__ inline void lds_read(const float* p, float* out) {
  if constexpr (CNT == 4) {
    f4 v = *reinterpret_cast<const f4*>(p);
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
  } else if constexpr (CNT == 2) {
    f2 v = *reinterpret_cast<const f2*>(p);
    out[0] = v[0]; out[1] = v[1];
  } else {
    out[0] = p[0];
  }
}

// Global -> register load of one float4 of an operand tile.  `row`/`col`
// index the stored matrix (row-major, leading dimension ld); the 4 elements
// run along the contiguous dimension.  Out-of-range elements read as 0.
__device__ inline f4 load4(const float* base, int ld, int row, int col, int rows, int cols, int vec) {
  const float* src = base + (long long)row * ld + col;
  if (vec && row < rows && col + 3 < cols) return *reinterpret_cast<const f4*>(src);
  f4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (row < rows && col + e < cols) ? src[e] : 0.0f;
  return v;
}

// One block's work: tile `bid` (already XCD-renumbered, in [0, tiles)) of
// K slice `split`.
//
// The block is KS groups of 2x2 waves.  Every group computes the whole
// BM x BN tile, each over its own share of every BK-wide K step (SUB
// sub-steps of 16), and at the end the groups' accumulators are summed
// through LDS in group order.  More waves per tile hide more load latency
// without shrinking the tile.  PF is how many K steps ahead the global loads
// run: 1 (one register stage) or 2 (two register stages, alternating).
template <int BM, int BN, bool A_KC, bool B_KC, int BK = 32, int KS = 1, int PF = 1>
struct F32Tile {
  static constexpr int THREADS = 256 * KS;
  static constexpr int PAD = 4;
  static constexpr int TM = BM / 32, TN = BN / 32;  // MFMA tiles per wave (2x2 waves of BM/2 x BN/2)
  static constexpr int A_STRIDE = A_KC ? (BK + PAD) : (BM + PAD);
  static constexpr int B_STRIDE = B_KC ? (BK + PAD) : (BN + PAD);
  static constexpr int A_ELEMS = A_KC ? BM * A_STRIDE : BK * A_STRIDE;
  static constexpr int B_ELEMS = B_KC ? BN * B_STRIDE : BK * B_STRIDE;
  static constexpr int PIPE = 2 * (A_ELEMS + B_ELEMS);  // floats: two stages of both operands
  static constexpr int RED = (KS - 1) * BM * BN;        // floats: accumulators of groups 1..KS-1
  static constexpr int SMEM = PIPE > RED ? PIPE : RED;
  static constexpr int A_LD = BM * BK / 4 / THREADS;  // float4 loads per thread per K step
  static constexpr int B_LD = BN * BK / 4 / THREADS;
  static constexpr int SUB = BK / 16 / KS;
  static_assert(BM % 32 == 0 && BN % 32 == 0 && BM <= 128 && BN <= 128, "tile");
  static_assert(A_LD >= 1 && B_LD >= 1 && BM * BK % (4 * THREADS) == 0 && BN * BK % (4 * THREADS) == 0,
                "tile loads must split evenly over the threads");
  static_assert(SUB >= 1 && BK % (16 * KS) == 0, "each group takes whole 16-wide sub-steps");
  static_assert(PF == 1 || PF == 2, "prefetch depth");

  __device__ static void run(const F32Args& p, int bid, int split, float* smem);
};

template <int BM, int BN, bool A_KC, bool B_KC, int BK, int KS, int PF>
__device__ void F32Tile<BM, BN, A_KC, B_KC, BK, KS, PF>::run(const F32Args& p, int bid, int split, float* smem) {
  float* const sA0 = smem;
  float* const sB0 = smem + 2 * A_ELEMS;
  auto sA = [&](int buf) { return sA0 + buf * A_ELEMS; };
  auto sB = [&](int buf) { return sB0 + buf * B_ELEMS; };

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int kg = wave >> 2, wq = wave & 3;  // K group, wave within the group
  const int g = lane >> 4, r = lane & 15;
  const int wm = (wq >> 1) * (BM / 2), wn = (wq & 1) * (BN / 2);

  constexpr int GROUP = 8;
  const int per_group = GROUP * p.tiles_n;
  const int grp = bid / per_group;
  const int first_m = grp * GROUP;
  const int gsize = min(p.tiles_m - first_m, GROUP);
  const int in_grp = bid - grp * per_group;
  const int tile_m = first_m + in_grp % gsize;
  const int tile_n = in_grp / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int kb = split * p.k_per_split;
  const int ke = min(p.K, kb + p.k_per_split);
  const int nk = ke > kb ? (ke - kb + BK - 1) / BK : 0;

  auto load_tiles = [&](f4 (&ra)[A_LD], f4 (&rb)[B_LD], int k0) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int idx = tid + THREADS * i;
      if constexpr (A_KC) {
        const int rr = idx / (BK / 4), kq = idx % (BK / 4);
        ra[i] = load4(p.A, p.lda, m0 + rr, k0 + 4 * kq, p.M, ke, p.vec_a);
      } else {
        constexpr int Q = BM / 4;
        const int kk = idx / Q, mq = idx % Q;
        ra[i] = load4(p.A, p.lda, k0 + kk, m0 + 4 * mq, ke, p.M, p.vec_a);
      }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int idx = tid + THREADS * i;
      if constexpr (B_KC) {
        const int rr = idx / (BK / 4), kq = idx % (BK / 4);
        rb[i] = load4(p.B, p.ldb, n0 + rr, k0 + 4 * kq, p.N, ke, p.vec_b);
      } else {
        constexpr int Q = BN / 4;
        const int kk = idx / Q, nq = idx % Q;
        rb[i] = load4(p.B, p.ldb, k0 + kk, n0 + 4 * nq, ke, p.N, p.vec_b);
      }
    }
  };
  auto store_tiles = [&](const f4 (&ra)[A_LD], const f4 (&rb)[B_LD], int buf) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int idx = tid + THREADS * i;
      if constexpr (A_KC) {
        *reinterpret_cast<f4*>(&sA(buf)[(idx / (BK / 4)) * A_STRIDE + 4 * (idx % (BK / 4))]) = ra[i];
      } else {
        constexpr int Q = BM / 4;
        *reinterpret_cast<f4*>(&sA(buf)[(idx / Q) * A_STRIDE + 4 * (idx % Q)]) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int idx = tid + THREADS * i;
      if constexpr (B_KC) {
        *reinterpret_cast<f4*>(&sB(buf)[(idx / (BK / 4)) * B_STRIDE + 4 * (idx % (BK / 4))]) = rb[i];
      } else {
        constexpr int Q = BN / 4;
        *reinterpret_cast<f4*>(&sB(buf)[(idx / Q) * B_STRIDE + 4 * (idx % Q)]) = rb[i];
      }
    }
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int u = 0; u < TN; ++u) acc[t][u] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int buf) {
    const float* as = sA(buf);
    const float* bs = sB(buf);
#pragma unroll
    for (int s2 = 0; s2 < SUB; ++s2) {
      const int ss = kg * SUB + s2;
      float af[TM][4], bf[TN][4];
      if constexpr (A_KC) {
#pragma unroll
        for (int t = 0; t < TM; ++t) lds_read<4>(&as[(wm + TM * r + t) * A_STRIDE + ss * 16 + 4 * g], af[t]);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float tmp[TM];
          lds_read<TM>(&as[(ss * 16 + 4 * g + s) * A_STRIDE + wm + TM * r], tmp);
#pragma unroll
          for (int t = 0; t < TM; ++t) af[t][s] = tmp[t];
        }
      }
      if constexpr (B_KC) {
#pragma unroll
        for (int u = 0; u < TN; ++u) lds_read<4>(&bs[(wn + TN * r + u) * B_STRIDE + ss * 16 + 4 * g], bf[u]);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float tmp[TN];
          lds_read<TN>(&bs[(ss * 16 + 4 * g + s) * B_STRIDE + wn + TN * r], tmp);
#pragma unroll
          for (int u = 0; u < TN; ++u) bf[u][s] = tmp[u];
        }
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int t = 0; t < TM; ++t)
#pragma unroll
          for (int u = 0; u < TN; ++u)
            acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[t][s], bf[u][s], acc[t][u], 0, 0, 0);
    }
  };

  // Column sums of B (the bias gradient when B = δ), from the LDS tiles of
  // the first M tile's blocks, summed over k in increasing order.
  const bool do_cs = !B_KC && p.colsum != nullptr && tile_m == 0 && tid < BN;
  float cs = 0.0f;
  auto colsum = [&](int buf) {
    if constexpr (!B_KC) {
      if (do_cs) {
        const float* bs = sB(buf);
#pragma unroll 8
        for (int kk = 0; kk < BK; ++kk) cs += bs[kk * B_STRIDE + tid];
      }
    }
  };

  if (nk > 0) {
    if constexpr (PF == 1) {
      f4 ra[A_LD], rb[B_LD];
      load_tiles(ra, rb, kb);
      store_tiles(ra, rb, 0);
      __syncthreads();
      for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_tiles(ra, rb, kb + (kt + 1) * BK);
        compute(cur);
        colsum(cur);
        if (kt + 1 < nk) store_tiles(ra, rb, cur ^ 1);
        __syncthreads();
      }
    } else {
      // Register stage j holds K step kt + j; the loads of step kt + 2 are
      // issued before step kt computes and stored after step kt + 1 does.
      f4 ra0[A_LD], rb0[B_LD], ra1[A_LD], rb1[B_LD];
      load_tiles(ra0, rb0, kb);
      if (nk > 1) load_tiles(ra1, rb1, kb + BK);
      store_tiles(ra0, rb0, 0);
      __syncthreads();
      auto iter = [&](int kt, f4 (&la)[A_LD], f4 (&lb)[B_LD], const f4 (&sa)[A_LD], const f4 (&sb)[B_LD]) {
        const int cur = kt & 1;
        if (kt + 2 < nk) load_tiles(la, lb, kb + (kt + 2) * BK);
        compute(cur);
        colsum(cur);
        if (kt + 1 < nk) store_tiles(sa, sb, cur ^ 1);
        __syncthreads();
      };
      for (int kt = 0; kt < nk; kt += 2) {
        iter(kt, ra0, rb0, ra1, rb1);
        if (kt + 1 < nk) iter(kt + 1, ra1, rb1, ra0, rb0);
      }
    }
  }

  if (do_cs && n0 + tid < p.N) p.colsum[(long long)split * p.N + n0 + tid] = cs;

  if constexpr (KS > 1) {
    // Groups 1.. park their accumulators (the main loop ended on a barrier,
    // so the pipeline buffers are free); group 0 adds them in group order.
    constexpr int PER = TM * TN * 4;
    if (kg > 0) {
      float* dst = smem + ((kg - 1) * 4 + wq) * PER * 64 + lane;
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
          for (int q = 0; q < 4; ++q) dst[((t * TN + u) * 4 + q) * 64] = acc[t][u][q];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int j = 1; j < KS; ++j) {
      const float* src = smem + ((j - 1) * 4 + wq) * PER * 64 + lane;
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[t][u][q] += src[((t * TN + u) * 4 + q) * 64];
    }
  }

  // Epilogue.  Lane owns rows m0+wm+TM*(4g+q)+t and columns n0+wn+TN*r+u.
  const bool partial = p.splits > 1;
  float* Cout = p.C + (long long)split * p.split_stride;
  const int col0 = n0 + wn + TN * r;
  float bias_v[TN];
#pragma unroll
  for (int u = 0; u < TN; ++u)
    bias_v[u] = (!partial && p.bias != nullptr && col0 + u < p.N) ? p.bias[col0 + u] : 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int row = m0 + wm + TM * (4 * g + q) + t;
      if (row >= p.M) continue;
      float v[TN];
#pragma unroll
      for (int u = 0; u < TN; ++u) v[u] = acc[t][u][q];
      if (!partial) {
        if (p.epi == RT_EPI_BIAS || p.epi == RT_EPI_BIAS_RELU) {
#pragma unroll
          for (int u = 0; u < TN; ++u) v[u] = v[u] + bias_v[u];
          if (p.epi == RT_EPI_BIAS_RELU) {
#pragma unroll
            for (int u = 0; u < TN; ++u) v[u] = fmaxf(v[u], 0.0f);
          }
        } else if (p.epi == RT_EPI_RELU_MASK) {
          const float* mrow = p.mask + (long long)row * p.ldc;
#pragma unroll
          for (int u = 0; u < TN; ++u)
            if (col0 + u < p.N && !(mrow[col0 + u] > 0.0f)) v[u] = 0.0f;
        }
      }
      float* dst = Cout + (long long)row * p.ldc + col0;
      if constexpr (TN == 4) {
        if (p.vec_c && col0 + 3 < p.N) {
          *reinterpret_cast<f4*>(dst) = f4{v[0], v[1], v[2], v[3]};
          continue;
        }
      }
#pragma unroll
      for (int u = 0; u < TN; ++u)
        if (col0 + u < p.N) dst[u] = v[u];
    }
  }
}

// ---------------------------------------------------------------- full-tile kernel
// For whole 64x64 tiles with 16-byte aligned operands the tiles go from
// global memory straight into LDS (buffer_load ... lds: lane l's 16 bytes
// land at the instruction's LDS base + 16 l), two stages of BK = 32 k.
// Within a stage the two 16-k halves are pipelined around one barrier:
//   A: read (k, half 1) fragments     | MFMAs of (k, half 0)
//   B: wait for stage k+1, barrier, DMA stage k+2 into stage k's buffer,
//      read (k+1, half 0) fragments   | MFMAs of (k, half 1)
// MFMAs take the operands swapped (D = op(B)·op(A)), so lane (g, r) ends with
// C(m0+wm+16t+r, n0+wn+16u+4g+q), q = 0..3: one float4 store per 16x16 tile.
//
// LDS layouts (unpadded, bank-conflict-free for the fragment reads):
//   K-contiguous [row][32]: 16-byte granule j of row r at j ^ ((r >> 1) & 7);
//     a fragment is one b128 read of row 16t + r at granule 4 half + g (the
//     four k of the lane's four MFMA steps);
//   M/N-contiguous [k][64]: 64-byte chunk c of row k at c ^ ((k >> 2) & 3); a
//     fragment is four b32 reads (k = 16 half + 4g + s, column 16u + r).
// A tile's plain stores (F32Dma::run's default epilogue).
struct NoEpi {
  static constexpr bool kOn = false;
};

struct F32Dma {
  static constexpr int BM = 64, BN = 64, BK = 32, THREADS = 256, WAVES = 4;
  static constexpr int TM = 2, TN = 2;                 // 16x16 MFMA tiles per wave (32x32 wave tile)
  static constexpr int ELEMS = 64 * BK;                // floats per operand per stage
  static constexpr int PER_WAVE = ELEMS / 256 / WAVES; // 1 KB DMA instructions per operand per wave
  static constexpr int STAGE = 2 * ELEMS;
  static constexpr int SMEM = 2 * STAGE;               // floats: two stages of both operands
  static constexpr int PER_STAGE = 2 * PER_WAVE;

  template <bool KC>
  struct Op {
    __amdgpu_buffer_rsrc_t rsrc;
    int voff;       // this lane's byte offset from the tile origin (first instruction)
    int istep;      // bytes between a lane's consecutive instructions (uniform)
    // Wave w's i-th instruction fills LDS floats [256 (4 i + w), +256); with
    // that spacing the lane's swizzle term is the same for every instruction.
    __device__ inline void init(const float* tile, int ld, int wave, int lane) {
      rsrc = rt_dev::raw_rsrc(tile);
      if constexpr (KC) {
        const int row = 8 * wave + (lane >> 3), slot = lane & 7;  // 8 rows of 128 B per instruction
        voff = 4 * (row * ld + 4 * (slot ^ ((row >> 1) & 7)));
        istep = 4 * 32 * ld;                                        // 32 rows
      } else {
        const int k = 4 * wave + (lane >> 4), s = lane & 15;        // 4 rows of 256 B per instruction
        voff = 4 * (k * ld + 16 * ((s >> 2) ^ ((k >> 2) & 3)) + 4 * (s & 3));
        istep = 4 * 16 * ld;                                        // 16 rows
      }
    }
    __device__ inline void issue(int stage_bytes, float* lds, int wave) const {
#pragma unroll
      for (int i = 0; i < PER_WAVE; ++i) rt_dev::dma16(rsrc, lds + 256 * (4 * i + wave), voff, stage_bytes + i * istep);
    }
    // Fragment of MFMA tile `base` (16 rows / columns) for k-half h: the
    // lane's four k values 16 h + 4 g + s, s = 0..3.
    __device__ static inline f4 frag(const float* lds, int h, int base, int g, int r) {
      if constexpr (KC) {
        const int row = base + r;
        return *reinterpret_cast<const f4*>(&lds[row * BK + 4 * ((4 * h + g) ^ ((row >> 1) & 7))]);
      } else {
        const int col = base + r;
        f4 v;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int k = 16 * h + 4 * g + s;  // (k >> 2) & 3 == g
          v[s] = lds[k * BM + 16 * ((col >> 4) ^ g) + (col & 15)];
        }
        return v;
      }
    }
    // Element (k, col) of an M/N-contiguous stage.
    __device__ static inline float at(const float* lds, int k, int col) {
      return lds[k * BM + 16 * ((col >> 4) ^ ((k >> 2) & 3)) + (col & 15)];
    }
  };

  template <bool A_KC, bool B_KC, class Epi = NoEpi>
  __device__ static void run(const F32Args& p, int bid, int split, float* smem, const Epi& e = Epi{});
};

template <int EPI>
__device__ __forceinline__ void f32_store_direct(const F32Args& p, const f4 (&acc)[2][2], int m0, int n0, int wm,
                                                 int wn, int g, int r, int split) {
  float* C = p.C + (p.splits > 1 ? (long long)split * p.split_stride : 0);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const long long row_off = (long long)(m0 + wm + 16 * t + r) * p.ldc;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int col = n0 + wn + 16 * u + 4 * g;
      f4 v = acc[t][u];
      if constexpr (EPI == RT_EPI_BIAS || EPI == RT_EPI_BIAS_RELU) {
        const f4 b = *reinterpret_cast<const f4*>(p.bias + col);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = v[e] + b[e];
          if constexpr (EPI == RT_EPI_BIAS_RELU) v[e] = fmaxf(v[e], 0.0f);
        }
      } else if constexpr (EPI == RT_EPI_RELU_MASK) {
        const f4 mk = *reinterpret_cast<const f4*>(p.mask + row_off + col);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (!(mk[e] > 0.0f)) v[e] = 0.0f;
      }
      *reinterpret_cast<f4*>(C + row_off + col) = v;
    }
  }
}

template <bool A_KC, bool B_KC, class Epi>
__device__ void F32Dma::run(const F32Args& p, int bid, int split, float* smem, const Epi& e) {
  using OpA = Op<A_KC>;
  using OpB = Op<B_KC>;
  auto sA = [&](int buf) { return smem + buf * STAGE; };
  auto sB = [&](int buf) { return smem + buf * STAGE + ELEMS; };

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;

  constexpr int GROUP = 8;
  const int per_group = GROUP * p.tiles_n;
  const int grp = bid / per_group;
  const int first_m = grp * GROUP;
  const int gsize = min(p.tiles_m - first_m, GROUP);
  const int in_grp = bid - grp * per_group;
  const int tile_m = first_m + in_grp % gsize;
  const int tile_n = in_grp / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int kb = split * p.k_per_split;
  const int nk = (min(p.K, kb + p.k_per_split) - kb) / BK;  // whole stages (checked by the host)

  OpA oa;
  OpB ob;
  oa.init(A_KC ? p.A + (long long)m0 * p.lda + kb : p.A + (long long)kb * p.lda + m0, p.lda, wave, lane);
  ob.init(B_KC ? p.B + (long long)n0 * p.ldb + kb : p.B + (long long)kb * p.ldb + n0, p.ldb, wave, lane);
  const int a_step = 4 * (A_KC ? BK : BK * p.lda);  // bytes per stage
  const int b_step = 4 * (B_KC ? BK : BK * p.ldb);
  auto issue = [&](int stage, int buf) {
    oa.issue(stage * a_step, sA(buf), wave);
    ob.issue(stage * b_step, sB(buf), wave);
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int u = 0; u < TN; ++u) acc[t][u] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto read_frags = [&](int buf, int h, f4 (&fa)[TM], f4 (&fb)[TN]) {
#pragma unroll
    for (int u = 0; u < TN; ++u) fb[u] = OpB::frag(sB(buf), h, wn + 16 * u, g, r);
#pragma unroll
    for (int t = 0; t < TM; ++t) fa[t] = OpA::frag(sA(buf), h, wm + 16 * t, g, r);
  };
  auto mfmas = [&](const f4 (&fa)[TM], const f4 (&fb)[TN]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < TM; ++t)
#pragma unroll
        for (int u = 0; u < TN; ++u)
          acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(fb[u][s], fa[t][s], acc[t][u], 0, 0, 0);
  };

  // Bias gradient (TN with a colsum target, first M tile): thread t sums
  // column t % 64 over the k rows 8 (t / 64) .. +7 of every stage; the four
  // partial rows are added in order at the end.
  const bool do_cs = !B_KC && p.colsum != nullptr && tile_m == 0;  // uniform over the block
  float cs = 0.0f;
  auto colsum = [&](int buf) {
    if constexpr (!B_KC) {
      if (do_cs) {
        const int col = tid & 63, k0 = 8 * (tid >> 6);
#pragma unroll
        for (int k = 0; k < 8; ++k) cs += OpB::at(sB(buf), k0 + k, col);
      }
    }
  };

  if (nk > 0) {
    f4 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    // Every B step waits for everything and issues one stage (past the last
    // stage it re-fetches stage nk-1 into a buffer nothing reads), so the
    // bookkeeping is the same in every stage.
    issue(0, 0);
    issue(min(1, nk - 1), 1);
    rt_dev::wait_vm<PER_STAGE>();
    rt_dev::barrier_lds();
    read_frags(0, 0, fa0, fb0);
    auto stage = [&](int k, auto bc) {
      constexpr int BUF = decltype(bc)::value;  // k % 2
      read_frags(BUF, 1, fa1, fb1);
      mfmas(fa0, fb0);
      colsum(BUF);
      rt_dev::wait_vm<0>();
      rt_dev::barrier_lds();  // stage k+1 everywhere; stage k no longer read
      issue(min(k + 2, nk - 1), BUF);
      read_frags(BUF ^ 1, 0, fa0, fb0);  // (k+1, half 0); discarded after the last stage
      mfmas(fa1, fb1);
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    for (int k = 0; k < nk; k += 2) {
      stage(k, B0{});
      if (k + 1 < nk) stage(k + 1, B1{});
    }
  }

  if (do_cs) {
    __syncthreads();  // main-loop LDS reads are finished
    float* red = smem;  // [4][64]
    red[tid] = cs;
    __syncthreads();
    if (tid < 64) {
      const float v = ((red[tid] + red[64 + tid]) + red[128 + tid]) + red[192 + tid];
      if constexpr (Epi::kOn)
        e.bias(p, n0 + tid, v);
      else
        p.colsum[(long long)split * p.N + n0 + tid] = v;
    }
  }

  if constexpr (Epi::kOn) return e.tile(p, acc, m0, n0, wm, wn, g, r);
  if (p.splits > 1) return f32_store_direct<RT_EPI_NONE>(p, acc, m0, n0, wm, wn, g, r, split);
  switch (p.epi) {
    case RT_EPI_BIAS: return f32_store_direct<RT_EPI_BIAS>(p, acc, m0, n0, wm, wn, g, r, split);
    case RT_EPI_BIAS_RELU: return f32_store_direct<RT_EPI_BIAS_RELU>(p, acc, m0, n0, wm, wn, g, r, split);
    case RT_EPI_RELU_MASK: return f32_store_direct<RT_EPI_RELU_MASK>(p, acc, m0, n0, wm, wn, g, r, split);
    default: return f32_store_direct<RT_EPI_NONE>(p, acc, m0, n0, wm, wn, g, r, split);
  }
}

// Adapter so the single and pair kernels can run an F32Dma layout like an
// F32Tile.
template <bool A_KC, bool B_KC>
struct F32DmaTile {
  static constexpr int THREADS = F32Dma::THREADS;
  static constexpr int SMEM = F32Dma::SMEM;
  __device__ static void run(const F32Args& p, int bid, int split, float* smem) {
    F32Dma::run<A_KC, B_KC>(p, bid, split, smem);
  }
};

template <class T>
__global__ __launch_bounds__(T::THREADS) void gemm_f32_kernel(F32Args p) {
  __shared__ __attribute__((aligned(16))) float smem[T::SMEM];
  T::run(p, xcd_local(blockIdx.x, gridDim.x), blockIdx.z, smem);
}

// C = A·Bᵀ (NT) for K <= 16, one 64x64 block of C per workgroup: the
// block's 64 rows of A and 64 rows of B go to LDS, and thread t computes
// rows 4(t/16) .. +3, columns 4(t%16) .. +3 with K multiply-adds each, in k
// order, then applies the epilogue.  A rank-K update is a stream of C (and
// of the mask): the MFMA tile's K pipeline padded to 32 only adds latency.
struct F32RankK {
  static constexpr int THREADS = 256;
  static constexpr int KMAX = 16;
  static constexpr int LD = KMAX + 1;  // LDS row stride (floats)
  static constexpr int SMEM = 2 * 64 * LD;
  __device__ static void run(const F32Args& p, int bid, int, float* smem) {
    float* sa = smem;
    float* sb = smem + 64 * LD;
    const int tile_m = bid / p.tiles_n, tile_n = bid - tile_m * p.tiles_n;
    const int m0 = 64 * tile_m, n0 = 64 * tile_n, K = p.K, tid = threadIdx.x;
    const int r0 = 4 * (tid / 16), c0 = 4 * (tid % 16);
    const int col = n0 + c0;
    // The ReLU mask of this thread's outputs, loaded first so that its
    // latency runs under the operand staging and the multiply-adds.
    const bool vec_mask = p.epi == RT_EPI_RELU_MASK && p.vec_c && col + 4 <= p.N;
    f4 mkv[4];
    if (vec_mask) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        mkv[i] = m0 + r0 + i < p.M ? *reinterpret_cast<const f4*>(p.mask + (long long)(m0 + r0 + i) * p.ldc + col)
                                   : f4{0, 0, 0, 0};
    }
    for (int i = tid; i < 64 * K; i += THREADS) {
      const int r = i / K, k = i - r * K;
      sa[r * LD + k] = m0 + r < p.M ? p.A[(long long)(m0 + r) * p.lda + k] : 0.0f;
      sb[r * LD + k] = n0 + r < p.N ? p.B[(long long)(n0 + r) * p.ldb + k] : 0.0f;
    }
    __syncthreads();
    f4 acc[4] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}, f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
    for (int k = 0; k < K; ++k) {
      const f4 b = f4{sb[c0 * LD + k], sb[(c0 + 1) * LD + k], sb[(c0 + 2) * LD + k], sb[(c0 + 3) * LD + k]};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] += sa[(r0 + i) * LD + k] * b;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = m0 + r0 + i;
      if (row >= p.M) break;
      f4 v = acc[i];
      float* c = p.C + (long long)row * p.ldc + col;
      const float* mk = p.mask + (long long)row * p.ldc + col;
      if (p.vec_c && col + 4 <= p.N) {
        if (p.epi == RT_EPI_BIAS || p.epi == RT_EPI_BIAS_RELU) {
          v += *reinterpret_cast<const f4*>(p.bias + col);
          if (p.epi == RT_EPI_BIAS_RELU)
            for (int q = 0; q < 4; ++q) v[q] = fmaxf(v[q], 0.0f);
        } else if (vec_mask) {
          for (int q = 0; q < 4; ++q)
            if (!(mkv[i][q] > 0.0f)) v[q] = 0.0f;
        }
        *reinterpret_cast<f4*>(c) = v;
      } else {
        for (int q = 0; q < 4 && col + q < p.N; ++q) {
          float x = v[q];
          if (p.epi == RT_EPI_BIAS || p.epi == RT_EPI_BIAS_RELU) {
            x = x + p.bias[col + q];
            if (p.epi == RT_EPI_BIAS_RELU) x = fmaxf(x, 0.0f);
          } else if (p.epi == RT_EPI_RELU_MASK && !(mk[q] > 0.0f)) {
            x = 0.0f;
          }
          c[q] = x;
        }
      }
    }
  }
};

// Two independent GEMMs in one launch (horizontal fusion): blocks
// [0, n0) run problem 0, the rest problem 1, each problem's split index
// folded into its block range.  n0 is a multiple of 8 so both problems are
// spread evenly over the XCDs; problem 0 is dispatched first.
template <class T0, class T1>
__global__ __launch_bounds__(T0::THREADS) void gemm_f32_pair_kernel(F32Args p0, F32Args p1, int n0) {
  static_assert(T0::THREADS == T1::THREADS, "one block size");
  constexpr int S = T0::SMEM > T1::SMEM ? T0::SMEM : T1::SMEM;
  __shared__ __attribute__((aligned(16))) float smem[S];
  const int b = blockIdx.x;
  if (b < n0) {
    const int tiles = p0.tiles_m * p0.tiles_n;
    const int nb = tiles * p0.splits;
    if (b >= nb) return;  // padding up to a multiple of 8
    const int loc = xcd_local(b, nb);
    T0::run(p0, loc % tiles, loc / tiles, smem);
  } else {
    const int tiles = p1.tiles_m * p1.tiles_n;
    const int nb = tiles * p1.splits;
    const int loc = xcd_local(b - n0, nb);
    T1::run(p1, loc % tiles, loc / tiles, smem);
  }
}

// A GEMM and an optimizer update that does not touch its operands in one
// launch: blocks [0, n_gemm) run the GEMM's (tile, K slice) items, the rest
// the optimizer blocks of b.  The GEMM is dispatched first; the update, which
// is HBM-bound, runs on the CUs next to its MFMA-bound tiles.
template <class T>
__global__ __launch_bounds__(T::THREADS) void gemm_f32_opt_kernel(F32Args p, rt_opt::OptBatch b, int n_gemm) {
  static_assert(T::THREADS == rt_opt::kThreads, "one block size");
  __shared__ __attribute__((aligned(16))) float smem[T::SMEM];
  const int blk = blockIdx.x;
  if (blk < n_gemm) {
    const int tiles = p.tiles_m * p.tiles_n;
    const int loc = xcd_local(blk, n_gemm);
    T::run(p, loc % tiles, loc / tiles, smem);
  } else {
    rt_opt::optimizer_block<false>(b, blk - n_gemm);
  }
}

// The update of the layer whose dW this unsplit TN launch computes, done by
// the tiles themselves: an element's gradient is final in the tile that
// computed it, so the tile stores it and updates the parameter and its
// optimizer state there, with the optimizer's per-element arithmetic (same
// bits as the separate update); the first row of tiles does the same for the
// bias from its column sums.  w / b index like dW / db (w.n = M·N, ldc = N).
struct UpdEpi {
  static constexpr bool kOn = true;
  rt::OptTensor w, b;
  rt::OptParams P;
  __device__ void tile(const F32Args& p, const f4 (&acc)[2][2], int m0, int n0, int wm, int wn, int g,
                       int r) const {
    const bool skip = rt_opt::skipped(P);
    const rt_opt::Coef c = rt_opt::coef(P);
    const bool adam = P.kind == 0, has_m = w.m != nullptr;
    long long idx[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) idx[t][u] = (long long)(m0 + wm + 16 * t + r) * p.ldc + n0 + wn + 16 * u + 4 * g;
    // Every load of θ and the state first, so that they go out together
    // (the stores below could alias them as far as the compiler knows).
    f4 th[2][2], m[2][2], v[2][2];
    if (!skip) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          th[t][u] = *reinterpret_cast<const f4*>(w.theta + idx[t][u]);
          m[t][u] = has_m ? *reinterpret_cast<const f4*>(w.m + idx[t][u]) : f4{0, 0, 0, 0};
          v[t][u] = adam ? *reinterpret_cast<const f4*>(w.v + idx[t][u]) : f4{0, 0, 0, 0};
        }
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const long long i = idx[t][u];
        const f4 gv = acc[t][u];
        *reinterpret_cast<f4*>(p.C + i) = gv;
        if (skip) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float te = th[t][u][q], me = m[t][u][q], ve = v[t][u][q];
          rt_opt::update(P, c, gv[q], te, &me, &ve);
          th[t][u][q] = te;
          m[t][u][q] = me;
          v[t][u][q] = ve;
        }
        *reinterpret_cast<f4*>(w.theta + i) = th[t][u];
        if (has_m) *reinterpret_cast<f4*>(w.m + i) = m[t][u];
        if (adam) *reinterpret_cast<f4*>(w.v + i) = v[t][u];
      }
  }
  __device__ void bias(const F32Args& p, int col, float gv) const {
    p.colsum[col] = gv;
    if (rt_opt::skipped(P)) return;
    const bool adam = P.kind == 0, has_m = b.m != nullptr;
    float th = b.theta[col], m = has_m ? b.m[col] : 0.0f, v = adam ? b.v[col] : 0.0f;
    rt_opt::update(P, rt_opt::coef(P), gv, th, &m, &v);
    b.theta[col] = th;
    if (has_m) b.m[col] = m;
    if (adam) b.v[col] = v;
  }
};

// gemm_f32_opt_kernel on 64x64 DMA tiles of an unsplit TN product whose
// tiles also update their own layer (UpdEpi).
__global__ __launch_bounds__(F32Dma::THREADS) void gemm_f32_opt_upd_kernel(F32Args p, rt_opt::OptBatch b, int n_gemm,
                                                                          UpdEpi u) {
  static_assert(F32Dma::THREADS == rt_opt::kThreads, "one block size");
  __shared__ __attribute__((aligned(16))) float smem[F32Dma::SMEM];
  const int blk = blockIdx.x;
  if (blk < n_gemm) {
    F32Dma::run<false, false>(p, xcd_local(blk, n_gemm), 0, smem, u);
  } else {
    rt_opt::optimizer_block<false>(b, blk - n_gemm);
  }
}

// Two such products (two layers' dW, each updating its own layer) and the
// optimizer blocks of b in one launch: blocks [0, n0) problem 0 (n0 a
// multiple of 8, the padding idle), [n0, n1) problem 1, the rest the update.
__global__ __launch_bounds__(F32Dma::THREADS) void gemm_f32_opt_upd2_kernel(F32Args p0, F32Args p1, rt_opt::OptBatch b,
                                                                           int n0, int n1, UpdEpi u0, UpdEpi u1) {
  static_assert(F32Dma::THREADS == rt_opt::kThreads, "one block size");
  __shared__ __attribute__((aligned(16))) float smem[F32Dma::SMEM];
  const int blk = blockIdx.x;
  if (blk < n0) {
    const int nb = p0.tiles_m * p0.tiles_n;
    if (blk >= nb) return;  // padding up to a multiple of 8
    F32Dma::run<false, false>(p0, xcd_local(blk, nb), 0, smem, u0);
  } else if (blk < n1) {
    F32Dma::run<false, false>(p1, xcd_local(blk - n0, n1 - n0), 0, smem, u1);
  } else {
    rt_opt::optimizer_block<false>(b, blk - n1);
  }
}

// The first cs_blocks blocks each take 256 columns of the column sums: they
// start first, so their chains of loads run under the plane sums; the rest
// sum the planes (grid-stride over M*N).
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ part, int S, long long stride,
                                                             int M, int N, float* C, int ldc, int epi,
                                                             const float* bias, const float* mask,
                                                             const float* __restrict__ cs_part, int cs_rows,
                                                             float* cs, int cs_blocks, int vec4) {
  if ((int)blockIdx.x < cs_blocks) {
    const long long j = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= N) return;
    // Slice s's column sum: cs_part[s, j], or with shares the cs_rows rows
    // cs_part[s, t, j] added in order from zero; then the slices in order.
    // Element e = s * rows + t of that sequence is at cs_part[e * N + j]; the
    // loads go out 16 at a time and the adds follow in sequence order.
    const int rows = cs_rows > 0 ? cs_rows : 1;
    const long long n = (long long)S * rows;
    float v = 0.0f, w = 0.0f;
    int t = 0;          // row of element e within its slice
    bool first = true;  // e lies in slice 0
    for (long long e0 = 0; e0 < n; e0 += 16) {
      float x[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) x[u] = e0 + u < n ? cs_part[(e0 + u) * N + j] : 0.0f;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (e0 + u >= n) break;
        w = cs_rows > 0 ? (t == 0 ? 0.0f : w) + x[u] : x[u];
        if (++t == rows) {
          v = first ? w : v + w;
          first = false;
          t = 0;
        }
      }
    }
    cs[j] = v;
    return;
  }
  const int plane_blocks = (int)gridDim.x - cs_blocks;
  const long long total = (long long)M * N;
  const long long first = (blockIdx.x - cs_blocks) * (long long)blockDim.x + threadIdx.x;
  const long long step = (long long)plane_blocks * blockDim.x;
  if (vec4) {
    // Four consecutive elements of one row per thread (N, ldc, stride and
    // every pointer 16-byte aligned); each element's sum is the scalar one.
    const f4* P = reinterpret_cast<const f4*>(part);
    const long long s4 = stride / 4, total4 = total / 4;
    for (long long i = first; i < total4; i += step) {
      f4 v = P[i];
      int s = 1;
      for (; s + 8 <= S; s += 8) {
        f4 t[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = P[(long long)(s + j) * s4 + i];
#pragma unroll
        for (int j = 0; j < 8; ++j) v += t[j];
      }
      f4 t[7];
#pragma unroll
      for (int j = 0; j < 7; ++j) t[j] = s + j < S ? P[(long long)(s + j) * s4 + i] : f4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < 7; ++j)
        if (s + j < S) v += t[j];
      const long long e = 4 * i, row = e / N;
      const int col = (int)(e - row * N);
      if (epi == RT_EPI_BIAS || epi == RT_EPI_BIAS_RELU) {
        const f4 b = *reinterpret_cast<const f4*>(bias + col);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[q] = v[q] + b[q];
          if (epi == RT_EPI_BIAS_RELU) v[q] = fmaxf(v[q], 0.0f);
        }
      } else if (epi == RT_EPI_RELU_MASK) {
        const f4 mk = *reinterpret_cast<const f4*>(mask + row * ldc + col);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (!(mk[q] > 0.0f)) v[q] = 0.0f;
      }
      *reinterpret_cast<f4*>(C + row * ldc + col) = v;
    }
    return;
  }
  for (long long i = first; i < total; i += step) {
    // v = plane 0 + plane 1 + ... in slice order; the loads go out 8 at a
    // time (the last S - 1 mod 8 together) so the chain of adds does not
    // wait on one load after another.
    float v = part[i];
    int s = 1;
    for (; s + 8 <= S; s += 8) {
      float t[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) t[j] = part[(long long)(s + j) * stride + i];
#pragma unroll
      for (int j = 0; j < 8; ++j) v += t[j];
    }
    float t[7];
#pragma unroll
    for (int j = 0; j < 7; ++j) t[j] = s + j < S ? part[(long long)(s + j) * stride + i] : 0.0f;
#pragma unroll
    for (int j = 0; j < 7; ++j)
      if (s + j < S) v += t[j];
    long long o = i;  // offset in C
    if (epi != RT_EPI_NONE || ldc != N) {
      const long long row = i / N;
      const int col = (int)(i - row * N);
      o = row * ldc + col;
      if (epi == RT_EPI_BIAS || epi == RT_EPI_BIAS_RELU) {
        v = v + bias[col];
        if (epi == RT_EPI_BIAS_RELU) v = fmaxf(v, 0.0f);
      } else if (epi == RT_EPI_RELU_MASK) {
        if (!(mask[o] > 0.0f)) v = 0.0f;
      }
    }
    C[o] = v;
  }
}

template <int BM, int BN, bool A_KC, bool B_KC, int BK = 32, int KS = 1, int PF = 1>
hipError_t launch_f32(hipStream_t s, F32Args a) {
  using T = F32Tile<BM, BN, A_KC, B_KC, BK, KS, PF>;
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  dim3 grid(a.tiles_m * a.tiles_n, 1, a.splits);
  rt::launch((gemm_f32_kernel<T>), grid, dim3(T::THREADS), 0, s, a);
  return hipGetLastError();
}

// 128x128 tiles when they alone give at least two waves of 256 CUs,
// otherwise 64x64 (4x the workgroups) so small GEMMs still fill the chip;
// 64x32 for narrow outputs.
enum TileCfg { kT128, kT64x32, kT64 };
TileCfg pick_tile(const F32Args& a) {
  const long long t128 = (long long)((a.M + 127) / 128) * ((a.N + 127) / 128) * a.splits;
  if (t128 >= 512) return kT128;
  if (a.N <= 32) return kT64x32;
  return kT64;
}

// Whole 64x64 tiles, every K slice (the last included) a multiple of 32,
// 16-byte aligned rows and pointers for the DMA and the float4 epilogue, and
// operands addressable with 32-bit byte offsets.
template <bool A_KC, bool B_KC>
bool dma_ok(const F32Args& a) {
  const int last = a.K - (a.splits - 1) * a.k_per_split;
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  const long long lim = 1LL << 31;
  const bool epi_ok = (a.epi != RT_EPI_BIAS && a.epi != RT_EPI_BIAS_RELU) || al(a.bias);
  const bool mask_ok = a.epi != RT_EPI_RELU_MASK || al(a.mask);
  return a.M % 64 == 0 && a.N % 64 == 0 && a.k_per_split % 32 == 0 && last > 0 && last % 32 == 0 && a.vec_a &&
         a.vec_b && a.vec_c && epi_ok && mask_ok && (long long)(A_KC ? a.M : a.K) * a.lda * 4 < lim &&
         (long long)(B_KC ? a.N : a.K) * a.ldb * 4 < lim;
}

template <bool A_KC, bool B_KC>
hipError_t launch_dma(hipStream_t s, F32Args a) {
  using T = F32DmaTile<A_KC, B_KC>;
  a.tiles_m = a.M / 64;
  a.tiles_n = a.N / 64;
  dim3 grid(a.tiles_m * a.tiles_n, 1, a.splits);
  rt::launch((gemm_f32_kernel<T>), grid, dim3(T::THREADS), 0, s, a);
  return hipGetLastError();
}

// Skinny products: at most 64 rows of output, A K-contiguous (the NN
// forward and the NT dX of a small batch).  A block owns 16 output columns
// over the whole K; its 8 waves take consecutive runs of 16-k sub-blocks and
// issue the loads of up to 8 sub-blocks together ahead of their MFMAs, so
// the K loop is a few memory round trips instead of one per step.  The
// waves' partial tiles are added in LDS in wave order, then the epilogue.
// One launch and no partial planes, where split-K needs a reduction launch.
//
// Within a sub-block at k0, lane (g, r) feeds MFMA step q the element
// k0 + 4g + q of its A row and B column (one float4 of A per sub-block); the
// accumulator of row block rb holds C[16 rb + 4g + q][n0 + r].
constexpr int kSkinnyWaves = 8, kSkinnyChunk = 8;

template <int RB, bool B_KC>
__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_f32_skinny_kernel(F32Args p) {
  __shared__ float red[kSkinnyWaves * RB * 16 * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r = lane & 15;
  const int n0 = blockIdx.x * 16;
  const int nsub = p.K / 16;  // K % 16 == 0 (checked by the host)
  const int per = (nsub + kSkinnyWaves - 1) / kSkinnyWaves;
  const int s_end = min(nsub, (wave + 1) * per);

  f4 acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int sb = wave * per; sb < s_end; sb += kSkinnyChunk) {
    f4 a[kSkinnyChunk][RB], b[kSkinnyChunk];
#pragma unroll
    for (int c = 0; c < kSkinnyChunk; ++c) {
      const int k = 16 * (sb + c) + 4 * g;
      const bool in = sb + c < s_end;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int row = 16 * rb + r;
        a[c][rb] = (in && row < p.M) ? *reinterpret_cast<const f4*>(p.A + (long long)row * p.lda + k)
                                     : f4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      if (!in) {
        b[c] = f4{0.0f, 0.0f, 0.0f, 0.0f};
      } else if constexpr (B_KC) {
        b[c] = *reinterpret_cast<const f4*>(p.B + (long long)(n0 + r) * p.ldb + k);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) b[c][q] = p.B[(long long)(k + q) * p.ldb + n0 + r];
      }
    }
#pragma unroll
    for (int c = 0; c < kSkinnyChunk; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c][rb][q], b[c][q], acc[rb], 0, 0, 0);
  }

  // red[w][row][col]: wave w's partial C[row][n0 + col].
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(wave * RB * 16 + 16 * rb + 4 * g + q) * 16 + r] = acc[rb][q];
  __syncthreads();
  for (int e = tid; e < RB * 16 * 16; e += 64 * kSkinnyWaves) {
    const int row = e >> 4, col = n0 + (e & 15);
    if (row >= p.M) continue;
    float v = red[e];
#pragma unroll
    for (int w = 1; w < kSkinnyWaves; ++w) v += red[w * RB * 16 * 16 + e];
    if (p.epi == RT_EPI_BIAS || p.epi == RT_EPI_BIAS_RELU) {
      v = v + p.bias[col];
      if (p.epi == RT_EPI_BIAS_RELU) v = fmaxf(v, 0.0f);
    } else if (p.epi == RT_EPI_RELU_MASK) {
      if (!(p.mask[(long long)row * p.ldc + col] > 0.0f)) v = 0.0f;
    }
    p.C[(long long)row * p.ldc + col] = v;
  }
}

// The skinny kernel takes a product when it has at most 64 rows, too few
// 64x64 tiles to fill the chip, whole 16-column and 16-k blocks, a
// K-contiguous A (NN or NT) with float4-loadable rows, and no K slices or
// column sums.
template <bool A_KC, bool B_KC>
bool skinny_ok(const F32Args& a) {
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  const long long tiles = (long long)((a.M + 63) / 64) * ((a.N + 63) / 64);
  return A_KC && a.splits == 1 && a.colsum == nullptr && rt::gemm_f32_skinny_shape(a.M, a.N, a.K) && tiles < 256 &&
         a.lda % 4 == 0 && al(a.A) && (!B_KC || (a.ldb % 4 == 0 && al(a.B)));
}

template <bool B_KC>
hipError_t launch_skinny(hipStream_t s, const F32Args& a) {
  const dim3 grid(a.N / 16), block(64 * kSkinnyWaves);
  if (a.M <= 32)
    rt::launch((gemm_f32_skinny_kernel<2, B_KC>), grid, block, 0, s, a);
  else
    rt::launch((gemm_f32_skinny_kernel<4, B_KC>), grid, block, 0, s, a);
  return hipGetLastError();
}

// dX of a narrow layer (K = that layer's outputs <= 16): the rank-K block.
bool rank_k_ok(const F32Args& a) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool epi_ok = (a.epi != RT_EPI_RELU_MASK || al16(a.mask)) &&
                      ((a.epi != RT_EPI_BIAS && a.epi != RT_EPI_BIAS_RELU) || al16(a.bias));
  return a.K >= 1 && a.K <= F32RankK::KMAX && a.splits <= 1 && epi_ok;
}

hipError_t launch_rank_k(hipStream_t s, F32Args a) {
  a.tiles_m = (a.M + 63) / 64;
  a.tiles_n = (a.N + 63) / 64;
  rt::launch((gemm_f32_kernel<F32RankK>), dim3(a.tiles_m * a.tiles_n), dim3(F32RankK::THREADS), 0, s, a);
  return hipGetLastError();
}

template <bool A_KC, bool B_KC>
hipError_t dispatch_tile(hipStream_t s, F32Args a) {
  if constexpr (A_KC) {
    if (skinny_ok<A_KC, B_KC>(a)) return launch_skinny<B_KC>(s, a);
  }
  if constexpr (A_KC && B_KC) {
    if (rank_k_ok(a)) return launch_rank_k(s, a);
  }
  switch (pick_tile(a)) {
    case kT128: return launch_f32<128, 128, A_KC, B_KC>(s, a);
    case kT64x32: return launch_f32<64, 32, A_KC, B_KC>(s, a);
    default:
      if (dma_ok<A_KC, B_KC>(a)) return launch_dma<A_KC, B_KC>(s, a);
      return launch_f32<64, 64, A_KC, B_KC>(s, a);
  }
}

F32Args make_args(const rt::GemmDesc& d) {
  F32Args a{};
  a.A = static_cast<const float*>(d.A);
  a.B = static_cast<const float*>(d.B);
  a.C = static_cast<float*>(d.C);
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.lda = d.lda;
  a.ldb = d.ldb;
  a.ldc = d.ldc;
  a.epi = d.epi;
  a.bias = d.bias;
  a.mask = static_cast<const float*>(d.mask);
  a.colsum = d.splits > 1 ? d.colsum_partials : d.colsum;
  a.splits = d.splits < 1 ? 1 : d.splits;
  // Slices are whole multiples of the 32-wide K step.
  int kps = (d.K + a.splits - 1) / a.splits;
  kps = ((kps + 31) / 32) * 32;
  a.k_per_split = a.splits > 1 ? kps : (d.K > 0 ? d.K : 1);
  a.split_stride = d.split_stride;
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  a.vec_a = (d.lda % 4 == 0) && al16(d.A);
  a.vec_b = (d.ldb % 4 == 0) && al16(d.B);
  a.vec_c = (d.ldc % 4 == 0) && al16(d.C);
  return a;
}

// The backward pair of a hidden layer: dW = Aᵀ·δ (TN, 64x64 or, for a
// narrow layer, 64x32 tiles; any number of K slices) and
// dX = (δ·Wᵀ) ⊙ mask (NT, 64x64 tiles, whole K).
template <class T0, class T1, int BN0>
hipError_t launch_pair_tn_nt(hipStream_t s, F32Args a0, F32Args a1) {
  a0.tiles_m = (a0.M + 63) / 64;
  a0.tiles_n = (a0.N + BN0 - 1) / BN0;
  a1.tiles_m = (a1.M + 63) / 64;
  a1.tiles_n = (a1.N + 63) / 64;
  const long long nb0 = (long long)a0.tiles_m * a0.tiles_n * a0.splits;
  const long long nb1 = (long long)a1.tiles_m * a1.tiles_n * a1.splits;
  const long long n0 = (nb0 + 7) / 8 * 8;
  if (n0 + nb1 > 0x7fffffffLL) return hipErrorInvalidValue;
  rt::launch((gemm_f32_pair_kernel<T0, T1>), dim3((unsigned)(n0 + nb1)), dim3(T0::THREADS), 0, s, a0,
                     a1, (int)n0);
  return hipGetLastError();
}

}  // namespace

namespace rt {

bool gemm_f32_skinny_shape(int M, int N, int K) {
  return M >= 1 && M <= 64 && N >= 16 && N % 16 == 0 && K >= 128 && K % 16 == 0;
}

hipError_t gemm_f32_launch(hipStream_t s, const GemmDesc& d) {
  const F32Args a = make_args(d);
  switch (d.layout) {
    case RT_NN: return dispatch_tile<true, false>(s, a);
    case RT_TN: return dispatch_tile<false, false>(s, a);
    case RT_NT: return dispatch_tile<true, true>(s, a);
  }
  return hipErrorInvalidValue;
}

template <class T, int BM, int BN>
hipError_t launch_gemm_opt(hipStream_t s, F32Args a, const rt_opt::OptBatch& b, long long opt_blocks) {
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
  const long long n_gemm = (long long)a.tiles_m * a.tiles_n * a.splits;
  if (n_gemm + opt_blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  rt::launch((gemm_f32_opt_kernel<T>), dim3((unsigned)(n_gemm + opt_blocks)), dim3(T::THREADS), 0, s, a, b,
             (int)n_gemm);
  return hipGetLastError();
}

bool gemm_opt_supported(const GemmDesc& d, const OptTensor* ts, int nt, const OptParams& P) {
  if (d.in_dtype != RT_F32 || d.layout != RT_TN || d.M <= 0 || d.N <= 0 || d.K <= 0) return false;
  return nt > 0 && optimizer_fits_cache(ts, nt, P);
}

bool gemm_opt_update_ok(const GemmDesc& d, const OptTensor* wb, const OptParams& P) {
  if (d.in_dtype != RT_F32 || d.layout != RT_TN || d.splits > 1 || d.epi != RT_EPI_NONE || d.colsum == nullptr ||
      d.ldc != d.N || d.M <= 0 || d.N <= 0 || d.K <= 0)
    return false;
  // The tile the TN GEMM's own launch would take: 64x64 DMA tiles.
  const F32Args a = make_args(d);
  if (pick_tile(a) != kT64 || !dma_ok<false, false>(a)) return false;
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  const OptTensor &W = wb[0], &Bt = wb[1];
  const bool adam = P.kind == 0, need_m = adam || P.momentum != 0.0f;
  for (const OptTensor* T : {&W, &Bt}) {
    if (T->theta == nullptr || T->parts != nullptr || T->half_copy != nullptr) return false;
    if (need_m != (T->m != nullptr) || (adam && T->v == nullptr)) return false;
  }
  return W.n == (size_t)d.M * d.N && Bt.n == (size_t)d.N && W.grad == d.C && Bt.grad == d.colsum &&
         al16(W.theta) && (W.m == nullptr || al16(W.m)) && (!adam || al16(W.v));
}

hipError_t gemm_opt_launch(hipStream_t s, const GemmDesc& d, const OptTensor* ts, int nt, const OptParams& P,
                           const OptTensor* upd) {
  if (!gemm_opt_supported(d, ts, nt, P)) return hipErrorInvalidValue;
  if (upd != nullptr && !gemm_opt_update_ok(d, upd, P)) return hipErrorInvalidValue;
  rt_opt::OptBatch b{};
  long long opt_blocks = 0;
  double bytes = 0.0;
  hipError_t e = rt_opt::make_batch(ts, nt, P, b, &opt_blocks, &bytes);
  if (e != hipSuccess) return e;
  // The tile the TN GEMM's own launch would take (same bits).
  F32Args a = make_args(d);
  if (upd != nullptr) {
    a.tiles_m = a.M / 64;
    a.tiles_n = a.N / 64;
    const long long n_gemm = (long long)a.tiles_m * a.tiles_n;
    if (n_gemm + opt_blocks > 0x7fffffffLL) return hipErrorInvalidValue;
    UpdEpi u{upd[0], upd[1], P};
    u.P.skip_count = nullptr;  // counted by the optimizer blocks of the launch
    rt::launch(gemm_f32_opt_upd_kernel, dim3((unsigned)(n_gemm + opt_blocks)), dim3(F32Dma::THREADS), 0, s, a, b,
               (int)n_gemm, u);
    return hipGetLastError();
  }
  switch (pick_tile(a)) {
    case kT128: return launch_gemm_opt<F32Tile<128, 128, false, false>, 128, 128>(s, a, b, opt_blocks);
    case kT64x32: return launch_gemm_opt<F32Tile<64, 32, false, false>, 64, 32>(s, a, b, opt_blocks);
    default:
      if (dma_ok<false, false>(a)) return launch_gemm_opt<F32DmaTile<false, false>, 64, 64>(s, a, b, opt_blocks);
      return launch_gemm_opt<F32Tile<64, 64, false, false>, 64, 64>(s, a, b, opt_blocks);
  }
}

hipError_t gemm_opt_update2_launch(hipStream_t s, const GemmDesc& d0, const OptTensor* upd0, const GemmDesc& d1,
                                   const OptTensor* upd1, const OptTensor* ts, int nt, const OptParams& P) {
  if (!gemm_opt_supported(d0, ts, nt, P) || !gemm_opt_update_ok(d0, upd0, P) || !gemm_opt_update_ok(d1, upd1, P))
    return hipErrorInvalidValue;
  rt_opt::OptBatch b{};
  long long opt_blocks = 0;
  double bytes = 0.0;
  hipError_t e = rt_opt::make_batch(ts, nt, P, b, &opt_blocks, &bytes);
  if (e != hipSuccess) return e;
  F32Args a0 = make_args(d0), a1 = make_args(d1);
  for (F32Args* a : {&a0, &a1}) {
    a->tiles_m = a->M / 64;
    a->tiles_n = a->N / 64;
  }
  const long long n0 = ((long long)a0.tiles_m * a0.tiles_n + 7) / 8 * 8;
  const long long n1 = n0 + (long long)a1.tiles_m * a1.tiles_n;
  if (n1 + opt_blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  UpdEpi u0{upd0[0], upd0[1], P}, u1{upd1[0], upd1[1], P};
  u0.P.skip_count = u1.P.skip_count = nullptr;  // counted by the optimizer blocks of the launch
  rt::launch(gemm_f32_opt_upd2_kernel, dim3((unsigned)(n1 + opt_blocks)), dim3(F32Dma::THREADS), 0, s, a0, a1, b,
             (int)n0, (int)n1, u0, u1);
  return hipGetLastError();
}

bool gemm_pair_supported(const GemmDesc& d0, const GemmDesc& d1) {
  if (d0.in_dtype != RT_F32 || d1.in_dtype != RT_F32) return false;
  if (d0.layout != RT_TN || d1.layout != RT_NT || d1.splits > 1) return false;
  // Only where the single launches would use the same tiles.
  const TileCfg t0 = pick_tile(make_args(d0));
  return (t0 == kT64 || t0 == kT64x32) && (pick_tile(make_args(d1)) == kT64 || rank_k_ok(make_args(d1)));
}

hipError_t gemm_pair_launch(hipStream_t s, const GemmDesc& d0, const GemmDesc& d1) {
  if (!gemm_pair_supported(d0, d1)) return hipErrorInvalidValue;
  const F32Args a0 = make_args(d0), a1 = make_args(d1);
  // dX takes the block its single launch would (the rank-K block for K <= 16).
  const bool rk = rank_k_ok(a1);
  if (pick_tile(a0) == kT64x32)
    return rk ? launch_pair_tn_nt<F32Tile<64, 32, false, false>, F32RankK, 32>(s, a0, a1)
              : launch_pair_tn_nt<F32Tile<64, 32, false, false>, F32Tile<64, 64, true, true>, 32>(s, a0, a1);
  if (rk)
    return dma_ok<false, false>(a0) ? launch_pair_tn_nt<F32DmaTile<false, false>, F32RankK, 64>(s, a0, a1)
                                    : launch_pair_tn_nt<F32Tile<64, 64, false, false>, F32RankK, 64>(s, a0, a1);
  if (dma_ok<false, false>(a0) && dma_ok<true, true>(a1))
    return launch_pair_tn_nt<F32DmaTile<false, false>, F32DmaTile<true, true>, 64>(s, a0, a1);
  return launch_pair_tn_nt<F32Tile<64, 64, false, false>, F32Tile<64, 64, true, true>, 64>(s, a0, a1);
}

hipError_t splitk_reduce_launch(hipStream_t s, const float* partials, int splits, long long stride, int M, int N,
                                void* C, int out_dtype, int ldc, int epi, const float* bias, const void* mask,
                                int mask_dtype, const float* colsum_partials, float* colsum, int cs_rows) {
  if (out_dtype != RT_F32 || mask_dtype != RT_F32) return hipErrorInvalidValue;
  const long long total = (long long)M * N;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec4 = N % 4 == 0 && ldc % 4 == 0 && stride % 4 == 0 && al16(partials) && al16(C) &&
                    (bias == nullptr || al16(bias)) && (mask == nullptr || al16(mask));
  const long long items = vec4 ? total / 4 : total;
  int blocks = (int)std::min<long long>((items + 255) / 256, 4096);
  if (blocks < 1) blocks = 1;
  const int cs_blocks = colsum != nullptr ? (N + 255) / 256 : 0;
  rt::launch(splitk_reduce_kernel, dim3(blocks + cs_blocks), dim3(256), 0, s, partials, splits, stride, M, N,
             static_cast<float*>(C), ldc, epi, bias, static_cast<const float*>(mask), colsum_partials, cs_rows, colsum,
             cs_blocks, vec4 ? 1 : 0);
  return hipGetLastError();
}

}  // namespace rt
