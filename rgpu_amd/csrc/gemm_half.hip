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

#include "device_util.h"
#include "rt_internal.h"

namespace {

using rt_dev::barrier_lds;
using rt_dev::static_for;
using rt_dev::wait_vm;

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
  float* cs_parts;  // non-null: per-M-tile column-sum shares [splits * tiles_m, N]
  int k_per_split;
  long long split_stride;
  int tiles_m, tiles_n;
  int vec_a, vec_b;
  int n_ragged;  // N is not a multiple of BN: B tiles read past column N, stores and sums stop at N
  int* nf_flag;  // non-null: set to 1 if any f32 result (C or column sums) is not finite
  // ReLU predicate bits (GemmDesc::relu_bits_out / relu_bits): written by a
  // bf16 bias+ReLU epilogue, read by the ReLU-mask epilogue instead of mask.
  unsigned* relu_bits_out;
  const unsigned* relu_bits;
};

__device__ inline int not_finite(float v) { return !(fabsf(v) <= 3.402823466e38f); }

__device__ inline float bf16_to_f32(unsigned short h) { return __uint_as_float((unsigned int)h << 16); }

// Round to nearest even; a NaN keeps its sign and top payload bits and is
// made quiet.  Both results are computed and one selected (no branch).
__device__ inline unsigned short f32_to_bf16_rne(float x) {
  const unsigned int u = __float_as_uint(x);
  const unsigned int rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const unsigned int nan = (u >> 16) | 0x40u;
  return (unsigned short)((u & 0x7fffffffu) > 0x7f800000u ? nan : rne);
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

// Epilogue through LDS, one 16-row slab of the wave tile at a time: the
// accumulators acc[t][u][q] = C(m0+wm+16t+4g+q, n0+wn+16u+r) are parked in
// a per-wave [16][WN+4] f32 region of smem, then each lane reads 4
// consecutive columns back, applies bias / ReLU / mask and stores 16 (f32) or
// 8 (bf16) bytes.  Bounded register use and coalesced stores.  The caller has
// finished every read of smem (barrier) before calling.
template <int BM, int BN, int WGM, int WGN, int SMEM_BYTES, int TM, int TN>
__device__ __forceinline__ void store_tile(const HalfArgs& p, f4 (&acc)[TM][TN], unsigned short* smem, int m0, int n0,
                                           int wm, int wn, int wave, int lane, int g, int r) {
  constexpr int WN = BN / WGN;
  constexpr int SROW = WN + 4;
  static_assert(16 * SROW * 4 * WGM * WGN <= SMEM_BYTES, "epilogue staging must fit in LDS");
  float* stage = reinterpret_cast<float*>(smem) + wave * 16 * SROW;
  const bool partial = gridDim.z > 1;
  const bool out_bf16 = !partial && p.out_bf16;
  const bool vec_c = (p.ldc % 4 == 0) && ((reinterpret_cast<uintptr_t>(p.C) & 15) == 0);
  float* Cf = static_cast<float*>(p.C) + (partial ? (long long)blockIdx.z * p.split_stride : 0);
  unsigned short* Ch = static_cast<unsigned short*>(p.C);
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

  __syncthreads();  // main-loop LDS reads are finished
  store_tile<BM, BN, WGM, WGN, (int)sizeof(smem)>(p, acc, smem, m0, n0, wm, wn, wave, lane, g, r);
}


// ---------------------------------------------------------------- full-tile kernel
// For full tiles (M % BM == 0, N % BN == 0, every K slice a whole number of
// BK steps, 16-byte aligned operands whose leading dimensions are multiples
// of 8 halves) the operand tiles go from global memory straight into LDS
// with global_load_lds_dwordx4: lane l's 16 bytes land at the instruction's
// LDS base + 16 l, so a wave fills 1 KB of LDS per instruction with no VGPR
// staging and no LDS write instructions, and the loads of stage k+1 run
// while stage k computes.  Each lane picks the global chunk whose swizzled
// LDS position is 16 l.  Layouts (unpadded):
//   K-contiguous [row][64]: 16-byte granule j of row r at j ^ ((r >> 1) & 7)
//     (b128 fragment reads of 16 rows at one granule are conflict-free);
//   M/N-contiguous [k][ROWS]: 32-byte granule G of row k at G ^ hm(k).  A
//     transposed fragment read touches, per 32 lanes, rows k0 + {0..3, 8..11}
//     at one granule; hm gives those eight rows distinct bank groups.
template <int ROWS, bool KC, int THREADS, int BKD>
struct DmaOperand {
  static constexpr int ELEMS = ROWS * BKD;    // halves per stage
  static constexpr int INSTR = ELEMS / 512;   // 1 KB DMA instructions per stage
  static constexpr int WAVES = THREADS / 64;
  static constexpr int PER_WAVE = INSTR / WAVES;
  static constexpr int GR = BKD / 8;          // 16-byte granules per K-contiguous row
  static_assert(INSTR % WAVES == 0 && PER_WAVE >= 1, "DMA instructions must split evenly over the waves");
  static_assert(ROWS % 64 == 0 && (BKD == 32 || BKD == 64), "tile shape");

  // Wave w's i-th DMA instruction fills LDS block i * WAVES + w, so a lane's
  // rows advance by RSTEP per instruction; with that spacing the swizzle term
  // of a lane's chunk is the same for every instruction (or, for 256-wide
  // M/N-contiguous tiles, alternates with the instruction's parity), and the
  // rest of the offset is uniform: it goes in the scalar offset.
  static constexpr int RSTEP = (KC ? 512 / BKD : 512 / ROWS) * WAVES;
  static constexpr bool PAR = !KC && (RSTEP % 16) == 8;  // hm(k + RSTEP) != hm(k)

  // Buffer descriptor based at the tile origin; this lane's byte offset from
  // it for its first instruction (voff[1]: the odd instructions when PAR).
  __amdgpu_buffer_rsrc_t rsrc;
  int voff[2];
  int row_bytes;  // bytes per stored row of the operand (2 ld)

  // K-contiguous: granule j of row r is stored at j ^ kc_sw(r).  16 lanes read
  // 16 consecutive rows at one granule; with 128-byte rows (BKD 64) two rows
  // share a 256-byte bank line, with 64-byte rows four do.
  __device__ static inline int kc_sw(int row) {
    if constexpr (BKD == 64) return (row >> 1) & 7;
    else return (row >> 2) & 3;
  }
  __device__ static inline int hm(int k) {
    if constexpr (ROWS >= 128) return (k & 3) | (((k >> 3) & 1) << 2);
    else return ((k >> 1) & 1) | (((k >> 3) & 1) << 1);
  }
  __device__ inline void init(const unsigned short* tile, int ld, int wave, int lane) {
    static_assert(KC ? (RSTEP % 16 == 0) : (RSTEP % 8 == 0), "swizzle period");
    // 0x00020000: raw (untyped) buffer, 32-bit data format.  The host only
    // takes this path when every operand byte lies below 2^31 of its base.
    rsrc = rt_dev::raw_rsrc(tile);
    row_bytes = 2 * ld;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      if constexpr (KC) {
        const int row = (512 / BKD) * wave + lane / GR, slot = lane % GR;
        voff[par] = 2 * (row * ld + 8 * (slot ^ kc_sw(row)));
      } else {
        constexpr int CH = ROWS / 8;  // 16-byte chunks per LDS row
        const int k = (512 / ROWS) * wave + lane / CH, s = lane % CH;
        voff[par] = 2 * (k * ld + 16 * ((s >> 1) ^ hm(k + par * RSTEP)) + 8 * (s & 1));
      }
    }
  }
  // This wave's DMA of the stage `stage_bytes` past the tile origin into `lds`
  // (ASM: through rt_dev::dma16_asm, ordered only by the kernel's own waits).
  template <bool ASM>
  __device__ inline void issue(int stage_bytes, unsigned short* lds, int wave) const {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int vo = voff[PAR ? (i & 1) : 0], so = stage_bytes + i * RSTEP * row_bytes;
      if constexpr (ASM)
        rt_dev::dma16_asm(rsrc, lds + 512 * (i * WAVES + wave), vo, so);
      else
        rt_dev::dma16(rsrc, lds + 512 * (i * WAVES + wave), vo, so);
    }
  }
  // Same fragment contract as Operand::frag.
  __device__ inline u4 frag(const unsigned short* lds, int kk, int rbase, int g, int r) const {
    if constexpr (KC) {
      const int row = rbase + r;
      return *reinterpret_cast<const u4*>(&lds[row * BKD + 8 * ((4 * kk + g) ^ kc_sw(row))]);
    } else {
      const int k = 32 * kk + 8 * g + (r >> 2);  // hm(k + 4) == hm(k)
      const unsigned short* q = &lds[k * ROWS + 16 * ((rbase >> 4) ^ hm(k)) + 4 * (r & 3)];
      const u2 lo = lds_tr(q), hi = lds_tr(q + 4 * ROWS);
      return u4{lo[0], lo[1], hi[0], hi[1]};
    }
  }
  // 8 consecutive halves [c8*8, c8*8+8) of LDS row k (M/N-contiguous tiles).
  __device__ static inline u4 row_chunk(const unsigned short* lds, int k, int c8) {
    return *reinterpret_cast<const u4*>(&lds[k * ROWS + 16 * ((c8 >> 1) ^ hm(k)) + 8 * (c8 & 1)]);
  }
};

// Full-tile epilogue straight from the accumulators.  The DMA kernel issues
// its MFMAs with the operands swapped (D = op(B)·op(A)), so lane (g, r) holds
// C(m0+wm+16t+r, n0+wn+16u+4g+q) for q = 0..3: four consecutive columns of
// one row.  Each 16x16 tile is then one 16-byte (f32) or 8-byte (bf16) store,
// with the bias / mask read the same way; no LDS round trip and no bounds
// checks (the host only takes this path for whole, aligned tiles).
template <int EPI, bool OUT_BF16, int TM, int TN>
__device__ __forceinline__ void store_direct(const HalfArgs& p, const f4 (&acc)[TM][TN], int m0, int n0, int wm,
                                             int wn, int g, int r, int slice) {
  float* Cf = static_cast<float*>(p.C) + (gridDim.z > 1 ? (long long)slice * p.split_stride : 0);
  unsigned short* Ch = static_cast<unsigned short*>(p.C);
  // ReLU predicate bits (layout in rt_internal.h): this lane's dword of the
  // 16-row x 64-column group of row block t, the byte of its 16x16 block
  // u = 0 and, within the byte, the nibble of lane 16g + r.
  static_assert(TN == 2 || TN == 4, "a wave tile spans half or all of a 64-column group");
  const int lane = 16 * g + r, byte0 = (wn & 63) >> 4;
  auto bits_dword = [&](int t) {
    return 32 * ((long long)((m0 + wm) / 16 + t) * (p.N / 64) + (n0 + wn) / 64) + (lane >> 1);
  };
  // Loads the stores do not feed, issued before the first store (the
  // compiler cannot move a load past a store it might alias, and each wait
  // for a load also waits for every store before it): the bias of the wave
  // tile's TN column groups, the same for all its rows, and the ReLU mask
  // bits of its rows.
  f4 bias[TN];
  unsigned mbits[TM];
#pragma unroll
  for (int u = 0; u < TN; ++u) bias[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < TM; ++t) mbits[t] = 0;
  if constexpr (EPI == RT_EPI_BIAS || EPI == RT_EPI_BIAS_RELU) {
#pragma unroll
    for (int u = 0; u < TN; ++u) {
      const int col = n0 + wn + 16 * u + 4 * g;
      if (!(p.n_ragged && col >= p.N)) bias[u] = *reinterpret_cast<const f4*>(p.bias + col);
    }
  } else if constexpr (EPI == RT_EPI_RELU_MASK) {
    if (p.relu_bits) {
#pragma unroll
      for (int t = 0; t < TM; ++t) mbits[t] = p.relu_bits[bits_dword(t)] >> (4 * (lane & 1));
    }
  }
  int bad = 0;
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    const long long row_off = (long long)(m0 + wm + 16 * t + r) * p.ldc;
    unsigned bits_w = 0;  // bias+ReLU with bits: this lane's and its neighbour's nibbles, by block
#pragma unroll
    for (int u = 0; u < TN; ++u) {
      const int col = n0 + wn + 16 * u + 4 * g;
      if (p.n_ragged && col >= p.N) continue;  // N % 4 == 0: a group is all in or all out
      const long long off = row_off + col;
      f4 v = acc[t][u];
      if constexpr (EPI == RT_EPI_BIAS || EPI == RT_EPI_BIAS_RELU) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = v[e] + bias[u][e];
          if constexpr (EPI == RT_EPI_BIAS_RELU) v[e] = fmaxf(v[e], 0.0f);
        }
      } else if constexpr (EPI == RT_EPI_RELU_MASK) {
        if (p.relu_bits) {
          const unsigned nib = mbits[t] >> (8 * (byte0 + u));  // bit e: column 4g + e
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (!((nib >> e) & 1u)) v[e] = 0.0f;
        } else {
          f4 mk;
          if (p.mask_bf16) {
            const u2 h = *reinterpret_cast<const u2*>(static_cast<const unsigned short*>(p.mask) + off);
            mk = f4{__uint_as_float(h[0] << 16), __uint_as_float(h[0] & 0xffff0000u), __uint_as_float(h[1] << 16),
                    __uint_as_float(h[1] & 0xffff0000u)};
          } else {
            mk = *reinterpret_cast<const f4*>(static_cast<const float*>(p.mask) + off);
          }
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (!(mk[e] > 0.0f)) v[e] = 0.0f;
        }
      }
      if constexpr (OUT_BF16) {
        u2 w;
        w[0] = (unsigned)f32_to_bf16_rne(v[0]) | ((unsigned)f32_to_bf16_rne(v[1]) << 16);
        w[1] = (unsigned)f32_to_bf16_rne(v[2]) | ((unsigned)f32_to_bf16_rne(v[3]) << 16);
        *reinterpret_cast<u2*>(Ch + off) = w;
        if constexpr (EPI == RT_EPI_BIAS_RELU) {
          if (p.relu_bits_out) {
            // The predicate the mask epilogue applies to the stored bf16
            // values (> 0) as a nibble, paired with the neighbour lane's
            // (DPP quad_perm [1,0,3,2]) into one byte.
            const unsigned nib = (unsigned)(__uint_as_float(w[0] << 16) > 0.0f) |
                                 ((unsigned)(__uint_as_float(w[0] & 0xffff0000u) > 0.0f) << 1) |
                                 ((unsigned)(__uint_as_float(w[1] << 16) > 0.0f) << 2) |
                                 ((unsigned)(__uint_as_float(w[1] & 0xffff0000u) > 0.0f) << 3);
            const unsigned other = (unsigned)__builtin_amdgcn_update_dpp(0, (int)nib, 0xB1, 0xF, 0xF, false);
            bits_w |= ((lane & 1) ? other | (nib << 4) : nib | (other << 4)) << (8 * (byte0 + u));
          }
        }
      } else {
        *reinterpret_cast<f4*>(Cf + off) = v;
        bad |= not_finite(v[0]) | not_finite(v[1]) | not_finite(v[2]) | not_finite(v[3]);
      }
    }
    if constexpr (EPI == RT_EPI_BIAS_RELU && OUT_BF16) {
      // Even lanes store the pair's bytes: 128 (or 64) contiguous bytes.
      if (p.relu_bits_out && !(lane & 1)) {
        if constexpr (TN == 4)
          p.relu_bits_out[bits_dword(t)] = bits_w;
        else
          reinterpret_cast<unsigned short*>(p.relu_bits_out + bits_dword(t))[byte0 >> 1] =
              (unsigned short)(bits_w >> (8 * byte0));
      }
    }
  }
  if (bad && p.nf_flag) *p.nf_flag = 1;
}

template <int TM, int TN>
__device__ __forceinline__ void store_direct_any(const HalfArgs& p, const f4 (&acc)[TM][TN], int m0, int n0, int wm,
                                                 int wn, int g, int r, int slice) {
  if (gridDim.z > 1) return store_direct<RT_EPI_NONE, false>(p, acc, m0, n0, wm, wn, g, r, slice);  // raw partial plane
  const bool hb = p.out_bf16;
  switch (p.epi) {
    case RT_EPI_BIAS:
      return hb ? store_direct<RT_EPI_BIAS, true>(p, acc, m0, n0, wm, wn, g, r, slice)
                : store_direct<RT_EPI_BIAS, false>(p, acc, m0, n0, wm, wn, g, r, slice);
    case RT_EPI_BIAS_RELU:
      return hb ? store_direct<RT_EPI_BIAS_RELU, true>(p, acc, m0, n0, wm, wn, g, r, slice)
                : store_direct<RT_EPI_BIAS_RELU, false>(p, acc, m0, n0, wm, wn, g, r, slice);
    case RT_EPI_RELU_MASK:
      return hb ? store_direct<RT_EPI_RELU_MASK, true>(p, acc, m0, n0, wm, wn, g, r, slice)
                : store_direct<RT_EPI_RELU_MASK, false>(p, acc, m0, n0, wm, wn, g, r, slice);
    default:
      return hb ? store_direct<RT_EPI_NONE, true>(p, acc, m0, n0, wm, wn, g, r, slice)
                : store_direct<RT_EPI_NONE, false>(p, acc, m0, n0, wm, wn, g, r, slice);
  }
}

// Two LDS stages of BKD = 64 k (two MFMA k-steps, kk = 0, 1).  With the
// fragments of (stage k, kk 0) already in registers, stage k runs as
//   A: read (k, kk 1) fragments       | MFMAs of (k, kk 0)
//   B: wait for stage k+1, barrier, DMA stage k+2 into stage k's buffer,
//      read (k+1, kk 0) fragments     | MFMAs of (k, kk 1)
// so every LDS read overlaps MFMAs and there is one barrier per 64 k.  The
// reads and the DMA are interleaved one per MFMA: a single wave per SIMD
// never stalls on a full memory queue with MFMAs still to issue.
template <int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC, bool IS_BF16, int BKD, int NS>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_half_dma_kernel(HalfArgs p) {
  constexpr int THREADS = 64 * WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  using OpA = DmaOperand<BM, A_KC, THREADS, BKD>;
  using OpB = DmaOperand<BN, B_KC, THREADS, BKD>;
  constexpr int STAGE = OpA::ELEMS + OpB::ELEMS;
  constexpr int PER_STAGE = OpA::PER_WAVE + OpB::PER_WAVE;  // DMA instructions per wave per stage
  static_assert(BKD == 64 && NS == 2, "two stages of two MFMA k-steps");
  __shared__ __attribute__((aligned(16))) unsigned short smem[NS * STAGE];
  auto sA = [&](int buf) { return smem + buf * STAGE; };
  auto sB = [&](int buf) { return smem + buf * STAGE + OpA::ELEMS; };

  const int tid = threadIdx.x;
  // Wave index as a scalar: the DMA's LDS destinations (M0) are then SALU
  // arithmetic instead of per-instruction VGPRs kept live across the loop.
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;

  // Work item (K slice, tile) of this workgroup.  Consecutive workgroup ids
  // go to the 8 XCDs in turn; when the grid divides by 8, each XCD takes a
  // contiguous run of items instead (the tiles of one slice, then the next
  // slice), so workgroups that read the same operand panels share an L2.
  const int nb = gridDim.x;
  int bid = blockIdx.x, slice = blockIdx.z;
  const int total = nb * (int)gridDim.z;
  if ((total & 7) == 0) {
    const int lin = blockIdx.x + nb * blockIdx.z;
    const int w = (lin & 7) * (total >> 3) + (lin >> 3);
    slice = w / nb;
    bid = w - slice * nb;
  }
  constexpr int GROUP = 8;
  const int per_group = GROUP * p.tiles_n;
  const int grp = bid / per_group;
  const int first_m = grp * GROUP;
  const int gsize = min(p.tiles_m - first_m, GROUP);
  const int in_grp = bid - grp * per_group;
  const int tile_m = first_m + in_grp % gsize;
  const int tile_n = in_grp / gsize;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int kb = slice * p.k_per_split;
  const int nk = (min(p.K, kb + p.k_per_split) - kb) / BKD;  // whole stages (checked by the host)

  OpA oa;
  OpB ob;
  oa.init(A_KC ? p.A + (long long)m0 * p.lda + kb : p.A + (long long)kb * p.lda + m0, p.lda, wave, lane);
  ob.init(B_KC ? p.B + (long long)n0 * p.ldb + kb : p.B + (long long)kb * p.ldb + n0, p.ldb, wave, lane);
  const int a_step = 2 * (A_KC ? BKD : BKD * p.lda);  // bytes per stage
  const int b_step = 2 * (B_KC ? BKD : BKD * p.ldb);
  // With an M/N-contiguous B the DMA goes through inline asm: the compiler's
  // own LDS-DMA ordering would wait for stage k+1's DMA before the first
  // fragment read of stage k, halving the time each stage has to arrive
  // (measured: 4096^3 NN 117 -> 105 us, the K = 262144 split-K dW 159 -> 143
  // us).  The NT kernel's schedule has no such wait and keeps the builtin.
  constexpr bool ASM_DMA = !B_KC;
  auto issue = [&](int stage, int buf) {
    oa.template issue<ASM_DMA>(stage * a_step, sA(buf), wave);
    ob.template issue<ASM_DMA>(stage * b_step, sB(buf), wave);
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int t = 0; t < TM; ++t)
#pragma unroll
    for (int u = 0; u < TN; ++u) acc[t][u] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto read_frags = [&](int buf, int kk, u4 (&fa)[TM], u4 (&fb)[TN]) {
#pragma unroll
    for (int u = 0; u < TN; ++u) fb[u] = ob.frag(sB(buf), kk, wn + 16 * u, g, r);
#pragma unroll
    for (int t = 0; t < TM; ++t) fa[t] = oa.frag(sA(buf), kk, wm + 16 * t, g, r);
  };
  // Operands swapped: acc[t][u] accumulates the transposed 16x16 tile, so a
  // lane ends up with four consecutive columns of one row (store_direct).
  auto mfmas = [&](const u4 (&fa)[TM], const u4 (&fb)[TN]) {
#pragma unroll
    for (int t = 0; t < TM; ++t)
#pragma unroll
      for (int u = 0; u < TN; ++u) {
        if constexpr (IS_BF16)
          acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, fb[u]),
                                                              __builtin_bit_cast(bf16x8, fa[t]), acc[t][u], 0, 0, 0);
        else
          acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, fb[u]),
                                                             __builtin_bit_cast(f16x8, fa[t]), acc[t][u], 0, 0, 0);
      }
  };
  constexpr int N_DS = (A_KC ? TM : 2 * TM) + (B_KC ? TN : 2 * TN);  // LDS read instructions per k-step
  constexpr int N_MF = TM * TN;
  // Scheduling hint for the region just emitted: one MFMA, then one of the
  // N_DS LDS reads, ...; one MFMA, then one of the N_VM DMA loads, ...; then
  // the remaining MFMAs.  Small tiles are left to the scheduler.
  auto interleave = [&](auto n_vm) {
    constexpr int N_VM = decltype(n_vm)::value;
    if constexpr (N_DS + N_VM <= N_MF) {
      static_for<0, N_DS>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      });
      static_for<0, N_VM>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global (DMA) load
      });
      __builtin_amdgcn_sched_group_barrier(0x008, N_MF - N_DS - N_VM, 0);
    }
  };

  // Column sums of the (M/N-contiguous) B tiles over k: thread t sums 8
  // consecutive columns (chunk t % (BN/8)) over the k rows t / (BN/8),
  // t / (BN/8) + KG, ... of a stage; the KG partial rows are added in a fixed
  // order at the end.  With cs_parts every M tile takes the stages s with
  // s % tiles_m == tile_m and writes its share (the shares are added by a
  // second launch); without it the first M tile sums every stage.
  constexpr int CH = BN / 8, KG = THREADS / CH;
  static_assert(B_KC || (THREADS % CH == 0 && BKD % KG == 0), "colsum split");
  const bool cs_shared = p.cs_parts != nullptr;
  const bool do_cs = !B_KC && p.colsum != nullptr && (cs_shared || tile_m == 0);  // uniform over the block
  float cs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto colsum = [&](int buf) {
    if constexpr (!B_KC) {
      if (do_cs) {
        const int c8 = tid % CH;
#pragma unroll
        for (int k = tid / CH; k < BKD; k += KG) {
          const u4 v = OpB::row_chunk(sB(buf), k, c8);
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            cs[2 * d] += half_to_f32<IS_BF16>((unsigned short)(v[d] & 0xffffu));
            cs[2 * d + 1] += half_to_f32<IS_BF16>((unsigned short)(v[d] >> 16));
          }
        }
      }
    }
  };

  if (nk > 0) {
    u4 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    // Every B step waits for everything and issues one stage of DMA (past
    // the last stage it re-fetches stage nk-1 into a buffer nothing reads),
    // so the bookkeeping is the same in every stage.
    issue(0, 0);
    issue(min(1, nk - 1), 1);
    wait_vm<PER_STAGE>();
    barrier_lds();
    read_frags(0, 0, fa0, fb0);
    auto stage = [&](int k, auto bc) {
      constexpr int BUF = decltype(bc)::value;  // k % 2
      // A: (k, kk 1) fragments in, (k, kk 0) MFMAs.
      read_frags(BUF, 1, fa1, fb1);
      mfmas(fa0, fb0);
      interleave(std::integral_constant<int, 0>{});
      if (!cs_shared || k % p.tiles_m == tile_m) colsum(BUF);
      // B: stage k+1 everywhere; stage k no longer read.
      wait_vm<0>();
      barrier_lds();
      // (k+1, kk 0) fragments (discarded after the last stage) and the DMA of
      // stage k+2 touch different buffers.  The DMA has one stage of MFMAs
      // to land, so it starts right after the barrier: NT issues all of it
      // first; with a transposed operand A's half goes first, then the
      // fragment reads, then B's half (measured fastest of the orders tried:
      // reads first, DMA first, and the B-first mirror).
      const int next = min(k + 2, nk - 1);
      if constexpr (A_KC && B_KC) {
        issue(next, BUF);
        read_frags(BUF ^ 1, 0, fa0, fb0);
      } else {
        oa.template issue<ASM_DMA>(next * a_step, sA(BUF), wave);
        read_frags(BUF ^ 1, 0, fa0, fb0);
        ob.template issue<ASM_DMA>(next * b_step, sB(BUF), wave);
      }
      mfmas(fa1, fb1);
      interleave(std::integral_constant<int, PER_STAGE>{});
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    for (int k = 0; k < nk; k += 2) {
      stage(k, B0{});
      if (k + 1 < nk) stage(k + 1, B1{});
    }
  }
  wait_vm<0>();     // no DMA (the re-fetches past the last stage) still writing LDS
  __syncthreads();  // main-loop LDS reads are finished

  if (do_cs) {
    float* red = reinterpret_cast<float*>(smem);  // [KG][BN]
    const int c8 = tid % CH, kg = tid / CH;
#pragma unroll
    for (int e = 0; e < 8; ++e) red[kg * BN + 8 * c8 + e] = cs[e];
    __syncthreads();
    float* dst = cs_shared ? p.cs_parts + ((long long)slice * p.tiles_m + tile_m) * p.N
                           : p.colsum + (long long)slice * p.N;
    int bad = 0;
    for (int col = tid; col < BN && n0 + col < p.N; col += THREADS) {
      float v = 0.0f;
      for (int j = 0; j < KG; ++j) v += red[j * BN + col];
      dst[n0 + col] = v;
      bad |= not_finite(v);
    }
    if (bad && p.nf_flag && !cs_shared) *p.nf_flag = 1;  // shares are checked once summed
  }

  store_direct_any<TM, TN>(p, acc, m0, n0, wm, wn, g, r, slice);
}

// dst[z, n] = sum over t of parts[z * rows + t, n], t in increasing order:
// the column-sum shares of the M tiles of each K slice z.
__global__ __launch_bounds__(256) void cs_shares_reduce_kernel(const float* __restrict__ parts, int rows, int splits,
                                                               int N, float* __restrict__ dst, int* nf_flag) {
  const long long i = blockIdx.x * 256LL + threadIdx.x;
  if (i >= (long long)splits * N) return;
  const int z = (int)(i / N), n = (int)(i % N);
  const float* q = parts + (long long)z * rows * N + n;
  float v = 0.0f;
  int t = 0;
  for (; t + 8 <= rows; t += 8) {  // eight loads in flight, added in order
    float w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = q[(long long)(t + u) * N];
#pragma unroll
    for (int u = 0; u < 8; ++u) v += w[u];
  }
  for (; t < rows; ++t) v += q[(long long)t * N];
  dst[i] = v;
  if (nf_flag && not_finite(v)) *nf_flag = 1;
}

// Direct-to-LDS pipeline shape: K per stage and number of stages.
constexpr int kDmaBK = 64, kDmaStages = 2;

template <int BM, int BN>
void set_tiles(HalfArgs& a) {
  a.tiles_m = (a.M + BM - 1) / BM;
  a.tiles_n = (a.N + BN - 1) / BN;
}

// Whole BM x BN tiles everywhere, every K slice (the last included) a
// multiple of the DMA stage, and operands the DMA can read 16 bytes at a time.
// With n_ragged_ok, N need only be a multiple of 8 (the caller guarantees
// that B may be read up to BN columns past its last element).
bool full_tiles(const HalfArgs& a, int splits, int BM, int BN, bool n_ragged_ok = false) {
  const int last = a.K - (splits - 1) * a.k_per_split;
  auto al = [](const void* ptr, unsigned n) { return (reinterpret_cast<uintptr_t>(ptr) & (n - 1)) == 0; };
  const bool bf16_out = splits == 1 && a.out_bf16;
  const bool epi_ok = (a.epi != RT_EPI_BIAS && a.epi != RT_EPI_BIAS_RELU) || al(a.bias, 16);
  const bool mask_ok = a.epi != RT_EPI_RELU_MASK || al(a.mask, a.mask_bf16 ? 8 : 16);
  const bool n_ok = a.N % BN == 0 || (n_ragged_ok && a.N % 8 == 0);
  return a.M % BM == 0 && n_ok && a.k_per_split % kDmaBK == 0 && last > 0 && last % kDmaBK == 0 &&
         a.vec_a && a.vec_b && a.ldc % 4 == 0 && al(a.C, bf16_out ? 8 : 16) && epi_ok && mask_ok;
}

// The DMA addresses operands through 32-bit byte offsets from a tile origin.
template <bool A_KC, bool B_KC>
bool dma_addressable(const HalfArgs& a) {
  const long long lim = 1LL << 31;
  return (long long)(A_KC ? a.M : a.K) * a.lda * 2 < lim && (long long)(B_KC ? a.N : a.K) * a.ldb * 2 < lim;
}

template <int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC>
hipError_t launch_dma(hipStream_t s, HalfArgs a, int splits, bool bf16, float* cs_scratch = nullptr,
                      size_t cs_scratch_elems = 0, bool shares_to_caller = false) {
  set_tiles<BM, BN>(a);
  // Column sums shared over the M tiles when there are several and room.
  a.cs_parts = nullptr;
  if (!B_KC && a.colsum && a.tiles_m > 1 && cs_scratch &&
      (size_t)splits * a.tiles_m * a.N <= cs_scratch_elems)
    a.cs_parts = cs_scratch;
  const dim3 grid(a.tiles_m * a.tiles_n, 1, splits), block(64 * WGM * WGN);
  if (bf16)
    rt::launch((gemm_half_dma_kernel<BM, BN, WGM, WGN, A_KC, B_KC, true, kDmaBK, kDmaStages>), grid, block, 0,
                       s, a);
  else
    rt::launch((gemm_half_dma_kernel<BM, BN, WGM, WGN, A_KC, B_KC, false, kDmaBK, kDmaStages>), grid, block,
                       0, s, a);
  if (a.cs_parts && !shares_to_caller) {
    const long long n = (long long)splits * a.N;
    rt::launch(cs_shares_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, a.cs_parts,
                       a.tiles_m, splits, a.N, a.colsum, a.nf_flag);
  }
  return hipGetLastError();
}

template <int BM, int BN, int WGM, int WGN, bool A_KC, bool B_KC>
hipError_t launch_regs(hipStream_t s, HalfArgs a, int splits, bool bf16) {
  set_tiles<BM, BN>(a);
  const dim3 grid(a.tiles_m * a.tiles_n, 1, splits), block(64 * WGM * WGN);
  if (bf16)
    rt::launch((gemm_half_kernel<BM, BN, WGM, WGN, A_KC, B_KC, true>), grid, block, 0, s, a);
  else
    rt::launch((gemm_half_kernel<BM, BN, WGM, WGN, A_KC, B_KC, false>), grid, block, 0, s, a);
  return hipGetLastError();
}

// Tile size (256, 128 or 64) and kernel (direct-to-LDS or register-staged)
// for a problem: 256x256 blocks when they give at least one block per CU,
// 128x128 for mid sizes, 64x64 for small ones.  Full tiles take the
// direct-to-LDS kernel (256x256: two waves per SIMD with 128x64 wave tiles);
// the rest the register-staged kernel.
struct HalfPath {
  int tile;
  bool dma;
};
template <bool A_KC, bool B_KC>
HalfPath pick_path(const HalfArgs& a, int splits, bool overread_ok) {
  const long long tbig = (long long)((a.M + 255) / 256) * ((a.N + 255) / 256) * splits;
  const long long t128 = (long long)((a.M + 127) / 128) * ((a.N + 127) / 128) * splits;
  const int tile = tbig >= 256 ? 256 : t128 >= 128 ? 128 : 64;
  // A ragged N is read past its end only along B's rows (N-contiguous B).
  return HalfPath{tile, full_tiles(a, splits, tile, tile, overread_ok && !B_KC) && dma_addressable<A_KC, B_KC>(a)};
}

template <bool A_KC, bool B_KC>
hipError_t launch_half(hipStream_t s, HalfArgs a, int splits, bool bf16, float* cs_scratch, size_t cs_elems,
                       bool overread_ok, bool shares_to_caller) {
  const HalfPath hp = pick_path<A_KC, B_KC>(a, splits, overread_ok);
  a.n_ragged = hp.dma && a.N % hp.tile != 0;
  if (!hp.dma || splits > 1) a.nf_flag = nullptr;  // gemm_checks_nonfinite says false for these
  // Predicate bits only where the direct epilogue writes or reads them
  // (gemm_relu_bits_ok): never leave them unwritten or ignored silently.
  if ((a.relu_bits_out || a.relu_bits) &&
      (!hp.dma || splits > 1 || a.n_ragged || a.M % 16 != 0 || a.N % 64 != 0 ||
       (a.relu_bits_out && !(a.epi == RT_EPI_BIAS_RELU && a.out_bf16)) || (a.relu_bits && a.epi != RT_EPI_RELU_MASK)))
    return hipErrorInvalidValue;
  switch (hp.tile) {
    case 256:
      return hp.dma ? launch_dma<256, 256, 2, 4, A_KC, B_KC>(s, a, splits, bf16, cs_scratch, cs_elems,
                                                             shares_to_caller)
                    : launch_regs<256, 256, 4, 2, A_KC, B_KC>(s, a, splits, bf16);
    case 128:
      return hp.dma ? launch_dma<128, 128, 2, 2, A_KC, B_KC>(s, a, splits, bf16, cs_scratch, cs_elems,
                                                             shares_to_caller)
                    : launch_regs<128, 128, 2, 2, A_KC, B_KC>(s, a, splits, bf16);
    default:
      return hp.dma ? launch_dma<64, 64, 2, 2, A_KC, B_KC>(s, a, splits, bf16, cs_scratch, cs_elems,
                                                           shares_to_caller)
                    : launch_regs<64, 64, 2, 2, A_KC, B_KC>(s, a, splits, bf16);
  }
}

// M tiles whose column-sum shares launch_half writes per K slice (launch_dma's
// rule), 0 when the column sums are not shared.
template <bool A_KC, bool B_KC>
int half_share_rows(const HalfArgs& a, int splits, size_t cs_elems, bool have_scratch, bool overread_ok) {
  if (B_KC || !a.colsum || !have_scratch) return 0;
  const HalfPath hp = pick_path<A_KC, B_KC>(a, splits, overread_ok);
  if (!hp.dma) return 0;
  const int tiles_m = (a.M + hp.tile - 1) / hp.tile;
  return (tiles_m > 1 && (size_t)splits * tiles_m * a.N <= cs_elems) ? tiles_m : 0;
}

}  // namespace

namespace rt {

static HalfArgs half_args(const GemmDesc& d, int splits) {
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
  a.out_bf16 = splits == 1 && d.out_dtype == RT_BF16;
  a.colsum = splits > 1 ? d.colsum_partials : d.colsum;
  int kps = (d.K + splits - 1) / splits;
  kps = ((kps + BK - 1) / BK) * BK;
  a.k_per_split = splits > 1 ? kps : (d.K > 0 ? d.K : 1);
  a.split_stride = splits > 1 ? d.split_stride : 0;
  auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  a.vec_a = (d.lda % 8 == 0) && al16(d.A);
  a.vec_b = (d.ldb % 8 == 0) && al16(d.B);
  a.nf_flag = d.nf_flag;
  a.relu_bits_out = d.relu_bits_out;
  a.relu_bits = d.relu_bits;
  return a;
}

hipError_t gemm_half_launch(hipStream_t s, const GemmDesc& d) {
  if (d.in_dtype != RT_BF16 && d.in_dtype != RT_F16) return hipErrorInvalidValue;
  const int splits = d.splits < 1 ? 1 : d.splits;
  const HalfArgs a = half_args(d, splits);
  const bool bf16 = d.in_dtype == RT_BF16;
  switch (d.layout) {
    case RT_NN:
      return launch_half<true, false>(s, a, splits, bf16, d.cs_scratch, d.cs_scratch_elems, d.overread_ok,
                                      d.cs_shares_to_caller);
    case RT_TN:
      return launch_half<false, false>(s, a, splits, bf16, d.cs_scratch, d.cs_scratch_elems, d.overread_ok,
                                       d.cs_shares_to_caller);
    case RT_NT:
      return launch_half<true, true>(s, a, splits, bf16, d.cs_scratch, d.cs_scratch_elems, d.overread_ok,
                                     d.cs_shares_to_caller);
  }
  return hipErrorInvalidValue;
}

bool gemm_relu_bits_ok(const GemmDesc& d) {
  if ((d.in_dtype != RT_BF16 && d.in_dtype != RT_F16) || d.splits > 1 || d.M % 16 != 0 || d.N % 64 != 0) return false;
  if (!(d.epi == RT_EPI_BIAS_RELU && d.out_dtype == RT_BF16) && d.epi != RT_EPI_RELU_MASK) return false;
  const HalfArgs a = half_args(d, 1);
  HalfPath hp{};
  switch (d.layout) {
    case RT_NN: hp = pick_path<true, false>(a, 1, d.overread_ok); break;
    case RT_TN: hp = pick_path<false, false>(a, 1, d.overread_ok); break;
    case RT_NT: hp = pick_path<true, true>(a, 1, d.overread_ok); break;
    default: return false;
  }
  return hp.dma && a.N % hp.tile == 0;
}

bool gemm_checks_nonfinite(const GemmDesc& d) {
  if (d.nf_flag == nullptr || (d.in_dtype != RT_BF16 && d.in_dtype != RT_F16) || d.splits > 1) return false;
  const HalfArgs a = half_args(d, 1);
  switch (d.layout) {
    case RT_NN: return pick_path<true, false>(a, 1, d.overread_ok).dma;
    case RT_TN: return pick_path<false, false>(a, 1, d.overread_ok).dma;
    case RT_NT: return pick_path<true, true>(a, 1, d.overread_ok).dma;
  }
  return false;
}

static int share_rows(const GemmDesc& d) {
  if (d.in_dtype != RT_BF16 && d.in_dtype != RT_F16) return 0;
  const int splits = d.splits < 1 ? 1 : d.splits;
  const HalfArgs a = half_args(d, splits);
  const bool have = d.cs_scratch != nullptr;
  switch (d.layout) {
    case RT_NN: return half_share_rows<true, false>(a, splits, d.cs_scratch_elems, have, d.overread_ok);
    case RT_TN: return half_share_rows<false, false>(a, splits, d.cs_scratch_elems, have, d.overread_ok);
    default: return 0;
  }
}

int gemm_launch_count(const GemmDesc& d) {
  if (share_rows(d) == 0) return 1;
  return d.cs_shares_to_caller ? 1 : 2;  // otherwise the shares are added by a second launch
}

int gemm_cs_share_rows(const GemmDesc& d) { return d.cs_shares_to_caller ? share_rows(d) : 0; }

size_t colsum_scratch_need(int M, int N, int splits) {
  // The most M tiles any half kernel uses (64-row tiles), per K slice.
  return (size_t)(splits < 1 ? 1 : splits) * (size_t)((M + 63) / 64) * (size_t)N;
}

}  // namespace rt
