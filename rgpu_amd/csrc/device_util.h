// Device-side helpers shared by the GEMM kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

namespace rt_dev {

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).  Used
// where the body indexes register arrays, which must stay in registers.
template <int B, int E, class F>
__device__ inline void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Workgroup barrier for the direct-to-LDS pipelines: this wave's LDS reads
// are complete (lgkmcnt 0), then s_barrier.  Unlike __syncthreads it does not
// wait for outstanding global loads (later stages in flight); the asm's
// memory clobber keeps the compiler from moving LDS accesses across it.
__device__ inline void barrier_lds() {
  __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4));  // lgkmcnt(0) only
  asm volatile("s_barrier" ::: "memory");
}

// s_waitcnt vmcnt(N), leaving the LDS and export counters alone.
template <int N>
__device__ inline void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Raw buffer descriptor over `base` (word 3 = 0x00020000: untyped, 32-bit
// data format).  Offsets are 32-bit bytes; callers keep every access below
// 2^31 bytes from base.
__device__ inline __amdgpu_buffer_rsrc_t raw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// One 16-byte-per-lane DMA from global memory (rsrc + voff + soff bytes) into
// LDS at lds + 16 * lane.  The scalar offset is made opaque to the optimiser,
// which would otherwise fold it into a separate VGPR offset per instruction.
__device__ inline void dma16(__amdgpu_buffer_rsrc_t rsrc, void* lds, int voff, int soff) {
  int so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("" : "+s"(so));
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voff, so, 0, 0);
}

// dma16 issued as inline asm.  The compiler orders its own LDS DMA against
// every later LDS read it cannot prove disjoint with a vmcnt(0) wait, so a
// pipeline that reads stage k while stage k+1 is in flight waits for stage
// k+1 before the first read of stage k.  This form is invisible to that
// bookkeeping: the caller's own wait_vm before its barrier is then the only
// ordering, and a caller must wait_vm<0>() before reusing the LDS it targets.
// M0 (the LDS destination) is set inside the asm; kernels that use this form
// must not also use the builtin, which may keep M0 live across it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void dma16_asm(__amdgpu_buffer_rsrc_t rsrc, void* lds, int voff, int soff) {
  const int so = __builtin_amdgcn_readfirstlane(soff);
  const unsigned dst = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(__attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(dst), "v"(voff), "s"(rsrc),
               "s"(so)
               : "m0");
}
#pragma clang diagnostic pop

}  // namespace rt_dev
