// rt_gemm_splitk_static: the split-K GEMM of rt_gemm_splitk for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// or training loops, harnesses that forbid hipMalloc).  The K-slice partial
// planes, their column-sum rows and the half GEMM's column-sum shares live in
// `scratch`, one static device array of this library, instead of in a
// caller's workspace and the context's grow-only scratch.
//
// Each GPU the library runs on holds its own copy of the array (64 MiB) from
// the first rt_open on it until the process ends.  Every call on a device
// uses that device's copy and leaves its contents behind: calls that overlap
// on one GPU (two contexts' streams, two threads) race on it.  Calls on one
// context are ordered by its stream and do not.  Nothing needs clearing
// between calls: every slice writes its whole plane and column-sum row (an
// empty K range writes zeros), and the column-sum shares are written whole.

#include "rt_internal.h"

namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr size_t kScratchFloats = kScratchBytes / sizeof(float);

// In host code `scratch` names a host-side stand-in, not device memory: the
// device address comes from hipGetSymbolAddress (per device, at rt_open).
static __device__ __align__(256) float scratch[kScratchFloats];

}  // namespace

namespace rt {

hipError_t static_scratch_address(float** out) {
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  *out = e == hipSuccess ? static_cast<float*>(ptr) : nullptr;
  return e;
}

size_t static_scratch_floats() { return kScratchFloats; }

}  // namespace rt

using namespace rt;

extern "C" int rt_gemm_splitk_static(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* out,
                                     size_t slices, rt_buf* colsum) {
  CHECK_CTX(c);
  if (!a || !b || !out) return fail(c, RT_ERR_INVALID, "null buffer");
  if (c->static_scratch == nullptr) return fail(c, RT_ERR_HIP, "the static scratch array has no device address");
  size_t M, N, K;
  int rc = splitk_check(c, layout, a, b, out, slices, colsum, &M, &N, &K);
  if (rc) return rc;
  const bool half = a->dtype == RT_BF16 || a->dtype == RT_F16;
  const size_t planes = slices > 1 ? slices * M * N + (colsum ? slices * N : 0) : 0;
  const size_t shares = (colsum && half) ? colsum_scratch_need((int)M, (int)N, (int)slices) : 0;
  if (planes + shares > kScratchFloats)
    return fail(c, RT_ERR_SHAPE,
                "%zu slices of a [%zu,%zu] product need %zu floats of scratch; the static array holds %zu (64 MiB)",
                slices, M, N, planes + shares, kScratchFloats);
  if (M == 0 || N == 0) return RT_OK;
  float* base = c->static_scratch;
  return splitk_run(c, layout, a, b, out, slices, colsum, M, N, K, base, base + planes, shares);
}
