// Host runtime of the C ABI: device context, buffers, transfers, argument
// validation and the op-level entry points (rtensor::gpu::Gpu, mod.rs:224-1237).

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>

#include "rt_internal.h"

namespace rt {

hipError_t gemm_f32_launch(hipStream_t s, const GemmDesc& d);
hipError_t gemm_half_launch(hipStream_t s, const GemmDesc& d);

hipError_t gemm_launch(hipStream_t s, const GemmDesc& d) {
  if (d.in_dtype == RT_F32) return gemm_f32_launch(s, d);
  return gemm_half_launch(s, d);
}

size_t dtype_size(rt_dtype d) {
  switch (d) {
    case RT_F32: return 4;
    case RT_BF16: return 2;
    case RT_F16: return 2;
    case RT_U32: return 4;
  }
  return 0;
}

int fail(rt_ctx* c, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  return code;
}

int hip_fail(rt_ctx* c, hipError_t e, const char* what) {
  return fail(c, e == hipErrorOutOfMemory ? RT_ERR_OOM : RT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int ensure_scratch(rt_ctx* c, size_t elems) {
  if (elems <= c->scratch_elems) return RT_OK;
  // Earlier work may still read the old scratch.
  HIP_TRY(c, hipStreamSynchronize(c->stream), "scratch sync");
  if (c->scratch) hipFree(c->scratch);
  c->scratch = nullptr;
  c->scratch_elems = 0;
  HIP_TRY(c, hipMalloc((void**)&c->scratch, elems * sizeof(float)), "scratch");
  c->scratch_elems = elems;
  return RT_OK;
}

thread_local LaunchEvents* g_launch_events = nullptr;

static hipEvent_t take_event(rt_ctx* c) {
  if (!c->event_pool.empty()) {
    hipEvent_t e = c->event_pool.back();
    c->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

Launch::Launch(rt_ctx* c, const char* label) : c_(c), label_(label) {
  if (!c_->profiling) return;
  ev_.start = take_event(c_);
  ev_.stop = take_event(c_);
  if (ev_.start == nullptr || ev_.stop == nullptr) {
    if (ev_.start) c_->event_pool.push_back(ev_.start);
    if (ev_.stop) c_->event_pool.push_back(ev_.stop);
    return;
  }
  prev_ = g_launch_events;
  g_launch_events = &ev_;
  on_ = true;
}

Launch::~Launch() {
  if (!on_) return;
  g_launch_events = prev_;
  if (ev_.used) {
    c_->prof.push_back(rt_prof_rec{std::string(label_), ev_.start, ev_.stop});
  } else {  // nothing was launched in the scope
    c_->event_pool.push_back(ev_.start);
    c_->event_pool.push_back(ev_.stop);
  }
}

}  // namespace rt

using namespace rt;

// rt_open's last failure, per calling thread (contexts opened on different
// threads do not share it).
static thread_local std::string g_open_err;

static bool is_half(rt_dtype d) { return d == RT_BF16 || d == RT_F16; }
// Row and column counts of the row kernels (column sums, bias add, softmax
// cross-entropy, argmax) and GEMM dimensions: their int indices and launch
// plans add a block's, tile's or chunk's extent to a count, so counts stay
// well below INT32_MAX.
static constexpr size_t kRowOpMax = size_t(1) << 30;
static size_t cols_of(const rt_buf* b) { return b->rank >= 2 ? b->shape[b->rank - 1] : b->n; }

extern "C" {

int rt_open(int device, rt_ctx** out) {
  if (out == nullptr) return RT_ERR_INVALID;
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    g_open_err = std::string("no HIP device: ") + (e != hipSuccess ? hipGetErrorString(e) : "count is 0");
    return RT_ERR_NO_DEVICE;
  }
  if (device < 0 || device >= count) {
    g_open_err = "device ordinal out of range";
    return RT_ERR_NO_DEVICE;
  }
  e = hipSetDevice(device);
  if (e != hipSuccess) {
    g_open_err = std::string("hipSetDevice: ") + hipGetErrorString(e);
    return RT_ERR_NO_DEVICE;
  }
  hipDeviceProp_t props;
  e = hipGetDeviceProperties(&props, device);
  if (e != hipSuccess) {
    g_open_err = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
    return RT_ERR_NO_DEVICE;
  }
  std::string arch = props.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0) {
    g_open_err = "unsupported device arch " + arch + " (this library is built for gfx950)";
    return RT_ERR_NO_DEVICE;
  }
  auto* c = new rt_ctx();
  c->device = device;
  c->arch = arch;
  c->name = props.name;
  c->num_cus = props.multiProcessorCount;
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  // The device address of this device's copy of the static scratch array
  // of rt_gemm_splitk_static (loads its code object on this device).
  if (e == hipSuccess) e = static_scratch_address(&c->static_scratch);
  if (e == hipSuccess) e = hipMalloc(&c->d_flags, 64 * sizeof(int));
  if (e == hipSuccess) e = fill_i32_launch(c->stream, c->d_flags, 0, 64);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    g_open_err = std::string("context setup: ") + hipGetErrorString(e);
    if (c->d_flags) hipFree(c->d_flags);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
    return RT_ERR_HIP;
  }
  *out = c;
  return RT_OK;
}

int rt_close(rt_ctx* c) {
  CHECK_CTX(c);
  hipSetDevice(c->device);
  hipStreamSynchronize(c->stream);
  // The context owns what was created on it: models and buffers the caller
  // did not free go with it (their handles become invalid).
  for (rt_mlp* p : c->mlps) mlp_release(p);
  c->mlps.clear();
  for (rt_buf* b : c->bufs) {
    if (b->ptr) hipFree(b->ptr);
    delete b;
  }
  c->bufs.clear();
  for (auto& kv : c->pool)
    for (void* ptr : kv.second) hipFree(ptr);
  c->pool.clear();
  for (auto& r : c->prof) {
    hipEventDestroy(r.e0);
    hipEventDestroy(r.e1);
  }
  for (auto e : c->event_pool) hipEventDestroy(e);
  if (c->timer0) hipEventDestroy(c->timer0);
  if (c->timer1) hipEventDestroy(c->timer1);
  hipFree(c->d_flags);
  if (c->scratch) hipFree(c->scratch);
  if (c->copy_stream) hipStreamDestroy(c->copy_stream);
  hipStreamDestroy(c->stream);
  delete c;
  return RT_OK;
}

const char* rt_last_error(const rt_ctx* c) { return c ? c->err.c_str() : g_open_err.c_str(); }

int rt_info(rt_ctx* c, char* buf, size_t len) {
  CHECK_CTX(c);
  if (buf == nullptr || len == 0) return RT_ERR_INVALID;
  snprintf(buf, len, "%s (%s, %d CUs)", c->name.c_str(), c->arch.c_str(), c->num_cus);
  return RT_OK;
}

int rt_sync(rt_ctx* c) {
  CHECK_CTX(c);
  int flag = 0;
  HIP_TRY(c, hipMemcpyAsync(&flag, c->d_flags, sizeof(int), hipMemcpyDeviceToHost, c->stream), "flag read");
  HIP_TRY(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  if (flag != 0) {
    // The label flag is sticky until reported once.
    HIP_TRY(c, fill_i32_launch(c->stream, c->d_flags, 0, 1), "flag reset");
    HIP_TRY(c, hipStreamSynchronize(c->stream), "flag reset sync");
    return fail(c, RT_ERR_LABEL, "a label was >= the number of classes");
  }
  return RT_OK;
}

// Size classes of the buffer cache: 256-byte steps up to 1 MiB, then 1 MiB
// steps.  Cached bytes above kPoolMax are given back instead of kept.
static size_t size_class(size_t bytes) {
  constexpr size_t kMiB = size_t(1) << 20;
  if (bytes <= kMiB) return (bytes + 255) & ~size_t(255);
  return (bytes + kMiB - 1) & ~(kMiB - 1);
}
static constexpr size_t kPoolMax = size_t(16) << 30;

static void pool_trim(rt_ctx* c) {
  hipStreamSynchronize(c->stream);
  for (auto& kv : c->pool)
    for (void* ptr : kv.second) hipFree(ptr);
  c->pool.clear();
  c->pool_bytes = 0;
}

static hipError_t pool_alloc(rt_ctx* c, size_t cap, void** ptr) {
  auto it = c->pool.find(cap);
  if (it != c->pool.end() && !it->second.empty()) {
    *ptr = it->second.back();
    it->second.pop_back();
    c->pool_bytes -= cap;
    return hipSuccess;
  }
  hipError_t e = hipMalloc(ptr, cap);
  if (e == hipErrorOutOfMemory && c->pool_bytes > 0) {
    (void)hipGetLastError();
    pool_trim(c);
    e = hipMalloc(ptr, cap);
  }
  return e;
}

// Returns an allocation to the cache.  Work already enqueued may still use
// it; anything that reuses it is enqueued later on the same stream.
static void pool_release(rt_ctx* c, void* ptr, size_t cap) {
  if (ptr == nullptr) return;
  if (c->pool_bytes + cap > kPoolMax) {
    hipStreamSynchronize(c->stream);
    hipFree(ptr);
    return;
  }
  c->pool[cap].push_back(ptr);
  c->pool_bytes += cap;
}

static int make_buf(rt_ctx* c, rt_dtype dtype, const size_t* shape, int rank, rt_buf** out) {
  if (out == nullptr || (rank > 0 && shape == nullptr) || rank < 0 || rank > 4)
    return fail(c, RT_ERR_INVALID, "bad shape arguments");
  if (dtype < RT_F32 || dtype > RT_U32) return fail(c, RT_ERR_DTYPE, "unknown dtype %d", (int)dtype);
  size_t n = 1;
  for (int i = 0; i < rank; ++i) {
    if (shape[i] != 0 && n > (SIZE_MAX >> 4) / shape[i]) return fail(c, RT_ERR_SHAPE, "shape too large");
    n *= shape[i];
  }
  auto* b = new rt_buf();
  b->dtype = dtype;
  b->rank = rank;
  for (int i = 0; i < rank; ++i) b->shape[i] = shape[i];
  b->n = n;
  b->bytes = n * dtype_size(dtype);
  if (b->bytes > 0) {
    // Whole 256-byte granules, so fills and vector loads never need a tail.
    b->cap = size_class(b->bytes);
    hipError_t e = pool_alloc(c, b->cap, &b->ptr);
    if (e != hipSuccess) {
      delete b;
      return hip_fail(c, e, "hipMalloc");
    }
  }
  c->bufs.insert(b);
  *out = b;
  return RT_OK;
}

// Undoes make_buf for a buffer whose initialisation failed.
static void drop_buf(rt_ctx* c, rt_buf* b) {
  c->bufs.erase(b);
  pool_release(c, b->ptr, b->cap);
  delete b;
}

int rt_zeros(rt_ctx* c, rt_dtype dtype, const size_t* shape, int rank, rt_buf** out) {
  CHECK_CTX(c);
  int rc = make_buf(c, dtype, shape, rank, out);
  if (rc != RT_OK) return rc;
  rt_buf* b = *out;
  if (b->bytes > 0) {
    // Zero fill with a kernel, not a memset node (graph-capture safe).
    size_t words = (b->bytes + 3) / 4;
    hipError_t e = fill_i32_launch(c->stream, static_cast<int*>(b->ptr), 0, words);
    if (e != hipSuccess) {
      drop_buf(c, b);
      *out = nullptr;
      return hip_fail(c, e, "zero fill");
    }
  }
  return RT_OK;
}

int rt_empty(rt_ctx* c, rt_dtype dtype, const size_t* shape, int rank, rt_buf** out) {
  CHECK_CTX(c);
  return make_buf(c, dtype, shape, rank, out);
}

int rt_upload(rt_ctx* c, rt_dtype dtype, const size_t* shape, int rank, const void* host, rt_buf** out) {
  CHECK_CTX(c);
  int rc = make_buf(c, dtype, shape, rank, out);
  if (rc != RT_OK) return rc;
  rt_buf* b = *out;
  if (b->bytes > 0) {
    if (host == nullptr) {
      drop_buf(c, b);
      *out = nullptr;
      return fail(c, RT_ERR_INVALID, "null host pointer");
    }
    hipError_t e = hipMemcpyAsync(b->ptr, host, b->bytes, hipMemcpyHostToDevice, c->stream);
    // The host buffer is caller-owned and may be reused on return.
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
      drop_buf(c, b);
      *out = nullptr;
      return hip_fail(c, e, "upload");
    }
  }
  return RT_OK;
}

int rt_download(rt_ctx* c, const rt_buf* b, void* host, size_t bytes) {
  CHECK_CTX(c);
  if (b == nullptr || (host == nullptr && b->bytes > 0)) return fail(c, RT_ERR_INVALID, "null argument");
  if (bytes != b->bytes) return fail(c, RT_ERR_SHAPE, "download of %zu bytes from a %zu-byte tensor", bytes, b->bytes);
  if (b->bytes == 0) return RT_OK;
  HIP_TRY(c, hipMemcpyAsync(host, b->ptr, b->bytes, hipMemcpyDeviceToHost, c->stream), "download");
  HIP_TRY(c, hipStreamSynchronize(c->stream), "download sync");
  return RT_OK;
}

int rt_write(rt_ctx* c, rt_buf* b, const void* host, size_t bytes) {
  CHECK_CTX(c);
  if (b == nullptr || (host == nullptr && bytes > 0)) return fail(c, RT_ERR_INVALID, "null argument");
  if (bytes != b->bytes) return fail(c, RT_ERR_SHAPE, "write of %zu bytes into a %zu-byte tensor", bytes, b->bytes);
  if (bytes == 0) return RT_OK;
  HIP_TRY(c, hipMemcpyAsync(b->ptr, host, bytes, hipMemcpyHostToDevice, c->stream), "write");
  // The host buffer is caller-owned and may be reused on return.
  HIP_TRY(c, hipStreamSynchronize(c->stream), "write sync");
  return RT_OK;
}

int rt_free(rt_ctx* c, rt_buf* b) {
  CHECK_CTX(c);
  if (b == nullptr) return RT_OK;
  if (c->bufs.find(b) == c->bufs.end()) return fail(c, RT_ERR_INVALID, "buffer does not belong to this context");
  drop_buf(c, b);
  return RT_OK;
}

int rt_buf_info(const rt_buf* b, rt_dtype* dtype, size_t* shape, int* rank) {
  if (b == nullptr) return RT_ERR_INVALID;
  if (dtype) *dtype = b->dtype;
  if (rank) *rank = b->rank;
  if (shape)
    for (int i = 0; i < b->rank; ++i) shape[i] = b->shape[i];
  return RT_OK;
}

int rt_upload_labels(rt_ctx* c, const uint64_t* labels, size_t n, rt_buf** out) {
  CHECK_CTX(c);
  if (labels == nullptr && n > 0) return fail(c, RT_ERR_INVALID, "null labels");
  std::vector<uint32_t> v(n);
  for (size_t i = 0; i < n; ++i) {
    if (labels[i] > 0xffffffffULL) return fail(c, RT_ERR_LABEL, "label %zu does not fit u32", i);
    v[i] = (uint32_t)labels[i];
  }
  size_t shape[1] = {n};
  return rt_upload(c, RT_U32, shape, 1, v.data(), out);
}

int rt_convert(rt_ctx* c, const rt_buf* src, rt_buf* dst) {
  CHECK_CTX(c);
  if (!src || !dst) return fail(c, RT_ERR_INVALID, "null buffer");
  if (src->n != dst->n) return fail(c, RT_ERR_SHAPE, "convert: %zu vs %zu elements", src->n, dst->n);
  if (src->dtype == RT_U32 || dst->dtype == RT_U32) return fail(c, RT_ERR_DTYPE, "convert: u32 not supported");
  Launch L(c, "convert");
  HIP_TRY(c, convert_launch(c->stream, src->ptr, src->dtype, dst->ptr, dst->dtype, src->n), "convert");
  return RT_OK;
}

// ------------------------------------------------------------------ GEMM
static int gemm_shapes(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, size_t* M, size_t* N,
                       size_t* K) {
  if (a->rank != 2 || b->rank != 2) return fail(c, RT_ERR_SHAPE, "gemm operands must be rank 2");
  size_t am = a->shape[0], ak = a->shape[1], bk = b->shape[0], bn = b->shape[1];
  switch (layout) {
    case RT_NN: *M = am; *K = ak; *N = bn; if (bk != ak) goto bad; break;
    case RT_TN: *K = am; *M = ak; *N = bn; if (bk != am) goto bad; break;   // A stored [K, M]
    case RT_NT: *M = am; *K = ak; *N = bk; if (bn != ak) goto bad; break;   // B stored [N, K]
    default: return fail(c, RT_ERR_INVALID, "unknown layout %d", (int)layout);
  }
  // The kernels index tiles with int and round M, N, K up to whole tiles.
  if (*M > kRowOpMax || *N > kRowOpMax || *K > kRowOpMax) return fail(c, RT_ERR_SHAPE, "dimension too large");
  return RT_OK;
bad:
  return fail(c, RT_ERR_SHAPE, "gemm inner dimensions differ: [%zu,%zu] x [%zu,%zu] (layout %d)", am, ak, bk, bn,
              (int)layout);
}

static int check_epilogue(rt_ctx* c, rt_epilogue epi, const rt_buf* aux, const rt_buf* out, size_t M, size_t N) {
  if (epi == RT_EPI_NONE) return RT_OK;
  if (aux == nullptr) return fail(c, RT_ERR_INVALID, "epilogue needs an aux buffer");
  if (epi == RT_EPI_BIAS || epi == RT_EPI_BIAS_RELU) {
    if (aux->dtype != RT_F32 || aux->n != N) return fail(c, RT_ERR_SHAPE, "bias must be f32 with %zu elements", N);
  } else if (epi == RT_EPI_RELU_MASK) {
    if (aux->n != M * N || aux->dtype == RT_U32) return fail(c, RT_ERR_SHAPE, "mask must match C [%zu,%zu]", M, N);
    if (aux->dtype != out->dtype && !(out->dtype == RT_F32 && aux->dtype == RT_F32))
      return fail(c, RT_ERR_DTYPE, "mask dtype must match C");
  } else {
    return fail(c, RT_ERR_INVALID, "unknown epilogue %d", (int)epi);
  }
  return RT_OK;
}

int rt_gemm(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* out, rt_epilogue epi,
            const rt_buf* aux, rt_buf* colsum) {
  CHECK_CTX(c);
  if (!a || !b || !out) return fail(c, RT_ERR_INVALID, "null buffer");
  size_t M, N, K;
  int rc = gemm_shapes(c, layout, a, b, &M, &N, &K);
  if (rc) return rc;
  if (out->n != M * N || (out->rank == 2 && (out->shape[0] != M || out->shape[1] != N)))
    return fail(c, RT_ERR_SHAPE, "C must be [%zu,%zu]", M, N);
  if (a->dtype != b->dtype || a->dtype == RT_U32) return fail(c, RT_ERR_DTYPE, "A and B must share a float dtype");
  if (a->dtype == RT_F32 && out->dtype != RT_F32) return fail(c, RT_ERR_DTYPE, "f32 GEMM writes f32");
  if (is_half(a->dtype) && !(out->dtype == RT_F32 || out->dtype == RT_BF16))
    return fail(c, RT_ERR_DTYPE, "half GEMM writes f32 or bf16");
  if ((rc = check_epilogue(c, epi, aux, out, M, N))) return rc;
  if (colsum) {
    if (layout != RT_TN) return fail(c, RT_ERR_INVALID, "fused colsum is only for the TN layout");
    if (colsum->dtype != RT_F32 || colsum->n != N) return fail(c, RT_ERR_SHAPE, "colsum must be f32 [%zu]", N);
  }
  if (M == 0 || N == 0) return RT_OK;
  GemmDesc d;
  d.layout = layout;
  d.in_dtype = a->dtype;
  d.out_dtype = out->dtype;
  d.A = a->ptr;
  d.B = b->ptr;
  d.C = out->ptr;
  d.M = (int)M;
  d.N = (int)N;
  d.K = (int)K;
  d.lda = (int)a->shape[1];
  d.ldb = (int)b->shape[1];
  d.ldc = (int)N;
  d.epi = epi;
  if (epi == RT_EPI_BIAS || epi == RT_EPI_BIAS_RELU) d.bias = static_cast<const float*>(aux->ptr);
  if (epi == RT_EPI_RELU_MASK) {
    d.mask = aux->ptr;
    d.mask_dtype = aux->dtype;
  }
  d.colsum = colsum ? static_cast<float*>(colsum->ptr) : nullptr;
  if (narrow_nn(d)) {
    Launch L(c, "gemm_nn");
    HIP_TRY(c, narrow_nn_launch(c->stream, d), "gemm launch");
    return RT_OK;
  }
  if (colsum && is_half(a->dtype)) {
    if ((rc = ensure_scratch(c, colsum_scratch_need(d.M, d.N, 1)))) return rc;
    d.cs_scratch = c->scratch;
    d.cs_scratch_elems = c->scratch_elems;
  }
  Launch L(c, layout == RT_NN ? "gemm_nn" : layout == RT_TN ? "gemm_tn" : "gemm_nt");
  HIP_TRY(c, gemm_launch(c->stream, d), "gemm launch");
  return RT_OK;
}

int rt_linear_backward(rt_ctx* c, const rt_buf* x, const rt_buf* delta, const rt_buf* w, rt_buf* dx, rt_buf* dw,
                       rt_buf* db) {
  CHECK_CTX(c);
  if (!x || !delta || !w || !dw) return fail(c, RT_ERR_INVALID, "null buffer");
  if (x->rank != 2 || delta->rank != 2 || w->rank != 2) return fail(c, RT_ERR_SHAPE, "linear backward takes rank 2");
  const size_t m = x->shape[0], k = x->shape[1], n = w->shape[1];
  if (delta->shape[0] != m || delta->shape[1] != n || w->shape[0] != k)
    return fail(c, RT_ERR_SHAPE, "x [%zu,%zu], delta [%zu,%zu], w [%zu,%zu] do not chain", m, k, delta->shape[0],
                delta->shape[1], w->shape[0], n);
  const bool f32 = x->dtype == RT_F32 && delta->dtype == RT_F32 && w->dtype == RT_F32;
  const bool outs_f32 = dw->dtype == RT_F32 && (!dx || dx->dtype == RT_F32) && (!db || db->dtype == RT_F32);
  if (f32 && outs_f32 && dx && dw->n == k * n && dx->n == m * k && (!db || db->n == n) && m && n && k &&
      m <= kRowOpMax && n <= kRowOpMax && k <= kRowOpMax) {
    GemmDesc d0;  // dW = Xᵀ·δ (+ db = 1ᵀδ)
    d0.layout = RT_TN;
    d0.A = x->ptr;
    d0.B = delta->ptr;
    d0.C = dw->ptr;
    d0.M = (int)k;
    d0.N = (int)n;
    d0.K = (int)m;
    d0.lda = (int)k;
    d0.ldb = (int)n;
    d0.ldc = (int)n;
    d0.colsum = db ? static_cast<float*>(db->ptr) : nullptr;
    GemmDesc d1;  // dX = δ·Wᵀ
    d1.layout = RT_NT;
    d1.A = delta->ptr;
    d1.B = w->ptr;
    d1.C = dx->ptr;
    d1.M = (int)m;
    d1.N = (int)k;
    d1.K = (int)n;
    d1.lda = (int)n;
    d1.ldb = (int)n;
    d1.ldc = (int)k;
    if (gemm_pair_supported(d0, d1)) {
      Launch L(c, "linear_bwd");
      HIP_TRY(c, gemm_pair_launch(c->stream, d0, d1), "linear backward");
      return RT_OK;
    }
  }
  // Otherwise the two GEMMs one after the other (rt_gemm checks the rest).
  int rc = rt_gemm(c, RT_TN, x, delta, dw, RT_EPI_NONE, nullptr, db);
  if (rc == RT_OK && dx) rc = rt_gemm(c, RT_NT, delta, w, dx, RT_EPI_NONE, nullptr, nullptr);
  return rc;
}

size_t rt_splitk_slices(size_t m, size_t n, size_t k) {
  // Split only when the output tiles alone cannot fill the 256 CUs: aim for
  // ~256 workgroups (one per CU), keep at least 4 K steps of 32 per slice,
  // and cap at 32 slices so the partial planes stay small next to A and B.
  // (Against ~512: the f32 MLP step 0.1753 -> 0.1733 ms at batch 2048,
  // 0.0744 -> 0.0714 at 256, 0.094 -> 0.088 at 512; fewer planes to write
  // and sum, and the layer-0 dW tiles leave room for the update blocks
  // launched beside them.)
  const size_t tiles = ((m + 63) / 64) * ((n + 63) / 64);
  const size_t ksteps = (k + 31) / 32;
  if (tiles >= 256 || ksteps < 8) return 1;
  size_t s = std::min<size_t>(256 / tiles, ksteps / 4);
  s = std::min<size_t>(s, 32);
  return std::max<size_t>(s, 1);
}

}  // extern "C"

namespace rt {

int splitk_check(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, const rt_buf* out, size_t slices,
                 const rt_buf* colsum, size_t* M, size_t* N, size_t* K) {
  if (layout != RT_NN && layout != RT_TN) return fail(c, RT_ERR_INVALID, "split-K takes RT_NN or RT_TN");
  if (slices < 1 || slices > 1024) return fail(c, RT_ERR_INVALID, "slices must be in [1, 1024]");
  int rc = gemm_shapes(c, layout, a, b, M, N, K);
  if (rc) return rc;
  if (out->n != *M * *N || out->dtype != RT_F32) return fail(c, RT_ERR_SHAPE, "C must be f32 [%zu,%zu]", *M, *N);
  if (a->dtype != b->dtype || a->dtype == RT_U32) return fail(c, RT_ERR_DTYPE, "A and B must share a float dtype");
  if (colsum) {
    if (layout != RT_TN) return fail(c, RT_ERR_INVALID, "fused colsum is only for the TN layout");
    if (colsum->dtype != RT_F32 || colsum->n != *N) return fail(c, RT_ERR_SHAPE, "colsum must be f32 [%zu]", *N);
  }
  return RT_OK;
}

// A narrow f32 NN product (an output layer's logits, <= 16 columns) has too
// few output tiles for the tiled kernels to be anything but latency bound;
// the output-layer kernel splits its K over 8 waves of a block per 16 rows
// instead.  rt_gemm and a one-slice split-K both route it there, so that a
// split-K of one slice gives the whole GEMM's bits.
bool narrow_nn(const GemmDesc& d) {
  return d.layout == RT_NN && d.in_dtype == RT_F32 && (d.epi == RT_EPI_NONE || d.epi == RT_EPI_BIAS) &&
         d.colsum == nullptr && d.splits <= 1 && head_xent_supported(d.K, d.N) && d.lda == d.K &&
         (reinterpret_cast<uintptr_t>(d.A) & 15) == 0;
}

hipError_t narrow_nn_launch(hipStream_t s, const GemmDesc& d) {
  return head_xent_launch(s, static_cast<const float*>(d.A), d.K, static_cast<const float*>(d.B), d.bias, nullptr,
                          static_cast<float*>(d.C), nullptr, nullptr, d.M, d.N, 0.0f, nullptr);
}

int splitk_run(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* out, size_t slices,
               rt_buf* colsum, size_t M, size_t N, size_t K, float* part, float* cs_scratch, size_t cs_elems) {
  GemmDesc d;
  d.layout = layout;
  d.in_dtype = a->dtype;
  d.out_dtype = RT_F32;
  d.A = a->ptr;
  d.B = b->ptr;
  d.M = (int)M;
  d.N = (int)N;
  d.K = (int)K;
  d.lda = (int)a->shape[1];
  d.ldb = (int)b->shape[1];
  d.ldc = (int)N;
  if (colsum && is_half(a->dtype) && cs_elems > 0) {
    d.cs_scratch = cs_scratch;
    d.cs_scratch_elems = cs_elems;
  }
  if (slices == 1) {
    d.C = out->ptr;
    d.colsum = colsum ? static_cast<float*>(colsum->ptr) : nullptr;
    Launch L(c, "splitk_gemm");
    HIP_TRY(c, narrow_nn(d) ? narrow_nn_launch(c->stream, d) : gemm_launch(c->stream, d), "split-K gemm");
    return RT_OK;
  }
  d.C = part;
  d.splits = (int)slices;
  d.split_stride = (long long)(M * N);
  d.colsum_partials = colsum ? part + slices * M * N : nullptr;
  d.cs_shares_to_caller = true;  // the reduction below adds the column-sum shares
  const int cs_rows = gemm_cs_share_rows(d);
  {
    Launch L(c, "splitk_gemm");
    HIP_TRY(c, gemm_launch(c->stream, d), "split-K gemm");
  }
  Launch L(c, "splitk_reduce");
  HIP_TRY(c,
          splitk_reduce_launch(c->stream, part, (int)slices, (long long)(M * N), (int)M, (int)N, out->ptr, RT_F32,
                               (int)N, RT_EPI_NONE, nullptr, nullptr, RT_F32, cs_rows ? d.cs_scratch : d.colsum_partials,
                               colsum ? static_cast<float*>(colsum->ptr) : nullptr, cs_rows),
          "split-K reduce");
  return RT_OK;
}

}  // namespace rt

extern "C" {

int rt_gemm_splitk(rt_ctx* c, rt_layout layout, const rt_buf* a, const rt_buf* b, rt_buf* out, rt_buf* partials,
                   size_t slices, rt_buf* colsum) {
  CHECK_CTX(c);
  if (!a || !b || !out || !partials) return fail(c, RT_ERR_INVALID, "null buffer");
  size_t M, N, K;
  int rc = splitk_check(c, layout, a, b, out, slices, colsum, &M, &N, &K);
  if (rc) return rc;
  if (partials->dtype != RT_F32 || partials->n < slices * M * N + (colsum ? slices * N : 0))
    return fail(c, RT_ERR_SHAPE, "partials need %zu f32 elements", slices * M * N + (colsum ? slices * N : 0));
  if (M == 0 || N == 0) return RT_OK;
  if (colsum && is_half(a->dtype)) {
    if ((rc = ensure_scratch(c, colsum_scratch_need((int)M, (int)N, (int)slices)))) return rc;
  }
  return splitk_run(c, layout, a, b, out, slices, colsum, M, N, K, static_cast<float*>(partials->ptr), c->scratch,
                    (colsum && is_half(a->dtype)) ? c->scratch_elems : 0);
}

// ------------------------------------------------------------------ row / column ops
int rt_colsum(rt_ctx* c, const rt_buf* src, rt_buf* dst) {
  CHECK_CTX(c);
  if (!src || !dst) return fail(c, RT_ERR_INVALID, "null buffer");
  if (src->rank != 2) return fail(c, RT_ERR_SHAPE, "colsum source must be rank 2");
  size_t R = src->shape[0], Cc = src->shape[1];
  if (dst->dtype != RT_F32 || dst->n != Cc) return fail(c, RT_ERR_SHAPE, "colsum target must be f32 [1,%zu]", Cc);
  if (src->dtype == RT_U32) return fail(c, RT_ERR_DTYPE, "colsum of u32");
  if (R > kRowOpMax || Cc > kRowOpMax) return fail(c, RT_ERR_SHAPE, "colsum source too large");
  int rc = ensure_scratch(c, colsum_scratch_elems((int)R, (int)Cc, src->dtype));
  if (rc) return rc;
  Launch L(c, "colsum");
  HIP_TRY(c, colsum_launch(c->stream, src->ptr, src->dtype, (int)R, (int)Cc, static_cast<float*>(dst->ptr), c->scratch,
                           c->scratch_elems),
          "colsum");
  return RT_OK;
}

int rt_bias_add(rt_ctx* c, rt_buf* z, const rt_buf* b) {
  CHECK_CTX(c);
  if (!z || !b) return fail(c, RT_ERR_INVALID, "null buffer");
  if (z->dtype != RT_F32 || b->dtype != RT_F32) return fail(c, RT_ERR_DTYPE, "bias_add is f32");
  size_t cols = cols_of(z);
  if (b->n != cols || z->n % std::max<size_t>(cols, 1)) return fail(c, RT_ERR_SHAPE, "bias must have %zu elements", cols);
  if (z->n == 0) return RT_OK;
  if (cols > kRowOpMax || z->n / cols > kRowOpMax) return fail(c, RT_ERR_SHAPE, "bias_add: too large");
  Launch L(c, "bias_add");
  HIP_TRY(c, bias_add_launch(c->stream, static_cast<float*>(z->ptr), static_cast<const float*>(b->ptr),
                             (int)(z->n / cols), (int)cols),
          "bias_add");
  return RT_OK;
}

int rt_relu(rt_ctx* c, const rt_buf* x, rt_buf* y) {
  CHECK_CTX(c);
  if (!x || !y) return fail(c, RT_ERR_INVALID, "null buffer");
  if (x->dtype != RT_F32 || y->dtype != RT_F32 || x->n != y->n) return fail(c, RT_ERR_SHAPE, "relu: f32, same size");
  if (x->n == 0) return RT_OK;
  Launch L(c, "relu");
  HIP_TRY(c, relu_launch(c->stream, static_cast<const float*>(x->ptr), static_cast<float*>(y->ptr), x->n), "relu");
  return RT_OK;
}

int rt_relu_bwd(rt_ctx* c, const rt_buf* a, rt_buf* delta) {
  CHECK_CTX(c);
  if (!a || !delta) return fail(c, RT_ERR_INVALID, "null buffer");
  if (delta->dtype != RT_F32 || a->dtype == RT_U32 || a->n != delta->n)
    return fail(c, RT_ERR_SHAPE, "relu_bwd: delta f32, same size as a");
  if (a->n == 0) return RT_OK;
  Launch L(c, "relu_bwd");
  HIP_TRY(c, relu_bwd_launch(c->stream, a->ptr, a->dtype, static_cast<float*>(delta->ptr), a->n), "relu_bwd");
  return RT_OK;
}

int rt_softmax_xent(rt_ctx* c, const rt_buf* logits, const rt_buf* labels, rt_buf* delta, rt_buf* loss_rows,
                    float scale) {
  CHECK_CTX(c);
  if (!logits || !labels || !delta || !loss_rows) return fail(c, RT_ERR_INVALID, "null buffer");
  if (logits->rank != 2 || logits->dtype != RT_F32) return fail(c, RT_ERR_SHAPE, "logits must be f32 [B, C]");
  size_t B = logits->shape[0], Cc = logits->shape[1];
  if (labels->dtype != RT_U32 || labels->n != B) return fail(c, RT_ERR_SHAPE, "labels must be u32 [%zu]", B);
  if (delta->dtype != RT_F32 || delta->n != B * Cc) return fail(c, RT_ERR_SHAPE, "delta must be f32 [%zu,%zu]", B, Cc);
  if (loss_rows->dtype != RT_F32 || loss_rows->n != B) return fail(c, RT_ERR_SHAPE, "loss_rows must be f32 [%zu]", B);
  if (Cc == 0) return fail(c, RT_ERR_SHAPE, "zero classes");
  if (B > kRowOpMax || Cc > kRowOpMax) return fail(c, RT_ERR_SHAPE, "softmax_xent: too large");
  if (B == 0) return RT_OK;
  Launch L(c, "softmax_xent");
  HIP_TRY(c,
          xent_launch(c->stream, static_cast<const float*>(logits->ptr), static_cast<const uint32_t*>(labels->ptr),
                      static_cast<float*>(delta->ptr), nullptr, static_cast<float*>(loss_rows->ptr), (int)B, (int)Cc,
                      scale / (float)B, c->d_flags),
          "softmax_xent");
  return RT_OK;
}

int rt_argmax_rows(rt_ctx* c, const rt_buf* logits, rt_buf* out) {
  CHECK_CTX(c);
  if (!logits || !out) return fail(c, RT_ERR_INVALID, "null buffer");
  if (logits->rank != 2 || logits->dtype != RT_F32) return fail(c, RT_ERR_SHAPE, "logits must be f32 [B, C]");
  const size_t B = logits->shape[0], Cc = logits->shape[1];
  if (out->dtype != RT_U32 || out->n != B) return fail(c, RT_ERR_SHAPE, "out must be u32 [%zu]", B);
  if (Cc == 0 && B > 0) return fail(c, RT_ERR_SHAPE, "zero classes");
  if (B > kRowOpMax || Cc > kRowOpMax) return fail(c, RT_ERR_SHAPE, "argmax: too large");
  if (B == 0) return RT_OK;
  Launch L(c, "argmax");
  HIP_TRY(c,
          argmax_launch(c->stream, static_cast<const float*>(logits->ptr), static_cast<uint32_t*>(out->ptr), (int)B,
                        (int)Cc),
          "argmax");
  return RT_OK;
}

int rt_accuracy(rt_ctx* c, const rt_buf* logits, const rt_buf* labels, float* out) {
  CHECK_CTX(c);
  if (!logits || !labels || !out) return fail(c, RT_ERR_INVALID, "null argument");
  if (logits->rank != 2 || logits->dtype != RT_F32) return fail(c, RT_ERR_SHAPE, "logits must be f32 [B, C]");
  const size_t B = logits->shape[0], Cc = logits->shape[1];
  if (labels->dtype != RT_U32 || labels->n != B) return fail(c, RT_ERR_SHAPE, "labels must be u32 [%zu]", B);
  // hits / labels.len() as the reference computes it: 0/0 = NaN for an empty
  // batch; zero columns give no predictions, hence no hits.
  if (B == 0 || Cc == 0) {
    *out = B == 0 ? std::nanf("") : 0.0f;
    return RT_OK;
  }
  if (B > kRowOpMax || Cc > kRowOpMax) return fail(c, RT_ERR_SHAPE, "argmax: too large");
  // Predictions in the context scratch (grow-only), then compared on the host.
  int rc = ensure_scratch(c, B);
  if (rc) return rc;
  uint32_t* pred = reinterpret_cast<uint32_t*>(c->scratch);
  {
    Launch L(c, "argmax");
    HIP_TRY(c, argmax_launch(c->stream, static_cast<const float*>(logits->ptr), pred, (int)B, (int)Cc), "argmax");
  }
  std::vector<uint32_t> hp(B), hl(B);
  HIP_TRY(c, hipMemcpyAsync(hp.data(), pred, B * 4, hipMemcpyDeviceToHost, c->stream), "download");
  HIP_TRY(c, hipMemcpyAsync(hl.data(), labels->ptr, B * 4, hipMemcpyDeviceToHost, c->stream), "download");
  HIP_TRY(c, hipStreamSynchronize(c->stream), "sync");
  size_t hits = 0;
  for (size_t i = 0; i < B; ++i) hits += hp[i] == hl[i];
  *out = (float)hits / (float)B;
  return RT_OK;
}

// One launch per run of at most kMaxOptTensors tensors.  A tensor listed again
// starts a new run: the tensors of one launch are updated concurrently, and a
// repeated one must see its first update before the second, as in a loop over
// the list.
static int launch_opt_list(rt_ctx* c, const std::vector<OptTensor>& ts, const OptParams& P) {
  size_t i = 0;
  while (i < ts.size()) {
    size_t j = i + 1;
    while (j < ts.size() && j - i < (size_t)kMaxOptTensors) {
      bool repeat = false;
      for (size_t q = i; q < j && !repeat; ++q) repeat = ts[q].theta == ts[j].theta;
      if (repeat) break;
      ++j;
    }
    Launch L(c, "optimizer");
    HIP_TRY(c, optimizer_launch(c->stream, ts.data() + i, (int)(j - i), P), "optimizer");
    i = j;
  }
  return RT_OK;
}

int rt_adam_many(rt_ctx* c, int n, rt_buf* const* theta, rt_buf* const* m, rt_buf* const* v, const rt_buf* const* g,
                 float lr, float beta1, float beta2, float eps, int t) {
  CHECK_CTX(c);
  if (n < 0 || (n > 0 && (!theta || !m || !v || !g))) return fail(c, RT_ERR_INVALID, "null tensor list");
  if (t < 1) return fail(c, RT_ERR_INVALID, "adam step t must be >= 1");
  std::vector<OptTensor> ts;
  ts.reserve(n);
  for (int i = 0; i < n; ++i) {
    if (!theta[i] || !m[i] || !v[i] || !g[i]) return fail(c, RT_ERR_INVALID, "null buffer (tensor %d)", i);
    if (theta[i]->dtype != RT_F32 || m[i]->dtype != RT_F32 || v[i]->dtype != RT_F32 || g[i]->dtype != RT_F32)
      return fail(c, RT_ERR_DTYPE, "adam is f32 (tensor %d)", i);
    const size_t len = theta[i]->n;
    if (m[i]->n != len || v[i]->n != len || g[i]->n != len) return fail(c, RT_ERR_SHAPE, "adam: sizes differ (tensor %d)", i);
    if (len == 0) continue;
    ts.push_back(OptTensor{static_cast<float*>(theta[i]->ptr), static_cast<const float*>(g[i]->ptr),
                           static_cast<float*>(m[i]->ptr), static_cast<float*>(v[i]->ptr), nullptr, len});
  }
  OptParams P;
  P.kind = 0;
  P.lr = lr;
  P.beta1 = beta1;
  P.beta2 = beta2;
  P.eps = eps;
  float c1 = 1.0f - powi_f32(beta1, t), c2 = 1.0f - powi_f32(beta2, t);
  P.inv_c1 = 1.0f / c1;
  P.inv_c2 = 1.0f / c2;
  return launch_opt_list(c, ts, P);
}

int rt_adam(rt_ctx* c, rt_buf* theta, rt_buf* m, rt_buf* v, const rt_buf* g, float lr, float beta1, float beta2,
            float eps, int t) {
  return rt_adam_many(c, 1, &theta, &m, &v, &g, lr, beta1, beta2, eps, t);
}

int rt_sgd_many(rt_ctx* c, int n, rt_buf* const* theta, rt_buf* const* velocity, const rt_buf* const* g, float lr,
                float momentum) {
  CHECK_CTX(c);
  if (n < 0 || (n > 0 && (!theta || !g))) return fail(c, RT_ERR_INVALID, "null tensor list");
  if (momentum != 0.0f && n > 0 && !velocity) return fail(c, RT_ERR_INVALID, "sgd with momentum needs velocities");
  std::vector<OptTensor> ts;
  ts.reserve(n);
  for (int i = 0; i < n; ++i) {
    if (!theta[i] || !g[i]) return fail(c, RT_ERR_INVALID, "null buffer (tensor %d)", i);
    if (theta[i]->dtype != RT_F32 || g[i]->dtype != RT_F32) return fail(c, RT_ERR_DTYPE, "sgd is f32 (tensor %d)", i);
    const size_t len = theta[i]->n;
    if (g[i]->n != len) return fail(c, RT_ERR_SHAPE, "sgd: sizes differ (tensor %d)", i);
    rt_buf* vel = momentum != 0.0f ? velocity[i] : nullptr;
    if (momentum != 0.0f && (vel == nullptr || vel->n != len || vel->dtype != RT_F32))
      return fail(c, RT_ERR_INVALID, "sgd with momentum needs an f32 velocity buffer (tensor %d)", i);
    if (len == 0) continue;
    ts.push_back(OptTensor{static_cast<float*>(theta[i]->ptr), static_cast<const float*>(g[i]->ptr),
                           vel ? static_cast<float*>(vel->ptr) : nullptr, nullptr, nullptr, len});
  }
  OptParams P;
  P.kind = 1;
  P.lr = lr;
  P.momentum = momentum;
  return launch_opt_list(c, ts, P);
}

int rt_sgd(rt_ctx* c, rt_buf* theta, rt_buf* velocity, const rt_buf* g, float lr, float momentum) {
  return rt_sgd_many(c, 1, &theta, &velocity, &g, lr, momentum);
}

// ------------------------------------------------------------------ profiling
int rt_profile_enable(rt_ctx* c, int on) {
  CHECK_CTX(c);
  c->profiling = on != 0;
  return RT_OK;
}

int rt_profile_reset(rt_ctx* c) {
  CHECK_CTX(c);
  HIP_TRY(c, hipStreamSynchronize(c->stream), "profile sync");
  for (auto& r : c->prof) {
    c->event_pool.push_back(r.e0);
    c->event_pool.push_back(r.e1);
  }
  c->prof.clear();
  return RT_OK;
}

int rt_profile_report(rt_ctx* c, char* names, size_t name_len, int* counts, double* ms, int cap, int* n_out) {
  CHECK_CTX(c);
  HIP_TRY(c, hipStreamSynchronize(c->stream), "profile sync");
  std::vector<std::string> order;
  std::map<std::string, std::pair<int, double>> agg;
  for (auto& r : c->prof) {
    float t = 0;
    HIP_TRY(c, hipEventElapsedTime(&t, r.e0, r.e1), "hipEventElapsedTime");
    auto it = agg.find(r.label);
    if (it == agg.end()) {
      order.push_back(r.label);
      agg[r.label] = {1, (double)t};
    } else {
      it->second.first += 1;
      it->second.second += t;
    }
  }
  int n = 0;
  for (auto& lbl : order) {
    if (n >= cap) break;
    if (names && name_len) {
      strncpy(names + (size_t)n * name_len, lbl.c_str(), name_len - 1);
      names[(size_t)n * name_len + name_len - 1] = 0;
    }
    if (counts) counts[n] = agg[lbl].first;
    if (ms) ms[n] = agg[lbl].second;
    ++n;
  }
  if (n_out) *n_out = n;
  return RT_OK;
}

int rt_timer_begin(rt_ctx* c) {
  CHECK_CTX(c);
  if (!c->timer0) HIP_TRY(c, hipEventCreate(&c->timer0), "timer event");
  if (!c->timer1) HIP_TRY(c, hipEventCreate(&c->timer1), "timer event");
  HIP_TRY(c, hipEventRecord(c->timer0, c->stream), "timer begin");
  c->timer_running = true;
  return RT_OK;
}

int rt_timer_end(rt_ctx* c, float* ms) {
  CHECK_CTX(c);
  if (!c->timer_running || ms == nullptr) return fail(c, RT_ERR_INVALID, "rt_timer_end without rt_timer_begin");
  c->timer_running = false;
  HIP_TRY(c, hipEventRecord(c->timer1, c->stream), "timer end");
  HIP_TRY(c, hipEventSynchronize(c->timer1), "timer sync");
  HIP_TRY(c, hipEventElapsedTime(ms, c->timer0, c->timer1), "timer elapsed");
  return RT_OK;
}

}  // extern "C"
