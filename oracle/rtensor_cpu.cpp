// oracle/rtensor_cpu.cpp -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// A C++ restatement of rtensor's single-threaded CPU path, the reference
// results that the HIP backend in rgpu_amd/ is checked against, and the CPU
// baseline that bench.py times next to it.  Only tests/, the smoke check in
// __graft_entry__.py and the cpu_baseline leg of bench.py load this library.
//
// What it restates (paths relative to the rtensor crate, crates/rtensor/):
//   Rng             src/rng.rs:3-49      xorshift64*, 24-bit uniform, Box-Muller
//   Tensor          src/tensor.rs        matmul (318-373), t (132-155),
//                                        zip/broadcast (183-246), reduce_to
//                                        (399-438), softmax_rows (455-472),
//                                        argmax_rows (476-493), sum/mean (279-286)
//   Tape / Var      src/tape.rs:43-229   reverse sweep with in-place accumulation
//   VJPs            src/ops.rs:38-322    add/sub/mul/div/matmul/scale/.../softmax
//   losses          src/losses.rs        mse, mae, softmax_cross_entropy,
//                                        binary_cross_entropy, one_hot, accuracy
//   optimizers      src/optim.rs:62-198  Sgd (with momentum), Adam
//   Dense           src/nn.rs:108-192    Glorot init order, forward order
//
// Numerics: compiled with -ffp-contract=off and without fast-math, so every
// a*b+c rounds twice exactly as rustc's output does.  Summations keep the
// reference's sequential order.  The row-parallel matmul splits the output
// rows across threads; each output element still sums k in order 0..k-1, so
// the result is bit-identical to the single-threaded one.
//
// Parity status of each function is recorded in the header of oracle.py.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace oc {

static int g_threads = 1;
static thread_local std::string g_err;

// ----------------------------------------------------------------- Rng
// rng.rs:3-49.  xorshift64* with the reference's shift triple and multiplier.
struct Rng {
  uint64_t state;
  explicit Rng(uint64_t seed) : state(seed == 0 ? 0x9E3779B97F4A7C15ULL : seed) {}
  uint64_t next_u64() {  // rng.rs:12-19
    uint64_t x = state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    state = x;
    return x * 0x2545F4914F6CDD1DULL;  // wrapping multiply
  }
  float uniform() {  // rng.rs:22-24: top 24 bits / 2^24
    return (float)(next_u64() >> 40) / (float)(1ULL << 24);
  }
  float range(float lo, float hi) { return lo + uniform() * (hi - lo); }  // rng.rs:27-29
  float normal() {  // rng.rs:32-36
    float u1 = std::fmax(uniform(), 1e-7f);
    float u2 = uniform();
    const float two_pi = 2.0f * 3.14159265358979323846f;  // 2 * f32::consts::PI, exact doubling
    return std::sqrt(-2.0f * std::log(u1)) * std::cos(two_pi * u2);
  }
  uint64_t below(uint64_t n) { return next_u64() % n; }  // rng.rs:38-40
};

// ----------------------------------------------------------------- Tensor
struct Tensor {
  std::vector<size_t> shape;
  std::vector<float> data;

  Tensor() = default;
  Tensor(std::vector<size_t> s, std::vector<float> d) : shape(std::move(s)), data(std::move(d)) {
    size_t n = 1;
    for (size_t v : shape) n *= v;
    if (n != data.size()) throw std::runtime_error("shape does not match element count");
  }
  static Tensor full(const std::vector<size_t>& s, float v) {
    size_t n = 1;
    for (size_t x : s) n *= x;
    return Tensor(s, std::vector<float>(n, v));
  }
  static Tensor zeros(const std::vector<size_t>& s) { return full(s, 0.0f); }
  static Tensor scalar(float v) { return Tensor({}, {v}); }
  size_t len() const { return data.size(); }
  size_t rank() const { return shape.size(); }
  bool is_scalar() const { return data.size() == 1; }
  float item() const {
    if (!is_scalar()) throw std::runtime_error("item() needs a one-element tensor");
    return data[0];
  }

  // tensor.rs:132-155: blocked 32x32 transpose (values only move, so the
  // blocking does not affect results).
  Tensor t() const {
    if (rank() != 2) throw std::runtime_error("t() needs rank 2");
    size_t r = shape[0], c = shape[1];
    std::vector<float> out(data.size());
    const size_t T = 32;
    for (size_t i0 = 0; i0 < r; i0 += T) {
      size_t i1 = std::min(i0 + T, r);
      for (size_t j0 = 0; j0 < c; j0 += T) {
        size_t j1 = std::min(j0 + T, c);
        for (size_t i = i0; i < i1; ++i)
          for (size_t j = j0; j < j1; ++j) out[j * r + i] = data[i * c + j];
      }
    }
    return Tensor({c, r}, std::move(out));
  }

  template <class F>
  Tensor map(F f) const {
    std::vector<float> out(data.size());
    for (size_t i = 0; i < data.size(); ++i) out[i] = f(data[i]);
    return Tensor(shape, std::move(out));
  }

  float sum_all() const {  // tensor.rs:279-281: sequential iterator sum
    float s = 0.0f;
    for (float v : data) s += v;
    return s;
  }
  float mean_all() const { return sum_all() / (float)data.size(); }  // tensor.rs:284-286
};

static std::vector<size_t> broadcast_shapes(const std::vector<size_t>& a, const std::vector<size_t>& b) {
  size_t rank = std::max(a.size(), b.size());
  std::vector<size_t> out(rank);
  for (size_t i = 0; i < rank; ++i) {
    size_t da = i < rank - a.size() ? 1 : a[i - (rank - a.size())];
    size_t db = i < rank - b.size() ? 1 : b[i - (rank - b.size())];
    if (da == db) out[i] = da;
    else if (da == 1) out[i] = db;
    else if (db == 1) out[i] = da;
    else throw std::runtime_error("shapes are not broadcast-compatible");
  }
  return out;
}

// Strides of `from` in the index space of `to` (0 on broadcast axes).
static std::vector<size_t> broadcast_strides(const std::vector<size_t>& from, const std::vector<size_t>& to) {
  std::vector<size_t> base(from.size());
  size_t acc = 1;
  for (size_t i = from.size(); i-- > 0;) {
    base[i] = acc;
    acc *= from[i];
  }
  size_t off = to.size() - from.size();
  std::vector<size_t> out(to.size(), 0);
  for (size_t i = off; i < to.size(); ++i) {
    size_t d = from[i - off];
    out[i] = (d == 1 && to[i] != 1) ? 0 : base[i - off];
  }
  return out;
}

static void bump(std::vector<size_t>& idx, const std::vector<size_t>& shape) {
  for (size_t ax = shape.size(); ax-- > 0;) {
    if (++idx[ax] < shape[ax]) return;
    idx[ax] = 0;
  }
}

// tensor.rs:183-246.  Every element is f(a[σa(i)], b[σb(i)]) whichever fast
// path the reference takes, so one strided loop gives identical values.
template <class F>
static Tensor zip(const Tensor& a, const Tensor& b, F f) {
  std::vector<size_t> shape = broadcast_shapes(a.shape, b.shape);
  size_t n = 1;
  for (size_t v : shape) n *= v;
  std::vector<float> out(n);
  if (a.shape == b.shape) {
    for (size_t i = 0; i < n; ++i) out[i] = f(a.data[i], b.data[i]);
    return Tensor(shape, std::move(out));
  }
  if (b.len() == 1 || a.len() == 1) {
    for (size_t i = 0; i < n; ++i) out[i] = f(a.data[a.len() == 1 ? 0 : i], b.data[b.len() == 1 ? 0 : i]);
    return Tensor(shape, std::move(out));
  }
  std::vector<size_t> sa = broadcast_strides(a.shape, shape), sb = broadcast_strides(b.shape, shape);
  std::vector<size_t> idx(shape.size(), 0);
  for (size_t l = 0; l < n; ++l) {
    size_t ia = 0, ib = 0;
    for (size_t ax = 0; ax < shape.size(); ++ax) {
      ia += idx[ax] * sa[ax];
      ib += idx[ax] * sb[ax];
    }
    out[l] = f(a.data[ia], b.data[ib]);
    bump(idx, shape);
  }
  return Tensor(shape, std::move(out));
}

static Tensor t_add(const Tensor& a, const Tensor& b) { return zip(a, b, [](float x, float y) { return x + y; }); }
static Tensor t_sub(const Tensor& a, const Tensor& b) { return zip(a, b, [](float x, float y) { return x - y; }); }
static Tensor t_mul(const Tensor& a, const Tensor& b) { return zip(a, b, [](float x, float y) { return x * y; }); }
static Tensor t_div(const Tensor& a, const Tensor& b) { return zip(a, b, [](float x, float y) { return x / y; }); }
static Tensor t_scale(const Tensor& a, float k) { return a.map([k](float x) { return x * k; }); }
static Tensor t_neg(const Tensor& a) { return a.map([](float x) { return -x; }); }

// tensor.rs:318-373.  ikj order, a==0 skipped, k*n <= 32768 single sweep,
// otherwise (JC=256 column panel) x (PC=128 depth panel) blocking.  Each
// output element accumulates p = 0..k-1 in order with a separately rounded
// product, which is what makes this bit-identical to the reference.
// Row-parallel: threads own disjoint row ranges and run the same loop nest.
static void matmul_raw(const float* A, const float* B, float* C, size_t m, size_t k, size_t n, int threads) {
  std::fill(C, C + m * n, 0.0f);
  if (m == 0 || n == 0 || k == 0) return;
  auto rows = [&](size_t r0, size_t r1) {
    if (k * n <= 32768) {
      for (size_t i = r0; i < r1; ++i) {
        float* dst = C + i * n;
        const float* arow = A + i * k;
        for (size_t p = 0; p < k; ++p) {
          float a = arow[p];
          if (a == 0.0f) continue;
          const float* brow = B + p * n;
          for (size_t j = 0; j < n; ++j) dst[j] += a * brow[j];
        }
      }
      return;
    }
    const size_t JC = 256, PC = 128;
    for (size_t j0 = 0; j0 < n; j0 += JC) {
      size_t j1 = std::min(j0 + JC, n);
      for (size_t p0 = 0; p0 < k; p0 += PC) {
        size_t p1 = std::min(p0 + PC, k);
        for (size_t i = r0; i < r1; ++i) {
          const float* arow = A + i * k;
          float* dst = C + i * n;
          for (size_t p = p0; p < p1; ++p) {
            float a = arow[p];
            if (a == 0.0f) continue;
            const float* brow = B + p * n;
            for (size_t j = j0; j < j1; ++j) dst[j] += a * brow[j];
          }
        }
      }
    }
  };
  int nt = std::max(1, std::min<int>(threads, (int)m));
  if (nt == 1) {
    rows(0, m);
    return;
  }
#ifdef _OPENMP
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int t = 0; t < nt; ++t) {
    size_t r0 = m * (size_t)t / (size_t)nt, r1 = m * (size_t)(t + 1) / (size_t)nt;
    rows(r0, r1);
  }
#else
  rows(0, m);
#endif
}

static Tensor matmul(const Tensor& a, const Tensor& b) {
  if (a.rank() != 2 || b.rank() != 2) throw std::runtime_error("matmul needs rank 2");
  size_t m = a.shape[0], k = a.shape[1], n = b.shape[1];
  if (b.shape[0] != k) throw std::runtime_error("matmul inner dimensions differ");
  std::vector<float> out(m * n);
  matmul_raw(a.data.data(), b.data.data(), out.data(), m, k, n, g_threads);
  return Tensor({m, n}, std::move(out));
}

// tensor.rs:399-438.  Undo a broadcast by summing over the broadcast axes.
// Every reference path adds contributions in increasing linear index of the
// source, which the single strided loop below also does.
static Tensor reduce_to(const Tensor& g, const std::vector<size_t>& target) {
  if (g.shape == target) return g;
  size_t n = 1;
  for (size_t v : target) n *= v;
  if (n == 1) return Tensor(target, {g.sum_all()});
  // [rows, cols] -> [1, cols]: out[j] += G[i, j], rows in order (tensor.rs:411-419)
  if (g.rank() == 2 && target.size() == 2 && target[0] == 1 && target[1] == g.shape[1]) {
    size_t c = g.shape[1];
    std::vector<float> out(c, 0.0f);
    for (size_t i = 0; i < g.shape[0]; ++i)
      for (size_t j = 0; j < c; ++j) out[j] += g.data[i * c + j];
    return Tensor(target, std::move(out));
  }
  // [rows, cols] -> [rows, 1]: sequential row sums (tensor.rs:422-426)
  if (g.rank() == 2 && target.size() == 2 && target[0] == g.shape[0] && target[1] == 1) {
    size_t c = g.shape[1];
    std::vector<float> out(g.shape[0]);
    for (size_t i = 0; i < g.shape[0]; ++i) {
      float s = 0.0f;
      for (size_t j = 0; j < c; ++j) s += g.data[i * c + j];
      out[i] = s;
    }
    return Tensor(target, std::move(out));
  }
  std::vector<float> out(n, 0.0f);
  std::vector<size_t> st = broadcast_strides(target, g.shape);
  std::vector<size_t> idx(g.shape.size(), 0);
  for (size_t l = 0; l < g.len(); ++l) {
    size_t it = 0;
    for (size_t ax = 0; ax < idx.size(); ++ax) it += idx[ax] * st[ax];
    out[it] += g.data[l];
    bump(idx, g.shape);
  }
  return Tensor(target, std::move(out));
}

// tensor.rs:455-472: max-stabilised row softmax; exp, sequential sum, divide.
static Tensor softmax_rows(const Tensor& z) {
  if (z.rank() != 2) throw std::runtime_error("softmax_rows needs rank 2");
  size_t r = z.shape[0], c = z.shape[1];
  std::vector<float> out(r * c);
  for (size_t i = 0; i < r; ++i) {
    const float* row = z.data.data() + i * c;
    float* dst = out.data() + i * c;
    float mx = -INFINITY;
    for (size_t j = 0; j < c; ++j) mx = std::fmax(mx, row[j]);
    float sum = 0.0f;
    for (size_t j = 0; j < c; ++j) {
      float e = std::exp(row[j] - mx);
      dst[j] = e;
      sum += e;
    }
    for (size_t j = 0; j < c; ++j) dst[j] /= sum;
  }
  return Tensor({r, c}, std::move(out));
}

// tensor.rs:476-493: first maximum wins ties.
// One prediction per chunk of max(c, 1) elements (chunks_exact): with zero
// columns the data is empty and there are no predictions at all.
static std::vector<size_t> argmax_rows(const Tensor& z) {
  size_t c = z.shape[1], r = c == 0 ? 0 : z.shape[0];
  std::vector<size_t> out(r, 0);
  for (size_t i = 0; i < r; ++i) {
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t j = 0; j < c; ++j) {
      float v = z.data[i * c + j];
      if (j == 0 || v > bv) {
        bv = v;
        best = j;
      }
    }
    out[i] = best;
  }
  return out;
}

// ----------------------------------------------------------------- Param / Tape
struct Param {
  size_t id;
  std::string name;
  std::shared_ptr<Tensor> value;
};

static std::mutex g_param_mu;
static size_t g_next_param_id = 0;
static std::unordered_map<size_t, Param> g_params;

static Param& param_ref(size_t id) {
  auto it = g_params.find(id);
  if (it == g_params.end()) throw std::runtime_error("unknown param id");
  return it->second;
}

static size_t param_new(const std::string& name, Tensor v) {
  std::lock_guard<std::mutex> lk(g_param_mu);
  size_t id = g_next_param_id++;
  g_params[id] = Param{id, name, std::make_shared<Tensor>(std::move(v))};
  return id;
}

using Backward = std::function<std::vector<Tensor>(const Tensor&)>;

struct Node {
  std::vector<size_t> parents;
  Backward backward;  // empty for leaves
};

// tape.rs:43-229.  Nodes are pushed in topological order; values live beside
// the nodes (a Var in the reference carries its value, here it is indexed).
struct Tape {
  std::vector<Node> nodes;
  std::vector<Tensor> values;
  std::unordered_map<size_t, size_t> param_nodes;
  std::vector<bool> have_grad;
  std::vector<Tensor> grads;

  size_t push(std::vector<size_t> parents, Backward bw, Tensor value) {
    nodes.push_back(Node{std::move(parents), std::move(bw)});
    values.push_back(std::move(value));
    return nodes.size() - 1;
  }
  size_t constant(Tensor v) { return push({}, nullptr, std::move(v)); }  // tape.rs:70-73
  size_t watch(size_t pid) {                                              // tape.rs:124-131
    auto it = param_nodes.find(pid);
    if (it != param_nodes.end()) return it->second;
    size_t idx = push({}, nullptr, *param_ref(pid).value);
    param_nodes[pid] = idx;
    return idx;
  }
  const Tensor& val(size_t v) const { return values.at(v); }

  size_t unary(size_t a, Tensor value, std::function<Tensor(const Tensor&)> f) {
    return push({a}, [f](const Tensor& g) { return std::vector<Tensor>{f(g)}; }, std::move(value));
  }
  size_t binary(size_t a, size_t b, Tensor value, std::function<std::pair<Tensor, Tensor>(const Tensor&)> f) {
    return push({a, b},
                [f](const Tensor& g) {
                  auto p = f(g);
                  return std::vector<Tensor>{std::move(p.first), std::move(p.second)};
                },
                std::move(value));
  }

  // tape.rs:187-229: seed ones, reverse sweep, in-place axpy accumulation.
  void backward(size_t root) {
    if (!values[root].is_scalar()) throw std::runtime_error("backward() must start at a scalar");
    size_t n = nodes.size();
    grads.assign(n, Tensor());
    have_grad.assign(n, false);
    grads[root] = Tensor::full(values[root].shape, 1.0f);
    have_grad[root] = true;
    for (size_t i = n; i-- > 0;) {
      if (!nodes[i].backward || !have_grad[i]) continue;
      std::vector<Tensor> outs = nodes[i].backward(grads[i]);
      for (size_t q = 0; q < nodes[i].parents.size(); ++q) {
        size_t p = nodes[i].parents[q];
        Tensor& gp = outs[q];
        if (have_grad[p]) {
          if (grads[p].shape == gp.shape) {
            for (size_t e = 0; e < gp.len(); ++e) grads[p].data[e] += gp.data[e];
          } else {
            grads[p] = t_add(grads[p], gp);
          }
        } else {
          grads[p] = std::move(gp);
          have_grad[p] = true;
        }
      }
    }
  }
  const Tensor* grad_of_param(size_t pid) const {
    auto it = param_nodes.find(pid);
    if (it == param_nodes.end() || it->second >= have_grad.size() || !have_grad[it->second]) return nullptr;
    return &grads[it->second];
  }
};

// ----------------------------------------------------------------- ops.rs
enum UnaryOp {
  U_SCALE = 0, U_OFFSET, U_NEG, U_SQUARE, U_SQRT, U_EXP, U_LN, U_RELU, U_LEAKY_RELU,
  U_SIGMOID, U_TANH, U_SUM, U_MEAN, U_SOFTMAX
};
enum BinaryOp { B_ADD = 0, B_SUB, B_MUL, B_DIV, B_MATMUL };

static size_t op_binary(Tape& tp, int op, size_t ia, size_t ib) {
  Tensor a = tp.val(ia), b = tp.val(ib);
  std::vector<size_t> sa = a.shape, sb = b.shape;
  switch (op) {
    case B_ADD:  // ops.rs:49-53
      return tp.binary(ia, ib, t_add(a, b), [sa, sb](const Tensor& g) {
        return std::make_pair(reduce_to(g, sa), reduce_to(g, sb));
      });
    case B_SUB:  // ops.rs:61-65
      return tp.binary(ia, ib, t_sub(a, b), [sa, sb](const Tensor& g) {
        return std::make_pair(reduce_to(g, sa), reduce_to(t_neg(g), sb));
      });
    case B_MUL:  // ops.rs:76-83
      return tp.binary(ia, ib, t_mul(a, b), [a, b, sa, sb](const Tensor& g) {
        return std::make_pair(reduce_to(t_mul(g, b), sa), reduce_to(t_mul(g, a), sb));
      });
    case B_DIV:  // ops.rs:93-102
      return tp.binary(ia, ib, t_div(a, b), [a, b, sa, sb](const Tensor& g) {
        Tensor da = reduce_to(t_div(g, b), sa);
        Tensor db = reduce_to(t_neg(t_div(t_mul(g, a), t_mul(b, b))), sb);
        return std::make_pair(std::move(da), std::move(db));
      });
    case B_MATMUL:  // ops.rs:125-129: both g·Bᵀ and Aᵀ·g, always
      return tp.binary(ia, ib, matmul(a, b), [a, b](const Tensor& g) {
        return std::make_pair(matmul(g, b.t()), matmul(a.t(), g));
      });
  }
  throw std::runtime_error("unknown binary op");
}

static size_t op_unary(Tape& tp, int op, size_t ia, float k) {
  const Tensor x = tp.val(ia);
  std::vector<size_t> shape = x.shape;
  switch (op) {
    case U_SCALE:  // ops.rs:132-135
      return tp.unary(ia, t_scale(x, k), [k](const Tensor& g) { return t_scale(g, k); });
    case U_OFFSET:  // ops.rs:139-142
      return tp.unary(ia, x.map([k](float v) { return v + k; }), [](const Tensor& g) { return g; });
    case U_NEG:  // ops.rs:145-147
      return tp.unary(ia, t_scale(x, -1.0f), [](const Tensor& g) { return t_scale(g, -1.0f); });
    case U_SQUARE:  // ops.rs:150-154
      return tp.unary(ia, x.map([](float v) { return v * v; }),
                      [x](const Tensor& g) { return t_scale(t_mul(g, x), 2.0f); });
    case U_SQRT: {  // ops.rs:158-162
      Tensor out = x.map([](float v) { return std::sqrt(v); });
      Tensor cached = out;
      return tp.unary(ia, std::move(out), [cached](const Tensor& g) { return t_div(g, t_scale(cached, 2.0f)); });
    }
    case U_EXP: {  // ops.rs:166-170
      Tensor out = x.map([](float v) { return std::exp(v); });
      Tensor cached = out;
      return tp.unary(ia, std::move(out), [cached](const Tensor& g) { return t_mul(g, cached); });
    }
    case U_LN:  // ops.rs:176-180
      return tp.unary(ia, x.map([](float v) { return std::log(std::fmax(v, 1e-12f)); }),
                      [x](const Tensor& g) { return t_div(g, x); });
    case U_RELU:  // ops.rs:190-194
      return tp.unary(ia, x.map([](float v) { return std::fmax(v, 0.0f); }), [x](const Tensor& g) {
        return t_mul(g, x.map([](float v) { return v > 0.0f ? 1.0f : 0.0f; }));
      });
    case U_LEAKY_RELU:  // ops.rs:197-203
      return tp.unary(ia, x.map([k](float v) { return v > 0.0f ? v : k * v; }), [x, k](const Tensor& g) {
        return t_mul(g, x.map([k](float v) { return v > 0.0f ? 1.0f : k; }));
      });
    case U_SIGMOID: {  // ops.rs:212-216
      Tensor out = x.map([](float v) { return 1.0f / (1.0f + std::exp(-v)); });
      Tensor cached = out;
      return tp.unary(ia, std::move(out), [cached](const Tensor& g) {
        return t_mul(g, cached.map([](float s) { return s * (1.0f - s); }));
      });
    }
    case U_TANH: {  // ops.rs:223-227
      Tensor out = x.map([](float v) { return std::tanh(v); });
      Tensor cached = out;
      return tp.unary(ia, std::move(out), [cached](const Tensor& g) {
        return t_mul(g, cached.map([](float t) { return 1.0f - t * t; }));
      });
    }
    case U_SUM:  // ops.rs:239-243
      return tp.unary(ia, Tensor::scalar(x.sum_all()),
                      [shape](const Tensor& g) { return Tensor::full(shape, g.item()); });
    case U_MEAN: {  // ops.rs:250-255
      float n = (float)x.len();
      return tp.unary(ia, Tensor::scalar(x.mean_all()),
                      [shape, n](const Tensor& g) { return Tensor::full(shape, g.item() / n); });
    }
    case U_SOFTMAX: {  // ops.rs:291-309
      Tensor out = softmax_rows(x);
      Tensor cached = out;
      return tp.unary(ia, std::move(out), [cached](const Tensor& g) {
        size_t r = cached.shape[0], c = cached.shape[1];
        std::vector<float> data(r * c);
        for (size_t i = 0; i < r; ++i) {
          const float* s = cached.data.data() + i * c;
          const float* gr = g.data.data() + i * c;
          float dot = 0.0f;
          for (size_t j = 0; j < c; ++j) dot += gr[j] * s[j];
          for (size_t j = 0; j < c; ++j) data[i * c + j] = s[j] * (gr[j] - dot);
        }
        return Tensor({r, c}, std::move(data));
      });
    }
  }
  throw std::runtime_error("unknown unary op");
}

// ----------------------------------------------------------------- losses.rs
enum LossKind { L_MSE = 0, L_MAE = 1, L_SOFTMAX_XENT = 2, L_BCE = 3 };

static size_t loss_op(Tape& tp, int kind, size_t pred, const Tensor& target) {
  switch (kind) {
    case L_MSE: {  // losses.rs:31-34: sub -> square -> mean
      size_t t = tp.constant(target);
      size_t d = op_binary(tp, B_SUB, pred, t);
      return op_unary(tp, U_MEAN, op_unary(tp, U_SQUARE, d, 0.0f), 0.0f);
    }
    case L_MAE: {  // losses.rs:46-53
      size_t t = tp.constant(target);
      size_t d = op_binary(tp, B_SUB, pred, t);
      const Tensor& dv = tp.val(d);
      Tensor sign = dv.map([](float v) { return v >= 0.0f ? 1.0f : -1.0f; });
      float value = dv.map([](float v) { return std::fabs(v); }).mean_all();
      float n = (float)dv.len();
      return tp.unary(d, Tensor::scalar(value), [sign, n](const Tensor& g) { return t_scale(sign, g.item() / n); });
    }
    case L_SOFTMAX_XENT: {  // losses.rs:99-115
      const Tensor& z = tp.val(pred);
      if (z.shape != target.shape) throw std::runtime_error("logits and targets differ in shape");
      Tensor probs = softmax_rows(z);
      float batch = (float)z.shape[0];
      float total = 0.0f;
      for (size_t i = 0; i < probs.len(); ++i) {
        float y = target.data[i];
        if (y != 0.0f) total -= y * std::log(std::fmax(probs.data[i], 1e-12f));
      }
      Tensor y = target;
      return tp.unary(pred, Tensor::scalar(total / batch), [probs, y, batch](const Tensor& g) {
        return t_scale(t_sub(probs, y), g.item() / batch);
      });
    }
    case L_BCE: {  // losses.rs:143-162
      Tensor p = tp.val(pred);
      Tensor y = target;
      float batch = (float)p.len();
      const float lo = 1e-7f, hi = 1.0f - 1e-7f;
      float total = 0.0f;
      for (size_t i = 0; i < p.len(); ++i) {
        float c = std::min(std::max(p.data[i], lo), hi);
        float yi = y.data[i];
        total -= yi * std::log(c) + (1.0f - yi) * std::log(1.0f - c);
      }
      return tp.unary(pred, Tensor::scalar(total / batch), [p, y, batch, lo, hi](const Tensor& g) {
        Tensor d = zip(p, y, [lo, hi](float pi, float yi) {
          float c = std::min(std::max(pi, lo), hi);
          return (c - yi) / (c * (1.0f - c));
        });
        return t_scale(d, g.item() / batch);
      });
    }
  }
  throw std::runtime_error("unknown loss");
}

static Tensor one_hot(const uint32_t* labels, size_t n, size_t classes) {  // losses.rs:169-175
  std::vector<float> data(n * classes, 0.0f);
  for (size_t i = 0; i < n; ++i) {
    if (labels[i] >= classes) throw std::runtime_error("label out of range");
    data[i * classes + labels[i]] = 1.0f;
  }
  return Tensor({n, classes}, std::move(data));
}

// ----------------------------------------------------------------- optim.rs
// f32::powi lowers to binary exponentiation from the least significant bit
// (square-and-multiply); restated here so c1/c2 round like the reference's.
static float powi_f32(float a, int b) {
  bool recip = b < 0;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

struct Optimizer {
  int kind = 0;  // 1 = Sgd, 2 = Adam
  float lr = 0, momentum = 0, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f;
  int t = 0;
  std::unordered_map<size_t, Tensor> m, v, velocity;

  // optim.rs:80-114 (Sgd) and 162-198 (Adam).
  void step(const std::vector<size_t>& pids, const Tape& tp) {
    if (kind == 1) {
      for (size_t pid : pids) {
        const Tensor* g = tp.grad_of_param(pid);
        if (!g) continue;
        Tensor& th = *param_ref(pid).value;
        if (momentum == 0.0f) {
          for (size_t i = 0; i < th.len(); ++i) th.data[i] -= g->data[i] * lr;
        } else {
          auto it = velocity.find(pid);
          if (it == velocity.end()) it = velocity.emplace(pid, Tensor::zeros(th.shape)).first;
          Tensor& vel = it->second;
          for (size_t i = 0; i < vel.len(); ++i) vel.data[i] = vel.data[i] * momentum + g->data[i] * lr;
          for (size_t i = 0; i < th.len(); ++i) th.data[i] -= vel.data[i];
        }
      }
      return;
    }
    t += 1;
    float c1 = 1.0f - powi_f32(beta1, t);
    float c2 = 1.0f - powi_f32(beta2, t);
    float inv_c1 = 1.0f / c1, inv_c2 = 1.0f / c2;
    float b1 = beta1, b2 = beta2, omb1 = 1.0f - b1, omb2 = 1.0f - b2;
    for (size_t pid : pids) {
      const Tensor* g = tp.grad_of_param(pid);
      if (!g) continue;
      Tensor& th = *param_ref(pid).value;
      auto im = m.find(pid);
      if (im == m.end()) im = m.emplace(pid, Tensor::zeros(th.shape)).first;
      auto iv = v.find(pid);
      if (iv == v.end()) iv = v.emplace(pid, Tensor::zeros(th.shape)).first;
      float* md = im->second.data.data();
      float* vd = iv->second.data.data();
      for (size_t i = 0; i < th.len(); ++i) {
        float gi = g->data[i];
        md[i] = md[i] * b1 + gi * omb1;
        vd[i] = vd[i] * b2 + (gi * gi) * omb2;
        float m_hat = md[i] * inv_c1;
        float v_hat = vd[i] * inv_c2;
        th.data[i] -= (m_hat / (std::sqrt(v_hat) + eps)) * lr;
      }
    }
  }
};

// ----------------------------------------------------------------- nn.rs
enum Act { A_LINEAR = 0, A_RELU = 1, A_LEAKY = 2, A_SIGMOID = 3, A_TANH = 4 };

struct Dense {
  size_t w, b;
  int act;
  float slope;
};

static size_t apply_act(Tape& tp, const Dense& d, size_t z) {  // nn.rs:52-60
  switch (d.act) {
    case A_LINEAR: return z;
    case A_RELU: return op_unary(tp, U_RELU, z, 0.0f);
    case A_LEAKY: return op_unary(tp, U_LEAKY_RELU, z, d.slope);
    case A_SIGMOID: return op_unary(tp, U_SIGMOID, z, 0.0f);
    case A_TANH: return op_unary(tp, U_TANH, z, 0.0f);
  }
  throw std::runtime_error("unknown activation");
}

// nn.rs:143-149: Z = X·W + 1ₙb (matmul, then broadcast add), A = φ(Z)
static size_t dense_forward(Tape& tp, const Dense& d, size_t x) {
  size_t w = tp.watch(d.w);
  size_t b = tp.watch(d.b);
  size_t z = op_binary(tp, B_ADD, op_binary(tp, B_MATMUL, x, w), b);
  return apply_act(tp, d, z);
}

// A Sequential of Dense layers with an optimizer: the CPU training step that
// the GPU plan is compared with (tests/gpu.rs:72-76, 116-121).
struct Mlp {
  std::vector<Dense> layers;
  Optimizer opt;
  std::unique_ptr<Tape> last;
  size_t last_logits = 0;

  std::vector<size_t> params() const {  // nn.rs:190-192: [W¹, b¹, W², b², …]
    std::vector<size_t> out;
    for (const Dense& d : layers) {
      out.push_back(d.w);
      out.push_back(d.b);
    }
    return out;
  }
};

}  // namespace oc

// =================================================================== C ABI
using namespace oc;

#define OC_TRY(expr)            \
  try {                         \
    expr;                       \
  } catch (const std::exception& e) { \
    oc::g_err = e.what();       \
    return -1;                  \
  }

extern "C" {

const char* ocpu_last_error(void) { return oc::g_err.c_str(); }
void ocpu_set_threads(int n) { oc::g_threads = n < 1 ? 1 : n; }
int ocpu_get_threads(void) { return oc::g_threads; }

// ---- Rng
void* ocpu_rng_new(uint64_t seed) { return new Rng(seed); }
void ocpu_rng_free(void* r) { delete static_cast<Rng*>(r); }
uint64_t ocpu_rng_next_u64(void* r) { return static_cast<Rng*>(r)->next_u64(); }
float ocpu_rng_uniform(void* r) { return static_cast<Rng*>(r)->uniform(); }
float ocpu_rng_range(void* r, float lo, float hi) { return static_cast<Rng*>(r)->range(lo, hi); }
float ocpu_rng_normal(void* r) { return static_cast<Rng*>(r)->normal(); }
uint64_t ocpu_rng_below(void* r, uint64_t n) { return static_cast<Rng*>(r)->below(n); }
void ocpu_rng_fill_normal(void* r, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = static_cast<Rng*>(r)->normal();
}
void ocpu_rng_fill_range(void* r, float* out, size_t n, float lo, float hi) {
  for (size_t i = 0; i < n; ++i) out[i] = static_cast<Rng*>(r)->range(lo, hi);
}
void ocpu_rng_fill_below(void* r, uint32_t* out, size_t n, uint64_t c) {
  for (size_t i = 0; i < n; ++i) out[i] = (uint32_t) static_cast<Rng*>(r)->below(c);
}
float ocpu_powi(float a, int b) { return powi_f32(a, b); }

// ---- Tensor kernels on raw row-major arrays
int ocpu_matmul(const float* a, const float* b, float* c, size_t m, size_t k, size_t n) {
  OC_TRY(matmul_raw(a, b, c, m, k, n, oc::g_threads));
  return 0;
}
int ocpu_transpose(const float* a, float* out, size_t r, size_t c) {
  OC_TRY({
    Tensor t({r, c}, std::vector<float>(a, a + r * c));
    Tensor tt = t.t();
    std::memcpy(out, tt.data.data(), r * c * sizeof(float));
  });
  return 0;
}
int ocpu_softmax_rows(const float* z, float* out, size_t r, size_t c) {
  OC_TRY({
    Tensor s = softmax_rows(Tensor({r, c}, std::vector<float>(z, z + r * c)));
    std::memcpy(out, s.data.data(), r * c * sizeof(float));
  });
  return 0;
}
// reduce_to for rank-2 sources: target [1,c] (column sums) or [r,1] (row sums)
int ocpu_reduce_to(const float* g, size_t r, size_t c, size_t t0, size_t t1, float* out) {
  OC_TRY({
    Tensor res = reduce_to(Tensor({r, c}, std::vector<float>(g, g + r * c)), {t0, t1});
    std::memcpy(out, res.data.data(), res.len() * sizeof(float));
  });
  return 0;
}
int ocpu_argmax_rows(const float* z, size_t r, size_t c, uint32_t* out) {
  OC_TRY({
    auto v = argmax_rows(Tensor({r, c}, std::vector<float>(z, z + r * c)));
    if (v.size() != r) throw std::runtime_error("argmax_rows: zero columns give no predictions");
    for (size_t i = 0; i < r; ++i) out[i] = (uint32_t)v[i];
  });
  return 0;
}
// losses.rs:181-185
float ocpu_accuracy(const float* z, size_t r, size_t c, const uint32_t* labels) {
  auto v = argmax_rows(Tensor({r, c}, std::vector<float>(z, z + r * c)));
  size_t hits = 0;  // zip of predictions and labels: the shorter one ends it
  for (size_t i = 0; i < v.size(); ++i) hits += (v[i] == labels[i]);
  return (float)hits / (float)r;
}
int ocpu_one_hot(const uint32_t* labels, size_t n, size_t classes, float* out) {
  OC_TRY({
    Tensor t = one_hot(labels, n, classes);
    std::memcpy(out, t.data.data(), t.len() * sizeof(float));
  });
  return 0;
}

// ---- Params (tape.rs:76-132)
int64_t ocpu_param_new(const size_t* shape, int rank, const float* data) {
  try {
    std::vector<size_t> s(shape, shape + rank);
    size_t n = 1;
    for (size_t v : s) n *= v;
    return (int64_t)param_new("p", Tensor(s, std::vector<float>(data, data + n)));
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return -1;
  }
}
int ocpu_param_get(int64_t pid, float* out) {
  OC_TRY({
    const Tensor& t = *param_ref((size_t)pid).value;
    std::memcpy(out, t.data.data(), t.len() * sizeof(float));
  });
  return 0;
}
int ocpu_param_set(int64_t pid, const float* data) {
  OC_TRY({
    Tensor& t = *param_ref((size_t)pid).value;
    std::memcpy(t.data.data(), data, t.len() * sizeof(float));
  });
  return 0;
}
int64_t ocpu_param_len(int64_t pid) {
  try {
    return (int64_t)param_ref((size_t)pid).value->len();
  } catch (...) {
    return -1;
  }
}
void ocpu_param_free(int64_t pid) {
  std::lock_guard<std::mutex> lk(g_param_mu);
  g_params.erase((size_t)pid);
}
// nn.rs:122-130: Glorot uniform, λ = sqrt(6/(d+m)), W drawn row-major, b = 0.
int ocpu_dense_new(size_t inputs, size_t units, void* rng, int64_t* w_out, int64_t* b_out) {
  OC_TRY({
    float limit = std::sqrt(6.0f / (float)(inputs + units));
    std::vector<float> w(inputs * units);
    for (float& v : w) v = static_cast<Rng*>(rng)->range(-limit, limit);
    *w_out = (int64_t)param_new("W", Tensor({inputs, units}, std::move(w)));
    *b_out = (int64_t)param_new("b", Tensor::zeros({1, units}));
  });
  return 0;
}

// ---- Tape interpreter (tape.rs / ops.rs / losses.rs)
void* ocpu_tape_new(void) { return new Tape(); }
void ocpu_tape_free(void* t) { delete static_cast<Tape*>(t); }
int64_t ocpu_var_constant(void* t, const size_t* shape, int rank, const float* data) {
  try {
    std::vector<size_t> s(shape, shape + rank);
    size_t n = 1;
    for (size_t v : s) n *= v;
    return (int64_t) static_cast<Tape*>(t)->constant(Tensor(s, std::vector<float>(data, data + n)));
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return -1;
  }
}
int64_t ocpu_var_watch(void* t, int64_t pid) {
  try {
    return (int64_t) static_cast<Tape*>(t)->watch((size_t)pid);
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return -1;
  }
}
int64_t ocpu_var_unary(void* t, int op, int64_t a, float k) {
  try {
    return (int64_t)op_unary(*static_cast<Tape*>(t), op, (size_t)a, k);
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return -1;
  }
}
int64_t ocpu_var_binary(void* t, int op, int64_t a, int64_t b) {
  try {
    return (int64_t)op_binary(*static_cast<Tape*>(t), op, (size_t)a, (size_t)b);
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return -1;
  }
}
int64_t ocpu_var_loss(void* t, int kind, int64_t pred, const size_t* shape, int rank, const float* target) {
  try {
    std::vector<size_t> s(shape, shape + rank);
    size_t n = 1;
    for (size_t v : s) n *= v;
    return (int64_t)loss_op(*static_cast<Tape*>(t), kind, (size_t)pred, Tensor(s, std::vector<float>(target, target + n)));
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return -1;
  }
}
int ocpu_var_shape(void* t, int64_t v, size_t* shape, int* rank) {
  OC_TRY({
    const Tensor& x = static_cast<Tape*>(t)->val((size_t)v);
    *rank = (int)x.rank();
    for (size_t i = 0; i < x.rank(); ++i) shape[i] = x.shape[i];
  });
  return 0;
}
int ocpu_var_value(void* t, int64_t v, float* out) {
  OC_TRY({
    const Tensor& x = static_cast<Tape*>(t)->val((size_t)v);
    std::memcpy(out, x.data.data(), x.len() * sizeof(float));
  });
  return 0;
}
int ocpu_backward(void* t, int64_t root) {
  OC_TRY(static_cast<Tape*>(t)->backward((size_t)root));
  return 0;
}
// 1 if the param has a gradient in this tape (copied to out), 0 if not.
int ocpu_grad_of_param(void* t, int64_t pid, float* out) {
  try {
    const Tensor* g = static_cast<Tape*>(t)->grad_of_param((size_t)pid);
    if (!g) return 0;
    std::memcpy(out, g->data.data(), g->len() * sizeof(float));
    return 1;
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return -1;
  }
}

// ---- Optimizers (optim.rs)
void* ocpu_opt_new(int kind, float lr, float a, float b) {
  auto* o = new Optimizer();
  o->kind = kind;
  o->lr = lr;
  if (kind == 1) o->momentum = a;
  if (kind == 2) {
    o->beta1 = a;
    o->beta2 = b;
  }
  return o;
}
void ocpu_opt_free(void* o) { delete static_cast<Optimizer*>(o); }
int ocpu_opt_step(void* o, void* tape, const int64_t* pids, size_t n) {
  OC_TRY({
    std::vector<size_t> p(n);
    for (size_t i = 0; i < n; ++i) p[i] = (size_t)pids[i];
    static_cast<Optimizer*>(o)->step(p, *static_cast<Tape*>(tape));
  });
  return 0;
}

// ---- MLP training step (the oracle for the GPU plan)
// dims[0..n_layers]; weights[l] is [dims[l], dims[l+1]] row-major, biases[l] is [1, dims[l+1]].
void* ocpu_mlp_new(int n_layers, const size_t* dims, const int* acts, const float* const* weights,
                   const float* const* biases) {
  try {
    auto* m = new Mlp();
    for (int l = 0; l < n_layers; ++l) {
      size_t din = dims[l], dout = dims[l + 1];
      Dense d;
      d.w = param_new("W", Tensor({din, dout}, std::vector<float>(weights[l], weights[l] + din * dout)));
      d.b = param_new("b", Tensor({1, dout}, std::vector<float>(biases[l], biases[l] + dout)));
      d.act = acts[l];
      d.slope = 0.01f;
      m->layers.push_back(d);
    }
    return m;
  } catch (const std::exception& e) {
    oc::g_err = e.what();
    return nullptr;
  }
}
void ocpu_mlp_free(void* p) {
  auto* m = static_cast<Mlp*>(p);
  if (!m) return;
  for (size_t pid : m->params()) ocpu_param_free((int64_t)pid);
  delete m;
}
// kind 0: no update (gradients only), 1: Sgd(lr, momentum=a), 2: Adam(lr, β1=a, β2=b)
int ocpu_mlp_set_optimizer(void* p, int kind, float lr, float a, float b) {
  auto* m = static_cast<Mlp*>(p);
  m->opt = Optimizer();
  m->opt.kind = kind;
  m->opt.lr = lr;
  if (kind == 1) m->opt.momentum = a;
  if (kind == 2) {
    m->opt.beta1 = a;
    m->opt.beta2 = b;
  }
  return 0;
}
// One step on a batch: tape forward, softmax cross-entropy over one_hot(labels),
// backward, optimizer update (tests/gpu.rs:116-121).  Returns the loss in *loss.
int ocpu_mlp_step(void* p, const float* x, size_t batch, const uint32_t* labels, float* loss) {
  auto* m = static_cast<Mlp*>(p);
  OC_TRY({
    size_t din = param_ref(m->layers[0].w).value->shape[0];
    size_t classes = param_ref(m->layers.back().w).value->shape[1];
    m->last.reset(new Tape());
    Tape& tp = *m->last;
    size_t h = tp.constant(Tensor({batch, din}, std::vector<float>(x, x + batch * din)));
    for (const Dense& d : m->layers) h = dense_forward(tp, d, h);
    m->last_logits = h;
    size_t l = loss_op(tp, L_SOFTMAX_XENT, h, one_hot(labels, batch, classes));
    *loss = tp.val(l).item();
    tp.backward(l);
    if (m->opt.kind != 0) m->opt.step(m->params(), tp);
  });
  return 0;
}
// Forward only (Sequential::predict, nn.rs:184-188): logits [batch, classes].
int ocpu_mlp_forward(void* p, const float* x, size_t batch, float* logits) {
  auto* m = static_cast<Mlp*>(p);
  OC_TRY({
    size_t din = param_ref(m->layers[0].w).value->shape[0];
    Tape tp;
    size_t h = tp.constant(Tensor({batch, din}, std::vector<float>(x, x + batch * din)));
    for (const Dense& d : m->layers) h = dense_forward(tp, d, h);
    const Tensor& z = tp.val(h);
    std::memcpy(logits, z.data.data(), z.len() * sizeof(float));
  });
  return 0;
}
// The optimizer's per-parameter state map that `which` names: 2 = Adam m or
// Sgd velocity, 3 = Adam v (optim.rs:100-103, 143-149: keyed by the param,
// created as zeros on its first update).
static std::unordered_map<size_t, Tensor>& opt_state_map(Mlp* m, int which) {
  if (which == 2) return m->opt.kind == 1 ? m->opt.velocity : m->opt.m;
  if (which == 3) return m->opt.v;
  throw std::runtime_error("unknown state kind");
}
// which: 0 = parameter value, 1 = gradient of the last step, 2 = Adam m (Sgd
// velocity), 3 = Adam v (zeros before the parameter's first update); idx over
// [W¹, b¹, …].
int ocpu_mlp_get(void* p, int which, int idx, float* out) {
  auto* m = static_cast<Mlp*>(p);
  OC_TRY({
    std::vector<size_t> ps = m->params();
    size_t pid = ps.at((size_t)idx);
    const Tensor& th = *param_ref(pid).value;
    if (which == 0) {
      std::memcpy(out, th.data.data(), th.len() * sizeof(float));
    } else if (which == 1) {
      if (!m->last) throw std::runtime_error("no step has run");
      const Tensor* g = m->last->grad_of_param(pid);
      if (!g) throw std::runtime_error("parameter has no gradient");
      std::memcpy(out, g->data.data(), g->len() * sizeof(float));
    } else {
      auto& st = opt_state_map(m, which);
      auto it = st.find(pid);
      if (it == st.end()) std::memset(out, 0, th.len() * sizeof(float));
      else std::memcpy(out, it->second.data.data(), th.len() * sizeof(float));
    }
  });
  return 0;
}
// The inverse for which = 0 (Param::set, tape.rs:119-121), 2 and 3.
int ocpu_mlp_set(void* p, int which, int idx, const float* in) {
  auto* m = static_cast<Mlp*>(p);
  OC_TRY({
    std::vector<size_t> ps = m->params();
    size_t pid = ps.at((size_t)idx);
    Tensor& th = *param_ref(pid).value;
    if (which == 0) {
      std::memcpy(th.data.data(), in, th.len() * sizeof(float));
    } else if (which == 2 || which == 3) {
      Tensor t(th.shape, std::vector<float>(in, in + th.len()));
      opt_state_map(m, which)[pid] = std::move(t);
    } else {
      throw std::runtime_error("gradients cannot be set");
    }
  });
  return 0;
}
// Adam's step count t (optim.rs:163).
int ocpu_mlp_get_t(void* p) { return static_cast<Mlp*>(p)->opt.t; }
void ocpu_mlp_set_t(void* p, int t) { static_cast<Mlp*>(p)->opt.t = t; }
int ocpu_mlp_logits(void* p, float* out) {
  auto* m = static_cast<Mlp*>(p);
  OC_TRY({
    if (!m->last) throw std::runtime_error("no step has run");
    const Tensor& z = m->last->val(m->last_logits);
    std::memcpy(out, z.data.data(), z.len() * sizeof(float));
  });
  return 0;
}

}  // extern "C"
